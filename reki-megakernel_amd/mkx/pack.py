"""Offline weight packer for the expert megakernel, and its on-disk layout (safetensors).

A packed expert holds exactly what ``mkx_create`` takes, under the field names of ``mkx_weights``:

=================  ==============================  ===========================================
tensor             shape                           dtype
=================  ==============================  ===========================================
wqkv               [L, 3H, H]  (rows q; k; v)      F8_E4M3 or BF16
wo, wqca, woca     [L, H, H]                       F8_E4M3 or BF16
wg, wu             [L, I, H]                       F8_E4M3 or BF16
wd                 [L, H, I]                       F8_E4M3 or BF16
<w>_scale          [L, N]  (fp8 only)              F32, per output channel: w[l, n, k] ~ q * s[l, n]
qn, kn, qcan       [L, HD]                         BF16 (q/k RMSNorm weights, used as 1 + w)
win                [A, H]  (action_in_proj^T)      F32
bin                [H]                             F32
wout               [A, H]                          F32
bout               [A]                             F32
reg_tok (opt.)     [R, H]                          BF16 register tokens
=================  ==============================  ===========================================

Linear stacks are [L, out, in] with q; k; v concatenated along out, the order the reference stacks its
weights in (src/mk_expert.py:445-460), so ``mkx_create`` reads a loaded file without a copy. The file's
metadata (strings) carries ``format`` = ``mkx-expert/1``, the shapes (L, H, NH, HD, I, A), ``eps``,
``qk_eps``, ``activation`` (``silu`` | ``gelu_tanh``) and ``weight_dtype`` (``bf16`` | ``fp8_e4m3``).

fp8 quantisation is e4m3 (OCP "fn": max 448, no infinities) with one fp32 scale per output channel,
``scale = max_k |w[n, k]| / 448`` and ``q = rne_e4m3(w / scale)``: the largest magnitude of a row maps to
+-448 exactly, and a zero row gets scale 1e-12 / 448 with all-zero codes.
"""
from __future__ import annotations

import json
from dataclasses import dataclass, field

import torch

FORMAT = "mkx-expert/1"
LINEARS = ("wqkv", "wo", "wqca", "woca", "wg", "wu", "wd")
E4M3_MAX = 448.0

# model attribute paths of each stack's linears, in concatenation order
_LIN_PATHS = {
    "wqkv": (("self_attn", "q_proj"), ("self_attn", "k_proj"), ("self_attn", "v_proj")),
    "wo": (("self_attn", "o_proj"),), "wqca": (("cross_attn", "q_proj"),), "woca": (("cross_attn", "o_proj"),),
    "wg": (("mlp", "gate_proj"),), "wu": (("mlp", "up_proj"),), "wd": (("mlp", "down_proj"),),
}


def quantize_e4m3(w: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel e4m3 quantisation of w [..., N, K]: returns (q [..., N, K] float8_e4m3fn,
    scale [..., N] fp32) with w ~ q * scale[..., None] (round to nearest even in w / scale)."""
    wf = w.float()
    scale = wf.abs().amax(-1, keepdim=True).clamp_min(1e-12) / E4M3_MAX
    q = (wf / scale).to(torch.float8_e4m3fn)
    return q, scale.squeeze(-1)


def dequantize_e4m3(q: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """q [..., N, K] e4m3 with scale [..., N] -> fp32 weights (what the kernel multiplies with)."""
    return q.to(torch.float32) * scale.float()[..., None]


@dataclass
class PackedExpert:
    """Stacked expert weights in the on-disk layout plus their metadata."""

    tensors: dict = field(default_factory=dict)
    meta: dict = field(default_factory=dict)

    @property
    def fp8(self) -> bool:
        return self.meta["weight_dtype"] == "fp8_e4m3"

    def to(self, device) -> "PackedExpert":
        return PackedExpert({k: v.to(device) for k, v in self.tensors.items()}, dict(self.meta))

    def dequantized(self, name: str) -> torch.Tensor:
        """Stack ``name`` (one of LINEARS) as fp32 [L, N, K], as the kernel sees it."""
        t = self.tensors[name]
        return dequantize_e4m3(t, self.tensors[name + "_scale"]) if self.fp8 else t.float()


def _get(mod, path):
    for p in path:
        mod = getattr(mod, p)
    return mod


def _activation_name(act) -> str:
    if isinstance(act, torch.nn.SiLU) or type(act).__name__ in ("SiLU", "SiLUActivation"):
        return "silu"
    if isinstance(act, torch.nn.GELU) and getattr(act, "approximate", "none") == "tanh":
        return "gelu_tanh"
    raise ValueError(f"unsupported MLP activation {type(act).__name__}")


def _has_fp8(lin) -> bool:
    q = getattr(lin, "weight_q", None)
    return q is not None and q.dtype == torch.float8_e4m3fn


def pack_expert(model, weight_dtype: str | None = None) -> PackedExpert:
    """Stack a REKI-shaped model's expert weights (on the model's device) into the packed layout.

    ``weight_dtype`` None keeps the model's own: fp8 when its linears carry ``weight_q`` (float8_e4m3fn) and
    ``weight_scale`` beside ``weight``, else bf16. ``"fp8_e4m3"`` uses those when present and otherwise
    quantises each linear's ``weight`` with ``quantize_e4m3`` (per linear, so q, k and v keep their own
    per-row scales); ``"bf16"`` stacks ``weight`` rounded to bf16. Shapes and eps values are read off the
    model as the reference reads them (src/mk_expert.py:438-464)."""
    vwe = model.vlm_with_expert
    layers = list(vwe.action_expert.layers)
    sa0 = layers[0].self_attn
    L, NH, HD = len(layers), sa0.n_q_heads, sa0.head_dim
    H = NH * HD
    I = layers[0].mlp.gate_proj.out_features  # noqa: E741
    A = model.action_in_proj.in_features
    if sa0.n_kv_heads != NH or layers[0].cross_attn.n_kv_heads != NH:
        raise ValueError("the megakernel implements multi-head attention only (n_kv_heads == n_q_heads)")
    eps = float(layers[0].input_layernorm.eps)
    if float(vwe.action_expert.norm.eps) != eps:
        raise ValueError("final norm eps differs from the layer norm eps")
    model_fp8 = _has_fp8(layers[0].self_attn.q_proj)
    wd = weight_dtype or ("fp8_e4m3" if model_fp8 else "bf16")
    if wd not in ("bf16", "fp8_e4m3"):
        raise ValueError(f"weight_dtype must be 'bf16' or 'fp8_e4m3', got {wd!r}")
    t = {}
    for name, paths in _LIN_PATHS.items():
        if wd == "fp8_e4m3":
            qs, ss = [], []
            for lay in layers:
                ql, sl = [], []
                for p in paths:
                    lin = _get(lay, p)
                    if _has_fp8(lin):
                        q, s = lin.weight_q.detach(), lin.weight_scale.detach().float().reshape(-1)
                    else:
                        q, s = quantize_e4m3(lin.weight.detach())
                    ql.append(q)
                    sl.append(s)
                qs.append(torch.cat(ql, 0))
                ss.append(torch.cat(sl, 0))
            t[name] = torch.stack(qs).contiguous()
            t[name + "_scale"] = torch.stack(ss).contiguous()
        else:
            t[name] = torch.stack([torch.cat([_get(lay, p).weight.detach() for p in paths], 0)
                                   for lay in layers]).to(torch.bfloat16).contiguous()
    for name, path in (("qn", ("self_attn", "q_norm")), ("kn", ("self_attn", "k_norm")), ("qcan", ("cross_attn", "q_norm"))):
        t[name] = torch.stack([_get(lay, path).weight.detach() for lay in layers]).to(torch.bfloat16).contiguous()
    t["win"] = model.action_in_proj.weight.detach().float().t().contiguous()  # [A, H]
    t["bin"] = model.action_in_proj.bias.detach().float().contiguous()
    t["wout"] = model.action_out_proj.weight.detach().float().contiguous()
    t["bout"] = model.action_out_proj.bias.detach().float().contiguous()
    reg = getattr(model, "register_tokens", None)
    if reg is not None:
        t["reg_tok"] = reg.detach().to(torch.bfloat16).contiguous()
    meta = {"format": FORMAT, "L": L, "H": H, "NH": NH, "HD": HD, "I": I, "A": A, "eps": eps,
            "qk_eps": float(sa0.q_norm.eps), "activation": _activation_name(layers[0].mlp.act_fn), "weight_dtype": wd}
    out = PackedExpert(t, meta)
    validate(out)
    return out


def validate(p: PackedExpert) -> None:
    """Raise ValueError unless every tensor of the layout is present with its shape and dtype."""
    m = p.meta
    if m.get("format") != FORMAT:
        raise ValueError(f"not an {FORMAT} file (format = {m.get('format')!r})")
    L, H, NH, HD, I, A = (int(m[k]) for k in ("L", "H", "NH", "HD", "I", "A"))  # noqa: E741
    if NH * HD != H:
        raise ValueError("H must equal NH * HD")
    if m["activation"] not in ("silu", "gelu_tanh") or m["weight_dtype"] not in ("bf16", "fp8_e4m3"):
        raise ValueError("unknown activation or weight dtype")
    wdt = torch.float8_e4m3fn if m["weight_dtype"] == "fp8_e4m3" else torch.bfloat16
    want = {"wqkv": ((L, 3 * H, H), wdt), "wo": ((L, H, H), wdt), "wqca": ((L, H, H), wdt), "woca": ((L, H, H), wdt),
            "wg": ((L, I, H), wdt), "wu": ((L, I, H), wdt), "wd": ((L, H, I), wdt),
            "qn": ((L, HD), torch.bfloat16), "kn": ((L, HD), torch.bfloat16), "qcan": ((L, HD), torch.bfloat16),
            "win": ((A, H), torch.float32), "bin": ((H,), torch.float32), "wout": ((A, H), torch.float32),
            "bout": ((A,), torch.float32)}
    if wdt == torch.float8_e4m3fn:
        for n in LINEARS:
            want[n + "_scale"] = ((L, want[n][0][1]), torch.float32)
    for k, (shape, dt) in want.items():
        v = p.tensors.get(k)
        if v is None:
            raise ValueError(f"packed expert lacks {k}")
        if tuple(v.shape) != shape or v.dtype != dt:
            raise ValueError(f"{k}: expected {shape} {dt}, got {tuple(v.shape)} {v.dtype}")
    extra = set(p.tensors) - set(want) - {"reg_tok"}
    if extra:
        raise ValueError(f"unknown tensors in packed expert: {sorted(extra)}")
    r = p.tensors.get("reg_tok")
    if r is not None and (r.dim() != 2 or r.shape[1] != H or r.dtype != torch.bfloat16):
        raise ValueError("reg_tok must be [R, H] bf16")


def save_packed(p: PackedExpert, path: str) -> None:
    """Write the packed expert as one safetensors file (tensors moved to the CPU)."""
    from safetensors.torch import save_file

    validate(p)
    save_file({k: v.detach().cpu().contiguous() for k, v in p.tensors.items()}, path,
              metadata={k: json.dumps(v) for k, v in p.meta.items()})


def load_packed(path: str, device="cpu") -> PackedExpert:
    """Read a file written by ``save_packed`` (safetensors: no code runs from the file) onto ``device``."""
    from safetensors import safe_open

    with safe_open(path, framework="pt", device="cpu") as f:
        meta = {k: json.loads(v) for k, v in (f.metadata() or {}).items()}
        tensors = {k: f.get_tensor(k) for k in f.keys()}
    p = PackedExpert(tensors, meta)
    validate(p)
    return p.to(device) if str(device) != "cpu" else p


def attach_fp8(model, p: PackedExpert) -> None:
    """Give each expert linear of ``model`` the ``weight_q`` / ``weight_scale`` of a packed fp8 expert
    (on the model's device), so ``ExpertMegakernel(model)`` and ``install(model)`` run in fp8."""
    if not p.fp8:
        raise ValueError("the packed expert holds bf16 weights")
    layers = list(model.vlm_with_expert.action_expert.layers)
    if len(layers) != int(p.meta["L"]):
        raise ValueError("layer count differs from the packed expert")
    for name, paths in _LIN_PATHS.items():
        for l, lay in enumerate(layers):
            row = 0
            for path in paths:
                lin = _get(lay, path)
                n = lin.out_features if hasattr(lin, "out_features") else lin.weight.shape[0]
                dev = lin.weight.device
                lin.weight_q = p.tensors[name][l, row: row + n].to(dev).contiguous()
                lin.weight_scale = p.tensors[name + "_scale"][l, row: row + n].to(dev).contiguous()
                row += n
            if row != p.tensors[name].shape[1]:
                raise ValueError(f"{name}: model rows {row} differ from the packed {p.tensors[name].shape[1]}")
