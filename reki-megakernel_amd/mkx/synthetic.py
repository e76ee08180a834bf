"""A REKI-shaped flow-matching action expert with random weights, and the parts of REKI's expert call
that run outside the megakernel (step modulations, cache preparation, Euler step 1).

REKI itself (kyutai-labs/reki @ b2a3393) is not available offline, so this module defines the model
the megakernel is measured on. Its attribute tree matches what the reference's ExpertMegakernel reads
(src/mk_expert.py:437-463): ``model.vlm_with_expert.action_expert.layers[l].{self_attn, cross_attn, mlp,
input_layernorm}``, ``action_expert.norm``, ``model.action_in_proj``, ``model.action_out_proj``; and its
methods have the names and argument order of the REKI calls the reference makes
(``_step_modulations``, ``_expert_first_step``, ``_expert_actions``; src/mk_expert.py:527-533,
test_mk.py:31-32). ``register_prepare`` builds the ``past`` object whose fields the reference's
``ExpertMegakernel.run`` consumes (src/mk_expert.py:486-496).

Weights are drawn from N(0, 0.02) with a seeded CPU generator and rounded to bf16 (the action
projections are kept as bf16-valued fp32 like the reference's ``.float()`` copies, :457-460). The
modulations and the cache preparation are plain PyTorch (library GEMMs) on the caller's device; the
expert layers themselves only ever run in the HIP megakernel.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field, replace

import torch
import torch.nn.functional as F

from . import _lib
from .pack import dequantize_e4m3, quantize_e4m3


@dataclass(frozen=True)
class ExpertConfig:
    """Shapes of the expert and of one call. ``R_reg`` register rows ride along with the ``T_act``
    action rows in every Euler step when ``registers_in_loop`` (the 42-row layout); otherwise only
    Euler step 1 carries them (the reference's 10-row layout, src/mk_expert.py:466, 488)."""
    L: int = 10
    H: int = 768
    NH: int = 12
    HD: int = 64
    I: int = 3072
    A: int = 32
    action_dim: int = 7
    T_act: int = 10
    R_reg: int = 32
    registers_in_loop: bool = True
    PM: int = 96
    kv_start: int = 0
    S: int = 300
    SP: int = 300
    B: int = 1
    ctx_dim: int = 2048
    tdim: int = 256
    num_steps: int = 10
    eps: float = 1e-6
    qk_eps: float = 1e-6
    act: str = "silu"
    weight_dtype: str = "bf16"  # or "fp8_e4m3"

    @property
    def modw(self) -> int:
        return 9 * self.L * self.H + 2 * self.H

    @property
    def m_q(self) -> int:
        """Own rows per sample in Euler steps 2..N."""
        return self.T_act + (self.R_reg if self.registers_in_loop else 0)

    @property
    def m_q_first(self) -> int:
        """Own rows per sample in Euler step 1 (always carries the register rows)."""
        return self.T_act + self.R_reg


# Named workloads (sizes as the workload list states them).
WORKLOADS = {
    # b1, L10 H768, 10 action + 32 register rows, 96 memory rows, 300 source rows
    "A": ExpertConfig(),
    # the reference's own layout: 10 action rows in steps 2..N, 2 valid memory frames of 3
    "A-ref": ExpertConfig(registers_in_loop=False, kv_start=32, S=182, SP=256),
    # 8 independent chunks
    "B": ExpertConfig(B=8),
    # long context: 1024 source rows, 8 memory frames
    "C": ExpertConfig(S=1024, SP=1024, PM=256),
    # wider fp8 expert, 50 action rows
    "D": ExpertConfig(L=16, H=1024, NH=16, I=4096, T_act=50, weight_dtype="fp8_e4m3"),
    "D-b4": ExpertConfig(L=16, H=1024, NH=16, I=4096, T_act=50, weight_dtype="fp8_e4m3", B=4),
}


def algorithmic_bytes_per_step(cfg: ExpertConfig) -> int:
    """Unique bytes one Euler step must read: linear weights + CA K/V + memory K/V + modulations +
    action projections (activations are negligible)."""
    wbytes = 1 if cfg.weight_dtype == "fp8_e4m3" else 2
    w = cfg.L * (6 * cfg.H * cfg.H + 3 * cfg.H * cfg.I) * wbytes
    if cfg.weight_dtype == "fp8_e4m3":
        w += cfg.L * (6 * cfg.H + 2 * cfg.I) * 4  # per-output-channel scales
    ca = cfg.B * 2 * cfg.L * cfg.S * cfg.H * 2
    mem = cfg.B * 2 * cfg.L * (cfg.PM - cfg.kv_start) * cfg.H * 2
    mods = cfg.B * cfg.modw * 4
    proj = 2 * cfg.A * cfg.H * 4
    return w + ca + mem + mods + proj


def flops_per_step(cfg: ExpertConfig) -> int:
    m = cfg.B * cfg.m_q
    lin = 2 * m * cfg.L * (6 * cfg.H * cfg.H + 3 * cfg.H * cfg.I)
    att = 4 * cfg.B * cfg.L * cfg.m_q * ((cfg.PM - cfg.kv_start) + cfg.m_q + cfg.S) * cfg.H
    return lin + att


# ------------------------------------------------------------------------------------------------
# weights


def _e4m3_round(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float8_e4m3fn).to(torch.float32)


def make_weights(cfg: ExpertConfig, seed: int = 0) -> dict:
    """Random-init weights, N(0, 0.02), CPU. Linear weights bf16 (or e4m3 values with per-output-
    channel fp32 scales absmax/448 for ``fp8_e4m3``, stored as ``<name>_q`` / ``<name>_scale`` beside the
    dequantised bf16-exact copy used by the oracle). Order of draws is fixed."""
    g = torch.Generator().manual_seed(seed)
    H, I, HD, L = cfg.H, cfg.I, cfg.HD, cfg.L

    def n(*shape):
        return torch.randn(*shape, generator=g) * 0.02

    def lin(*shape):
        w = n(*shape)
        if cfg.weight_dtype == "fp8_e4m3":
            q, scale = quantize_e4m3(w)
            return {"w": dequantize_e4m3(q, scale), "q": q, "scale": scale}
        return {"w": w.to(torch.bfloat16)}

    layers = []
    for _ in range(L):
        ly = {}
        for name, shape in (("q", (H, H)), ("k", (H, H)), ("v", (H, H)), ("o", (H, H)),
                            ("ca_q", (H, H)), ("ca_o", (H, H)), ("gate", (I, H)), ("up", (I, H)), ("down", (H, I))):
            r = lin(*shape)
            ly[name] = r["w"]
            if "q" in r:
                ly[name + "_q"], ly[name + "_scale"] = r["q"], r["scale"]
        ly["ca_k"] = n(H, cfg.ctx_dim).to(torch.bfloat16)
        ly["ca_v"] = n(H, cfg.ctx_dim).to(torch.bfloat16)
        for nm in ("q_norm", "k_norm", "ca_q_norm", "ca_k_norm"):
            ly[nm] = n(HD).to(torch.bfloat16)
        layers.append(ly)
    bf = lambda t: t.to(torch.bfloat16).to(torch.float32)  # noqa: E731
    W = {
        "layers": layers,
        "in_w": bf(n(H, cfg.A)), "in_b": bf(n(H)), "out_w": bf(n(cfg.A, H)), "out_b": bf(n(cfg.A)),
        "reg_tok": n(cfg.R_reg, H).to(torch.bfloat16),
        "t1_w": n(H, cfg.tdim).to(torch.bfloat16), "t1_b": n(H).to(torch.bfloat16),
        "t2_w": n(H, H).to(torch.bfloat16), "t2_b": n(H).to(torch.bfloat16),
        "mod_w": n(cfg.modw, H).to(torch.bfloat16), "mod_b": n(cfg.modw).to(torch.bfloat16),
    }
    return W


def oracle_weights(W: dict) -> dict:
    """The weight dict with every tensor as fp32 (what the CPU oracle consumes)."""
    out = {k: (v.float() if torch.is_tensor(v) else v) for k, v in W.items() if k != "layers"}
    out["layers"] = [{k: v.float() for k, v in ly.items() if not (k.endswith("_q") and ly[k].dtype == torch.float8_e4m3fn)
                      and not k.endswith("_scale")} for ly in W["layers"]]
    return out


def make_inputs(cfg: ExpertConfig, seed_ctx: int = 1, seed_noise: int = 1234, seed_state: int = 2) -> dict:
    """Synthetic call inputs on CPU: VLM context [B, SP, ctx_dim] ~ N(0,1) bf16 (rows >= S zero), memory
    states [B, PM, H] ~ N(0,1), flow noise [B, T_act, A] ~ N(0,1) fp32 with seed seed_noise + b (the
    reference's FixedNoise convention, harness.py:53-66), state conditioning [B, H] ~ N(0,1)."""
    g = torch.Generator().manual_seed(seed_ctx)
    ctx = torch.randn(cfg.B, cfg.SP, cfg.ctx_dim, generator=g).to(torch.bfloat16)
    ctx[:, cfg.S:] = 0
    mem = torch.randn(cfg.B, cfg.PM, cfg.H, generator=g)
    noise = torch.stack([torch.randn(cfg.T_act, cfg.A, generator=torch.Generator().manual_seed(seed_noise + b))
                         for b in range(cfg.B)])
    state = torch.randn(cfg.B, cfg.H, generator=torch.Generator().manual_seed(seed_state))
    return {"ctx": ctx, "mem_states": mem, "noise": noise, "state_cond": state}


# ------------------------------------------------------------------------------------------------
# REKI-shaped module tree


class _Param:
    def __init__(self, w):
        self.weight = w


class _Linear:
    def __init__(self, w, b=None, q=None, scale=None):
        self.weight = w
        self.bias = b
        self.weight_q = q
        self.weight_scale = scale
        self.out_features, self.in_features = w.shape


class _Norm:
    def __init__(self, w, eps):
        self.weight = w
        self.eps = eps


class _Attn:
    def __init__(self, ly, prefix, cfg):
        g = lambda nm: _Linear(ly[prefix + nm], q=ly.get(prefix + nm + "_q"), scale=ly.get(prefix + nm + "_scale"))  # noqa: E731
        self.q_proj, self.k_proj, self.v_proj, self.o_proj = g("q"), g("k"), g("v"), g("o")
        self.q_norm = _Norm(ly[prefix + "q_norm"], cfg.qk_eps)
        self.k_norm = _Norm(ly[prefix + "k_norm"], cfg.qk_eps)
        self.n_q_heads = self.n_kv_heads = cfg.NH
        self.head_dim = cfg.HD


class _CrossAttn(_Attn):
    def __init__(self, ly, cfg):
        lyc = {"ca_" + k if not k.startswith("ca_") else k: v for k, v in ly.items()}
        super().__init__(lyc, "ca_", cfg)


class _MLP:
    def __init__(self, ly, cfg):
        g = lambda nm: _Linear(ly[nm], q=ly.get(nm + "_q"), scale=ly.get(nm + "_scale"))  # noqa: E731
        self.gate_proj, self.up_proj, self.down_proj = g("gate"), g("up"), g("down")
        self.act_fn = torch.nn.SiLU() if cfg.act == "silu" else torch.nn.GELU(approximate="tanh")


class _Layer:
    def __init__(self, ly, cfg):
        self.self_attn = _Attn(ly, "", cfg)
        self.cross_attn = _CrossAttn(ly, cfg)
        self.mlp = _MLP(ly, cfg)
        self.input_layernorm = _Norm(None, cfg.eps)


class _Expert:
    def __init__(self, layers, cfg):
        self.layers = layers
        self.norm = _Norm(None, cfg.eps)


class _VLMWithExpert:
    def __init__(self, expert):
        self.action_expert = expert


class Past:
    """The cache object the expert reads: ``register_step`` (memory K/V per layer, cu_kv, cu_src, RoPE
    tables) and ``cross_attn_kv`` (per-layer CA K/V), the fields src/mk_expert.py:486-496 consumes."""

    def __init__(self, register_step: dict, cross_attn_kv: list):
        self.register_step = register_step
        self.cross_attn_kv = cross_attn_kv


def rope_cos_sin(pos: torch.Tensor, hd: int, theta: float = 10000.0):
    inv = theta ** (-torch.arange(0, hd, 2, dtype=torch.float64, device=pos.device) / hd)
    f = pos.to(torch.float64)[:, None] * inv[None, :]
    emb = torch.cat([f, f], -1)
    return torch.cos(emb).float(), torch.sin(emb).float()


def _bf(t):
    return t.to(torch.bfloat16).to(torch.float32)


def _norm_rope_bf16(x, w, cos, sin, eps):
    """q/k RMSNorm (weight 1 + w) then rotate-half RoPE with bf16 rounding after each, in fp32."""
    hd = x.shape[-1]
    xn = _bf(x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * (1.0 + w.float()))
    rot = torch.cat([-xn[..., hd // 2:], xn[..., : hd // 2]], -1)
    return _bf(xn * cos[:, None, :] + rot * sin[:, None, :])


class SyntheticReki:
    """The model object: REKI's attribute tree plus its expert-side methods."""

    def __init__(self, cfg: ExpertConfig, W: dict | None = None, device="cuda", seed: int = 0):
        self.cfg = cfg
        self.device = torch.device(device)
        W = make_weights(cfg, seed) if W is None else W
        self.W_cpu = W
        dev = self.device
        mv = lambda t: t.to(dev) if torch.is_tensor(t) else t  # noqa: E731
        layers = [_Layer({k: mv(v) for k, v in ly.items()}, cfg) for ly in W["layers"]]
        self.vlm_with_expert = _VLMWithExpert(_Expert(layers, cfg))
        self.action_in_proj = _Linear(mv(W["in_w"]), mv(W["in_b"]))
        self.action_out_proj = _Linear(mv(W["out_w"]), mv(W["out_b"]))
        self.register_tokens = mv(W["reg_tok"])
        self._t1 = (mv(W["t1_w"]).float(), mv(W["t1_b"]).float())
        self._t2 = (mv(W["t2_w"]).float(), mv(W["t2_b"]).float())
        self._mod = (mv(W["mod_w"]).float(), mv(W["mod_b"]).float())
        self._first = None  # lazily built one-step megakernel (Euler step 1 with register rows)

    # -- REKI: _step_modulations(num_steps, state_cond) -> (mods, dt)
    def _step_modulations(self, num_steps: int, state_cond: torch.Tensor):
        """mods [N, MODW] (B = 1) or [B, N, MODW] fp32 and dt [1]: t_k = 1 - k/N, dt = -1/N;
        c = silu(temb(t) W1^T + b1) W2^T + b2 + state_cond; mods = silu(c) Wmod^T + bmod."""
        cfg = self.cfg
        dev = self.device
        c = self.modulation_input(num_steps, state_cond)
        sc = state_cond.reshape(-1, cfg.H)
        mods = F.silu(c) @ self._mod[0].T + self._mod[1]
        dt = torch.full((1,), -1.0 / num_steps, device=dev, dtype=torch.float32)
        return (mods[0] if sc.shape[0] == 1 else mods.contiguous()), dt

    def modulation_input(self, num_steps: int, state_cond: torch.Tensor) -> torch.Tensor:
        """c [B, N, H] fp32 = silu(temb(t) W1^T + b1) W2^T + b2 + state_cond, the input of the final
        modulation projection (mods = silu(c) Wmod^T + bmod)."""
        cfg = self.cfg
        dev = self.device
        t = 1.0 - torch.arange(num_steps, dtype=torch.float64, device=dev) / num_steps
        half = cfg.tdim // 2
        freqs = torch.exp(-math.log(10000.0) * torch.arange(half, dtype=torch.float64, device=dev) / half)
        args = (t * 1000.0)[:, None] * freqs[None, :]
        e = torch.cat([torch.cos(args), torch.sin(args)], -1).float()
        c = F.silu(e @ self._t1[0].T + self._t1[1]) @ self._t2[0].T + self._t2[1]
        sc = state_cond.to(dev).float().reshape(-1, cfg.H)
        return c[None] + sc[:, None, :]

    # -- REKI: register_prepare -> past
    def register_prepare(self, ctx: torch.Tensor, mem_states: torch.Tensor, ca_len=None, kv_start=None) -> Past:
        """CA source K (ca_k_norm + RoPE at positions 0..S-1) and V from ctx [B, SP, ctx_dim]; memory K
        (k_norm + RoPE at 0..PM-1) and V from mem_states [B, PM, H]; RoPE tables of the own rows
        (self-attention positions PM + i, cross-attention positions i). bf16 outputs with bf16 rounding
        after each projection, norm and rotation; rows >= ca_len and < kv_start are zero."""
        cfg = self.cfg
        dev = self.device
        B, SP, _ = ctx.shape
        PM = mem_states.shape[1]
        ca_len = [cfg.S] * B if ca_len is None else list(ca_len)
        kv_start = [cfg.kv_start] * B if kv_start is None else list(kv_start)
        ctx = ctx.to(dev)
        mem = mem_states.to(dev)
        ccos, csin = rope_cos_sin(torch.arange(SP, device=dev), cfg.HD)
        mcos, msin = rope_cos_sin(torch.arange(PM, device=dev), cfg.HD)
        mem_kv, ca_kv = [], []
        for ly in self.vlm_with_expert.action_expert.layers:
            kc = torch.zeros(B, SP, cfg.NH, cfg.HD, device=dev, dtype=torch.bfloat16)
            vc = torch.zeros_like(kc)
            km = torch.zeros(B, PM, cfg.NH, cfg.HD, device=dev, dtype=torch.bfloat16)
            vm = torch.zeros_like(km)
            for b in range(B):
                S = ca_len[b]
                c = ctx[b, :S].float()
                k = _bf(c @ ly.cross_attn.k_proj.weight.float().T).view(S, cfg.NH, cfg.HD)
                kc[b, :S] = _norm_rope_bf16(k, ly.cross_attn.k_norm.weight, ccos[:S], csin[:S], cfg.qk_eps).to(torch.bfloat16)
                vc[b, :S] = (c @ ly.cross_attn.v_proj.weight.float().T).view(S, cfg.NH, cfg.HD).to(torch.bfloat16)
                ks = kv_start[b]
                m = mem[b, ks:].float()
                k = _bf(m @ ly.self_attn.k_proj.weight.float().T).view(PM - ks, cfg.NH, cfg.HD)
                km[b, ks:] = _norm_rope_bf16(k, ly.self_attn.k_norm.weight, mcos[ks:], msin[ks:], cfg.qk_eps).to(torch.bfloat16)
                vm[b, ks:] = (m @ ly.self_attn.v_proj.weight.float().T).view(PM - ks, cfg.NH, cfg.HD).to(torch.bfloat16)
            if B == 1:
                kc, vc, km, vm = kc[0], vc[0], km[0], vm[0]
            mem_kv.append((km.contiguous(), vm.contiguous()))
            ca_kv.append((kc.contiguous(), vc.contiguous()))
        m_q = cfg.m_q
        sa = rope_cos_sin(PM + torch.arange(m_q, device=dev), cfg.HD)
        ca = rope_cos_sin(torch.arange(m_q, device=dev), cfg.HD)
        mf = cfg.m_q_first
        sa1 = rope_cos_sin(PM + torch.arange(mf, device=dev), cfg.HD)
        ca1 = rope_cos_sin(torch.arange(mf, device=dev), cfg.HD)
        i32 = lambda v: torch.tensor(v, device=dev, dtype=torch.int32)  # noqa: E731
        step = {
            "mem_kv": mem_kv, "sa_pe": sa, "ca_pe": ca, "sa_pe_first": sa1, "ca_pe_first": ca1,
            "cu_kv": i32([kv_start[0], PM]), "cu_src": i32([0, ca_len[0]]),
            "kv_start": i32(kv_start), "ca_len": i32(ca_len),
        }
        return Past(step, ca_kv)

    def register_ring(self, past: Past):
        """A ``RegisterRing`` over ``past``'s memory for this model's position convention: memory K is rotated
        at its row index and a call's register row r at PM + T_act + r (step 1's own rows are
        [T_act action rows || R_reg register rows] at PM + i), so kept rows turn by -R_reg and appended
        rows by -(T_act + R_reg). ``ring.append_frame(cur_k, cur_v)`` after a call, then
        ``ring.update_past(past)`` before the next."""
        from .ring import RegisterRing
        cfg = self.cfg
        st = past.register_step
        return RegisterRing(st["mem_kv"], st["kv_start"], cfg.R_reg, kept_delta=-cfg.R_reg,
                            new_delta=-(cfg.T_act + cfg.R_reg))

    # -- REKI: _expert_first_step(noise, past, register_cache, mods[:1], dt, action_dim) -> (x_t, cur_k, cur_v)
    def _expert_first_step(self, noise, past: Past, register_cache, mods1, dt, action_dim: int):
        """Euler step 1 over [action rows || register rows], run by the megakernel with one step and
        mod_row0 = 0; also returns the register rows' K (normed, rotated) and V per layer."""
        from .mk_expert import ExpertMegakernel
        if self._first is None:
            self._first = ExpertMegakernel(self, registers_in_loop=True)
        return self._first.run_first(noise, mods1, dt, past, action_dim)

    # -- REKI: _expert_actions(noise, cross_attn_cache, register_cache, state_cond, action_dim, num_steps)
    def _expert_actions(self, noise, cross_attn_cache, register_cache, state_cond, action_dim, num_steps):
        """Without install(): step 1, then steps 2..N as one megakernel launch per step (the per-step
        structure of REKI's own loop). install() replaces this with one launch for steps 2..N."""
        from .mk_expert import ExpertMegakernel
        mods, dt = self._step_modulations(num_steps, state_cond)
        x_t, cur_k, cur_v = self._expert_first_step(noise, cross_attn_cache, register_cache, mods[..., :1, :], dt, action_dim)
        if num_steps > 1:
            if getattr(self, "_per_step", None) is None:
                self._per_step = ExpertMegakernel(self)
            for s in range(1, num_steps):
                x_t = self._per_step.run(x_t, mods[..., [0, s], :], dt, cross_attn_cache, action_dim)
        return x_t, cur_k, cur_v
