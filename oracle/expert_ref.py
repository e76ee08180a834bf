"""CPU oracle for the flow-matching action expert's Euler loop.

TEST INFRASTRUCTURE ONLY. This module is the reference result the HIP megakernel is tested against: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import it. The product path
(``reki-megakernel_amd/``) never imports, calls or links it, and must fail loudly when its HIP
library is missing instead of falling back here.

What it restates. The arithmetic of the reference's Triton megakernel ``expert_megakernel``
(src/mk_expert.py:302-426) and of the REKI eager expert that kernel restates (NOTICE:7-12):
AdaRMS modulation, gated residuals, q/k RMSNorm + rotate-half RoPE, self-attention over
[cached memory rows || own rows], cross-attention to a pre-projected VLM source, a gated MLP, and
the fp32 step tail (final AdaRMS, action out-projection, Euler update, action in-projection).
Every function cites the reference lines it follows.

Modes.
  ``fp32``   every activation in fp32; weights are bf16-valued (the parity metric: the eager fp32
             expert). ``R`` (the rounding hook) is the identity.
  ``mirror`` rounds to bf16 at every point the reference kernel rounds (marked ``bf16(.)`` in the
             citations), including the residual stream.
  ``mixed``  rounds where a bf16 MFMA kernel must (GEMM inputs and outputs, attention operands) but keeps
             the residual stream (h0, h2, h3, h_l and the gated branch added to it) in fp32: the numerics
             of a bf16-activation kernel, reported beside the GPU results for comparison.
  ``f16``    the numerics of this library's HIP kernel: every GEMM operand is rounded to fp16 (round to
             nearest even) where the kernel stores it — the AdaRMS operand h (1 + scale) and the shift
             (the GEMM computes rstd(h) * (Q(h (1 + scale)) W^T) + Q(shift) W^T), the attention outputs
             before the out-projections, and the gated MLP product before the down projection — and
             everything else stays fp32. Not a reference mode: it models the kernel's rounding points.
             Over tens of layers these rounding decisions are chaotic (a 1e-7 relative change of the input
             moves the result as much as the rounding itself), so this mode gives the error level the kernel
             should show against ``fp32``, not a per-element reference.
  ``fp64``   like ``fp32`` but in float64; used by the oracle's own pin tests.

Parts REKI would have supplied (its code is not available offline): the timestep embedding and
modulation MLP (``step_modulations``), the cache preparation (``register_prepare``), RoPE positions
and the register-row layout. They are defined here and in ``mkx.synthetic`` by this library, are pinned
by closed forms and invariants in tests/test_oracle_pins.py, and are *parity unpinned against REKI*.

Pinning (tests/test_oracle_pins.py): ``rstd``/``adarms`` against ``torch.nn.functional.rms_norm``
in fp64; ``norm_rope`` against a complex-number rotation; ``attend`` against
``scaled_dot_product_attention`` in fp64 and a brute-force loop; the step against invariants
(zero gates => identity layers, zero out-projection => x unchanged, scale = -1 => AdaRMS = shift,
one valid key => output = V, memory-row permutation invariance, padded/invalid rows have no
effect, dims >= action_dim never feed back) and fp64 vs fp32 vs mirror consistency.
``layer_forward``'s wiring (tests/test_oracle_wiring.py): an independent fp64 restatement of one layer with
torch.nn.functional.linear / rms_norm / scaled_dot_product_attention and boolean key masks, on random
non-symmetric weights and open gates; planted mutants (a transposed square projection, h instead of h2 or
h3 into an AdaRMS) must differ from it; a cyclic-shift out-projection must move each column by one.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

__all__ = [
    "ExpertDims", "rounder", "operand_rounder", "rstd", "adarms", "norm_rope", "attend", "act_fn", "layer_forward",
    "step_tail", "in_proj", "run_steps", "timestep_embedding", "step_modulations", "rope_cos_sin",
    "register_prepare", "mods_offsets",
]


@dataclass(frozen=True)
class ExpertDims:
    """Shapes of one expert. ``A`` is the padded action width (``action_in_proj.in_features``,
    mk_expert.py:443); ``M_q = T_act + R_reg`` own rows per sample."""
    L: int = 10
    H: int = 768
    NH: int = 12
    HD: int = 64
    I: int = 3072
    A: int = 32
    ctx_dim: int = 2048
    tdim: int = 256
    eps: float = 1e-6
    qk_eps: float = 1e-6
    act: str = "silu"  # "silu" (reference, mk_expert.py:464) or "gelu_tanh"

    @property
    def modw(self) -> int:
        """Modulation row width: 9 H per layer + final [scale|shift] (mk_expert.py:336-340, 423)."""
        return 9 * self.L * self.H + 2 * self.H


def mods_offsets(d: ExpertDims, l: int) -> dict[str, int]:
    """Column offsets of layer ``l``'s modulation blocks inside one step row.
    mk_expert.py:338-340: m_sa = 9 l H, m_ca = m_sa + 3H, m_mlp = m_ca + 3H; each [scale|shift|gate]."""
    base = 9 * l * d.H
    return {"sa": base, "ca": base + 3 * d.H, "mlp": base + 6 * d.H}


def rounder(mode: str):
    """The rounding hook R: bf16 round trip in ``mirror`` and ``mixed`` modes, identity otherwise."""
    if mode in ("mirror", "mixed"):
        return lambda t: t.to(torch.bfloat16).to(torch.float32)
    return lambda t: t


def operand_rounder(mode: str):
    """Rounding of the GEMM operands: fp16 round trip (round to nearest even) in ``f16`` mode; in ``f8``
    mode fp8 e4m3 with one absmax scale per row (per token: the finest scaling an fp8 MFMA with
    per-row epilogue scales could apply), which gives the error an fp8-activation kernel would have;
    identity otherwise."""
    if mode == "f16":
        return lambda t: t.to(torch.float16).to(t.dtype)
    if mode == "f8":
        def f8(t):
            s = t.abs().amax(-1, keepdim=True).clamp_min(1e-30) / 448.0
            return (t / s).to(torch.float8_e4m3fn).to(t.dtype) * s
        return f8
    return lambda t: t


def res_rounder(mode: str):
    """Rounding of the residual stream: bf16 only in ``mirror`` mode."""
    return rounder(mode) if mode == "mirror" else (lambda t: t)


def _dtype(mode: str) -> torch.dtype:
    return torch.float64 if mode == "fp64" else torch.float32


def rstd(x: torch.Tensor, eps: float) -> torch.Tensor:
    """rsqrt(mean(x^2) + eps) over the last dim (mk_expert.py:93-103, fp32)."""
    return torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)


def adarms(h: torch.Tensor, scale: torch.Tensor, shift: torch.Tensor, eps: float, R) -> torch.Tensor:
    """AdaRMS: bf16(h * rstd(h) * (1 + scale) + shift); no affine weight, no mean subtraction
    (mk_expert.py:106-122 prologue, :119)."""
    return R(h * rstd(h, eps) * (1.0 + scale) + shift)


def norm_rope(x: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, eps: float, R) -> torch.Tensor:
    """Per-head RMSNorm with weight (1 + w), rounded, then rotate-half RoPE, rounded
    (mk_expert.py:175-193). x: [..., rows, NH, HD]; cos/sin: [rows, HD]; w: [HD].
    out_d = xn_d cos_d + sgn_d xn_{(d+HD/2) % HD} sin_d, sgn_d = -1 for d < HD/2."""
    hd = x.shape[-1]
    r = torch.rsqrt((x * x).mean(-1, keepdim=True) + eps)
    xn = R(x * r * (1.0 + w))
    half = hd // 2
    rot = torch.cat([-xn[..., half:], xn[..., :half]], dim=-1)
    return R(xn * cos[:, None, :] + rot * sin[:, None, :])


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, R, mirror: bool) -> torch.Tensor:
    """Softmax attention of queries q [Mq, NH, HD] over keys/values k, v [Nk, NH, HD] (all valid).
    fp32 max-subtracted softmax; in ``mirror`` mode the unnormalised P is rounded to bf16 before
    P.V and the sum of unrounded P divides afterwards (mk_expert.py:212-222, 242-250); the result is
    rounded to bf16 (:222, :251)."""
    s = torch.einsum("mhd,nhd->hmn", q, k) * scale
    mx = s.amax(-1, keepdim=True)
    p = torch.exp(s - mx)
    den = p.sum(-1, keepdim=True)
    if mirror:
        o = torch.einsum("hmn,nhd->hmd", R(p), v) / den
    else:
        o = torch.einsum("hmn,nhd->hmd", p / den, v)
    return R(o.permute(1, 0, 2))  # [Mq, NH, HD]


def act_fn(x: torch.Tensor, act: str) -> torch.Tensor:
    """Gate activation: SiLU x / (1 + exp(-x)) (mk_expert.py:410) or tanh-GELU."""
    if act == "silu":
        return x / (1.0 + torch.exp(-x))
    if act == "gelu_tanh":
        return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x * x * x)))
    raise ValueError(f"unknown activation {act!r}")


def layer_forward(h: torch.Tensor, l: int, W: dict, mrow: torch.Tensor, cache: dict, b: int, d: ExpertDims,
                  mode: str, reg_kv: list | None = None, t_act: int = 0) -> torch.Tensor:
    """One expert layer on the own rows h [M_q, H] of sample b (Appendix-A stages 1-8;
    mk_expert.py:342-419). ``mrow`` is the step's modulation row [MODW].
    If ``reg_kv`` is a list, the normed+rotated K and raw V of rows >= t_act (register rows) are
    appended as (k, v) [R, NH, HD] (what REKI's step 1 returns as cur_k / cur_v)."""
    R = rounder(mode)
    Rr = res_rounder(mode)
    Q = operand_rounder(mode)
    mirror = mode in ("mirror", "mixed")
    H, NH, HD = d.H, d.NH, d.HD
    M = h.shape[0]
    lw = W["layers"][l]

    def ada(x, sc, sh):
        # AdaRMS as a GEMM operand: mode f16 rounds the unnormalised operand and the shift where the kernel
        # stores them (rstd(x) is applied to the product; AdaRMS is linear in both)
        if mode in ("f16", "f8"):
            return rstd(x, d.eps) * Q(x * (1.0 + sc)) + Q(sh)
        return adarms(x, sc, sh, d.eps, R)

    off = mods_offsets(d, l)
    sa_sc, sa_sh, sa_g = (mrow[off["sa"] + i * H: off["sa"] + (i + 1) * H] for i in range(3))
    ca_sc, ca_sh, ca_g = (mrow[off["ca"] + i * H: off["ca"] + (i + 1) * H] for i in range(3))
    m_sc, m_sh, m_g = (mrow[off["mlp"] + i * H: off["mlp"] + (i + 1) * H] for i in range(3))
    scale = HD ** -0.5

    # 1. qkv = bf16(AdaRMS(h) @ [Wq;Wk;Wv]^T)  (mk_expert.py:343-348, weight packing :446-447)
    a = ada(h, sa_sc, sa_sh)
    q = R(a @ lw["q"].T).view(M, NH, HD)
    k = R(a @ lw["k"].T).view(M, NH, HD)
    v = R(a @ lw["v"].T).view(M, NH, HD)
    # 2. self-attention over [memory rows kv_start..PM || own rows] (mk_expert.py:196-222)
    qr = norm_rope(q, lw["q_norm"], cache["sa_cos"], cache["sa_sin"], d.qk_eps, R)
    kr = norm_rope(k, lw["k_norm"], cache["sa_cos"], cache["sa_sin"], d.qk_eps, R)
    if reg_kv is not None:
        reg_kv.append((kr[t_act:].clone(), v[t_act:].clone()))
    ks = int(cache["kv_start"][b])
    pm = cache["memk"].shape[2]
    mk = cache["memk"][l, b, ks:pm]
    mv = cache["memv"][l, b, ks:pm]
    y = attend(qr, torch.cat([mk, kr], 0), torch.cat([mv, v], 0), scale, R, mirror).reshape(M, H)
    # 3. h2 = bf16(h + bf16(y @ Wo^T) * gate_sa)  (mk_expert.py:364-366, 162-172)
    h2 = Rr(h + Rr(Q(y) @ lw["o"].T) * sa_g)
    # 4. qca = bf16(AdaRMS_ca(h2) @ Wqca^T)  (mk_expert.py:373-378)
    a = ada(h2, ca_sc, ca_sh)
    qca = R(a @ lw["ca_q"].T).view(M, NH, HD)
    # 5. cross-attention over the S valid source rows (mk_expert.py:225-251)
    qr = norm_rope(qca, lw["ca_q_norm"], cache["ca_cos"], cache["ca_sin"], d.qk_eps, R)
    S = int(cache["ca_len"][b])
    y = attend(qr, cache["kca"][l, b, :S], cache["vca"][l, b, :S], scale, R, mirror).reshape(M, H)
    # 6. h3 = bf16(h2 + bf16(y @ Woca^T) * gate_ca)  (mk_expert.py:395-397)
    h3 = Rr(h2 + Rr(Q(y) @ lw["ca_o"].T) * ca_g)
    # 7. g = bf16(act(bf16(A Wg^T)) * bf16(A Wu^T)), A = AdaRMS_mlp(h3)  (mk_expert.py:404-413)
    a = ada(h3, m_sc, m_sh)
    gf = R(a @ lw["gate"].T)
    uf = R(a @ lw["up"].T)
    g = R(act_fn(gf, d.act) * uf)
    # 8. h = bf16(h3 + bf16(g @ Wd^T) * gate_mlp)  (mk_expert.py:417-419)
    return Rr(h3 + Rr(Q(g) @ lw["down"].T) * m_g)


def in_proj(x: torch.Tensor, W: dict, action_dim: int, R) -> torch.Tensor:
    """h0 = bf16(x_pad @ Win^T + bin) with x_pad zero in dims >= action_dim, fp32 products
    (mk_expert.py:280-293 with FIRST, :326-327)."""
    xp = x.clone()
    xp[..., action_dim:] = 0
    return R(xp @ W["in_w"].T + W["in_b"])


def step_tail(hL: torch.Tensor, x: torch.Tensor, mrow: torch.Tensor, dt: float, W: dict, d: ExpertDims,
              action_dim: int, R) -> torch.Tensor:
    """Step tail on the T_act action rows (mk_expert.py:254-299):
    o = bf16(AdaRMS_final(h_L)); v = o Wout^T + bout (fp32); x' = x_pad + dt v (all A dims, so
    padded dims hold dt v only). Returns x' [T, A]."""
    f_sc = mrow[9 * d.L * d.H: 9 * d.L * d.H + d.H]
    f_sh = mrow[9 * d.L * d.H + d.H: 9 * d.L * d.H + 2 * d.H]
    o = adarms(hL, f_sc, f_sh, d.eps, R)
    v = o @ W["out_w"].T + W["out_b"]
    xp = x.clone()
    xp[..., action_dim:] = 0
    return xp + dt * v


def run_steps(x: torch.Tensor, mods: torch.Tensor, dt: float, W: dict, cache: dict, d: ExpertDims,
              action_dim: int, mode: str = "fp32", reg_kv_out: list | None = None) -> torch.Tensor:
    """Integrate ``mods.shape[1]`` Euler steps from x, the contract of ExpertMegakernel.run
    (mk_expert.py:483-515): x [B, T, A] fp32; mods [B, n, MODW] (one row per step, in order).
    Each step: in-proj of x (first step only; later steps take it from the previous tail,
    mk_expert.py:326-327, 423-424), the L layers, the tail. Register rows (rows T..M_q-1) take
    ``cache['reg_tok']`` as their layer-0 input every step and their outputs are discarded.
    Returns x after the last step [B, T, A] (fp32 / fp64)."""
    dtp = _dtype(mode)
    R = rounder(mode)
    Rr = res_rounder(mode)
    B, T, _ = x.shape
    out = []
    W = _cast_tree(W, dtp)
    cache = _cast_tree(cache, dtp)
    mods = mods.to(dtp)
    reg = cache.get("reg_tok")
    for b in range(B):
        xb = x[b].to(dtp)
        h0a = in_proj(xb, W, action_dim, Rr)
        for s in range(mods.shape[1]):
            h = h0a if reg is None or reg.shape[0] == 0 else torch.cat([h0a, reg], 0)
            kv = [] if (reg_kv_out is not None and s == 0) else None
            for l in range(d.L):
                h = layer_forward(h, l, W, mods[b, s], cache, b, d, mode, reg_kv=kv, t_act=T)
            if kv is not None:
                reg_kv_out.append(kv)
            xb = step_tail(h[:T], xb, mods[b, s], dt, W, d, action_dim, R)
            h0a = in_proj(xb, W, action_dim, Rr)
        out.append(xb)
    return torch.stack(out, 0)


def _cast_tree(t, dtp):
    if isinstance(t, torch.Tensor):
        return t.to(dtp) if t.is_floating_point() else t
    if isinstance(t, dict):
        return {k: _cast_tree(v, dtp) for k, v in t.items()}
    if isinstance(t, (list, tuple)):
        return type(t)(_cast_tree(v, dtp) for v in t)
    return t


# ---------------------------------------------------------------------------------------------
# Parts REKI supplies outside the megakernel (step modulations, cache preparation). REKI's code is
# unavailable offline, so these are this library's own definitions (parity unpinned against REKI);
# mkx.synthetic computes the same on the GPU.
# ---------------------------------------------------------------------------------------------

def timestep_embedding(t: torch.Tensor, dim: int, max_period: float = 10000.0, t_scale: float = 1000.0) -> torch.Tensor:
    """Sinusoidal embedding [cos | sin] of t * t_scale with geometric frequencies."""
    half = dim // 2
    freqs = torch.exp(-math.log(max_period) * torch.arange(half, dtype=torch.float64) / half)
    args = (t.to(torch.float64) * t_scale)[:, None] * freqs[None, :]
    return torch.cat([torch.cos(args), torch.sin(args)], -1)


def step_modulations(num_steps: int, state_cond: torch.Tensor, W: dict, d: ExpertDims):
    """mods [B, N, MODW] and dt for an N-step Euler schedule from t = 1 (noise) toward 0:
    t_k = 1 - k/N, dt = -1/N. c = silu(temb(t) W1^T + b1) W2^T + b2 + state_cond;
    mods = silu(c) Wmod^T + bmod (fp32). The kernel only sees mods and dt
    (mk_expert.py:336-340, 529)."""
    c = modulation_input(num_steps, state_cond, W, d)
    mods = F.silu(c) @ W["mod_w"].float().T + W["mod_b"].float()
    return mods, -1.0 / num_steps


def modulation_input(num_steps: int, state_cond: torch.Tensor, W: dict, d: ExpertDims) -> torch.Tensor:
    """c [B, N, H] = silu(temb(t) W1^T + b1) W2^T + b2 + state_cond, the input of the modulation
    projection (``step_modulations``)."""
    t = 1.0 - torch.arange(num_steps, dtype=torch.float64) / num_steps
    e = timestep_embedding(t, d.tdim).to(torch.float32)
    c = F.silu(e @ W["t1_w"].float().T + W["t1_b"].float()) @ W["t2_w"].float().T + W["t2_b"].float()
    return c[None, :, :] + state_cond.float()[:, None, :]


def rope_cos_sin(pos: torch.Tensor, hd: int, theta: float = 10000.0):
    """cos/sin tables [len(pos), hd] for rotate-half RoPE (frequencies repeated over both halves)."""
    inv = theta ** (-torch.arange(0, hd, 2, dtype=torch.float64) / hd)
    f = pos.to(torch.float64)[:, None] * inv[None, :]
    emb = torch.cat([f, f], -1)
    return torch.cos(emb).float(), torch.sin(emb).float()


def register_prepare(ctx: torch.Tensor, ca_len: list[int], mem_states: torch.Tensor, kv_start: list[int],
                     W: dict, d: ExpertDims, m_q: int, mode: str = "fp32") -> dict:
    """Caches the megakernel reads (what REKI's register_prepare / step 1 provide,
    mk_expert.py:22-24, 486-496): per layer the CA source K (K-normed with ca_k_norm, RoPE at
    positions 0..S-1) and V projected from ctx [B, SP, ctx_dim]; the memory K (k_norm, RoPE at
    positions 0..PM-1) and V projected from mem_states [B, PM, H]; RoPE tables for the own rows
    (SA positions PM + i, CA positions i). Rows >= ca_len[b] of kca/vca and rows < kv_start[b] of
    memk/memv are zero. Outputs are bf16 in ``mirror`` mode, fp32 otherwise."""
    R = rounder(mode)
    B, SP, _ = ctx.shape
    PM = mem_states.shape[1]
    L, NH, HD = d.L, d.NH, d.HD
    kca = torch.zeros(L, B, SP, NH, HD)
    vca = torch.zeros(L, B, SP, NH, HD)
    memk = torch.zeros(L, B, PM, NH, HD)
    memv = torch.zeros(L, B, PM, NH, HD)
    ccos, csin = rope_cos_sin(torch.arange(SP), HD)
    mcos, msin = rope_cos_sin(torch.arange(PM), HD)
    for l in range(L):
        lw = W["layers"][l]
        for b in range(B):
            S = ca_len[b]
            c = ctx[b, :S].float()
            k = (c @ lw["ca_k"].float().T).view(S, NH, HD)
            kca[l, b, :S] = norm_rope(R(k), lw["ca_k_norm"].float(), ccos[:S], csin[:S], d.qk_eps, R)
            vca[l, b, :S] = R(c @ lw["ca_v"].float().T).view(S, NH, HD)
            ks = kv_start[b]
            m = mem_states[b, ks:].float()
            k = (m @ lw["k"].float().T).view(PM - ks, NH, HD)
            memk[l, b, ks:] = norm_rope(R(k), lw["k_norm"].float(), mcos[ks:], msin[ks:], d.qk_eps, R)
            memv[l, b, ks:] = R(m @ lw["v"].float().T).view(PM - ks, NH, HD)
    sa_cos, sa_sin = rope_cos_sin(PM + torch.arange(m_q), HD)
    ca_cos, ca_sin = rope_cos_sin(torch.arange(m_q), HD)
    return {"kca": kca, "vca": vca, "memk": memk, "memv": memv, "kv_start": torch.tensor(kv_start),
            "ca_len": torch.tensor(ca_len), "sa_cos": sa_cos, "sa_sin": sa_sin, "ca_cos": ca_cos, "ca_sin": ca_sin}
