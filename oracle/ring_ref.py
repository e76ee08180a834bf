"""CPU oracle for the register-memory ring append (the step after an expert call).

TEST INFRASTRUCTURE ONLY: only ``tests/`` imports it, for the expected results of ``mkx_ring_append``;
the product path never imports, calls or links it.

What it restates. The expert reads its self-attention memory from ``past.register_step['mem_kv']``, per
layer K and V of PM rows, valid from ``kv_start = cu_kv[0]`` (src/mk_expert.py:489-490, :321). After each
call REKI's register cache appends the call's register rows to that memory (``append_frame``, timed at
src/profile_breakdown.py:97-104; "32 register tokens per frame are cached over 3 frames as memory",
README.md:27). The cache itself is Kyutai's code, absent from the reference, so the rule below is this
library's, with memory K normed and rotated at its row index (as ``register_prepare`` in ``mkx.synthetic``
prepares it):

    out row j = in row j + R               for kv_start' <= j < PM - R  (K turned by the ``shift`` angles)
              = call's register row j-PM+R for j >= PM - R               (K turned by the ``new`` angles)
              = 0                          for j < kv_start' = max(min(max(kv_start, 0), PM) - R, 0)

Rotation is rotate-half RoPE by fixed angles, ``y = x * cos + rotate_half(x) * sin`` in fp32 (each
product rounded, then one sum) and rounded to bf16 to nearest even. V rows move unchanged.

Pins (tests/test_ring.py): a brute-force per-row loop; V and unrotated K moved bit for bit; rotation
composition (turning by a then by b equals turning by a + b, to bf16 rounding); the shifted memory equals
the memory ``register_prepare`` builds from the shifted states (to bf16 rounding); kv_start arithmetic
and zeroed rows. *Parity unpinned against REKI's register cache*: its source is not in the reference.
"""
from __future__ import annotations

import torch


def rope_rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [..., 64] (any float dtype) rotated by per-dimension angles (cos, sin [64]) in fp32, rounded to
    bf16: the order x * cos + rotate_half(x) * sin with rotate_half(x) = [-x_hi, x_lo]."""
    xf = x.float()
    half = xf.shape[-1] // 2
    rot = torch.cat([-xf[..., half:], xf[..., :half]], -1)
    return (xf * cos.float() + rot * sin.float()).to(torch.bfloat16)


def ring_append(memk, memv, cur_k, cur_v, kv_start, shift=None, new=None):
    """memk, memv [L, B, PM, NH, 64] bf16; cur_k, cur_v [L, B, R, NH, 64] bf16; kv_start [B] int;
    shift, new: (cos, sin) [64] fp32 or None (no rotation). Returns (memk', memv', kv_start')."""
    L, B, PM = memk.shape[:3]
    R = cur_k.shape[2]
    if not 1 <= R <= PM:
        raise ValueError("need 1 <= R <= PM")
    ks_new = (kv_start.long().clamp(0, PM) - R).clamp_min(0)
    kept_k, new_k = memk[:, :, R:], cur_k
    if shift is not None:
        kept_k = rope_rotate(kept_k, *shift)
    if new is not None:
        new_k = rope_rotate(new_k, *new)
    ok = torch.cat([kept_k.to(torch.bfloat16), new_k.to(torch.bfloat16)], 2)
    ov = torch.cat([memv[:, :, R:], cur_v], 2).to(torch.bfloat16)
    rows = torch.arange(PM)
    dead = rows[None, :] < ks_new[:, None]  # [B, PM]
    m = dead[None, :, :, None, None]
    ok = ok.masked_fill(m, 0)
    ov = ov.masked_fill(m, 0)
    return ok, ov, ks_new.to(torch.int32)


def ring_append_loops(memk, memv, cur_k, cur_v, kv_start, shift=None, new=None):
    """The same rule as ``ring_append`` written row by row (small inputs only): the oracle's own check."""
    L, B, PM, NH, HD = memk.shape
    R = cur_k.shape[2]
    ok = torch.zeros_like(memk)
    ov = torch.zeros_like(memv)
    ks_out = torch.zeros(B, dtype=torch.int32)
    for b in range(B):
        ks = max(min(max(int(kv_start[b]), 0), PM) - R, 0)
        ks_out[b] = ks
        for l in range(L):
            for j in range(ks, PM):
                if j < PM - R:
                    k, v, tab = memk[l, b, j + R], memv[l, b, j + R], shift
                else:
                    k, v, tab = cur_k[l, b, j - (PM - R)], cur_v[l, b, j - (PM - R)], new
                for h in range(NH):
                    kk = k[h].float()
                    if tab is not None:
                        c, s = tab[0].float(), tab[1].float()
                        y = torch.empty(HD)
                        for d in range(HD // 2):
                            y[d] = kk[d] * c[d] - kk[d + HD // 2] * s[d]
                            y[d + HD // 2] = kk[d + HD // 2] * c[d + HD // 2] + kk[d] * s[d + HD // 2]
                        kk = y
                    ok[l, b, j, h] = kk.to(memk.dtype)
                    ov[l, b, j, h] = v[h]
    return ok, ov, ks_out
