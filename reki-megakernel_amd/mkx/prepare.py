"""Cross-attention source caches on the GPU: the part of REKI's ``register_prepare`` that projects the VLM
context onto each layer's cross-attention K and V (README.md:279-281, "the cross-attention K/V projections
of the VLM source (31 M weights)"; the expert reads the result as ``past.cross_attn_kv``,
src/mk_expert.py:491-492).

``SourcePrepare(model)`` stacks the layers' ``cross_attn.k_proj`` / ``v_proj`` weights and ``k_norm``
and hands them to ``mkx_source_create`` (repacked once); ``prep(ctx, ca_len)`` runs ``mkx_source_run``
(a context packing launch, then one launch for all layers, heads and samples)
and returns per-layer (K, V) bf16 [B, SP, NH, 64] ([SP, NH, 64] for a 2-D ctx): K = per-head RMSNorm
(weight 1 + w, bf16) then rotate-half RoPE at source positions 0..SP-1 (bf16), V = the projection
rounded to bf16, rows >= ca_len zero. Nothing here runs without libmkx.so.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import MAX_LAYERS, MkxSourceArgs, MkxSourceDims, check, lib, require_device


def rope_table(n: int, hd: int = 64, theta: float = 10000.0, device="cuda"):
    """(cos, sin) [n, hd] fp32 of rotate-half RoPE at positions 0..n-1 (frequencies theta^(-2i/hd),
    duplicated over the two halves), evaluated in float64 and rounded once."""
    inv = theta ** (-torch.arange(0, hd, 2, dtype=torch.float64) / hd)
    f = torch.arange(n, dtype=torch.float64)[:, None] * inv[None, :]
    emb = torch.cat([f, f], -1)
    return torch.cos(emb).float().to(device), torch.sin(emb).float().to(device)


class SourcePrepare:
    """Cross-attention source K/V of every layer from the VLM context, on the GPU."""

    def __init__(self, model, theta: float = 10000.0, max_rows: int = 1 << 14):
        layers = list(model.vlm_with_expert.action_expert.layers)
        ca = [lay.cross_attn for lay in layers]
        self.L, self.NH, self.HD = len(layers), ca[0].n_kv_heads, ca[0].head_dim
        if self.HD != 64:
            raise ValueError("head dim must be 64")
        if self.L > MAX_LAYERS:
            raise ValueError(f"at most {MAX_LAYERS} layers")
        bf = torch.bfloat16
        self.wk = torch.stack([c.k_proj.weight.detach() for c in ca]).to(bf).contiguous()  # [L, H, C]
        self.wv = torch.stack([c.v_proj.weight.detach() for c in ca]).to(bf).contiguous()
        self.k_norm = torch.stack([c.k_norm.weight.detach() for c in ca]).to(bf).contiguous()  # [L, 64]
        self.eps = float(ca[0].k_norm.eps)
        self.device = self.wk.device
        if self.device.type != "cuda":
            raise ValueError("the cross-attention projections must sit on the GPU")
        self.C = self.wk.shape[2]
        if self.wk.shape[1] != self.NH * 64 or self.C % 32:
            raise ValueError("k_proj must be [NH * 64, C] with C a multiple of 32")
        self.theta = theta
        self._tables = {}
        self.max_rows = max_rows
        dims = MkxSourceDims(L=self.L, NH=self.NH, HD=64, C=self.C, max_rows=max_rows, eps=self.eps)
        h = ctypes.c_void_p()
        check(lib().mkx_source_create(ctypes.byref(dims), ctypes.c_void_p(self.wk.data_ptr()),
                                      ctypes.c_void_p(self.wv.data_ptr()), ctypes.c_void_p(self.k_norm.data_ptr()),
                                      ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), ctypes.byref(h)),
              "mkx_source_create")
        self._h = h
        del self.wk, self.wv  # the handle holds its own packed copy

    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().mkx_source_destroy(h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass

    def __call__(self, ctx: torch.Tensor, ca_len, cos=None, sin=None, static_scratch: bool = False):
        """static_scratch: run ``mkx_source_run_noalloc`` (the context staged in the library's static device
        array; for callers that cannot allocate) instead of ``mkx_source_run``."""
        require_device(self.device, ctx=ctx, ca_len=ca_len if torch.is_tensor(ca_len) else None,
                       cos=cos, sin=sin)
        batched = ctx.dim() == 3
        x = (ctx if batched else ctx[None]).to(torch.bfloat16).contiguous()
        B, SP, C = x.shape
        if C != self.C:
            raise ValueError(f"context width {C} differs from the projections' {self.C}")
        dev = x.device
        if cos is None:
            key = (SP, dev)
            if key not in self._tables:
                self._tables[key] = rope_table(SP, 64, self.theta, dev)
            cos, sin = self._tables[key]
        cos, sin = cos.float().contiguous(), sin.float().contiguous()
        if cos.shape != (SP, 64) or sin.shape != (SP, 64):
            raise ValueError("cos / sin must be [SP, 64]")
        cal = torch.as_tensor(ca_len, dtype=torch.int32).reshape(-1).to(dev).contiguous()
        if cal.numel() != B:
            raise ValueError("ca_len needs one entry per sample")
        ks = [torch.empty(B, SP, self.NH, 64, dtype=torch.bfloat16, device=dev) for _ in range(self.L)]
        vs = [torch.empty_like(ks[0]) for _ in range(self.L)]
        a = MkxSourceArgs(B=B, SP=SP)
        a.ctx, a.ca_len = x.data_ptr(), cal.data_ptr()
        a.cos, a.sin = cos.data_ptr(), sin.data_ptr()
        for l in range(self.L):
            a.kca[l], a.vca[l] = ks[l].data_ptr(), vs[l].data_ptr()
        a.src_stride_b = SP * self.NH * 64
        fn = lib().mkx_source_run_noalloc if static_scratch else lib().mkx_source_run
        check(fn(self._h, ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
              "mkx_source_run_noalloc" if static_scratch else "mkx_source_run")
        self._keep = (x, cal, cos, sin)  # inputs outlive the asynchronous launch
        if batched:
            return list(zip(ks, vs))
        return [(k[0], v[0]) for k, v in zip(ks, vs)]
