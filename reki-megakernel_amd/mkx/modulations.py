"""The modulation projection on the GPU: the last layer of REKI's ``_step_modulations``
(src/mk_expert.py:529), ``mods = silu(c) W^T + b`` with W [MODW, H] (MODW = 9 L H + 2 H), which makes every
AdaRMS scale, shift and gate of every layer and Euler step of a call — the rows the expert kernel reads
(src/mk_expert.py:336-340).

``ModulationProjection(weight, bias)`` keeps W as bf16 (repacked once into MFMA fragment order, so every
weight load of the kernel is one contiguous 1 KB block per wave) and b as fp32 on the GPU; ``proj(c)`` runs
``mkx_modulations`` (one launch, each weight byte read once) on fp32 c [..., H] and returns fp32
[..., MODW]. Nothing here runs without libmkx.so.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import MkxModprojArgs, check, lib, require_device


class ModulationProjection:
    def __init__(self, weight: torch.Tensor, bias: torch.Tensor, fragment_order: bool = True):
        if weight.dim() != 2 or bias.shape != (weight.shape[0],):
            raise ValueError("weight must be [N, K] and bias [N]")
        if weight.device.type != "cuda" or bias.device != weight.device:
            raise ValueError("weight and bias must sit on one GPU")
        w = weight.detach().to(torch.bfloat16).contiguous()
        self.N, self.K = w.shape
        if self.N % 16 or self.K % 32:
            raise ValueError("N must be a multiple of 16 and K of 32")
        self.fragment_order = fragment_order
        # fragment order [N/16][K/32][64 lanes][8]: lane l of k-step t holds W[16 g + l % 16][32 t + 8 (l / 16) ..]
        self.w = (w.view(self.N // 16, 16, self.K // 32, 4, 8).permute(0, 2, 3, 1, 4).contiguous()
                  if fragment_order else w)
        self.b = bias.detach().float().contiguous()

    def __call__(self, c: torch.Tensor) -> torch.Tensor:
        if c.shape[-1] != self.K:
            raise ValueError(f"c must end in {self.K}, got {tuple(c.shape)}")
        require_device(self.w.device, c=c)
        lead = c.shape[:-1]
        x = c.float().reshape(-1, self.K).contiguous()
        out = torch.empty(x.shape[0], self.N, dtype=torch.float32, device=x.device)
        a = MkxModprojArgs(R=x.shape[0], K=self.K, N=self.N, c=x.data_ptr(), c_stride=self.K, w=self.w.data_ptr(),
                           bias=self.b.data_ptr(), out=out.data_ptr(), out_stride=self.N,
                           w_fragment_order=int(self.fragment_order))
        check(lib().mkx_modulations(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
              "mkx_modulations")
        self._keep = x  # the input outlives the asynchronous launch
        return out.reshape(*lead, self.N)
