"""The modulation projection on the GPU: the last layer of REKI's ``_step_modulations``
(src/mk_expert.py:529), ``mods = silu(c) W^T + b`` with W [MODW, H] (MODW = 9 L H + 2 H), which makes every
AdaRMS scale, shift and gate of every layer and Euler step of a call — the rows the expert kernel reads
(src/mk_expert.py:336-340).

``StepModulations`` runs the whole of ``_step_modulations`` on this library's kernels: ``mkx_modulation_input``
(the timestep embedding and the small MLP, c = silu(temb(t) W1^T + b1) W2^T + b2 + state_cond, one launch)
and then the projection, two launches in all.

``ModulationProjection(weight, bias)`` keeps W as bf16 (repacked once into MFMA fragment order, so every
weight load of the kernel is one contiguous 1 KB block per wave) and b as fp32 on the GPU; ``proj(c)`` runs
``mkx_modulations`` (one launch, each weight byte read once) on fp32 c [..., H] and returns fp32
[..., MODW]. Nothing here runs without libmkx.so.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import MkxModinArgs, MkxModprojArgs, check, lib, require_device


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


class StepModulations:
    """``mods, dt = step(num_steps, state_cond)`` with the result layout of REKI's ``_step_modulations``
    (src/mk_expert.py:529): mods [N, MODW] for one sample (state_cond [H] or [1, H]), [B, N, MODW] for B, and
    dt = -1 / N as a [1] tensor. t1_w [H, tdim], t2_w [H, H] and mod_w [MODW, H] are kept as bf16, the
    biases as fp32, on the weights' GPU."""

    def __init__(self, t1_w: torch.Tensor, t1_b: torch.Tensor, t2_w: torch.Tensor, t2_b: torch.Tensor,
                 mod_w: torch.Tensor, mod_b: torch.Tensor):
        dev = t1_w.device
        if dev.type != "cuda" or any(t.device != dev for t in (t1_b, t2_w, t2_b, mod_w, mod_b)):
            raise ValueError("the weights must sit on one GPU")
        self.H, self.tdim = t1_w.shape
        if t2_w.shape != (self.H, self.H) or t1_b.shape != (self.H,) or t2_b.shape != (self.H,) or mod_w.shape[1] != self.H:
            raise ValueError("expected t1_w [H, tdim], t1_b [H], t2_w [H, H], t2_b [H], mod_w [MODW, H]")
        self.t1_w = t1_w.detach().to(torch.bfloat16).contiguous()
        self.t2_w = t2_w.detach().to(torch.bfloat16).contiguous()
        self.t1_b = t1_b.detach().float().contiguous()
        self.t2_b = t2_b.detach().float().contiguous()
        self.device = dev
        self.proj = ModulationProjection(mod_w, mod_b.float())

    def input(self, num_steps: int, state_cond: torch.Tensor) -> torch.Tensor:
        """c [B, N, H] fp32 (the projection's input) for state_cond [B, H] (or [H])."""
        require_device(self.device, state_cond=state_cond)
        sc = state_cond.float().reshape(-1, self.H).contiguous()
        B = sc.shape[0]
        out = torch.empty(B, num_steps, self.H, dtype=torch.float32, device=self.device)
        a = MkxModinArgs(N=int(num_steps), B=B, H=self.H, tdim=self.tdim, t1_w=self.t1_w.data_ptr(),
                         t1_b=self.t1_b.data_ptr(), t2_w=self.t2_w.data_ptr(), t2_b=self.t2_b.data_ptr(),
                         state_cond=sc.data_ptr(), sc_stride=self.H, out=out.data_ptr(),
                         out_stride_b=num_steps * self.H, out_stride_k=self.H)
        check(lib().mkx_modulation_input(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
              "mkx_modulation_input")
        self._keep = sc  # the input outlives the asynchronous launch
        return out

    def __call__(self, num_steps: int, state_cond: torch.Tensor):
        one = state_cond.dim() == 1 or state_cond.shape[0] == 1
        mods = self.proj(self.input(num_steps, state_cond))
        dt = torch.full((1,), -1.0 / num_steps, device=self.device, dtype=torch.float32)
        return (mods[0] if one else mods), dt
