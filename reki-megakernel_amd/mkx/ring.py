"""Register-memory ring: the step after an expert call, refilling the memory the next call attends to.

REKI keeps the register rows of the last few calls (frames) as self-attention memory: "32 register
tokens per frame are cached over 3 frames" (README.md:27), appended by its register cache after every
call (``append_frame``, src/profile_breakdown.py:97-104) and read by the expert as
``past.register_step['mem_kv']`` with ``kv_start = cu_kv[0]`` (src/mk_expert.py:489-490, :321).

``RegisterRing`` owns two sets of per-layer memory buffers [B, PM, NH, 64] bf16 and swaps them on each
``append_frame(cur_k, cur_v)``, which launches ``mkx_ring_append`` once for all layers and samples:
the oldest R rows drop out, the call's R register rows (``run_first`` / ``run_all``'s cur_k, cur_v) come
in at the end, and ``kv_start`` drops by R (floor 0). Memory K is normed and rotated at its row index, so
kept rows are turned back by R positions and the new rows from their position in the call to their
memory row; the angles come from ``rope_delta`` (rotate-half RoPE with the model's base), or no
rotation when the deltas are None. Nothing here runs without libmkx.so.
"""
from __future__ import annotations

import ctypes

import torch

from ._lib import MkxRingArgs, check, lib, require_device


def rope_delta(delta: int, hd: int = 64, theta: float = 10000.0, device="cuda"):
    """(cos, sin) [hd] fp32 turning a rotate-half RoPE vector by ``delta`` positions (frequencies
    theta^(-2i/hd), duplicated over the two halves), evaluated in float64 and rounded once."""
    inv = theta ** (-torch.arange(0, hd, 2, dtype=torch.float64) / hd)
    f = torch.cat([inv, inv]) * float(delta)
    return torch.cos(f).float().to(device), torch.sin(f).float().to(device)


class RegisterRing:
    """Ping-pong register memory for one stream of calls.

    mem_kv: per-layer (K, V) bf16, [B, PM, NH, 64] or [PM, NH, 64] (the ``past.register_step['mem_kv']``
    format), copied in; kv_start: [B] ints (first valid row per sample); rows: R, the register rows one
    call appends; kept_delta / new_delta: RoPE position change of kept and of appended rows (None = no
    rotation); theta: the RoPE base."""

    def __init__(self, mem_kv, kv_start, rows: int, kept_delta: int | None = None, new_delta: int | None = None,
                 theta: float = 10000.0):
        k0 = mem_kv[0][0]
        self.batched = k0.dim() == 4
        as4 = lambda t: (t if self.batched else t[None]).to(torch.bfloat16).contiguous()  # noqa: E731
        self.L = len(mem_kv)
        B, PM, NH, HD = as4(k0).shape
        if HD != 64:
            raise ValueError("head dim must be 64")
        if not 1 <= rows <= PM:
            raise ValueError("need 1 <= rows <= PM")
        self.B, self.PM, self.NH, self.HD, self.R = B, PM, NH, HD, rows
        dev = k0.device
        if dev.type != "cuda":
            raise ValueError("the register memory must sit on the GPU")
        for l, (k, v) in enumerate(mem_kv):
            require_device(dev, **{f"mem_kv[{l}].k": k, f"mem_kv[{l}].v": v})
        self.device = dev
        self._k = [[as4(k).clone() for k, _ in mem_kv], [torch.empty(B, PM, NH, HD, dtype=torch.bfloat16, device=dev) for _ in mem_kv]]
        self._v = [[as4(v).clone() for _, v in mem_kv], [torch.empty(B, PM, NH, HD, dtype=torch.bfloat16, device=dev) for _ in mem_kv]]
        ks = torch.as_tensor(kv_start, dtype=torch.int32).reshape(-1)
        if ks.numel() != B:
            raise ValueError("kv_start needs one entry per sample")
        # a copy: the two kv_start buffers alternate as append outputs, so the caller's tensor must not be one
        self._ks = [ks.to(dev).clone(), torch.empty(B, dtype=torch.int32, device=dev)]
        self._cur = 0
        self._shift = None if kept_delta is None else rope_delta(kept_delta, HD, theta, dev)
        self._new = None if new_delta is None else rope_delta(new_delta, HD, theta, dev)
        self._pm = torch.full((1,), PM, dtype=torch.int32, device=dev)
        self.frames = 0

    @property
    def mem_kv(self):
        """Current per-layer (K, V), in the layout given at construction."""
        c = self._cur
        if self.batched:
            return [(k, v) for k, v in zip(self._k[c], self._v[c])]
        return [(k[0], v[0]) for k, v in zip(self._k[c], self._v[c])]

    @property
    def kv_start(self) -> torch.Tensor:
        return self._ks[self._cur]

    def append_frame(self, cur_k: torch.Tensor, cur_v: torch.Tensor) -> None:
        """Append one call's register K/V ([L, B, R, NH, 64] bf16) on the current stream."""
        shape = (self.L, self.B, self.R, self.NH, self.HD)
        require_device(self.device, cur_k=cur_k, cur_v=cur_v)
        for t, nm in ((cur_k, "cur_k"), (cur_v, "cur_v")):
            if tuple(t.shape) != shape or t.dtype != torch.bfloat16 or not t.is_contiguous():
                raise ValueError(f"{nm} must be contiguous bf16 {shape}, got {tuple(t.shape)} {t.dtype}")
        src, dst = self._cur, 1 - self._cur
        a = MkxRingArgs(L=self.L, B=self.B, NH=self.NH, HD=self.HD, PM=self.PM, R=self.R)
        a.cur_k, a.cur_v = cur_k.data_ptr(), cur_v.data_ptr()
        for l in range(self.L):
            a.memk_in[l], a.memv_in[l] = self._k[src][l].data_ptr(), self._v[src][l].data_ptr()
            a.memk_out[l], a.memv_out[l] = self._k[dst][l].data_ptr(), self._v[dst][l].data_ptr()
        a.mem_stride_b = self.PM * self.NH * self.HD
        a.kv_start_in, a.kv_start_out = self._ks[src].data_ptr(), self._ks[dst].data_ptr()
        if self._shift is not None:
            a.shift_cos, a.shift_sin = self._shift[0].data_ptr(), self._shift[1].data_ptr()
        if self._new is not None:
            a.new_cos, a.new_sin = self._new[0].data_ptr(), self._new[1].data_ptr()
        check(lib().mkx_ring_append(ctypes.byref(a), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)),
              "mkx_ring_append")
        self._keep = (cur_k, cur_v)  # inputs outlive the asynchronous launch
        self._cur = dst
        self.frames += 1

    def update_past(self, past) -> None:
        """Point ``past.register_step`` at the current memory: 'mem_kv', 'kv_start' and 'cu_kv' =
        [kv_start[0], PM] (the reference reads kv_start from cu_kv[0], src/mk_expert.py:321)."""
        st = past.register_step
        st["mem_kv"] = self.mem_kv
        st["kv_start"] = self.kv_start
        st["cu_kv"] = torch.cat([self.kv_start[:1], self._pm])
