"""Host-side mirror of the reference's expert-call boundary (src/mk_expert.py:429-536).

``ExpertMegakernel(model)`` reads the REKI-shaped expert, stacks its weights exactly as the reference
does (src/mk_expert.py:445-460) and hands them to ``mkx_create``, which repacks them for the HIP
megakernel. ``run(x_t, mods, dt, past, action_dim)`` integrates Euler steps 2..N in one persistent launch
on the current stream (src/mk_expert.py:483-515); ``barriers(n_steps)`` and ``install(model)`` keep the
reference's names and meaning (:517-536). Argument checks raise ``ValueError`` where the reference
asserts; a failing library call raises ``MkxError``. There is no fallback: without libmkx.so nothing
here runs.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import MkxDims, MkxStepArgs, MkxWeights, check, lib, require_device
from .pack import LINEARS, PackedExpert, pack_expert, validate


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


class ExpertMegakernel:
    """Packs the expert weights once; ``run`` integrates Euler steps 2..N in one launch."""

    def __init__(self, model, registers_in_loop: bool | None = None, max_rows: int = 128, max_batch: int = 16,
                 max_mem_rows: int = 256, max_src_rows: int = 1 << 16):
        # stacked exactly as the reference stacks them (src/mk_expert.py:445-460); fp8 e4m3 linear weights
        # (a ``weight_q`` tensor with per-output-channel ``weight_scale`` beside each linear) go as bytes
        # plus fp32 scales, otherwise bf16
        packed = pack_expert(model)
        packed.tensors.pop("reg_tok", None)
        self._create(packed, getattr(model, "register_tokens", None), registers_in_loop, max_rows, max_batch,
                     max_mem_rows, max_src_rows)

    @classmethod
    def from_packed(cls, packed: PackedExpert, registers_in_loop: bool | None = None, max_rows: int = 128,
                    max_batch: int = 16, max_mem_rows: int = 256, max_src_rows: int = 1 << 16) -> "ExpertMegakernel":
        """A handle built from a packed expert (``pack.load_packed(path, device)``) instead of a model; its
        ``reg_tok`` tensor, when present, gives the register rows' layer-0 input."""
        self = cls.__new__(cls)
        self._create(packed, packed.tensors.get("reg_tok"), registers_in_loop, max_rows, max_batch, max_mem_rows,
                     max_src_rows)
        return self

    def _create(self, packed: PackedExpert, register_tokens, registers_in_loop, max_rows, max_batch, max_mem_rows,
                max_src_rows) -> None:
        validate(packed)
        m, t = packed.meta, packed.tensors
        self.L, self.NH, self.HD, self.I, self.A = (int(m[k]) for k in ("L", "NH", "HD", "I", "A"))
        self.H = self.NH * self.HD
        self.fp8 = packed.fp8
        self.eps, self.qk_eps = float(m["eps"]), float(m["qk_eps"])
        self.activation = _lib.ACT_SILU if m["activation"] == "silu" else _lib.ACT_GELU_TANH
        self.register_tokens = register_tokens
        self.registers_in_loop = registers_in_loop
        dev = t["wqkv"].device
        if dev.type != "cuda" or any(v.device != dev for v in t.values()):
            raise ValueError("packed expert tensors must all sit on one GPU")
        # the library reads e4m3 weights as bytes
        t = {k: (v.view(torch.uint8) if v.dtype == torch.float8_e4m3fn else v).contiguous() for k, v in t.items()}
        dims = MkxDims(L=self.L, H=self.H, NH=self.NH, HD=self.HD, I=self.I, A=self.A, max_rows=max_rows,
                       max_batch=max_batch, max_mem_rows=max_mem_rows, max_src_rows=max_src_rows,
                       weight_dtype=_lib.WEIGHTS_FP8_E4M3 if self.fp8 else _lib.WEIGHTS_BF16, activation=self.activation,
                       eps=self.eps, qk_eps=self.qk_eps)
        w = MkxWeights(**{k: _ptr(t[k]) for k in LINEARS + ("qn", "kn", "qcan", "win", "bin", "wout", "bout")})
        if self.fp8:
            for k in LINEARS:
                setattr(w, k + "_scale", _ptr(t[k + "_scale"]))
        h = ctypes.c_void_p()
        check(lib().mkx_create(ctypes.byref(dims), ctypes.byref(w), ctypes.c_void_p(_stream()), ctypes.byref(h)), "mkx_create")
        self._h = h
        self.nprog = int(lib().mkx_query(h, _lib.Q_GRID))
        self.weight_bytes = int(lib().mkx_query(h, _lib.Q_WEIGHT_BYTES))
        self.device = dev
        self.cfg = {"block": int(lib().mkx_query(h, _lib.Q_BLOCK)), "lds_bytes": int(lib().mkx_query(h, _lib.Q_LDS_BYTES)),
                    "grid": self.nprog, "PROFILE": False}

    def close(self) -> None:
        """Releases the handle's device memory now (also done at garbage collection)."""
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().mkx_destroy(h)
        self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:  # interpreter shutdown
            pass

    # ------------------------------------------------------------------------------------------
    def _check_devices(self, x_t, mods, dt, past) -> None:
        """Every tensor the launch reads must sit on the handle's GPU (checked before anything is marshalled)."""
        step = past.register_step
        tensors = {"x_t": x_t, "mods": mods, "dt": dt if torch.is_tensor(dt) else None,
                   "register_tokens": self.register_tokens}
        for key in ("kv_start", "ca_len", "cu_kv", "cu_src"):
            if torch.is_tensor(step.get(key)):
                tensors[key] = step[key]
        for key in ("sa_pe", "ca_pe", "sa_pe_first", "ca_pe_first"):
            for i, t in enumerate(step.get(key, ())):
                tensors[f"{key}[{i}]"] = t
        for name, pairs in (("mem_kv", step["mem_kv"]), ("cross_attn_kv", past.cross_attn_kv)):
            for l, (k, v) in enumerate(pairs):
                tensors[f"{name}[{l}].k"], tensors[f"{name}[{l}].v"] = k, v
        require_device(self.device, **tensors)

    def set_operand_shift(self, shift: int) -> None:
        """AdaRMS operands of later launches stored as y 2^-shift (0 = the default, every result bit as without
        it): the remedy when ``check`` raises MKX_ERANGE, a residual stream beyond the fp16 operand range."""
        check(lib().mkx_set_operand_shift(self._h, int(shift)), "mkx_set_operand_shift")

    @property
    def operand_shift(self) -> int:
        return int(lib().mkx_query(self._h, _lib.Q_OPERAND_SHIFT))

    def run_checked(self, x_t: torch.Tensor, mods: torch.Tensor, dt, past, action_dim: int, shift_step: int = 8,
                    max_shift: int = 24) -> torch.Tensor:
        """``run``, then ``check`` (synchronises); a launch that overflowed an fp16 operand (MKX_ERANGE) is run
        again with the operand shift raised by ``shift_step``, up to ``max_shift``, and the handle keeps the shift
        that worked. Any other error is raised."""
        while True:
            x = self.run(x_t, mods, dt, past, action_dim)
            try:
                self.check()
                return x
            except _lib.MkxError as e:
                shift = self.operand_shift
                if e.status != _lib.ERANGE or shift + shift_step > max_shift:
                    raise
                self.set_operand_shift(shift + shift_step)

    def set_spin_limit(self, polls: int | None) -> None:
        """Spin bound (polls) of every wait of later launches; None restores the default (about 0.5 s)."""
        check(lib().mkx_set_spin_limit(self._h, 0 if polls is None else int(polls)), "mkx_set_spin_limit")

    def _args(self, x_t, mods, dt, past, action_dim, n_steps, mod_row0, first, cur_k=None, cur_v=None):
        self._check_devices(x_t, mods, dt, past)
        step = past.register_step
        if x_t.dim() != 3 or x_t.shape[2] != self.A:
            raise ValueError(f"x_t must be [B, T, {self.A}], got {tuple(x_t.shape)}")
        x = x_t.float().contiguous()
        B, T = x.shape[0], x.shape[1]
        if not 1 <= action_dim <= self.A:
            raise ValueError("action_dim out of range")
        m = mods.float()
        if m.dim() == 2:
            if B != 1:
                raise ValueError("mods [N, MODW] is for batch 1; pass [B, N, MODW]")
            m = m[None]
        m = m.contiguous()
        modw = 9 * self.L * self.H + 2 * self.H
        if m.shape[0] != B or m.shape[2] < modw:
            raise ValueError(f"mods must be [B, N, >= {modw}], got {tuple(m.shape)}")
        if m.shape[1] < mod_row0 + n_steps:
            raise ValueError("mods has fewer rows than the steps to run")
        sa_cos, sa_sin = step["sa_pe_first" if first and "sa_pe_first" in step else "sa_pe"]
        ca_cos, ca_sin = step["ca_pe_first" if first and "ca_pe_first" in step else "ca_pe"]
        sa_cos, sa_sin, ca_cos, ca_sin = (t.float().contiguous() for t in (sa_cos, sa_sin, ca_cos, ca_sin))
        m_q = sa_cos.shape[0]
        if sa_cos.shape != (m_q, self.HD) or ca_cos.shape != (m_q, self.HD) or m_q < T:
            raise ValueError(f"RoPE tables must be [M_q >= T, {self.HD}]: {tuple(sa_cos.shape)}, {tuple(ca_cos.shape)}")
        R = m_q - T
        reg = None
        if R > 0:
            if self.register_tokens is None or self.register_tokens.shape[0] != R:
                raise ValueError("RoPE tables cover register rows but the model has no matching register_tokens")
            reg = self.register_tokens.to(torch.bfloat16).contiguous()
        mem_kv = step["mem_kv"]
        ca_kv = past.cross_attn_kv
        if len(mem_kv) != self.L or len(ca_kv) != self.L:
            raise ValueError("caches must hold one (k, v) pair per layer")

        def bcheck(t, name):
            if t.dtype != torch.bfloat16 or not t.is_contiguous():
                raise ValueError(f"{name} must be contiguous bf16")
            t4 = t if t.dim() == 4 else t[None]
            if t4.shape[0] != B or t4.shape[2] != self.NH or t4.shape[3] != self.HD:
                raise ValueError(f"{name} must be [B, rows, {self.NH}, {self.HD}], got {tuple(t.shape)}")
            return t4

        mk = [bcheck(k, "memory K") for k, _ in mem_kv]
        mv = [bcheck(v, "memory V") for _, v in mem_kv]
        kc = [bcheck(k, "source K") for k, _ in ca_kv]
        vc = [bcheck(v, "source V") for _, v in ca_kv]
        PM, SP = mk[0].shape[1], kc[0].shape[1]
        if any(t.shape != mk[0].shape for t in mk + mv) or any(t.shape != kc[0].shape for t in kc + vc):
            raise ValueError("per-layer caches must share one shape")
        # kv_start[B] / ca_len[B] when the past holds them (the register ring keeps kv_start in device buffers
        # that its append updates, so a captured launch reads the current value); otherwise, batch 1 in the
        # reference layout, kv_start = cu_kv[0] and S = cu_src[1] (src/mk_expert.py:321-322)
        if B != 1 and not ("kv_start" in step and "ca_len" in step):
            raise ValueError("batched caches need register_step['kv_start'] and ['ca_len']")
        if "kv_start" in step:
            kvs = step["kv_start"].to(torch.int32).contiguous()
            kv_ptr = kvs.data_ptr()
        else:
            kvs = step["cu_kv"].to(torch.int32).contiguous()
            kv_ptr = kvs.data_ptr()
        if "ca_len" in step:
            cal = step["ca_len"].to(torch.int32).contiguous()
            ca_ptr = cal.data_ptr()
        else:
            cal = step["cu_src"].to(torch.int32).contiguous()
            ca_ptr = cal.data_ptr() + 4
        x_out = torch.empty_like(x)
        dtt = dt.float().reshape(-1)[:1].contiguous() if torch.is_tensor(dt) else torch.full((1,), float(dt), device=x.device)
        a = MkxStepArgs()
        a.x_in, a.x_out = x.data_ptr(), x_out.data_ptr()
        a.mods, a.mods_stride_b, a.mods_stride_step, a.mod_row0 = m.data_ptr(), m.stride(0), m.stride(1), mod_row0
        a.dt = dtt.data_ptr()
        for l in range(self.L):
            a.memk[l], a.memv[l], a.kca[l], a.vca[l] = mk[l].data_ptr(), mv[l].data_ptr(), kc[l].data_ptr(), vc[l].data_ptr()
        a.mem_stride_b, a.src_stride_b = mk[0].stride(0), kc[0].stride(0)
        a.kv_start, a.ca_len = kv_ptr, ca_ptr
        a.sa_cos, a.sa_sin, a.ca_cos, a.ca_sin = sa_cos.data_ptr(), sa_sin.data_ptr(), ca_cos.data_ptr(), ca_sin.data_ptr()
        a.reg_tok = _ptr(reg)
        a.cur_k, a.cur_v = _ptr(cur_k), _ptr(cur_v)
        a.n_steps, a.action_dim, a.T_act, a.R_reg, a.B, a.PM, a.SP = n_steps, action_dim, T, R, B, PM, SP
        keep = (x, m, dtt, sa_cos, sa_sin, ca_cos, ca_sin, reg, kvs, cal, mk, mv, kc, vc)
        return a, x_out, keep

    def run(self, x_t: torch.Tensor, mods: torch.Tensor, dt, past, action_dim: int) -> torch.Tensor:
        """x_t: [B, T, A] fp32 after Euler step 1; mods: [N, MODW] (B = 1) or [B, N, MODW], row 0 = step 1
        (used already); returns x_t after step N (padded dims as the reference: 0 + dt * v)."""
        n_steps = (mods.shape[-2]) - 1
        if n_steps < 1:
            raise ValueError("mods must hold at least two rows (step 1 and one more)")
        a, x_out, keep = self._args(x_t, mods, dt, past, action_dim, n_steps, 1, first=False)
        check(lib().mkx_run(self._h, ctypes.byref(a), ctypes.c_void_p(_stream())), "mkx_run")
        self._keep = keep  # inputs must outlive the asynchronous launch
        return x_out

    def plan(self, x_t: torch.Tensor, mods: torch.Tensor, dt, past, action_dim: int) -> "LaunchPlan":
        """Marshal the arguments of ``run`` once; ``LaunchPlan.launch()`` then enqueues the same launch with
        no host-side work beyond the library call (the analogue of replaying the reference's captured graph,
        profile_breakdown.py:107-130). The plan keeps its inputs alive; the output is ``plan.x_out``."""
        n_steps = (mods.shape[-2]) - 1
        a, x_out, keep = self._args(x_t, mods, dt, past, action_dim, n_steps, 1, first=False)
        return LaunchPlan(self, a, x_out, keep)

    def run_first(self, noise: torch.Tensor, mods1: torch.Tensor, dt, past, action_dim: int):
        """Euler step 1 over [action rows || register rows] (what REKI's _expert_first_step computes):
        returns (x after step 1, cur_k, cur_v) with cur_k/cur_v [L, B, R, NH, HD] bf16, the register rows'
        normed+rotated K and V of each layer."""
        R = 0 if self.register_tokens is None else self.register_tokens.shape[0]
        B = noise.shape[0]
        cur_k = torch.empty(self.L, B, R, self.NH, self.HD, device=noise.device, dtype=torch.bfloat16) if R else None
        cur_v = torch.empty_like(cur_k) if R else None
        a, x_out, keep = self._args(noise, mods1, dt, past, action_dim, 1, 0, first=True, cur_k=cur_k, cur_v=cur_v)
        check(lib().mkx_run(self._h, ctypes.byref(a), ctypes.c_void_p(_stream())), "mkx_run")
        self._keep = keep
        return x_out, cur_k, cur_v

    def can_run_all(self, past) -> bool:
        """Whether Euler step 1 and steps 2..N can share one launch: every step has the same own rows (the
        register rows are in the loop), so step 1's RoPE tables are the later steps' tables."""
        st = past.register_step
        if "sa_pe_first" not in st:
            return True
        pairs = list(zip(st["sa_pe_first"], st["sa_pe"])) + list(zip(st["ca_pe_first"], st["ca_pe"]))
        key = tuple((a.data_ptr(), b.data_ptr(), tuple(a.shape), tuple(b.shape)) for a, b in pairs)
        cache = self.__dict__.setdefault("_run_all_ok", {})
        if key not in cache:  # compared once per set of tables (the comparison synchronises the device)
            cache[key] = all(a.shape == b.shape and torch.equal(a, b) for a, b in pairs)
        return cache[key]

    def run_all(self, noise: torch.Tensor, mods: torch.Tensor, dt, past, action_dim: int):
        """Euler steps 1..N in one launch (mods rows 0..N-1): returns (x after step N, cur_k, cur_v) like
        ``run_first`` followed by ``run``, which it matches bit for bit. Requires ``can_run_all(past)``."""
        if not self.can_run_all(past):
            raise ValueError("step 1 has other own rows than steps 2..N (register rows outside the loop): use run_first + run")
        n_steps = mods.shape[-2]
        R = 0 if self.register_tokens is None else self.register_tokens.shape[0]
        B = noise.shape[0]
        cur_k = torch.empty(self.L, B, R, self.NH, self.HD, device=noise.device, dtype=torch.bfloat16) if R else None
        cur_v = torch.empty_like(cur_k) if R else None
        a, x_out, keep = self._args(noise, mods, dt, past, action_dim, n_steps, 0, first=True, cur_k=cur_k, cur_v=cur_v)
        check(lib().mkx_run(self._h, ctypes.byref(a), ctypes.c_void_p(_stream())), "mkx_run")
        self._keep = keep
        return x_out, cur_k, cur_v

    def barriers(self, n_steps: int) -> int:
        return int(lib().mkx_barriers(self._h, n_steps))

    def barrier_arrivals(self) -> int:
        """Workgroup arrivals at grid barriers since the previous call (synchronises the device); equals
        nprog * barriers(n_steps) after one launch (the reference's check, test_mk.py:44-45)."""
        return int(lib().mkx_query(self._h, _lib.Q_BARRIER_COUNT))

    def check(self) -> None:
        """Synchronise and raise MkxError if a barrier wait of the last launch timed out."""
        check(lib().mkx_check(self._h, ctypes.c_void_p(_stream())), "mkx_check")

    def set_profile(self, n_steps: int | None) -> None:
        """Per-barrier timestamps for later launches of up to n_steps steps (None turns them off)."""
        if n_steps is None:
            check(lib().mkx_set_profile(self._h, None, 0), "mkx_set_profile")
            self._prof = None
        else:
            self._prof = torch.zeros(self.barriers(n_steps) + 2, dtype=torch.int64, device=self.device)
            check(lib().mkx_set_profile(self._h, ctypes.c_void_p(self._prof.data_ptr()), self._prof.numel()), "mkx_set_profile")
        self.cfg["PROFILE"] = n_steps is not None

    def barrier_timestamps(self) -> torch.Tensor:
        """ns clock taken by workgroup 0 at launch start (entry 0) and after each barrier of the last
        profiled launch."""
        if getattr(self, "_prof", None) is None:
            raise RuntimeError("profiling is off")
        torch.cuda.synchronize()
        return self._prof.cpu()


class LaunchPlan:
    """A marshalled ``run`` call: launch() enqueues it on the current stream."""

    def __init__(self, mk: ExpertMegakernel, args: MkxStepArgs, x_out: torch.Tensor, keep):
        self.mk, self.args, self.x_out, self._keep = mk, args, x_out, keep
        self._ref = ctypes.byref(self.args)

    def launch(self, stream: int | None = None) -> torch.Tensor:
        s = _stream() if stream is None else stream
        check(lib().mkx_run(self.mk._h, self._ref, ctypes.c_void_p(s)), "mkx_run")
        return self.x_out


def install(model, fold_first_step: bool = False) -> ExpertMegakernel:
    """Route the model's ``_expert_actions`` through the megakernel for steps 2..N; modulations and step 1
    stay the model's own callables (src/mk_expert.py:521-536). With ``fold_first_step`` (and when the
    register rows are in the loop) step 1 runs in the same launch as steps 2..N instead."""
    mk = ExpertMegakernel(model)
    model._mk = mk

    def _expert_actions(noise, cross_attn_cache, register_cache, state_cond, action_dim, num_steps):
        mods, dt = model._step_modulations(num_steps, state_cond)
        if fold_first_step and num_steps > 1 and mk.can_run_all(cross_attn_cache):
            return mk.run_all(noise, mods, dt, cross_attn_cache, action_dim)
        x_t, cur_k, cur_v = model._expert_first_step(noise, cross_attn_cache, register_cache, mods[..., :1, :], dt, action_dim)
        if num_steps > 1:
            x_t = mk.run(x_t, mods, dt, cross_attn_cache, action_dim)
        return x_t, cur_k, cur_v

    model._expert_actions = _expert_actions
    return mk
