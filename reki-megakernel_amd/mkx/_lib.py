"""ctypes binding of libmkx.so (include/mkx.h). Loading fails loudly when the library is missing: there is
no fallback path."""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmkx.so")
MAX_LAYERS = 32

OK, EINVAL, ENORESIDENT, EHIP, ETIMEOUT, ENOMEM, EUNSUPPORTED, ERANGE = range(8)
WEIGHTS_BF16, WEIGHTS_FP8_E4M3 = 0, 1
ACT_SILU, ACT_GELU_TANH = 0, 1
Q_GRID, Q_BLOCK, Q_BARRIER_COUNT, Q_ERROR_FLAG, _Q_RESERVED, Q_PROFILE_LEN, Q_WEIGHT_BYTES, Q_LDS_BYTES, Q_GEMM_FORM, \
    Q_OPERAND_SHIFT = range(10)

EXPORTS = ("mkx_create", "mkx_run", "mkx_check", "mkx_barriers", "mkx_set_profile", "mkx_query", "mkx_destroy",
           "mkx_last_error", "mkx_status_string", "mkx_abi_version", "mkx_ring_append", "mkx_source_create", "mkx_source_run", "mkx_source_destroy",
           "mkx_modulations", "mkx_set_spin_limit", "mkx_source_run_noalloc", "mkx_modulation_input", "mkx_probe",
           "mkx_set_operand_shift")
PROBE_BARRIER, PROBE_HANDOFF = 0, 1

_vp = ctypes.c_void_p


class MkxDims(ctypes.Structure):
    _fields_ = [("L", ctypes.c_int32), ("H", ctypes.c_int32), ("NH", ctypes.c_int32), ("HD", ctypes.c_int32),
                ("I", ctypes.c_int32), ("A", ctypes.c_int32), ("max_rows", ctypes.c_int32),
                ("max_batch", ctypes.c_int32), ("max_mem_rows", ctypes.c_int32), ("max_src_rows", ctypes.c_int32),
                ("weight_dtype", ctypes.c_int32), ("activation", ctypes.c_int32), ("eps", ctypes.c_float),
                ("qk_eps", ctypes.c_float)]


class MkxWeights(ctypes.Structure):
    _fields_ = [(n, _vp) for n in ("wqkv", "wo", "wqca", "woca", "wg", "wu", "wd",
                                   "wqkv_scale", "wo_scale", "wqca_scale", "woca_scale", "wg_scale", "wu_scale", "wd_scale",
                                   "qn", "kn", "qcan", "win", "bin", "wout", "bout")]


class MkxStepArgs(ctypes.Structure):
    _fields_ = [("x_in", _vp), ("x_out", _vp), ("mods", _vp), ("mods_stride_b", ctypes.c_int64),
                ("mods_stride_step", ctypes.c_int64), ("mod_row0", ctypes.c_int32), ("dt", _vp),
                ("memk", _vp * MAX_LAYERS), ("memv", _vp * MAX_LAYERS), ("mem_stride_b", ctypes.c_int64),
                ("kv_start", _vp), ("kca", _vp * MAX_LAYERS), ("vca", _vp * MAX_LAYERS),
                ("src_stride_b", ctypes.c_int64), ("ca_len", _vp), ("sa_cos", _vp), ("sa_sin", _vp),
                ("ca_cos", _vp), ("ca_sin", _vp), ("reg_tok", _vp), ("cur_k", _vp), ("cur_v", _vp),
                ("n_steps", ctypes.c_int32), ("action_dim", ctypes.c_int32), ("T_act", ctypes.c_int32),
                ("R_reg", ctypes.c_int32), ("B", ctypes.c_int32), ("PM", ctypes.c_int32), ("SP", ctypes.c_int32)]


class MkxRingArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("L", "B", "NH", "HD", "PM", "R")] + \
               [("cur_k", _vp), ("cur_v", _vp), ("memk_in", _vp * MAX_LAYERS), ("memv_in", _vp * MAX_LAYERS),
                ("memk_out", _vp * MAX_LAYERS), ("memv_out", _vp * MAX_LAYERS), ("mem_stride_b", ctypes.c_int64),
                ("kv_start_in", _vp), ("kv_start_out", _vp), ("shift_cos", _vp), ("shift_sin", _vp),
                ("new_cos", _vp), ("new_sin", _vp)]


class MkxSourceDims(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("L", "NH", "HD", "C", "max_rows")] + [("eps", ctypes.c_float)]


class MkxSourceArgs(ctypes.Structure):
    _fields_ = [("B", ctypes.c_int32), ("SP", ctypes.c_int32), ("ctx", _vp), ("ca_len", _vp), ("cos", _vp), ("sin", _vp),
                ("kca", _vp * MAX_LAYERS), ("vca", _vp * MAX_LAYERS), ("src_stride_b", ctypes.c_int64)]


class MkxModprojArgs(ctypes.Structure):
    _fields_ = [("R", ctypes.c_int32), ("K", ctypes.c_int32), ("N", ctypes.c_int32), ("c", _vp), ("c_stride", ctypes.c_int64),
                ("w", _vp), ("bias", _vp), ("out", _vp), ("out_stride", ctypes.c_int64), ("w_fragment_order", ctypes.c_int32)]


class MkxModinArgs(ctypes.Structure):
    _fields_ = [("N", ctypes.c_int32), ("B", ctypes.c_int32), ("H", ctypes.c_int32), ("tdim", ctypes.c_int32),
                ("t1_w", _vp), ("t1_b", _vp), ("t2_w", _vp), ("t2_b", _vp), ("state_cond", _vp),
                ("sc_stride", ctypes.c_int64), ("out", _vp), ("out_stride_b", ctypes.c_int64),
                ("out_stride_k", ctypes.c_int64)]


class MkxProbeArgs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("kind", "n", "bytes", "fan", "reps", "timed_out")] + \
               [("xcd_first", ctypes.c_int32 * 2), ("us_median", ctypes.c_double), ("us_min", ctypes.c_double)]


class MkxError(RuntimeError):
    def __init__(self, status: int, where: str, detail: str):
        super().__init__(f"{where}: mkx status {status} ({detail})")
        self.status = status


_LIB = None


def lib() -> ctypes.CDLL:
    """Load libmkx.so (once). Raises when it has not been built: the expert has no other implementation."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build the HIP library first (python -c 'import __graft_entry__ as g; g.build()')")
        L = ctypes.CDLL(LIB_PATH)
        L.mkx_create.argtypes = [ctypes.POINTER(MkxDims), ctypes.POINTER(MkxWeights), _vp, ctypes.POINTER(_vp)]
        L.mkx_run.argtypes = [_vp, ctypes.POINTER(MkxStepArgs), _vp]
        L.mkx_check.argtypes = [_vp, _vp]
        L.mkx_barriers.argtypes = [_vp, ctypes.c_int32]
        L.mkx_barriers.restype = ctypes.c_int64
        L.mkx_set_profile.argtypes = [_vp, _vp, ctypes.c_int32]
        L.mkx_query.argtypes = [_vp, ctypes.c_int32]
        L.mkx_query.restype = ctypes.c_int64
        L.mkx_destroy.argtypes = [_vp]
        L.mkx_last_error.restype = ctypes.c_char_p
        L.mkx_status_string.argtypes = [ctypes.c_int]
        L.mkx_status_string.restype = ctypes.c_char_p
        L.mkx_abi_version.restype = ctypes.c_int32
        L.mkx_ring_append.argtypes = [ctypes.POINTER(MkxRingArgs), _vp]
        L.mkx_source_create.argtypes = [ctypes.POINTER(MkxSourceDims), _vp, _vp, _vp, _vp, ctypes.POINTER(_vp)]
        L.mkx_source_run.argtypes = [_vp, ctypes.POINTER(MkxSourceArgs), _vp]
        L.mkx_source_run_noalloc.argtypes = [_vp, ctypes.POINTER(MkxSourceArgs), _vp]
        L.mkx_source_destroy.argtypes = [_vp]
        L.mkx_modulations.argtypes = [ctypes.POINTER(MkxModprojArgs), _vp]
        L.mkx_modulation_input.argtypes = [ctypes.POINTER(MkxModinArgs), _vp]
        L.mkx_set_spin_limit.argtypes = [_vp, ctypes.c_uint32]
        L.mkx_set_operand_shift.argtypes = [_vp, ctypes.c_int32]
        L.mkx_probe.argtypes = [ctypes.POINTER(MkxProbeArgs), _vp]
        _LIB = L
    return _LIB


def require_device(device, **tensors) -> None:
    """Raise ValueError unless every given tensor (None skipped) sits on ``device``, the GPU the handle was
    made for: the library takes raw device pointers, so a host or other-device tensor would be read or
    written by the GPU as if it were this device's memory."""
    for name, t in tensors.items():
        if t is not None and t.device != device:
            raise ValueError(f"{name} is on {t.device}, the handle's tensors must be on {device}")


def check(status: int, where: str) -> None:
    if status != OK:
        L = lib()
        raise MkxError(status, where, f"{L.mkx_status_string(status).decode()}: {L.mkx_last_error().decode()}")
