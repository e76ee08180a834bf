"""The C ABI library (no GPU needed): it loads, exports every entry point include/mkx.h declares, reports
errors through status codes, and validates arguments before touching the device."""
import ctypes
import os
import re

import pytest

from mkx import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "mkx.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mkx_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = header_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(L, n), n
    assert set(_lib.EXPORTS) == set(names)


def test_abi_version_and_status_strings():
    L = _lib.lib()
    assert L.mkx_abi_version() == 1
    for s in range(8):
        assert L.mkx_status_string(s).decode() != "unknown status"
    assert L.mkx_status_string(_lib.ETIMEOUT).decode().startswith("grid barrier")
    assert "fp16" in L.mkx_status_string(_lib.ERANGE).decode()


def _dims(**over):
    d = dict(L=10, H=768, NH=12, HD=64, I=3072, A=32, max_rows=64, max_batch=1, max_mem_rows=96, max_src_rows=300,
             weight_dtype=_lib.WEIGHTS_BF16, activation=_lib.ACT_SILU, eps=1e-6, qk_eps=1e-6)
    d.update(over)
    return _lib.MkxDims(**d)


@pytest.mark.parametrize("over,status", [
    (dict(L=0), _lib.EINVAL), (dict(L=33), _lib.EINVAL), (dict(HD=128), _lib.EUNSUPPORTED),
    (dict(NH=10), _lib.EINVAL), (dict(A=16), _lib.EUNSUPPORTED), (dict(weight_dtype=7), _lib.EUNSUPPORTED),
    (dict(activation=5), _lib.EINVAL), (dict(max_batch=0), _lib.EINVAL), (dict(max_rows=200), _lib.EINVAL),
    (dict(max_mem_rows=300), _lib.EINVAL), (dict(H=512, NH=8), _lib.EUNSUPPORTED), (dict(H=128, NH=2, I=256), _lib.EUNSUPPORTED),
])
def test_create_validates_dims_before_touching_the_device(over, status):
    L = _lib.lib()
    h = ctypes.c_void_p()
    w = _lib.MkxWeights()
    rc = L.mkx_create(ctypes.byref(_dims(**over)), ctypes.byref(w), None, ctypes.byref(h))
    assert rc == status, L.mkx_last_error()
    assert not h.value
    assert L.mkx_last_error().decode()


def test_create_rejects_null_weights_and_null_arguments():
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.mkx_create(ctypes.byref(_dims()), ctypes.byref(_lib.MkxWeights()), None, ctypes.byref(h)) == _lib.EINVAL
    assert L.mkx_create(None, None, None, ctypes.byref(h)) == _lib.EINVAL
    assert L.mkx_run(None, None, None) == _lib.EINVAL
    assert L.mkx_destroy(None) == _lib.OK
    assert L.mkx_barriers(None, 9) == -1


def test_struct_layouts_match_header_sizes():
    # mkx_step_args: 4 per-layer tables of MKX_MAX_LAYERS pointers dominate the size
    assert ctypes.sizeof(_lib.MkxStepArgs) > 4 * 32 * 8
    assert ctypes.sizeof(_lib.MkxDims) == 14 * 4
    assert ctypes.sizeof(_lib.MkxWeights) == 21 * 8


def test_every_args_struct_matches_the_header_layout(tmp_path):
    # sizes and field offsets of every struct in include/mkx.h, as a C compiler lays them out, against the
    # ctypes mirrors the Python side passes to the library
    import subprocess
    structs = {"mkx_dims": _lib.MkxDims, "mkx_weights": _lib.MkxWeights, "mkx_step_args": _lib.MkxStepArgs,
               "mkx_ring_args": _lib.MkxRingArgs, "mkx_source_dims": _lib.MkxSourceDims,
               "mkx_source_args": _lib.MkxSourceArgs, "mkx_modproj_args": _lib.MkxModprojArgs,
               "mkx_modin_args": _lib.MkxModinArgs, "mkx_probe_args": _lib.MkxProbeArgs}
    lines = ['#include <stdio.h>', '#include "mkx.h"', "int main(void) {"]
    for cname, cls in structs.items():
        lines.append(f'  printf("{cname} size %zu\\n", sizeof({cname}));')
        for f, _ in cls._fields_:
            lines.append(f'  printf("{cname} {f} %zu\\n", offsetof({cname}, {f}));')
    lines += ["  return 0;", "}"]
    src, exe = tmp_path / "layout.c", tmp_path / "layout"
    src.write_text("\n".join(lines))
    subprocess.run(["gcc", "-std=c11", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = {tuple(ln.split()[:2]): int(ln.split()[2]) for ln in out if ln}
    for cname, cls in structs.items():
        assert got[(cname, "size")] == ctypes.sizeof(cls), cname
        for f, _ in cls._fields_:
            assert got[(cname, f)] == getattr(cls, f).offset, (cname, f)


def test_spin_limit_setter_rejects_a_null_handle():
    L = _lib.lib()
    assert L.mkx_set_spin_limit(None, 5) == _lib.EINVAL


def test_operand_shift_setter_rejects_a_null_handle():
    L = _lib.lib()
    assert L.mkx_set_operand_shift(None, 8) == _lib.EINVAL
    assert L.mkx_query(None, _lib.Q_OPERAND_SHIFT) == -1


class _Past:
    def __init__(self, step, ca):
        self.register_step, self.cross_attn_kv = step, ca


def test_host_tensors_are_refused_before_any_launch():
    # the library takes raw device pointers: host tensors must raise ValueError before anything is marshalled
    import torch
    from mkx.mk_expert import ExpertMegakernel
    from mkx.modulations import ModulationProjection
    mk = ExpertMegakernel.__new__(ExpertMegakernel)  # no handle: the check must come before any library call
    mk.L, mk.NH, mk.HD, mk.H, mk.A, mk.register_tokens = 1, 1, 64, 64, 32, None
    mk.device, mk._h = torch.device("cuda", 0), None
    bf = torch.bfloat16
    kv = (torch.zeros(1, 8, 1, 64, dtype=bf), torch.zeros(1, 8, 1, 64, dtype=bf))
    pe = (torch.zeros(2, 64), torch.zeros(2, 64))
    step = {"mem_kv": [kv], "cu_kv": torch.tensor([0, 8], dtype=torch.int32),
            "cu_src": torch.tensor([0, 8], dtype=torch.int32), "sa_pe": pe, "ca_pe": pe}
    past = _Past(step, [kv])
    with pytest.raises(ValueError, match="x_t is on cpu"):
        mk.run(torch.zeros(1, 2, 32), torch.zeros(2, 9 * 64 + 2 * 64), -0.1, past, 7)
    with pytest.raises(ValueError, match="GPU"):
        ModulationProjection(torch.zeros(32, 64), torch.zeros(32))
    from mkx.modulations import StepModulations
    with pytest.raises(ValueError, match="GPU"):
        StepModulations(torch.zeros(256, 32), torch.zeros(256), torch.zeros(256, 256), torch.zeros(256),
                        torch.zeros(2 * 256, 256), torch.zeros(2 * 256))


def test_modulation_input_rejects_bad_arguments_without_launching():
    L = _lib.lib()
    assert L.mkx_modulation_input(None, None) == _lib.EINVAL
    a = _lib.MkxModinArgs(N=10, B=1, H=768, tdim=256, sc_stride=768, out_stride_b=7680, out_stride_k=768)
    assert L.mkx_modulation_input(ctypes.byref(a), None) == _lib.EINVAL  # NULL pointers
    a.H = 640
    assert L.mkx_modulation_input(ctypes.byref(a), None) == _lib.EUNSUPPORTED
    a.H, a.tdim = 768, 48
    assert L.mkx_modulation_input(ctypes.byref(a), None) == _lib.EUNSUPPORTED
    a.tdim, a.N = 256, 0
    assert L.mkx_modulation_input(ctypes.byref(a), None) == _lib.EINVAL


def test_query_keys_match_the_header():
    """mkx_query_key values in include/mkx.h equal the binding's constants (a drifted key would query
    something else without any error)."""
    text = open(os.path.join(ROOT, "include", "mkx.h")).read()
    keys = dict((k, int(v)) for k, v in re.findall(r"\bMKX_(Q_[A-Z_]+)\s*=\s*(\d+)", text))
    assert keys, "no query keys found"
    for name, val in keys.items():
        assert getattr(_lib, name) == val, name
    assert keys["Q_GEMM_FORM"] == 8 and keys["Q_OPERAND_SHIFT"] == 9


@pytest.mark.parametrize("over", [dict(kind=5), dict(n=3), dict(n=0), dict(n=4096), dict(reps=0), dict(bytes=1000)])
def test_probe_validates_arguments_before_touching_the_device(over):
    L = _lib.lib()
    a = dict(kind=_lib.PROBE_HANDOFF, n=200, bytes=24576, fan=1, reps=3)
    a.update(over)
    args = _lib.MkxProbeArgs(**a)
    assert L.mkx_probe(ctypes.byref(args), None) == _lib.EINVAL
    assert "mkx_probe" in L.mkx_last_error().decode()
    assert L.mkx_probe(None, None) == _lib.EINVAL
