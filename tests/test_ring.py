"""The register-memory ring's oracle (CPU), and the C ABI's argument checks for ``mkx_ring_append`` and
``mkx_source_create`` / ``mkx_source_run`` and ``mkx_modulations``.

The oracle is pinned by a row-by-row restatement, by RoPE's composition law, by the memory that
``register_prepare`` builds from shifted states, and by the kv_start sequence over frames."""
import ctypes
from dataclasses import replace

import pytest
import torch

from _cases import TINY
from mkx import _lib, synthetic as SY
from mkx.ring import rope_delta
from oracle.ring_ref import ring_append, ring_append_loops, rope_rotate


def _rand(shape, g):
    return torch.randn(*shape, generator=g).to(torch.bfloat16)


def _tab(delta):
    return rope_delta(delta, 64, device="cpu")


@pytest.mark.parametrize("R,tables", [(3, True), (3, False), (8, True), (1, True)])
def test_vectorised_oracle_equals_row_loops(R, tables):
    g = torch.Generator().manual_seed(R)
    L, B, PM, NH = 2, 5, 8, 2
    memk, memv = _rand((L, B, PM, NH, 64), g), _rand((L, B, PM, NH, 64), g)
    cur_k, cur_v = _rand((L, B, R, NH, 64), g), _rand((L, B, R, NH, 64), g)
    ks = torch.tensor([0, 5, PM, 11, -2])  # valid, partial, empty, clamped above, clamped below
    sh, nw = (_tab(-R), _tab(-7)) if tables else (None, None)
    a = ring_append(memk, memv, cur_k, cur_v, ks, sh, nw)
    b = ring_append_loops(memk, memv, cur_k, cur_v, ks, sh, nw)
    for x, y in zip(a, b):
        assert x.dtype == y.dtype and torch.equal(x, y)
    assert a[2].tolist() == [0, max(5 - R, 0), PM - R, PM - R, 0]


def test_rotation_identity_and_composition():
    g = torch.Generator().manual_seed(1)
    x = _rand((64, 4, 64), g)
    assert torch.equal(rope_rotate(x, *_tab(0)), x)  # cos 1, sin 0: exact
    for a, b in ((5, -5), (-32, 10), (96, -37)):
        two = rope_rotate(rope_rotate(x, *_tab(a)), *_tab(b)).float()
        one = rope_rotate(x, *_tab(a + b)).float()
        pn = torch.sqrt(one[..., :32] ** 2 + one[..., 32:] ** 2).repeat(1, 1, 2)
        assert ((two - one).abs() <= 2.0 ** -6 * pn + 1e-6).all(), (a, b)
    # against a complex-number rotation in float64: pair (x_d, x_{d+32}) times e^{i theta_d}
    xf = x.double()
    z = torch.complex(xf[..., :32], xf[..., 32:])
    inv = 10000.0 ** (-torch.arange(0, 64, 2, dtype=torch.float64) / 64)
    zr = z * torch.exp(1j * inv * 17)
    want = torch.cat([zr.real, zr.imag], -1)
    assert (rope_rotate(x, *_tab(17)).double() - want).abs().max() <= 2.0 ** -7 * want.abs().max()


def test_append_equals_prepare_of_shifted_states():
    """Memory after one append equals the memory register_prepare builds from the states shifted by one
    frame: kept rows turned back by R positions, the call's register rows (K rotated at PM + T + r) turned
    to rows PM - R + r. A wrong delta or sign fails by orders of magnitude."""
    cfg = replace(TINY, B=2, kv_start=0)
    model = SY.SyntheticReki(cfg, SY.make_weights(cfg, 0), device="cpu")
    g = torch.Generator().manual_seed(3)
    PM, T, R = cfg.PM, cfg.T_act, cfg.R_reg
    states = torch.randn(2, PM + T + R, cfg.H, generator=g)
    ctx = SY.make_inputs(cfg)["ctx"]
    stack = lambda p, i: torch.stack([kv[i] for kv in p.register_step["mem_kv"]])  # noqa: E731
    big = model.register_prepare(ctx, states, kv_start=[0, 0])  # rows at positions 0 .. PM + T + R - 1
    K, V = stack(big, 0), stack(big, 1)
    exp = model.register_prepare(ctx, torch.cat([states[:, R:PM], states[:, PM + T:]], 1), kv_start=[0, 0])
    ek, ev = stack(exp, 0).float(), stack(exp, 1)
    pn = torch.sqrt(ek[..., :32] ** 2 + ek[..., 32:] ** 2).repeat(1, 1, 1, 1, 2)
    ks0 = torch.zeros(2, dtype=torch.int32)
    ok, ov, ks = ring_append(K[:, :, :PM], V[:, :, :PM], K[:, :, PM + T:], V[:, :, PM + T:], ks0, _tab(-R), _tab(-(T + R)))
    assert torch.equal(ov, ev) and ks.tolist() == [0, 0]
    assert ((ok.float() - ek).abs() <= 2.0 ** -6 * pn + 1e-6).all()
    bad, _, _ = ring_append(K[:, :, :PM], V[:, :, :PM], K[:, :, PM + T:], V[:, :, PM + T:], ks0, _tab(R), _tab(-(T + R)))
    assert (bad.float() - ek).abs().max() > 0.5


def test_kv_start_over_frames_and_zeroed_rows():
    g = torch.Generator().manual_seed(4)
    L, B, R, NH = 1, 1, 4, 2
    PM = 3 * R
    memk = torch.zeros(L, B, PM, NH, 64, dtype=torch.bfloat16)
    memv = torch.zeros_like(memk)
    ks = torch.tensor([PM])  # empty memory before the first frame
    frames = []
    for f in range(5):
        ck, cv = _rand((L, B, R, NH, 64), g), _rand((L, B, R, NH, 64), g)
        frames.append(cv)
        memk, memv, ks = ring_append(memk, memv, ck, cv, ks)
        assert int(ks[0]) == max(PM - (f + 1) * R, 0)
        assert (memv[0, 0, : int(ks[0])] == 0).all()
        # the last min(f + 1, 3) frames' rows, oldest first, fill [kv_start, PM)
        live = torch.cat([fr[0, 0] for fr in frames[-3:]], 0)
        assert torch.equal(memv[0, 0, int(ks[0]):], live[-(PM - int(ks[0])):])


def _ring_args(**over):
    a = _lib.MkxRingArgs(L=2, B=1, NH=2, HD=64, PM=8, R=2)
    a.cur_k, a.cur_v = 0x100000, 0x200000
    for l in range(2):
        a.memk_in[l], a.memv_in[l] = 0x1000000 + l * 0x100000, 0x2000000 + l * 0x100000
        a.memk_out[l], a.memv_out[l] = 0x3000000 + l * 0x100000, 0x4000000 + l * 0x100000
    a.mem_stride_b = 8 * 2 * 64
    a.kv_start_in, a.kv_start_out = 0x5000000, 0x5001000
    for k, v in over.items():
        if k.endswith("]"):
            name, idx = k[:-1].split("[")
            getattr(a, name)[int(idx)] = v
        else:
            setattr(a, k, v)
    return a


@pytest.mark.parametrize("over", [
    dict(L=0), dict(L=33), dict(HD=128), dict(R=0), dict(R=9), dict(PM=0), dict(B=0), dict(cur_k=0),
    dict(kv_start_out=0x5000000), dict(shift_cos=0x6000000), dict(new_sin=0x6000000), dict(cur_v=0x100008),
    {"memk_out[1]": 0x1000000 + 0x80}, {"memv_out[0]": 0x200100}, {"memk_in[1]": 0}, dict(mem_stride_b=12),
])
def test_ring_append_rejects_bad_arguments_before_touching_the_device(over):
    L = _lib.lib()
    rc = L.mkx_ring_append(ctypes.byref(_ring_args(**over)), None)
    assert rc == _lib.EINVAL, L.mkx_last_error()
    assert L.mkx_last_error().decode().startswith("mkx_ring_append")
    assert L.mkx_ring_append(None, None) == _lib.EINVAL


def test_source_create_rejects_bad_dims_before_touching_the_device():
    L = _lib.lib()
    good = dict(L=2, NH=2, HD=64, C=64, max_rows=64, eps=1e-6)
    for over in (dict(L=0), dict(L=33), dict(HD=32), dict(C=48), dict(C=0), dict(NH=0), dict(max_rows=0),
                 dict(eps=-1.0), dict(eps=float("nan"))):
        h = ctypes.c_void_p()
        d = _lib.MkxSourceDims(**{**good, **over})
        rc = L.mkx_source_create(ctypes.byref(d), ctypes.c_void_p(0x100000), ctypes.c_void_p(0x200000),
                                 ctypes.c_void_p(0x300000), None, ctypes.byref(h))
        assert rc == _lib.EINVAL and not h.value, (over, L.mkx_last_error())
        assert L.mkx_last_error().decode().startswith("mkx_source_create")
    h = ctypes.c_void_p()
    d = _lib.MkxSourceDims(**good)
    for wk, wv, kn in ((0, 0x200000, 0x300000), (0x100008, 0x200000, 0x300000), (0x100000, 0x200000, 0)):
        rc = L.mkx_source_create(ctypes.byref(d), ctypes.c_void_p(wk), ctypes.c_void_p(wv), ctypes.c_void_p(kn), None,
                                 ctypes.byref(h))
        assert rc == _lib.EINVAL and not h.value
    assert L.mkx_source_create(None, None, None, None, None, ctypes.byref(h)) == _lib.EINVAL
    assert L.mkx_source_run(None, None, None) == _lib.EINVAL


@pytest.mark.parametrize("over,status", [
    (dict(R=0), _lib.EINVAL), (dict(N=8), _lib.EINVAL), (dict(N=24), _lib.EINVAL), (dict(K=384), _lib.EUNSUPPORTED),
    (dict(c_stride=100), _lib.EINVAL), (dict(out_stride=30), _lib.EINVAL), (dict(c=0x100008), _lib.EINVAL),
    (dict(w=0), _lib.EINVAL), (dict(bias=0x300004), _lib.EINVAL), (dict(out=0), _lib.EINVAL),
])
def test_modulations_reject_bad_arguments_before_touching_the_device(over, status):
    L = _lib.lib()
    kw = dict(R=10, K=256, N=32, c=0x100000, c_stride=256, w=0x200000, bias=0x300000, out=0x400000, out_stride=32,
              w_fragment_order=1)
    kw.update(over)
    rc = L.mkx_modulations(ctypes.byref(_lib.MkxModprojArgs(**kw)), None)
    assert rc == status, L.mkx_last_error()
    assert L.mkx_last_error().decode().startswith("mkx_modulations")
    assert L.mkx_modulations(None, None) == _lib.EINVAL


def test_register_ring_rejects_host_memory():
    # the ring's buffers are device pointers handed to the library: host memory is refused at construction
    from mkx.ring import RegisterRing
    mem = [(torch.zeros(8, 2, 64, dtype=torch.bfloat16), torch.zeros(8, 2, 64, dtype=torch.bfloat16))]
    with pytest.raises(ValueError, match="GPU"):
        RegisterRing(mem, torch.tensor([8], dtype=torch.int32), 2)
