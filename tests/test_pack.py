"""The offline packer and its safetensors layout (CPU): the e4m3 quantiser against a brute-force
nearest-value search over all 256 codes, the layout's keys, shapes and dtypes, file round trips, and
attaching a packed fp8 expert to a bf16 model."""
from dataclasses import replace

import pytest
import torch

from _cases import TINY
from mkx import synthetic as SY
from mkx.pack import (FORMAT, LINEARS, PackedExpert, attach_fp8, dequantize_e4m3, load_packed, pack_expert,
                      quantize_e4m3, save_packed, validate)


def _e4m3_table() -> torch.Tensor:
    """Values of the 256 e4m3fn codes from the format's definition (1 sign, 4 exponent bits with bias 7,
    3 mantissa bits; exponent 0 is subnormal m/8 * 2^-6; S.1111.111 is NaN; no infinities)."""
    vals = []
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            v = float("nan")
        elif e == 0:
            v = m / 8 * 2.0 ** -6
        else:
            v = (1 + m / 8) * 2.0 ** (e - 7)
        vals.append(-v if s else v)
    return torch.tensor(vals, dtype=torch.float64)


def _nearest_e4m3(x: torch.Tensor) -> torch.Tensor:
    """Brute force: the finite code value nearest each x, ties to the code with an even mantissa."""
    tab = _e4m3_table()
    fin = torch.isfinite(tab)
    codes = torch.arange(256)[fin]
    v = tab[fin]
    d = (x.double()[:, None] - v[None, :]).abs()
    best = d.min(1, keepdim=True).values
    cand = d == best
    even = (codes & 1) == 0
    pick = torch.where((cand & even[None, :]).any(1), (cand & even[None, :]).double().argmax(1), cand.double().argmax(1))
    return v[pick]


def test_table_spot_values():
    tab = _e4m3_table()
    assert tab[0x7E] == 448 and tab[0x01] == 2.0 ** -9 and tab[0x08] == 2.0 ** -6 and tab[0x38] == 1.0
    assert torch.isnan(tab[0x7F]) and torch.isnan(tab[0xFF])
    # torch's decoder agrees with the definition on every finite code
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).double()
    fin = torch.isfinite(tab)
    assert torch.equal(t[fin], tab[fin])


def test_quantiser_rounds_to_nearest_even_per_row():
    g = torch.Generator().manual_seed(5)
    tab = _e4m3_table()
    fin = tab[torch.isfinite(tab)].unique()
    pos = fin[fin >= 0]
    mids = (pos[1:] + pos[:-1]) / 2  # exact ties between neighbouring codes
    vals = torch.cat([mids, -mids, torch.rand(2000, generator=g, dtype=torch.float64) * 896 - 448,
                      (torch.rand(500, generator=g, dtype=torch.float64) - 0.5) * 2 ** -5])
    # rows whose largest magnitude is 448 have scale exactly 1, so w / scale is w itself
    rows = vals.reshape(-1, 1).repeat(1, 2)
    rows[:, 1] = 448.0
    q, s = quantize_e4m3(rows.float())
    assert torch.equal(s, torch.ones(rows.shape[0]))
    got = q[:, 0].double()
    want = _nearest_e4m3(rows[:, 0].float())  # fp32 inputs, as the quantiser sees them
    assert torch.equal(got, want)
    assert (q[:, 1].double() == 448).all()


def test_quantiser_scale_and_error_bound():
    g = torch.Generator().manual_seed(6)
    w = torch.randn(64, 96, generator=g) * 0.02
    w[3] = 0.0  # a zero row
    w[7, 11] = -0.5  # a negative row maximum
    q, s = quantize_e4m3(w)
    assert q.dtype == torch.float8_e4m3fn and s.dtype == torch.float32 and s.shape == (64,)
    assert torch.allclose(s, w.abs().amax(-1).clamp_min(1e-12) / 448)
    assert q[7, 11].float() == -448 and (q[3].float() == 0).all()
    amax = q.float().abs().amax(-1)
    assert (amax[torch.arange(64) != 3] == 448).all()
    # round to nearest: error within half a code step (2^-4 relative for normals, 2^-10 absolute below 2^-6)
    deq = dequantize_e4m3(q, s)
    bound = torch.maximum(w.abs() * 2.0 ** -4, s[:, None] * 2.0 ** -10) * (1 + 1e-6)
    assert ((deq - w).abs() <= bound).all()


def _cpu_model(cfg):
    return SY.SyntheticReki(cfg, SY.make_weights(cfg, 0), device="cpu")


def test_layout_of_a_packed_fp8_model_and_file_round_trip(tmp_path):
    cfg = replace(TINY, weight_dtype="fp8_e4m3")
    model = _cpu_model(cfg)
    p = pack_expert(model)
    assert p.fp8 and p.meta["format"] == FORMAT
    L, H, I, HD, A = cfg.L, cfg.H, cfg.I, cfg.HD, cfg.A  # noqa: E741
    assert p.tensors["wqkv"].shape == (L, 3 * H, H) and p.tensors["wd"].shape == (L, H, I)
    assert p.tensors["wg_scale"].shape == (L, I) and p.tensors["qn"].shape == (L, HD)
    assert p.tensors["win"].shape == (A, H) and p.tensors["reg_tok"].shape == (cfg.R_reg, H)
    # stacks are the model's own codes and scales, q; k; v concatenated along the output rows
    ly = model.W_cpu["layers"][1]
    assert torch.equal(p.tensors["wqkv"][1, H: 2 * H].view(torch.uint8), ly["k_q"].view(torch.uint8))
    assert torch.equal(p.tensors["wqkv_scale"][1, 2 * H:], ly["v_scale"])
    assert torch.equal(p.tensors["wd"][0].view(torch.uint8), model.W_cpu["layers"][0]["down_q"].view(torch.uint8))
    assert torch.equal(p.dequantized("wu")[0], model.W_cpu["layers"][0]["up"])
    path = str(tmp_path / "expert.safetensors")
    save_packed(p, path)
    r = load_packed(path)
    assert r.meta == p.meta and set(r.tensors) == set(p.tensors)
    for k, v in p.tensors.items():
        a, b = (t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t for t in (v, r.tensors[k]))
        assert a.dtype == b.dtype and torch.equal(a, b), k


def test_packing_a_bf16_model_to_fp8_and_attaching_it(tmp_path):
    model = _cpu_model(TINY)
    p = pack_expert(model, "fp8_e4m3")
    assert p.fp8
    # quantised per linear: every row of q, k and v has its own scale and reaches 448
    for k in LINEARS:
        assert (p.tensors[k].float().abs().amax(-1) == 448).all(), k
        w = pack_expert(model, "bf16").tensors[k].float()
        deq = p.dequantized(k)
        bound = torch.maximum(w.abs() * 2.0 ** -4, p.tensors[k + "_scale"][..., None] * 2.0 ** -10) * (1 + 1e-6)
        assert ((deq - w).abs() <= bound).all(), k
    path = str(tmp_path / "e.safetensors")
    save_packed(p, path)
    model2 = _cpu_model(TINY)
    attach_fp8(model2, load_packed(path))
    p2 = pack_expert(model2)  # the model now carries fp8 codes and is packed as such
    assert p2.fp8
    for k in LINEARS:
        assert torch.equal(p2.tensors[k].view(torch.uint8), p.tensors[k].view(torch.uint8)), k
        assert torch.equal(p2.tensors[k + "_scale"], p.tensors[k + "_scale"]), k
    assert torch.equal(model2.vlm_with_expert.action_expert.layers[0].self_attn.v_proj.weight_q.view(torch.uint8),
                       p.tensors["wqkv"][0, 2 * TINY.H:].view(torch.uint8))
    with pytest.raises(ValueError):
        attach_fp8(model2, pack_expert(model, "bf16"))


def test_bf16_pack_and_validation_errors():
    model = _cpu_model(TINY)
    p = pack_expert(model)
    assert not p.fp8 and "wqkv_scale" not in p.tensors and p.tensors["wo"].dtype == torch.bfloat16
    assert torch.equal(p.tensors["wqkv"][0, : TINY.H], model.W_cpu["layers"][0]["q"])
    validate(p)
    bad = PackedExpert(dict(p.tensors), dict(p.meta))
    bad.tensors["wg"] = bad.tensors["wg"][:, :-1]
    with pytest.raises(ValueError, match="wg"):
        validate(bad)
    bad = PackedExpert({k: v for k, v in p.tensors.items() if k != "bout"}, dict(p.meta))
    with pytest.raises(ValueError, match="bout"):
        validate(bad)
    with pytest.raises(ValueError, match="format"):
        validate(PackedExpert(dict(p.tensors), {**p.meta, "format": "other"}))
    bad = PackedExpert({**p.tensors, "wo": p.tensors["wo"].float()}, dict(p.meta))
    with pytest.raises(ValueError, match="wo"):
        validate(bad)
    with pytest.raises(ValueError):
        pack_expert(model, "int8")
