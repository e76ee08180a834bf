"""GPU parity of the HIP megakernel against the CPU oracle, through the C ABI (via mkx.ExpertMegakernel).

Tolerances: the parity metric is max |delta| <= 1e-2 and mean |delta| <= 2e-3 over the real action dims
against the fp32 oracle (the eager fp32 expert). Against the ``mixed`` oracle, which rounds where this
kernel rounds, the bound is tighter (accumulation order and exp/rsqrt approximations remain).
"""
import json
import math

import pytest
import torch

from _cases import TINY, diff, make_case, oracle_steps
from mkx import ExpertMegakernel, install, synthetic as SY
from mkx._lib import MkxError

pytestmark = pytest.mark.gpu
torch.set_grad_enabled(False)

FP32_MAX, FP32_MEAN = 1e-2, 2e-3
# Against the ``mixed`` oracle: at small depth the kernel reproduces its roundings almost exactly; at full
# depth (90 layer evaluations) any two bf16-activation computations drift apart by the rounding-noise floor
# of the model (a 1e-7 relative input perturbation of the mixed oracle itself moves its output by ~1.7e-3
# mean), so the full-size bound is a consistency bound at that floor.
MIXED_MAX, MIXED_MEAN = 4e-3, 5e-4
MIXED_FULL = (1.5e-2, 3e-3)


def _report(name, **kv):
    print(json.dumps({"case": name, **kv}), flush=True)


def _steps_2_to_n(case):
    cfg = case["cfg"]
    x1, _, _ = case["model"]._expert_first_step(case["noise"], case["past"], None, case["mods"][..., :1, :], case["dt"], cfg.action_dim)
    mk = ExpertMegakernel(case["model"])
    x = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    mk.check()
    torch.cuda.synchronize()
    return mk, x1, x


def _check_loop(name, case, fp32=(FP32_MAX, FP32_MEAN), mixed=(MIXED_MAX, MIXED_MEAN)):
    cfg = case["cfg"]
    mk, x1, x = _steps_2_to_n(case)
    assert torch.isfinite(x).all(), "non-finite output"
    n = cfg.num_steps - 1
    r32 = oracle_steps(case, x1, 1, n, "fp32")
    rmx = oracle_steps(case, x1, 1, n, "mixed")
    m32, a32 = diff(x, r32, cfg.action_dim)
    mmx, amx = diff(x, rmx, cfg.action_dim)
    mall, _ = diff(x, r32, cfg.A)
    _report(name, vs_fp32_max=m32, vs_fp32_mean=a32, vs_mixed_max=mmx, vs_mixed_mean=amx, all_dims_max=mall,
            max_abs_x=float(r32[..., : cfg.action_dim].abs().max()))
    assert m32 <= fp32[0] and a32 <= fp32[1], (m32, a32)
    assert mmx <= mixed[0] and amx <= mixed[1], (mmx, amx)
    return mk, x1, x


def test_tiny_first_step_and_loop():
    case = make_case(TINY)
    cfg = case["cfg"]
    x1, ck, cv = case["model"]._expert_first_step(case["noise"], case["past"], None, case["mods"][..., :1, :], case["dt"], cfg.action_dim)
    torch.cuda.synchronize()
    kv = []
    r1 = oracle_steps(case, case["noise"], 0, 1, "mixed", first=True, reg_kv_out=kv)
    m, a = diff(x1, r1, cfg.action_dim)
    _report("tiny step 1 vs mixed", max=m, mean=a)
    assert m <= MIXED_MAX and a <= MIXED_MEAN
    # register K/V of step 1: [L, B, R, NH, HD]
    for l, (k_ref, v_ref) in enumerate(kv[0]):
        dk = (ck[l, 0].float().cpu() - k_ref).abs().max().item()
        dv = (cv[l, 0].float().cpu() - v_ref).abs().max().item()
        assert dk <= 3e-2 and dv <= 3e-2, (l, dk, dv)
    _check_loop("tiny loop", case)


def test_config_A_steps_2_to_10():
    _check_loop("A (b1, 10+32 rows, PM 96, S 300)", make_case(SY.WORKLOADS["A"]), mixed=MIXED_FULL)


def test_config_A_ref_layout_with_invalid_rows_nan():
    # the reference's own layout: 10 action rows in steps 2..N, memory rows below kv_start and source rows
    # beyond S hold NaN and must have no effect
    _check_loop("A-ref (10 rows, kv_start 32, S 182/256, NaN pads)", make_case(SY.WORKLOADS["A-ref"], nan_pads=True),
                mixed=MIXED_FULL)


def test_random_per_step_modulations():
    # strongly step-dependent modulation rows: a wrong step or layer offset cannot hide
    _check_loop("A random mods", make_case(SY.WORKLOADS["A"], random_mods=True), fp32=(3e-2, 6e-3), mixed=(3e-2, 6e-3))


def test_batch_of_two_independent_chunks():
    from dataclasses import replace
    cfg = replace(SY.WORKLOADS["A"], B=2)
    case = make_case(cfg)
    _check_loop("A batch 2", case, mixed=MIXED_FULL)


def test_long_context_C():
    _check_loop("C (S 1024, PM 256)", make_case(SY.WORKLOADS["C"]), mixed=MIXED_FULL)


def test_gelu_variant_tiny():
    from dataclasses import replace
    _check_loop("tiny gelu_tanh", make_case(replace(TINY, act="gelu_tanh")))


def test_barrier_count_invariant_and_determinism():
    case = make_case(TINY)
    cfg = case["cfg"]
    mk, x1, x = _steps_2_to_n(case)
    mk.barrier_arrivals()  # reset the counter window
    xa = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    arrivals = mk.barrier_arrivals()
    xb = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    mk.check()
    n = cfg.num_steps - 1
    _report("barriers", arrivals=arrivals, expected=mk.nprog * mk.barriers(n))
    assert arrivals == mk.nprog * mk.barriers(n)
    assert torch.equal(xa, xb) and torch.equal(xa, x)


def test_install_matches_first_step_plus_run():
    case = make_case(TINY)
    cfg = case["cfg"]
    model = case["model"]
    x_ref = _steps_2_to_n(case)[2]
    mk = install(model)
    x, ck, cv = model._expert_actions(case["noise"], case["past"], None, case["inp"]["state_cond"].cuda(), cfg.action_dim,
                                      cfg.num_steps)
    torch.cuda.synchronize()
    assert torch.equal(x, x_ref)
    assert ck.shape == (cfg.L, 1, cfg.R_reg, cfg.NH, cfg.HD)


def test_invalid_arguments_raise():
    case = make_case(TINY)
    cfg = case["cfg"]
    mk = ExpertMegakernel(case["model"])
    x1 = case["noise"]
    with pytest.raises(ValueError):
        mk.run(x1, case["mods"][:1], case["dt"], case["past"], cfg.action_dim)  # no step to run
    with pytest.raises(ValueError):
        mk.run(x1[..., :16], case["mods"], case["dt"], case["past"], cfg.action_dim)  # wrong action width
    with pytest.raises(ValueError):
        mk.run(x1, case["mods"], case["dt"], case["past"], 40)  # action_dim > A
