"""GPU: ``mkx_modulations`` (through the C ABI, via mkx.modulations.ModulationProjection) against the CPU
oracle's ``step_modulations`` on the same input c, and the expert run on the kernel's modulation rows.
Tolerance: fp32 products from split-bf16 operands and a hardware exp in SiLU, |delta| <= 1e-4 max|mods|."""
import json
from dataclasses import replace

import pytest
import torch

from _cases import TINY, diff, make_case, oracle_dims, oracle_steps
from mkx import ExpertMegakernel, synthetic as SY
from mkx.modulations import ModulationProjection, StepModulations
from oracle import expert_ref as ER

pytestmark = pytest.mark.gpu
torch.set_grad_enabled(False)


def _report(name, **kv):
    print(json.dumps({"case": name, **kv}), flush=True)


def _check(name, cfg, n_steps=10):
    W = SY.make_weights(cfg, 0)
    d = oracle_dims(cfg)
    sc = SY.make_inputs(cfg)["state_cond"]
    c = ER.modulation_input(n_steps, sc, W, d)  # [B, N, H]
    ref, _ = ER.step_modulations(n_steps, sc, W, d)
    proj = ModulationProjection(W["mod_w"].cuda(), W["mod_b"].float().cuda())
    out = proj(c.cuda())
    out_rm = ModulationProjection(W["mod_w"].cuda(), W["mod_b"].float().cuda(), fragment_order=False)(c.cuda())
    torch.cuda.synchronize()
    assert torch.equal(out, out_rm)  # both weight layouts give the same bits
    dd = (out.cpu() - ref).abs()
    _report(name, max=float(dd.max()), mean=float(dd.mean()), max_abs_ref=float(ref.abs().max()))
    assert out.shape == ref.shape
    assert float(dd.max()) <= 1e-4 * float(ref.abs().max())


def test_modulations_tiny():
    _check("modulations tiny (H 256)", TINY, 4)


def test_modulations_config_A():
    _check("modulations A (L10 H768, 10 steps)", SY.WORKLOADS["A"])


def test_modulations_batch_and_wide():
    _check("modulations B8 (80 rows)", SY.WORKLOADS["B"])
    _check("modulations D shape (L16 H1024)", replace(SY.WORKLOADS["D"], weight_dtype="bf16"))


def test_expert_on_kernel_modulations():
    case = make_case(SY.WORKLOADS["A"])
    cfg, model = case["cfg"], case["model"]
    W = case["W"]
    c = ER.modulation_input(cfg.num_steps, case["inp"]["state_cond"], W, oracle_dims(cfg))
    mods_k = ModulationProjection(W["mod_w"].cuda(), W["mod_b"].float().cuda())(c.cuda())[0]  # [N, MODW], B = 1
    mk = ExpertMegakernel(model)
    x_t, _, _ = mk.run_all(case["noise"], case["mods"], case["dt"], case["past"], cfg.action_dim)
    x_k, _, _ = mk.run_all(case["noise"], mods_k, case["dt"], case["past"], cfg.action_dim)
    mk.check()
    torch.cuda.synchronize()
    case_k = dict(case, mods=mods_k)
    r32 = oracle_steps(case_k, case["noise"], 0, cfg.num_steps, "fp32", first=True)
    m, a = diff(x_k, r32, cfg.action_dim)
    mt, _ = diff(x_k, x_t, cfg.action_dim)
    _report("expert on kernel modulations (A)", vs_fp32_max=m, vs_fp32_mean=a, vs_torch_mods_max=mt)
    assert m <= 1e-3 and a <= 2e-4 and mt <= 1e-3


def test_modulations_timing_config_A():
    """Kernel vs the PyTorch projection (fp32 weights) on config A's 10 rows; reported, not asserted."""
    cfg = SY.WORKLOADS["A"]
    W = SY.make_weights(cfg, 0)
    c = ER.modulation_input(cfg.num_steps, SY.make_inputs(cfg)["state_cond"], W, oracle_dims(cfg)).cuda()
    proj = ModulationProjection(W["mod_w"].cuda(), W["mod_b"].float().cuda())
    wf, bf = W["mod_w"].float().cuda(), W["mod_b"].float().cuda()

    def t(fn, n=50):
        for _ in range(3):
            fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(n):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3 / n

    proj_rm = ModulationProjection(W["mod_w"].cuda(), W["mod_b"].float().cuda(), fragment_order=False)
    _report("modulations timing A", kernel_us=t(lambda: proj(c)), kernel_row_major_us=t(lambda: proj_rm(c)),
            torch_fp32_us=t(lambda: torch.nn.functional.silu(c) @ wf.T + bf),
            weight_bytes=int(proj.w.numel() * 2))


def _step_mods(W):
    return StepModulations(W["t1_w"].cuda(), W["t1_b"].cuda(), W["t2_w"].cuda(), W["t2_b"].cuda(), W["mod_w"].cuda(),
                           W["mod_b"].cuda())


def _check_input(name, cfg, n_steps):
    """mkx_modulation_input (timestep embedding and the small MLP) against the oracle's modulation_input,
    then the whole _step_modulations (input kernel + projection) against the oracle's step_modulations:
    fp32 products from split-bf16 operands and a hardware exp in SiLU, |delta| <= 1e-4 of the largest value."""
    W = SY.make_weights(cfg, 0)
    d = oracle_dims(cfg)
    sc = SY.make_inputs(cfg)["state_cond"]
    sm = _step_mods(W)
    c = sm.input(n_steps, sc.cuda())
    ref_c = ER.modulation_input(n_steps, sc, W, d)
    mods, dt = sm(n_steps, sc.cuda())
    ref, ref_dt = ER.step_modulations(n_steps, sc, W, d)
    torch.cuda.synchronize()
    ref = ref[0] if cfg.B == 1 else ref
    dc, dm = (c.cpu() - ref_c).abs(), (mods.cpu() - ref).abs()
    _report(name, c_max=float(dc.max()), c_max_abs_ref=float(ref_c.abs().max()), mods_max=float(dm.max()),
            mods_max_abs_ref=float(ref.abs().max()))
    assert c.shape == ref_c.shape and mods.shape == ref.shape
    assert float(dc.max()) <= 1e-4 * float(ref_c.abs().max())
    assert float(dm.max()) <= 1e-4 * float(ref.abs().max())
    assert float(dt.item()) == pytest.approx(ref_dt)


def test_modulation_input_tiny():
    _check_input("modulation input tiny (H 256, tdim 32)", TINY, TINY.num_steps)


def test_modulation_input_config_A():
    _check_input("modulation input A (10 steps)", SY.WORKLOADS["A"], 10)


def test_modulation_input_batch_of_8():
    _check_input("modulation input B (8 samples)", SY.WORKLOADS["B"], 10)


def test_modulation_input_one_step_and_two_row_tiles():
    _check_input("modulation input A, 1 step", SY.WORKLOADS["A"], 1)
    _check_input("modulation input A, 20 steps (two row tiles)", SY.WORKLOADS["A"], 20)


def test_modulation_input_wide_expert():
    _check_input("modulation input D shape (H 1024)", replace(SY.WORKLOADS["D"], L=2), 10)


def test_step_modulations_drive_the_expert_like_the_pytorch_ones():
    """The expert run (Euler steps 1..N in one launch) on the kernels' modulation rows against the run on the
    synthetic model's PyTorch rows: the same up to the modulations' rounding."""
    cfg = SY.WORKLOADS["A"]
    case = make_case(cfg)
    model, past, noise = case["model"], case["past"], case["noise"]
    mk = ExpertMegakernel(model)
    sc = case["inp"]["state_cond"].cuda()
    mods_k, dt_k = _step_mods(case["W"])(cfg.num_steps, sc)
    mods_t, dt_t = model._step_modulations(cfg.num_steps, sc)
    x_k, _, _ = mk.run_all(noise, mods_k, dt_k, past, cfg.action_dim)
    x_t, _, _ = mk.run_all(noise, mods_t, dt_t, past, cfg.action_dim)
    mk.check()
    torch.cuda.synchronize()
    m, a = diff(x_k, x_t, cfg.action_dim)
    _report("expert on kernel step modulations vs PyTorch step modulations (A)", max=m, mean=a)
    assert m <= 1e-3 and a <= 2e-4
