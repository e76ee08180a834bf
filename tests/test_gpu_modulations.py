"""GPU: ``mkx_modulations`` (through the C ABI, via mkx.modulations.ModulationProjection) against the CPU
oracle's ``step_modulations`` on the same input c, and the expert run on the kernel's modulation rows.
Tolerance: fp32 products from split-bf16 operands and a hardware exp in SiLU, |delta| <= 1e-4 max|mods|."""
import json
from dataclasses import replace

import pytest
import torch

from _cases import TINY, diff, make_case, oracle_dims, oracle_steps
from mkx import ExpertMegakernel, synthetic as SY
from mkx.modulations import ModulationProjection
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
