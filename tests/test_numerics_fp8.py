"""Why the wide fp8 expert (workload D) runs fp8 weights on fp16 MFMAs rather than on the fp8 MFMA.

An fp8 MFMA multiplies fp8 operands on both sides, so the activations would have to be rounded to e4m3 as
well. The oracle's ``f8`` mode rounds every GEMM operand where the kernel stores it, to e4m3 with one absmax
scale per row (per token: the finest scaling such a kernel could apply in its epilogue). Over workload D's
16 layers and 9 Euler steps that error exceeds the parity bound (max |delta| <= 1e-2, mean <= 2e-3) several
times over, while the ``f16`` mode (the kernel's actual operand rounding) stays far inside it.
"""
import torch

import _cases as C
from mkx import synthetic as SY
from oracle import expert_ref as ER

torch.set_grad_enabled(False)


def test_f8_operand_rounding_is_per_row_e4m3():
    """Each row is scaled so its absmax maps to 448 (exact), every value lands on the e4m3 grid times the
    row's scale, and the rounding error is within half an e4m3 spacing: 2^-4 relative for normal values,
    2^-10 of the scale in the subnormal range."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(6, 96, generator=g, dtype=torch.float64) * torch.logspace(-3, 2, 6, dtype=torch.float64)[:, None]
    q = ER.operand_rounder("f8")(x)
    s = x.abs().amax(-1, keepdim=True) / 448.0
    assert torch.equal(q.abs().amax(-1, keepdim=True), x.abs().amax(-1, keepdim=True))
    codes = q / s  # on the grid (up to the fp64 rounding of the division)
    assert torch.allclose(codes.to(torch.float8_e4m3fn).to(torch.float64), codes, rtol=1e-12, atol=0)
    bound = torch.maximum(x.abs() * 2.0 ** -4, s * 2.0 ** -10)
    assert bool(((q - x).abs() <= bound * (1 + 1e-12)).all())
    # identity in the modes that keep fp32 operands, fp16 in f16 mode
    assert torch.equal(ER.operand_rounder("fp32")(x), x)
    assert torch.equal(ER.operand_rounder("f16")(x.float()), x.float().half().float())


def test_fp8_activations_miss_the_parity_bound_on_the_wide_expert():
    cfg = SY.WORKLOADS["D"]
    case = C.make_case(cfg, device="cpu")
    n = cfg.num_steps - 1
    x1 = torch.randn(cfg.B, cfg.T_act, cfg.A, generator=torch.Generator().manual_seed(5))
    r32 = C.oracle_steps(case, x1, 1, n, "fp32")
    m16, a16 = C.diff(C.oracle_steps(case, x1, 1, n, "f16"), r32, cfg.action_dim)
    m8, a8 = C.diff(C.oracle_steps(case, x1, 1, n, "f8"), r32, cfg.action_dim)
    print({"f16_vs_fp32": (m16, a16), "f8_vs_fp32": (m8, a8)})
    assert m16 <= 1e-2 / 5 and a16 <= 2e-3 / 5  # fp16 operands: well inside the bound
    assert m8 > 1e-2 and a8 > 2e-3                # fp8 operands: outside it
