"""GPU parity of the HIP megakernel against the CPU oracle, through the C ABI (via mkx.ExpertMegakernel).

Tolerances: the parity metric is max |delta| <= 1e-2 and mean |delta| <= 2e-3 over the real action dims
against the fp32 oracle (the eager fp32 expert). The kernel's own error level is that of the ``f16`` oracle,
which rounds the GEMM operands to fp16 where this kernel stores them: over tens of layers the rounding
decisions are chaotic (a 1e-7 relative change of the input re-rolls them and moves the result as much as the
rounding itself), so the ``f16`` oracle fixes the size of the error the kernel should show against fp32, not
its per-element value.
"""
import json
import math

import pytest
import torch

from _cases import TINY, diff, make_case, oracle_steps
from mkx import ExpertMegakernel, install, synthetic as SY
from mkx._lib import MkxError
from mkx.pack import attach_fp8, load_packed, pack_expert, save_packed

pytestmark = pytest.mark.gpu
torch.set_grad_enabled(False)

# Parity bound (against the fp32 oracle, real action dims): max |delta| <= 1e-2, mean <= 2e-3.
FP32_MAX, FP32_MEAN = 1e-2, 2e-3
# The kernel multiplies fp16 GEMM operands (activations rounded to nearest even where they are stored) with
# fp16 or fp8 weights into fp32 accumulators and keeps everything else fp32, so it tracks the fp32 oracle
# five times inside the parity bound (a bf16-activation kernel, the ``mixed`` oracle, uses most of it) ...
TIGHT_MAX, TIGHT_MEAN = 2e-3, 4e-4
# ... and its error against fp32 is at most this factor above that of the ``f16`` oracle (same rounding
# points, different accumulation order and exp / rsqrt approximations)
F16_FACTOR_MAX, F16_FACTOR_MEAN = 3.0, 2.0


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


def _check_loop(name, case, tight=(TIGHT_MAX, TIGHT_MEAN)):
    cfg = case["cfg"]
    mk, x1, x = _steps_2_to_n(case)
    assert torch.isfinite(x).all(), "non-finite output"
    n = cfg.num_steps - 1
    r32 = oracle_steps(case, x1, 1, n, "fp32")
    m32, a32 = diff(x, r32, cfg.action_dim)
    mall, _ = diff(x, r32, cfg.A)
    rmx = oracle_steps(case, x1, 1, n, "mixed")  # bf16-activation numerics, reported for comparison
    mmx, amx = diff(rmx, r32, cfg.action_dim)
    r16 = oracle_steps(case, x1, 1, n, "f16")  # the kernel's own rounding points: its expected error level
    m16, a16 = diff(r16, r32, cfg.action_dim)
    _report(name, vs_fp32_max=m32, vs_fp32_mean=a32, all_dims_max=mall, f16_oracle_vs_fp32_max=m16, f16_oracle_vs_fp32_mean=a16,
            bf16_activation_oracle_vs_fp32_max=mmx, bf16_activation_oracle_vs_fp32_mean=amx,
            max_abs_x=float(r32[..., : cfg.action_dim].abs().max()))
    assert m32 <= FP32_MAX and a32 <= FP32_MEAN, (m32, a32)
    assert m32 <= tight[0] and a32 <= tight[1], (m32, a32)
    assert m32 <= F16_FACTOR_MAX * m16 + 1e-5 and a32 <= F16_FACTOR_MEAN * a16 + 1e-6, (m32, a32, m16, a16)
    assert mall <= FP32_MAX
    return mk, x1, x


def test_tiny_first_step_and_loop():
    case = make_case(TINY)
    cfg = case["cfg"]
    x1, ck, cv = case["model"]._expert_first_step(case["noise"], case["past"], None, case["mods"][..., :1, :], case["dt"], cfg.action_dim)
    torch.cuda.synchronize()
    kv = []
    r1 = oracle_steps(case, case["noise"], 0, 1, "fp32", first=True, reg_kv_out=kv)
    m, a = diff(x1, r1, cfg.action_dim)
    _report("tiny step 1 vs fp32", max=m, mean=a)
    assert m <= TIGHT_MAX and a <= TIGHT_MEAN
    # register K/V of step 1: [L, B, R, NH, HD]
    for l, (k_ref, v_ref) in enumerate(kv[0]):
        dk = (ck[l, 0].float().cpu() - k_ref).abs().max().item()
        dv = (cv[l, 0].float().cpu() - v_ref).abs().max().item()
        assert dk <= 3e-2 and dv <= 3e-2, (l, dk, dv)
    _check_loop("tiny loop", case)


def test_config_A_steps_2_to_10():
    _check_loop("A (b1, 10+32 rows, PM 96, S 300)", make_case(SY.WORKLOADS["A"]))


def test_config_A_ref_layout_with_invalid_rows_nan():
    # the reference's own layout: 10 action rows in steps 2..N, memory rows below kv_start and source rows
    # beyond S hold NaN and must have no effect
    _check_loop("A-ref (10 rows, kv_start 32, S 182/256, NaN pads)", make_case(SY.WORKLOADS["A-ref"], nan_pads=True))


def test_random_per_step_modulations():
    # strongly step-dependent modulation rows: a wrong step or layer offset cannot hide
    _check_loop("A random mods", make_case(SY.WORKLOADS["A"], random_mods=True))


def test_batch_of_two_independent_chunks():
    from dataclasses import replace
    cfg = replace(SY.WORKLOADS["A"], B=2)
    case = make_case(cfg)
    _check_loop("A batch 2", case)


def test_config_B_batch_of_eight():
    # eight independent chunks (M = 8 x 48 rows): several row groups per tile in every GEMM stage
    _check_loop("B (b8)", make_case(SY.WORKLOADS["B"]))


def test_wide_expert_D_shape_bf16():
    # the wide expert's shape (L16 H1024 NH16 I4096, 50 action + 32 register rows) with bf16 weights
    from dataclasses import replace
    _check_loop("D shape, bf16 weights", make_case(replace(SY.WORKLOADS["D"], weight_dtype="bf16")))


def test_fp8_weights_tiny():
    # e4m3 weights with per-output-channel scales: the kernel converts them to bf16 operands exactly and
    # applies the scales in the epilogues, so it tracks the oracle run with the dequantised weights
    from dataclasses import replace
    _check_loop("tiny fp8", make_case(replace(TINY, weight_dtype="fp8_e4m3")))


def test_wide_expert_D_fp8():
    _check_loop("D (L16 H1024, fp8 weights)", make_case(SY.WORKLOADS["D"]))


def test_wide_expert_D_fp8_batch_of_four():
    _check_loop("D-b4 (fp8 weights, batch 4)", make_case(SY.WORKLOADS["D-b4"]))


def test_long_context_C():
    _check_loop("C (S 1024, PM 256)", make_case(SY.WORKLOADS["C"]))


def test_gelu_variant_tiny():
    from dataclasses import replace
    _check_loop("tiny gelu_tanh", make_case(replace(TINY, act="gelu_tanh")))


def test_gelu_variant_at_config_A_size():
    # the GELU(tanh) MLP of the benchmark's expert description, at the headline shape (H 768, I 3072, 10 layers)
    from dataclasses import replace
    _check_loop("A gelu_tanh", make_case(replace(SY.WORKLOADS["A"], act="gelu_tanh")))


class _gemm_form:
    """Forces the megakernel's GEMM form for the handles created inside the block (MKX_GEMM_FORM is read when
    a handle is created): "passes" (row tiles in passes, the K quarters of the four waves summed through LDS)
    or "rows" (each wave whole-K products of its own row tiles)."""

    def __init__(self, form):
        self.form = form

    def __enter__(self):
        import os
        self.old = os.environ.get("MKX_GEMM_FORM")
        os.environ["MKX_GEMM_FORM"] = self.form

    def __exit__(self, *exc):
        import os
        if self.old is None:
            os.environ.pop("MKX_GEMM_FORM", None)
        else:
            os.environ["MKX_GEMM_FORM"] = self.old


def test_tiny_batch_of_four_both_gemm_forms():
    # 4 x 16 rows: more row tiles than one GEMM pass holds, so the launch takes the row-wise form by itself;
    # forced into passes it must agree with the oracle as well
    from dataclasses import replace
    case = make_case(replace(TINY, B=4))
    _check_loop("tiny b4 (row-wise GEMMs)", case)
    with _gemm_form("passes"):
        _check_loop("tiny b4 (GEMM passes)", case)


def test_tiny_fp8_gelu_rowwise():
    # fp8 weights (scales in every row-wise epilogue kind) and the GELU MLP on the row-wise form
    from dataclasses import replace
    with _gemm_form("rows"):
        _check_loop("tiny fp8 gelu (row-wise GEMMs)", make_case(replace(TINY, B=3, weight_dtype="fp8_e4m3", act="gelu_tanh")))


def test_batch_of_eight_long_source_rowwise():
    # batch 8 at H 768 in the row-wise form with 520 source rows: the cross-attention K/V are streamed through
    # the LDS ring, and the workgroups with two attention tasks stream them once per task
    from dataclasses import replace
    _check_loop("b8 S 520 (row-wise, tile pairs, streamed source)", make_case(replace(SY.WORKLOADS["B"], L=2, S=520, SP=520)))


def test_two_tile_attention_tasks_with_a_lone_last_tile():
    # fp8 weights, batch 4 of 40 action + 32 register rows: 5 query tiles per sample, 320 one-tile attention
    # tasks on 256 workgroups, so both attention stages run in tasks of two query tiles (the fp8 two-tile
    # instantiations), the fifth tile of each sample-head alone
    from dataclasses import replace
    _check_loop("fp8 b4 T40 (two-tile attention tasks, lone last tile)",
                make_case(replace(SY.WORKLOADS["D-b4"], L=2, T_act=40)))


def test_two_tile_self_attention_with_a_streamed_source():
    # the same shape with 520 source rows: two-tile self-attention tasks, one-tile cross-attention tasks that
    # stream their K/V through the LDS ring (sources beyond the three ring slots)
    from dataclasses import replace
    _check_loop("fp8 b4 T40 S520 (two-tile self-attention, streamed source)",
                make_case(replace(SY.WORKLOADS["D-b4"], L=2, T_act=40, S=520, SP=520)))


def test_ragged_lengths_in_two_tile_cross_attention_fp16():
    # batch 8 at H 768 (two-tile cross-attention tasks; the second self-attention tiles resident) with a
    # source length and a memory start of its own per sample: 1 to 300 source rows, 1 to 96 memory rows
    from dataclasses import replace
    case = make_case(replace(SY.WORKLOADS["B"], L=2), ca_len=[300, 1, 33, 150, 299, 32, 128, 7],
                     kv_start=[0, 32, 64, 95, 16, 0, 48, 80])
    _check_loop("b8 ragged source and memory (two-tile cross-attention)", case)


def test_ragged_lengths_in_two_tile_attention_fp8():
    # the fp8 two-tile instantiations (both attention stages in two-tile tasks) with ragged samples
    from dataclasses import replace
    case = make_case(replace(SY.WORKLOADS["D-b4"], L=2), ca_len=[300, 1, 129, 257], kv_start=[0, 95, 33, 64])
    _check_loop("fp8 b4 ragged source and memory (two-tile attention tasks)", case)


def test_config_A_rowwise_form():
    # the headline shape forced into the row-wise form (one-tile tasks, row-wise GEMMs and step tail)
    with _gemm_form("rows"):
        _check_loop("A (row-wise form)", make_case(SY.WORKLOADS["A"]))


def test_tiny_single_row_tile_rowwise():
    # one row tile per sample: groups of two row tiles whose second repeats the first and stores nothing
    with _gemm_form("rows"):
        _check_loop("tiny (row-wise GEMMs)", make_case(TINY))


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


def test_graph_capture_replays_match_eager():
    """The launch captured in a HIP graph (the library falls back to a plain launch under capture; the ready
    epochs advance on the device, so replays need no host work): every replay, with eager work and a
    synchronisation between replays, reproduces the eager result bit for bit."""
    case = make_case(TINY)
    cfg = case["cfg"]
    x1, _, _ = case["model"]._expert_first_step(case["noise"], case["past"], None, case["mods"][..., :1, :], case["dt"],
                                                cfg.action_dim)
    mk = ExpertMegakernel(case["model"])
    plan = mk.plan(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    plan.launch()
    mk.check()
    x_eager = plan.x_out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan.launch()
    torch.cuda.synchronize()
    for i in range(3):
        plan.x_out.zero_()
        graph.replay()
        noise = torch.randn(4096, device=x1.device).square().sum()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        assert torch.equal(plan.x_out, x_eager), f"replay {i} differs from the eager launch"
    mk.check()
    plan.launch()  # an eager launch after the replays still matches
    mk.check()
    assert torch.equal(plan.x_out, x_eager)
    _report("graph replays", replays=3, max_abs_x=float(x_eager.abs().max()))


def test_run_all_folds_step_one_into_the_launch():
    """Euler steps 1..N as one launch (register rows in the loop) equal step 1's launch followed by the
    launch of steps 2..N, bit for bit, including the register rows' K/V of step 1; and install(...,
    fold_first_step=True) returns the same."""
    import time
    case = make_case(TINY)
    cfg = case["cfg"]
    model = case["model"]
    mk = ExpertMegakernel(model)
    assert mk.can_run_all(case["past"])
    x1, ck1, cv1 = model._expert_first_step(case["noise"], case["past"], None, case["mods"][..., :1, :], case["dt"], cfg.action_dim)
    x_two = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    x_all, ck, cv = mk.run_all(case["noise"], case["mods"], case["dt"], case["past"], cfg.action_dim)
    mk.check()
    torch.cuda.synchronize()
    assert torch.equal(x_all, x_two)
    assert torch.equal(ck, ck1) and torch.equal(cv, cv1)
    inst = install(model, fold_first_step=True)
    x_i, ck_i, cv_i = model._expert_actions(case["noise"], case["past"], None, case["inp"]["state_cond"].cuda(), cfg.action_dim,
                                            cfg.num_steps)
    torch.cuda.synchronize()
    assert torch.equal(x_i, x_all) and torch.equal(ck_i, ck)
    # wall time of the two forms (reported, not asserted)
    def wall(fn, n=20):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / n * 1e3
    t_two = wall(lambda: mk.run(model._expert_first_step(case["noise"], case["past"], None, case["mods"][..., :1, :], case["dt"],
                                                         cfg.action_dim)[0], case["mods"], case["dt"], case["past"], cfg.action_dim))
    t_all = wall(lambda: mk.run_all(case["noise"], case["mods"], case["dt"], case["past"], cfg.action_dim))
    _report("run_all", ms_step1_then_rest=round(t_two, 3), ms_one_launch=round(t_all, 3))
    # the reference layout (register rows only in step 1) cannot share a launch
    ref_case = make_case(replace_cfg(TINY, registers_in_loop=False))
    mk_ref = ExpertMegakernel(ref_case["model"])
    assert not mk_ref.can_run_all(ref_case["past"])
    with pytest.raises(ValueError):
        mk_ref.run_all(ref_case["noise"], ref_case["mods"], ref_case["dt"], ref_case["past"], cfg.action_dim)


def replace_cfg(cfg, **kw):
    from dataclasses import replace
    return replace(cfg, **kw)


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


def test_packed_fp8_file_drives_the_kernel(tmp_path):
    """An fp8 file packed offline from a bf16 model: the handle built from the loaded file equals, bit for
    bit, the one built from the model with the file's codes attached, and tracks the fp32 oracle run on
    the file's dequantised weights."""
    case = make_case(TINY)
    cfg = case["cfg"]
    path = str(tmp_path / "expert_fp8.safetensors")
    save_packed(pack_expert(case["model"], "fp8_e4m3"), path)
    p = load_packed(path, "cuda")
    x1, _, _ = case["model"]._expert_first_step(case["noise"], case["past"], None, case["mods"][..., :1, :], case["dt"], cfg.action_dim)
    mk_file = ExpertMegakernel.from_packed(p)
    assert mk_file.fp8
    x_file = mk_file.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    mk_file.check()
    attach_fp8(case["model"], p)
    mk_model = ExpertMegakernel(case["model"])
    x_model = mk_model.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    mk_model.check()
    torch.cuda.synchronize()
    assert torch.equal(x_file, x_model)
    pc = p.to("cpu")
    split = {"wqkv": ("q", "k", "v"), "wo": ("o",), "wqca": ("ca_q",), "woca": ("ca_o",), "wg": ("gate",),
             "wu": ("up",), "wd": ("down",)}
    layers = []
    for l, ly in enumerate(case["W"]["layers"]):
        ly = dict(ly)
        for stack, names in split.items():
            deq = pc.dequantized(stack)[l]
            for i, nm in enumerate(names):
                ly[nm] = deq[i * ly[nm].shape[0]: (i + 1) * ly[nm].shape[0]]
        layers.append(ly)
    case_q = dict(case, W={**case["W"], "layers": layers})
    r32 = oracle_steps(case_q, x1, 1, cfg.num_steps - 1, "fp32")
    m32, a32 = diff(x_file, r32, cfg.action_dim)
    _report("packed fp8 file (tiny)", vs_fp32_max=m32, vs_fp32_mean=a32)
    assert m32 <= TIGHT_MAX and a32 <= TIGHT_MEAN, (m32, a32)


def test_packed_fp8_file_of_the_wide_expert_D(tmp_path):
    """The wide fp8 expert (L16 H1024) written to a packed file and read back: a handle from the file gives
    the same result, bit for bit, as one from the model."""
    case = make_case(SY.WORKLOADS["D"])
    cfg = case["cfg"]
    path = str(tmp_path / "expert_D.safetensors")
    save_packed(pack_expert(case["model"]), path)
    mk_file = ExpertMegakernel.from_packed(load_packed(path, "cuda"))
    mk_model, x1, x_model = _steps_2_to_n(case)
    x_file = mk_file.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    mk_file.check()
    torch.cuda.synchronize()
    _report("packed fp8 file (D)", equal=bool(torch.equal(x_file, x_model)), weight_bytes=mk_file.weight_bytes)
    assert mk_file.fp8 and torch.equal(x_file, x_model)


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
