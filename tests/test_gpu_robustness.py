"""GPU tests of the boundary's failure handling and instrumentation, through the C ABI: bounded waits that
give up (forced from the host with a tiny spin bound, so every kernel still exits normally), GEMM operands
beyond the fp16 range (forced with huge inputs; the launch completes and reports it), per-boundary
timestamps, scratch growth under and after graph capture, and a reference-layout past captured with the
register ring. The reference has none of these paths: its grid barrier spins without bound
(README.md:262-263) and its timestamps are only binned by tune_mk.py (:82-95)."""
import json
import math
from dataclasses import replace

import pytest
import torch

from _cases import TINY, diff, make_case, oracle_steps
from mkx import ExpertMegakernel, synthetic as SY
from mkx import _lib
from mkx._lib import MkxError

pytestmark = pytest.mark.gpu
torch.set_grad_enabled(False)


def _report(name, **kv):
    print(json.dumps({"case": name, **kv}), flush=True)


def _first_step(case):
    cfg = case["cfg"]
    return case["model"]._expert_first_step(case["noise"], case["past"], None, case["mods"][..., :1, :], case["dt"],
                                            cfg.action_dim)[0]


def test_timeout_drains_returns_nan_and_recovers():
    """A tiny spin bound makes waits give up: the launch still ends (every wait after the first failure
    returns at once), its output is NaN, a second launch before mkx_check also returns NaN, mkx_check reports
    MKX_ETIMEOUT and resets, and the next launch with the default bound matches the oracle."""
    case = make_case(TINY)
    cfg = case["cfg"]
    x1 = _first_step(case)
    mk = ExpertMegakernel(case["model"])
    mk.set_spin_limit(1)
    x_bad = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    torch.cuda.synchronize()
    assert torch.isnan(x_bad).all(), "a launch whose waits gave up must return NaN"
    x_bad2 = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)  # no mkx_check in between
    torch.cuda.synchronize()
    assert torch.isnan(x_bad2).all(), "a launch after an unchecked timeout must return NaN"
    with pytest.raises(MkxError) as ei:
        mk.check()
    assert ei.value.status == _lib.ETIMEOUT
    mk.check()  # reset: the flag is clear now
    mk.set_spin_limit(None)
    x = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    mk.check()
    ref = oracle_steps(case, x1, 1, cfg.num_steps - 1, "fp32")
    m, a = diff(x, ref, cfg.action_dim)
    _report("timeout then recovery (tiny)", vs_fp32_max=m, vs_fp32_mean=a)
    assert m <= 1e-3 and a <= 2e-4


def test_operands_beyond_the_fp16_range_are_reported():
    """GEMM operands are stored as fp16: a launch whose activations exceed 65504 (inputs scaled by 1e9) still
    completes, returns NaN, and mkx_check reports MKX_ERANGE and resets; the next launch with the ordinary
    inputs matches the oracle. A bf16 weight beyond the fp16 range is refused when the handle is created."""
    case = make_case(TINY)
    cfg = case["cfg"]
    x1 = _first_step(case)
    mk = ExpertMegakernel(case["model"])
    x_bad = mk.run(x1 * 1e9, case["mods"], case["dt"], case["past"], cfg.action_dim)
    torch.cuda.synchronize()
    assert torch.isnan(x_bad).all(), "a launch with an operand beyond the fp16 range must return NaN"
    with pytest.raises(MkxError) as ei:
        mk.check()
    assert ei.value.status == _lib.ERANGE
    x = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    mk.check()
    ref = oracle_steps(case, x1, 1, cfg.num_steps - 1, "fp32")
    m, a = diff(x, ref, cfg.action_dim)
    _report("fp16 range error then recovery (tiny)", vs_fp32_max=m, vs_fp32_mean=a)
    assert m <= 1e-3 and a <= 2e-4
    W = SY.make_weights(TINY, 0)
    W["layers"][1]["down"][3, 5] = 1.0e5  # bf16 1e5 > 65504
    with pytest.raises(MkxError) as ei:
        ExpertMegakernel(SY.SyntheticReki(TINY, W, device="cuda"))
    assert ei.value.status == _lib.ERANGE


def test_boundary_timestamps_are_monotonic_and_inside_the_launch():
    """mkx_set_profile: workgroup 0 stamps the launch start and every one of the barriers(n) stage boundaries
    (the reference's prof buffer, src/mk_expert.py:66-69): nondecreasing, and spanning no more than the
    launch's own duration on the HIP event clock."""
    case = make_case(TINY)
    cfg = case["cfg"]
    x1 = _first_step(case)
    mk = ExpertMegakernel(case["model"])
    n = cfg.num_steps - 1
    mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)  # warm (scratch sized)
    mk.set_profile(n)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    x = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    e1.record()
    mk.check()
    ts = mk.barrier_timestamps()
    nb = mk.barriers(n)
    assert nb == 1 + n * (7 * cfg.L + 1)
    stamps = ts[: nb + 1]
    assert (stamps > 0).all(), "every boundary must be stamped"
    d = stamps[1:] - stamps[:-1]
    assert (d >= 0).all(), "timestamps must not decrease"
    span_ns = float(stamps[-1] - stamps[0])
    ev_ns = e0.elapsed_time(e1) * 1e6
    _report("boundary timestamps (tiny)", boundaries=nb, span_us=span_ns / 1e3, event_us=ev_ns / 1e3,
            median_stage_us=float(d.float().median()) / 1e3)
    assert 0 < span_ns <= ev_ns + 2000.0, (span_ns, ev_ns)
    mk.set_profile(None)
    ref = oracle_steps(case, x1, 1, n, "fp32")
    assert diff(x, ref, cfg.action_dim)[0] <= 1e-3  # profiling changes no result


# the refused capture records nothing, so torch reports its graph as empty: that is the expected outcome
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_scratch_growth_is_refused_under_and_after_capture():
    """A call that needs more scratch than the handle holds reallocates it. Under stream capture that is
    refused (MKX_EINVAL, nothing recorded); after a launch of the handle has been captured it is refused too
    (MKX_EUNSUPPORTED), and the graph, which holds the current scratch, still replays the eager result."""
    case = make_case(TINY)
    cfg, model = case["cfg"], case["model"]
    x1 = _first_step(case)
    mods8, dt8 = model._step_modulations(8, case["inp"]["state_cond"])
    # capture without an eager call at this shape first: refused before anything is recorded
    fresh = ExpertMegakernel(model)
    s = torch.cuda.Stream()
    g0 = torch.cuda.CUDAGraph()
    with pytest.raises(MkxError) as ei:
        with torch.cuda.graph(g0, stream=s):
            fresh.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    assert ei.value.status == _lib.EINVAL
    torch.cuda.synchronize()
    # eager at the small shape, capture it, then a larger eager call is refused
    mk = ExpertMegakernel(model)
    x_e = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim).clone()
    mk.check()
    g = torch.cuda.CUDAGraph()
    out = {}
    with torch.cuda.graph(g, stream=s):
        out["x"] = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    torch.cuda.synchronize()
    with pytest.raises(MkxError) as ei:
        mk.run(x1, mods8, dt8, case["past"], cfg.action_dim)
    assert ei.value.status == _lib.EUNSUPPORTED
    # a call that fits the current scratch still runs, and the graph replays the eager result
    x_small = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    torch.cuda.synchronize()
    assert torch.equal(x_small, x_e)
    out["x"].zero_()
    g.replay()
    torch.cuda.synchronize()
    mk.check()
    assert torch.equal(out["x"], x_e)
    # a second handle warmed at the larger shape runs it
    big = ExpertMegakernel(model)
    x8 = big.run(x1, mods8, dt8, case["past"], cfg.action_dim)
    big.check()
    assert torch.isfinite(x8).all()


def test_reference_layout_past_with_ring_as_two_graphs_matches_eager():
    """A past in the reference's layout (memory validity in cu_kv[0], source length in cu_src[1], no
    kv_start / ca_len keys) refilled by the register ring between calls and captured as one graph per ring
    parity: the kernel reads kv_start from the ring's device buffer (which the captured append updates), not
    from a cu_kv snapshot, so every replayed frame equals the eager frame."""
    from mkx.ring import RegisterRing
    cfg = replace(SY.WORKLOADS["A"], kv_start=SY.WORKLOADS["A"].PM)
    case = make_case(cfg)
    model, past = case["model"], case["past"]
    st = past.register_step
    cu_kv = torch.tensor([int(st["kv_start"][0]), cfg.PM], dtype=torch.int32, device="cuda")
    cu_src = torch.tensor([0, int(st["ca_len"][0])], dtype=torch.int32, device="cuda")
    del st["kv_start"], st["ca_len"]
    st["cu_kv"], st["cu_src"] = cu_kv, cu_src
    mk = ExpertMegakernel(model)
    mem0 = [(k.clone(), v.clone()) for k, v in st["mem_kv"]]
    ks0 = cu_kv[:1].clone()
    R, T = cfg.R_reg, cfg.T_act
    out = {}

    def call():
        out["x"], out["k"], out["v"] = mk.run_all(case["noise"], case["mods"], case["dt"], past, cfg.action_dim)

    ring_e = RegisterRing(mem0, ks0, R, kept_delta=-R, new_delta=-(T + R))
    ring_e.update_past(past)
    xs = []
    for _ in range(4):
        call()
        xs.append(out["x"].clone())
        ring_e.append_frame(out["k"], out["v"])
        ring_e.update_past(past)
    mk.check()
    torch.cuda.synchronize()
    assert not torch.equal(xs[0], xs[1])
    ring_g = RegisterRing(mem0, ks0, R, kept_delta=-R, new_delta=-(T + R))
    ring_g.update_past(past)
    call()  # warm-up, no append
    torch.cuda.synchronize()
    graphs, x_of = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            call()
            ring_g.append_frame(out["k"], out["v"])
        ring_g.update_past(past)
        graphs.append(g)
        x_of.append(out["x"])
    torch.cuda.synchronize()
    for f in range(4):
        graphs[f % 2].replay()
        torch.cuda.synchronize()
        assert torch.equal(x_of[f % 2], xs[f]), f"frame {f} differs from the eager sequence"
    mk.check()
    _report("reference-layout past, ring, two graphs (A)", frames=4)


def test_ring_copies_its_inputs():
    # the ring's two kv_start buffers alternate as append outputs: the caller's tensors must not be among them
    from mkx.ring import RegisterRing
    mem = [(torch.zeros(8, 2, 64, dtype=torch.bfloat16, device="cuda"),
            torch.zeros(8, 2, 64, dtype=torch.bfloat16, device="cuda"))]
    ks = torch.tensor([8], dtype=torch.int32, device="cuda")
    ring = RegisterRing(mem, ks, 2)
    ring._ks[0].fill_(0)
    ring._k[0][0].fill_(1)
    torch.cuda.synchronize()
    assert int(ks[0]) == 8 and bool((mem[0][0] == 0).all())
    assert ring.mem_kv[0][0].shape == (8, 2, 64) and int(ring.kv_start[0]) == 0
    with pytest.raises(ValueError, match="cur_k is on cpu"):
        ring.append_frame(torch.zeros(1, 1, 2, 2, 64, dtype=torch.bfloat16), torch.zeros(1, 1, 2, 2, 64, dtype=torch.bfloat16))


def test_fp16_operand_range_headroom_of_workload_a():
    """How far workload A's residual stream can grow before a GEMM operand leaves the fp16 range (the
    drop-in limit of this kernel's fp16 operands; a bf16-operand kernel has none): the step input x is
    scaled by 4^k, which scales the action rows' residual stream (h0 = x Win + bin, and every later
    residual add keeps it), until a launch reports MKX_ERANGE. The CPU oracle, run with the kernel's operand
    rounding and its largest GEMM operand recorded, must put 65504 between the last factor that passed and
    the first that failed; at factor 1 it gives the margin of the synthetic weights."""
    from oracle import expert_ref as ER

    cfg = SY.WORKLOADS["A"]
    case = make_case(cfg)
    x1 = _first_step(case)
    mk = ExpertMegakernel(case["model"])
    n = cfg.num_steps - 1

    def oracle_max_operand(f):
        seen = [0.0]
        orig = ER.operand_rounder

        def recording(mode):
            q = orig(mode)

            def rq(t):
                seen[0] = max(seen[0], float(t.abs().max()))
                return q(t)
            return rq
        ER.operand_rounder = recording
        try:
            oracle_steps(case, x1 * f, 1, n, "f16")
        finally:
            ER.operand_rounder = orig
        return seen[0]

    k_bad = None
    for k in range(0, 16):
        x = mk.run(x1 * float(4 ** k), case["mods"], case["dt"], case["past"], cfg.action_dim)
        torch.cuda.synchronize()
        try:
            mk.check()
        except MkxError as e:
            assert e.status == _lib.ERANGE, e
            assert torch.isnan(x).all()
            k_bad = k
            break
        assert torch.isfinite(x).all(), k
    assert k_bad is not None and k_bad >= 1, k_bad
    y1 = oracle_max_operand(1.0)
    y_ok = oracle_max_operand(float(4 ** (k_bad - 1)))
    y_bad = oracle_max_operand(float(4 ** k_bad))
    _report("fp16 operand headroom (A)", largest_operand_at_1=y1, headroom=65504.0 / y1, first_failing_scale=4 ** k_bad,
            largest_operand_last_passing=y_ok, largest_operand_first_failing=y_bad)
    assert y_ok <= 65504.0 * 1.01 and y_bad >= 65504.0 * 0.99, (y_ok, y_bad)
    assert 65504.0 / y1 >= 100.0  # the synthetic residual stream is far inside the range
    x = mk.run(x1, case["mods"], case["dt"], case["past"], cfg.action_dim)
    mk.check()
    assert torch.isfinite(x).all()
    mk.close()


def test_operand_shift_runs_a_residual_stream_beyond_the_fp16_range():
    """The remedy for MKX_ERANGE. The register tokens are scaled by 4^k (exact in bf16) until the register
    rows' residual stream makes an AdaRMS operand leave the fp16 range: the launch reports MKX_ERANGE at the
    default operand shift, and run_checked raises the shift by 8 (as often as needed) and returns actions (O(1):
    the action rows see the register rows only through normalised keys and values) that track the fp32
    oracle run with the same tokens within the parity bounds; the handle keeps the shift. At the unscaled
    tokens, shift 8 also stays within the bounds (operands of y below 6.1e-5 x 256 lose bits to fp16
    subnormals), and shift 0 again gives the default result bit for bit."""
    cfg = SY.WORKLOADS["A"]
    case = make_case(cfg)
    x1 = _first_step(case)
    mk = ExpertMegakernel(case["model"])
    n = cfg.num_steps - 1
    args = (case["mods"], case["dt"], case["past"], cfg.action_dim)
    x0 = mk.run(x1, *args).clone()
    mk.check()
    assert mk.operand_shift == 0
    tok = case["W"]["reg_tok"]
    k_bad = None
    for k in range(1, 20):
        mk.register_tokens = (tok.float() * float(4 ** k)).to(torch.bfloat16).to(x1.device)
        mk.run(x1, *args)
        torch.cuda.synchronize()
        try:
            mk.check()
        except MkxError as e:
            assert e.status == _lib.ERANGE, e
            k_bad = k
            break
    assert k_bad is not None
    x = mk.run_checked(x1, *args).clone()
    shift = mk.operand_shift
    assert shift >= 8 and torch.isfinite(x).all()
    W0 = dict(case["W"])
    case["W"] = dict(W0, reg_tok=(tok.float() * float(4 ** k_bad)).to(torch.bfloat16))
    try:
        ref = oracle_steps(case, x1, 1, n, "fp32")
    finally:
        case["W"] = W0
    mx, mean = diff(x, ref, cfg.action_dim)
    _report("operand shift past the fp16 range (A, register tokens x 4^k)", token_scale=4 ** k_bad, shift=shift,
            max_abs=mx, mean_abs=mean)
    assert mx <= 1e-2 and mean <= 2e-3, (mx, mean)
    mk.register_tokens = tok.to(x1.device)
    mk.set_operand_shift(8)
    x8 = mk.run(x1, *args).clone()
    mk.check()
    ref1 = oracle_steps(case, x1, 1, n, "fp32")
    mx8, mean8 = diff(x8, ref1, cfg.action_dim)
    mx0, mean0 = diff(x0, ref1, cfg.action_dim)
    _report("operand shift 8 at the unscaled tokens (A)", max_abs=mx8, mean_abs=mean8, shift0_max_abs=mx0,
            shift0_mean_abs=mean0)
    assert mx8 <= 1e-2 and mean8 <= 2e-3, (mx8, mean8)
    mk.set_operand_shift(0)
    x = mk.run(x1, *args)
    mk.check()
    assert torch.equal(x, x0)
    with pytest.raises(MkxError):
        mk.set_operand_shift(31)
    mk.close()


@pytest.mark.parametrize("name", ["B", "tiny fp8 b3", "D-b4"])
def test_operand_shift_in_the_row_wise_form(name):
    """The operand shift in the row-wise kernels (fp16-packed and fp8 weights; D-b4: the fp8 instantiations with
    two-tile attention tasks, 384 one-tile tasks on 256 workgroups): their shift twins track the fp32 oracle at
    shift 8 and, with register tokens scaled past the fp16 range (MKX_ERANGE at shift 0), after run_checked has
    raised the shift; shift 0 again gives the default result bit for bit."""
    cfg = SY.WORKLOADS[name] if name in SY.WORKLOADS else replace(TINY, B=3, weight_dtype="fp8_e4m3")
    import os
    old = os.environ.get("MKX_GEMM_FORM")
    os.environ["MKX_GEMM_FORM"] = "rows"
    try:
        case = make_case(cfg)
        mk = ExpertMegakernel(case["model"])
    finally:
        if old is None:
            os.environ.pop("MKX_GEMM_FORM", None)
        else:
            os.environ["MKX_GEMM_FORM"] = old
    x1 = _first_step(case)
    n = cfg.num_steps - 1
    args = (case["mods"], case["dt"], case["past"], cfg.action_dim)
    x0 = mk.run(x1, *args).clone()
    mk.check()
    assert int(_lib.lib().mkx_query(mk._h, _lib.Q_GEMM_FORM)) == 1  # the form of the last launch
    ref = oracle_steps(case, x1, 1, n, "fp32")
    mk.set_operand_shift(8)
    x8 = mk.run(x1, *args).clone()
    mk.check()
    mx8, mean8 = diff(x8, ref, cfg.action_dim)
    mx0, mean0 = diff(x0, ref, cfg.action_dim)
    assert mx8 <= 1e-2 and mean8 <= 2e-3, (mx8, mean8)
    mk.set_operand_shift(0)
    assert torch.equal(mk.run(x1, *args), x0)
    mk.check()
    tok = case["W"]["reg_tok"]
    k_bad = None
    for k in range(1, 20):
        mk.register_tokens = (tok.float() * float(4 ** k)).to(torch.bfloat16).to(x1.device)
        mk.run(x1, *args)
        torch.cuda.synchronize()
        try:
            mk.check()
        except MkxError as e:
            assert e.status == _lib.ERANGE, e
            k_bad = k
            break
    assert k_bad is not None
    x = mk.run_checked(x1, *args).clone()
    shift = mk.operand_shift
    W0 = dict(case["W"])
    case["W"] = dict(W0, reg_tok=(tok.float() * float(4 ** k_bad)).to(torch.bfloat16))
    try:
        ref_big = oracle_steps(case, x1, 1, n, "fp32")
    finally:
        case["W"] = W0
    mx, mean = diff(x, ref_big, cfg.action_dim)
    _report(f"operand shift, row-wise form ({name})", shift8_max_abs=mx8, shift8_mean_abs=mean8, shift0_max_abs=mx0,
            shift0_mean_abs=mean0, token_scale=4 ** k_bad, shift=shift, max_abs=mx, mean_abs=mean)
    assert shift >= 8 and mx <= 1e-2 and mean <= 2e-3, (shift, mx, mean)
    mk.close()
