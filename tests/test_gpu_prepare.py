"""GPU: ``mkx_prepare_source`` (through the C ABI, via mkx.prepare.SourcePrepare) against the CPU oracle's
``register_prepare`` in ``mirror`` mode (bf16 rounding after the projection, the norm and the rotation,
the points the kernel rounds at), and the expert run on the kernel's caches against the fp32 oracle.

Tolerance: accumulation order (MFMA vs the CPU's) and rsqrt can move a bf16 rounding by one unit, and the
rotation mixes the two halves of a head, so K is bounded per RoPE pair, |delta| <= 2^-6 |(x_d, x_d+32)|,
and V per element, |delta| <= 2^-7 |v| + 2^-12. A wrong position, sign, norm weight or head fails both by
orders of magnitude."""
import json
from dataclasses import replace

import pytest
import torch

from _cases import TINY, diff, make_case, oracle_dims, oracle_steps
from mkx import ExpertMegakernel, synthetic as SY
from mkx.prepare import SourcePrepare
from oracle import expert_ref as ER

pytestmark = pytest.mark.gpu
torch.set_grad_enabled(False)


def _report(name, **kv):
    print(json.dumps({"case": name, **kv}), flush=True)


def _check_prepare(name, cfg, ca_len=None):
    W = SY.make_weights(cfg, 0)
    model = SY.SyntheticReki(cfg, W, device="cuda")
    inp = SY.make_inputs(cfg)
    ca_len = [cfg.S] * cfg.B if ca_len is None else ca_len
    ctx = inp["ctx"]
    prep = SourcePrepare(model)
    kv = prep(ctx.cuda(), ca_len)
    torch.cuda.synchronize()
    ref = ER.register_prepare(ctx, ca_len, inp["mem_states"][:, :0], [0] * cfg.B, SY.oracle_weights(W), oracle_dims(cfg),
                              cfg.m_q, mode="mirror")
    gk = torch.stack([k for k, _ in kv]).float().cpu()  # [L, B, SP, NH, 64]
    gv = torch.stack([v for _, v in kv]).float().cpu()
    rk, rv = ref["kca"].float(), ref["vca"].float()
    pn = torch.sqrt(rk[..., :32] ** 2 + rk[..., 32:] ** 2).repeat(1, 1, 1, 1, 2)
    dk, dv = (gk - rk).abs(), (gv - rv).abs()
    exact_k = float((dk == 0).float().mean())
    exact_v = float((dv == 0).float().mean())
    _report(name, k_max=float(dk.max()), v_max=float(dv.max()), k_exact_frac=exact_k, v_exact_frac=exact_v)
    assert (dk <= 2.0 ** -6 * pn + 1e-6).all()
    assert (dv <= 2.0 ** -7 * rv.abs() + 2.0 ** -12).all()
    for b, n in enumerate(ca_len):
        n = min(max(n, 0), cfg.SP)
        assert (gk[:, b, n:] == 0).all() and (gv[:, b, n:] == 0).all()
    return model, kv


def test_prepare_tiny():
    _check_prepare("prepare tiny (C 96, SP 48)", TINY)


def test_prepare_odd_head_count():
    # three heads: the workgroups take heads in pairs, so the last pair's second head is computed and not stored
    _check_prepare("prepare NH 3 (odd head pair)", replace(TINY, H=192, NH=3, I=384))


def test_prepare_config_A_context():
    _check_prepare("prepare A (L10, C 2048, S 300)", SY.WORKLOADS["A"])


def test_prepare_batch_with_ragged_lengths():
    cfg = replace(SY.WORKLOADS["A"], B=4, L=3)
    _check_prepare("prepare B4 ragged", cfg, ca_len=[300, 1, 0, 150])


def test_prepare_wide_expert():
    cfg = replace(SY.WORKLOADS["D"], L=4)
    _check_prepare("prepare D shape (NH16, 4 layers)", cfg)


def test_expert_on_kernel_prepared_caches():
    """Euler steps 2..N on caches from the kernel: within the tight bound of the fp32 oracle run on the
    same caches, and close to the run on the PyTorch-prepared caches."""
    case = make_case(SY.WORKLOADS["A"])
    cfg, model, past = case["cfg"], case["model"], case["past"]
    x1, _, _ = model._expert_first_step(case["noise"], past, None, case["mods"][..., :1, :], case["dt"], cfg.action_dim)
    mk = ExpertMegakernel(model)
    x_torch = mk.run(x1, case["mods"], case["dt"], past, cfg.action_dim)
    past.cross_attn_kv = SourcePrepare(model)(case["inp"]["ctx"].cuda()[0], [cfg.S])
    x_kern = mk.run(x1, case["mods"], case["dt"], past, cfg.action_dim)
    mk.check()
    torch.cuda.synchronize()
    r32 = oracle_steps(case, x1, 1, cfg.num_steps - 1, "fp32")
    m, a = diff(x_kern, r32, cfg.action_dim)
    mt, _ = diff(x_kern, x_torch, cfg.action_dim)
    _report("expert on kernel caches (A)", vs_fp32_max=m, vs_fp32_mean=a, vs_torch_caches_max=mt)
    assert m <= 1e-3 and a <= 2e-4
    assert mt <= 1e-2


def test_prepare_timing_config_A():
    """Times one preparation of config A's source (10 layers, 300 x 2048 context); reported, not asserted."""
    cfg = SY.WORKLOADS["A"]
    model = SY.SyntheticReki(cfg, SY.make_weights(cfg, 0), device="cuda")
    ctx = SY.make_inputs(cfg)["ctx"].cuda()
    prep = SourcePrepare(model)
    for _ in range(3):
        prep(ctx, [cfg.S])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(20):
        prep(ctx, [cfg.S])
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / 20
    inp = SY.make_inputs(cfg)
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(5):
        model.register_prepare(inp["ctx"], inp["mem_states"])
    t1.record()
    torch.cuda.synchronize()
    _report("prepare timing A", kernel_us=us, torch_register_prepare_us=t0.elapsed_time(t1) * 1e3 / 5)


def test_prepare_rejects_more_rows_than_the_handle_stages():
    from mkx._lib import MkxError
    model = SY.SyntheticReki(TINY, SY.make_weights(TINY, 0), device="cuda")
    prep = SourcePrepare(model, max_rows=TINY.SP - 1)
    with pytest.raises(MkxError):
        prep(SY.make_inputs(TINY)["ctx"].cuda(), [TINY.S])
    prep.close()


def test_whole_call_captured_in_one_graph_replays_match_eager():
    """Step modulations (modulation input and projection), source caches and Euler steps 1..N captured as one
    HIP graph: every replay, with eager work and a synchronisation between replays, equals the eager call bit
    for bit."""
    from mkx.modulations import StepModulations
    case = make_case(SY.WORKLOADS["A"])
    cfg, model, past, W = case["cfg"], case["model"], case["past"], case["W"]
    mk = ExpertMegakernel(model)
    prep = SourcePrepare(model)
    step_mods = StepModulations(*(W[k].cuda() for k in ("t1_w", "t1_b", "t2_w", "t2_b", "mod_w", "mod_b")))
    sc = case["inp"]["state_cond"].cuda()
    ctx = case["inp"]["ctx"].cuda()
    ca_len = torch.tensor([cfg.S], dtype=torch.int32, device="cuda")
    out = {}

    def call():
        mods, dt = step_mods(cfg.num_steps, sc)
        past.cross_attn_kv = [(k[0], v[0]) for k, v in prep(ctx, ca_len)]
        out["x"], out["k"], out["v"] = mk.run_all(case["noise"], mods, dt, past, cfg.action_dim)

    call()
    mk.check()
    torch.cuda.synchronize()
    x_e, k_e = out["x"].clone(), out["k"].clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()  # warm-up on a side stream, as capture requires
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    torch.cuda.synchronize()
    times = []
    for i in range(3):
        out["x"].zero_()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        g.replay()
        e1.record()
        noise = torch.randn(4096, device="cuda").square().sum()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        times.append(e0.elapsed_time(e1))
        assert torch.equal(out["x"], x_e) and torch.equal(out["k"], k_e), f"replay {i} differs from the eager call"
    mk.check()
    _report("whole call graph replays (A)", replays=3, ms=times)


def test_frames_with_ring_append_as_two_graphs_match_eager():
    """Four calls (frames) of modulations + source caches + steps 1..N + register append, replayed as two
    captured graphs, one per buffer parity of the ring (G0 reads set 0 and appends into set 1, G1 the
    reverse): every frame's result equals the eager sequence's, bit for bit, and kv_start evolves on the
    device (from an empty memory: kv_start = PM, then PM - R, ... 0)."""
    from mkx.modulations import ModulationProjection
    from mkx.ring import RegisterRing
    case = make_case(replace(SY.WORKLOADS["A"], kv_start=SY.WORKLOADS["A"].PM))
    cfg, model, past, W = case["cfg"], case["model"], case["past"], case["W"]
    mk = ExpertMegakernel(model)
    prep = SourcePrepare(model)
    proj = ModulationProjection(W["mod_w"].cuda(), W["mod_b"].float().cuda())
    sc = case["inp"]["state_cond"].cuda()
    ctx = case["inp"]["ctx"].cuda()
    ca_len = torch.tensor([cfg.S], dtype=torch.int32, device="cuda")
    dt = torch.full((1,), -1.0 / cfg.num_steps, device="cuda")
    mem0 = [(k.clone(), v.clone()) for k, v in past.register_step["mem_kv"]]
    ks0 = past.register_step["kv_start"].clone()
    R, T = cfg.R_reg, cfg.T_act
    out = {}

    def call():
        mods = proj(model.modulation_input(cfg.num_steps, sc))[0]
        past.cross_attn_kv = [(k[0], v[0]) for k, v in prep(ctx, ca_len)]
        out["x"], out["k"], out["v"] = mk.run_all(case["noise"], mods, dt, past, cfg.action_dim)

    ring_e = RegisterRing(mem0, ks0, R, kept_delta=-R, new_delta=-(T + R))
    ring_e.update_past(past)
    xs, kss = [], []
    for _ in range(4):
        call()
        xs.append(out["x"].clone())
        ring_e.append_frame(out["k"], out["v"])
        ring_e.update_past(past)
        kss.append(int(ring_e.kv_start[0]))
    mk.check()
    torch.cuda.synchronize()
    assert not torch.equal(xs[0], xs[1])  # the memory changes between frames

    ring_g = RegisterRing(mem0, ks0, R, kept_delta=-R, new_delta=-(T + R))
    ring_g.update_past(past)
    call()  # warm-up (no append: the ring's state is untouched)
    torch.cuda.synchronize()
    graphs, x_of = [], []
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            call()
            ring_g.append_frame(out["k"], out["v"])
        ring_g.update_past(past)  # the next graph reads the other buffer set
        graphs.append(g)
        x_of.append(out["x"])
    torch.cuda.synchronize()
    for f in range(4):
        graphs[f % 2].replay()
        noise = torch.randn(4096, device="cuda").square().sum()  # eager work between replays
        torch.cuda.synchronize()
        assert torch.isfinite(noise)
        assert torch.equal(x_of[f % 2], xs[f]), f"frame {f} differs from the eager sequence"
        assert int(ring_g._ks[(f + 1) % 2][0]) == kss[f]
    mk.check()
    assert kss == [max(cfg.PM - (f + 1) * R, 0) for f in range(4)]
    _report("frames as two graphs (A)", frames=4, kv_start=kss)
