"""GPU: ``mkx_ring_append`` (through the C ABI, via mkx.ring.RegisterRing) against the CPU oracle, bit for
bit, and an episode of calls where each call's register rows feed the next call's memory."""
import json
from dataclasses import replace

import pytest
import torch

from _cases import TINY, diff, make_case, oracle_steps
from mkx import ExpertMegakernel, synthetic as SY
from mkx.ring import RegisterRing, rope_delta
from oracle.ring_ref import ring_append

pytestmark = pytest.mark.gpu
torch.set_grad_enabled(False)


def _report(name, **kv):
    print(json.dumps({"case": name, **kv}), flush=True)


def _check_append(name, L, B, PM, NH, R, kv_start, kept=-1, new=-2, seed=0, frames=2):
    g = torch.Generator().manual_seed(seed)
    rnd = lambda *s: torch.randn(*s, generator=g).to(torch.bfloat16)  # noqa: E731
    memk, memv = rnd(L, B, PM, NH, 64), rnd(L, B, PM, NH, 64)
    mem_kv = [(memk[l].cuda(), memv[l].cuda()) for l in range(L)]
    ring = RegisterRing(mem_kv, kv_start, R, kept_delta=kept, new_delta=new)
    sh = None if kept is None else rope_delta(kept, 64, device="cpu")
    nw = None if new is None else rope_delta(new, 64, device="cpu")
    ks = torch.tensor(kv_start, dtype=torch.int32)
    for f in range(frames):
        ck, cv = rnd(L, B, R, NH, 64), rnd(L, B, R, NH, 64)
        ring.append_frame(ck.cuda(), cv.cuda())
        memk, memv, ks = ring_append(memk, memv, ck, cv, ks, sh, nw)
        torch.cuda.synchronize()
        gk = torch.stack([k for k, _ in ring.mem_kv]).cpu()
        gv = torch.stack([v for _, v in ring.mem_kv]).cpu()
        assert torch.equal(ring.kv_start.cpu(), ks), (name, f)
        assert torch.equal(gv, memv), (name, f, "V")
        assert torch.equal(gk.view(torch.int16), memk.view(torch.int16)), (name, f, "K")
    _report(name, frames=frames, kv_start=ks.tolist())


def test_append_config_A_shape():
    _check_append("ring A (L10 B1 PM96 NH12 R32)", 10, 1, 96, 12, 32, [64], kept=-32, new=-42)


def test_append_batch_with_every_kv_start_case():
    # valid, partial, empty, full, clamped above and below, exactly R
    _check_append("ring B8 kv_start cases", 3, 8, 96, 12, 32, [0, 5, 96, 64, 200, -7, 32, 95], seed=1, frames=3)


def test_append_wide_expert_shape():
    _check_append("ring D (L16 NH16)", 16, 4, 96, 16, 32, [0, 32, 64, 96], kept=-32, new=-82, seed=2)


def test_append_edges():
    _check_append("ring R = PM", 2, 2, 16, 4, 16, [0, 8], seed=3)
    _check_append("ring R = 1, odd NH", 2, 3, 7, 3, 1, [0, 3, 7], seed=4, frames=4)
    _check_append("ring no rotation", 2, 2, 12, 2, 4, [4, 12], kept=None, new=None, seed=5)


def test_episode_register_rows_feed_the_next_call():
    """Three calls: each call's step-1 register K/V enter the memory of the next through the ring; every
    call's result tracks the fp32 oracle run on the memory the ring produced, and that memory equals the
    oracle ring's, bit for bit."""
    case = make_case(replace(TINY, kv_start=TINY.PM))  # empty memory before the first call
    cfg, model, past = case["cfg"], case["model"], case["past"]
    mk = ExpertMegakernel(model)
    ring = model.register_ring(past)
    R, T = cfg.R_reg, cfg.T_act
    sh, nw = rope_delta(-R, 64, device="cpu"), rope_delta(-(T + R), 64, device="cpu")
    memk = torch.stack([k for k, _ in ring.mem_kv]).cpu()[:, None]  # [L, 1, PM, NH, 64]
    memv = torch.stack([v for _, v in ring.mem_kv]).cpu()[:, None]
    ks = torch.tensor([cfg.PM], dtype=torch.int32)
    for call in range(3):
        x, ck, cv = mk.run_all(case["noise"], case["mods"], case["dt"], past, cfg.action_dim)
        mk.check()
        torch.cuda.synchronize()
        ref = oracle_steps(case, case["noise"], 0, cfg.num_steps, "fp32", first=True)
        m, a = diff(x, ref, cfg.action_dim)
        _report("episode call", call=call, kv_start=int(ks[0]), vs_fp32_max=m, vs_fp32_mean=a)
        assert m <= 1e-3 and a <= 2e-4, (call, m, a)
        ring.append_frame(ck, cv)
        ring.update_past(past)
        memk, memv, ks = ring_append(memk, memv, ck.cpu(), cv.cpu(), ks, sh, nw)
        torch.cuda.synchronize()
        assert torch.equal(torch.stack([k for k, _ in past.register_step["mem_kv"]]).cpu().view(torch.int16), memk[:, 0].view(torch.int16))
        assert torch.equal(torch.stack([v for _, v in past.register_step["mem_kv"]]).cpu(), memv[:, 0])
        assert int(past.register_step["kv_start"][0]) == int(ks[0]) == int(past.register_step["cu_kv"][0])
    assert int(ks[0]) == max(cfg.PM - 3 * R, 0)


def test_append_throughput_config_B_memory():
    """Times the append over config B's memory (8 samples, L10, PM96, NH12, R32): 2 x read + write of
    K and V; reported, not asserted."""
    L, B, PM, NH, R = 10, 8, 96, 12, 32
    mem_kv = [(torch.randn(B, PM, NH, 64, device="cuda").to(torch.bfloat16),
               torch.randn(B, PM, NH, 64, device="cuda").to(torch.bfloat16)) for _ in range(L)]
    ring = RegisterRing(mem_kv, [0] * B, R, kept_delta=-R, new_delta=-42)
    ck = torch.randn(L, B, R, NH, 64, device="cuda").to(torch.bfloat16)
    cv = torch.randn_like(ck)
    for _ in range(5):
        ring.append_frame(ck, cv)
    torch.cuda.synchronize()
    n = 200
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        ring.append_frame(ck, cv)
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / n
    nbytes = 2 * L * B * PM * NH * 64 * 2 * 2  # K and V, read + write
    _report("ring append B8 throughput", us=us, GB_s=nbytes / us / 1e3)
