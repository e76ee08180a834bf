"""The synthetic REKI-shaped model's step-1-side code (modulations, cache preparation) on the CPU, against
the oracle's restatement of the same definitions; workload bookkeeping."""
import torch

from _cases import TINY, oracle_dims
from mkx import synthetic as SY
from oracle import expert_ref as ER

torch.set_grad_enabled(False)


def test_modulations_match_oracle():
    W = SY.make_weights(TINY)
    model = SY.SyntheticReki(TINY, W, device="cpu")
    inp = SY.make_inputs(TINY)
    mods, dt = model._step_modulations(TINY.num_steps, inp["state_cond"])
    ref, rdt = ER.step_modulations(TINY.num_steps, inp["state_cond"], SY.oracle_weights(W), oracle_dims(TINY))
    assert mods.shape == (TINY.num_steps, TINY.modw)
    assert float(dt) == rdt == -1.0 / TINY.num_steps
    torch.testing.assert_close(mods, ref[0], rtol=1e-5, atol=1e-5)


def test_register_prepare_matches_oracle_mirror():
    W = SY.make_weights(TINY)
    model = SY.SyntheticReki(TINY, W, device="cpu")
    inp = SY.make_inputs(TINY)
    past = model.register_prepare(inp["ctx"], inp["mem_states"])
    ref = ER.register_prepare(inp["ctx"].float(), [TINY.S], inp["mem_states"], [TINY.kv_start], SY.oracle_weights(W),
                              oracle_dims(TINY), m_q=TINY.m_q, mode="mirror")
    kca = torch.stack([k.float()[None] for k, _ in past.cross_attn_kv])
    memk = torch.stack([k.float()[None] for k, _ in past.register_step["mem_kv"]])
    memv = torch.stack([v.float()[None] for _, v in past.register_step["mem_kv"]])
    torch.testing.assert_close(kca, ref["kca"], rtol=0, atol=0)
    torch.testing.assert_close(memk, ref["memk"], rtol=0, atol=0)
    torch.testing.assert_close(memv, ref["memv"], rtol=0, atol=0)
    torch.testing.assert_close(past.register_step["sa_pe"][0], ref["sa_cos"], rtol=0, atol=0)
    assert int(past.register_step["cu_kv"][0]) == TINY.kv_start and int(past.register_step["cu_src"][1]) == TINY.S


def test_weights_are_seeded_bf16_and_reki_shaped():
    a = SY.make_weights(TINY, seed=0)
    b = SY.make_weights(TINY, seed=0)
    assert torch.equal(a["layers"][1]["down"], b["layers"][1]["down"])
    assert a["layers"][0]["q"].dtype == torch.bfloat16
    assert abs(float(a["layers"][0]["gate"].float().std()) - 0.02) < 2e-3
    model = SY.SyntheticReki(TINY, a, device="cpu")
    lay = model.vlm_with_expert.action_expert.layers[0]
    assert lay.self_attn.q_proj.weight.shape == (TINY.H, TINY.H)
    assert lay.mlp.gate_proj.out_features == TINY.I
    assert model.action_in_proj.in_features == TINY.A


def test_fp8_weights_dequantise_exactly_from_e4m3_and_scale():
    from dataclasses import replace
    cfg = replace(TINY, weight_dtype="fp8_e4m3")
    W = SY.make_weights(cfg)
    ly = W["layers"][0]
    deq = ly["gate_q"].float() * ly["gate_scale"][:, None]
    torch.testing.assert_close(ly["gate"], deq, rtol=0, atol=0)
    assert ly["gate_q"].float().abs().max() <= 448


def test_algorithmic_bytes_of_workload_A():
    # 10 x (6 H^2 + 3 H I) x 2 B = 212.3 MB of weights; + CA K/V 9.22 MB + memory K/V 2.95 MB + mods + projections
    b = SY.algorithmic_bytes_per_step(SY.WORKLOADS["A"])
    assert abs(b / 1e6 - 225.0) < 0.2
    assert abs(SY.algorithmic_bytes_per_step(SY.WORKLOADS["C"]) / 1e6 - 252.1) < 0.2
