"""Case builder shared by the parity tests: a synthetic expert, its call inputs, and the same inputs in
the CPU oracle's format. The oracle only supplies the expected results here."""
from __future__ import annotations

import torch

from mkx import synthetic as SY
from oracle import expert_ref as ER

TINY = SY.ExpertConfig(L=2, H=256, NH=4, I=512, T_act=5, R_reg=3, PM=16, kv_start=4, S=40, SP=48, ctx_dim=96,
                       tdim=32, num_steps=4)


def oracle_dims(cfg: SY.ExpertConfig) -> ER.ExpertDims:
    return ER.ExpertDims(L=cfg.L, H=cfg.H, NH=cfg.NH, HD=cfg.HD, I=cfg.I, A=cfg.A, ctx_dim=cfg.ctx_dim,
                         tdim=cfg.tdim, eps=cfg.eps, qk_eps=cfg.qk_eps, act=cfg.act)


def make_case(cfg: SY.ExpertConfig, device="cuda", seed=0, random_mods=False, nan_pads=False, ca_len=None,
              kv_start=None):
    """ca_len / kv_start: per-sample source lengths and first valid memory rows (default cfg.S, cfg.kv_start)."""
    W = SY.make_weights(cfg, seed)
    model = SY.SyntheticReki(cfg, W, device=device)
    inp = SY.make_inputs(cfg)
    past = model.register_prepare(inp["ctx"], inp["mem_states"], ca_len=ca_len, kv_start=kv_start)
    mods, dt = model._step_modulations(cfg.num_steps, inp["state_cond"])
    if random_mods:
        g = torch.Generator().manual_seed(99)
        mods = (torch.randn(tuple(mods.shape), generator=g) * 0.3).to(mods.device)
    if nan_pads:
        for (k, v) in past.register_step["mem_kv"]:
            (k if k.dim() == 4 else k[None])[:, : cfg.kv_start] = float("nan")
            (v if v.dim() == 4 else v[None])[:, : cfg.kv_start] = float("nan")
        for (k, v) in past.cross_attn_kv:
            (k if k.dim() == 4 else k[None])[:, cfg.S:] = float("nan")
            (v if v.dim() == 4 else v[None])[:, cfg.S:] = float("nan")
    return {"cfg": cfg, "W": W, "model": model, "inp": inp, "past": past, "mods": mods, "dt": dt,
            "noise": inp["noise"].to(device)}


def oracle_cache(case, first=False) -> dict:
    cfg, past, W = case["cfg"], case["past"], case["W"]
    st = past.register_step
    as5 = lambda t: (t if t.dim() == 4 else t[None]).float().cpu()  # noqa: E731
    sa = st["sa_pe_first" if first else "sa_pe"]
    ca = st["ca_pe_first" if first else "ca_pe"]
    m_q = sa[0].shape[0]
    c = {
        "memk": torch.stack([as5(k) for k, _ in st["mem_kv"]]), "memv": torch.stack([as5(v) for _, v in st["mem_kv"]]),
        "kca": torch.stack([as5(k) for k, _ in past.cross_attn_kv]), "vca": torch.stack([as5(v) for _, v in past.cross_attn_kv]),
        "kv_start": st["kv_start"].cpu().long(), "ca_len": st["ca_len"].cpu().long(),
        "sa_cos": sa[0].cpu(), "sa_sin": sa[1].cpu(), "ca_cos": ca[0].cpu(), "ca_sin": ca[1].cpu(),
    }
    if m_q > cfg.T_act:
        c["reg_tok"] = W["reg_tok"].float()[: m_q - cfg.T_act]
    return c


def oracle_mods(case) -> torch.Tensor:
    m = case["mods"].float().cpu()
    return m[None] if m.dim() == 2 else m


def oracle_steps(case, x_in: torch.Tensor, first_row: int, n: int, mode: str, first=False, reg_kv_out=None):
    cfg = case["cfg"]
    return ER.run_steps(x_in.float().cpu(), oracle_mods(case)[:, first_row: first_row + n], float(case["dt"].item()),
                        SY.oracle_weights(case["W"]), oracle_cache(case, first), oracle_dims(cfg), cfg.action_dim, mode,
                        reg_kv_out=reg_kv_out)


def diff(a: torch.Tensor, b: torch.Tensor, adim: int) -> tuple[float, float]:
    d = (a.float().cpu()[..., :adim] - b.float().cpu()[..., :adim]).abs()
    return float(d.max()), float(d.mean())
