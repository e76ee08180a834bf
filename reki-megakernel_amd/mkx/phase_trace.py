"""Phase timeline of one Euler launch (diagnostic; not used by the expert call).

``python3 reki-megakernel_amd/mkx/phase_trace.py --build`` compiles the library with MKX_TRACE into
libmkx_trace.so beside libmkx.so: every workgroup then stamps the 100 MHz clock (s_memrealtime) at fixed
points of each stage (wait passed, operands landed, MFMAs and cross-wave sum done, epilogue done, stage
done; the down projection's reducers when they publish). ``--workload W --out F`` loads that library
instead of libmkx.so, runs one profiled launch of Euler steps 2..N of the named synthetic workload and writes,
per stage kind, medians over the launch's layers of:

- ``wait``: from the last producer task of the stage before finishing (its workgroup's stage-done stamp)
  to the last consumer task passing its ready-epoch wait: the time a stage boundary costs beyond the work;
- ``work``: from there to the stage's last task finishing;
- for GEMM stages in the pass form, the phases of a median task after its wait: first operands landed,
  MFMAs and cross-wave sum, epilogue, publish (store acknowledgements and the ready epoch);
- for the attention stages in the pass form, likewise: self-attention's query tile and own keys landed
  (with the barrier after them), attention over every key block, merge of the four waves' states, store and
  publish; cross-attention's query rows landed, query projection MFMAs, its epilogue (norm, RoPE, the query
  tile into LDS and the barrier), attention, merge and store, publish.

The trace build times slightly differently from libmkx.so (its stamps are stores on the critical path).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

TRACE_LIB = os.path.join(PKG, "libmkx_trace.so")
TRACE_BASE, TRACE_SLOTS = 8192, 16  # the kernel's trace layout (csrc/mkx_kernel.h)
STAGES = ["qkv", "sa_attn", "sa_o", "ca_attn", "ca_o", "gate_up", "down"]
GEMM = {"qkv", "sa_o", "ca_o", "gate_up", "down"}
# attention stages in the pass form: phase -> (from stamp slot, to stamp slot) of sa_stage / ca_stage
ATTN = {
    "sa_attn": {"operands": (0, 1), "attention": (1, 2), "merge_store_publish": (2, 4)},
    "ca_attn": {"query_rows": (0, 3), "query_projection": (3, 7), "query_epilogue": (7, 1), "attention": (1, 2),
                "merge_store": (2, 13), "publish": (13, 4)},
}


def build() -> str:
    from mkx import _build
    return _build.build_library(out=TRACE_LIB, extra=("-DMKX_TRACE",))


def _nanmed(v):
    v = [x for x in v if x == x]
    return statistics.median(v) if v else float("nan")


def trace(workload: str, raw_out: str = "") -> dict:
    from mkx import _lib
    _lib.LIB_PATH = TRACE_LIB
    import torch
    from mkx import ExpertMegakernel, synthetic as SY

    torch.set_grad_enabled(False)
    cfg = SY.WORKLOADS[workload]
    dev = torch.device("cuda:0")
    W = SY.make_weights(cfg, seed=0)
    model = SY.SyntheticReki(cfg, W, device=dev)
    inp = SY.make_inputs(cfg)
    past = model.register_prepare(inp["ctx"], inp["mem_states"])
    mods, dt = model._step_modulations(cfg.num_steps, inp["state_cond"])
    x1, _, _ = model._expert_first_step(inp["noise"].to(dev), past, None, mods[..., :1, :], dt, cfg.action_dim)
    mk = ExpertMegakernel(model)
    plan = mk.plan(x1, mods, dt, past, cfg.action_dim)
    n = cfg.num_steps - 1
    G = int(_lib.lib().mkx_query(mk._h, _lib.Q_GRID))
    total = mk.barriers(n)
    plen = TRACE_BASE + (total + 2) * G * TRACE_SLOTS
    prof = torch.zeros(plen, dtype=torch.int64, device=dev)
    for _ in range(5):
        plan.launch()
    torch.cuda.synchronize()
    _lib.check(_lib.lib().mkx_set_profile(mk._h, ctypes.c_void_p(prof.data_ptr()), plen), "mkx_set_profile")
    plan.launch()
    torch.cuda.synchronize()
    mk.check()
    raw = prof.cpu()[TRACE_BASE: TRACE_BASE + (total + 1) * G * TRACE_SLOTS].view(total + 1, G, TRACE_SLOTS)
    if raw_out:  # every workgroup's stamps, [boundary][workgroup][slot] (100 MHz ticks; 0 = not stamped)
        torch.save(raw.clone(), raw_out)
    t0 = int(raw[raw > 0].min())
    us = torch.where(raw > 0, (raw - t0).double() * 0.01, torch.full_like(raw, float("nan"), dtype=torch.float64))
    per = 7 * cfg.L + 1
    # the form the library chose for the traced launch (row-wise GEMM stages stamp other points, so only the
    # pass form's phases are reported)
    rows_form = int(_lib.lib().mkx_query(mk._h, _lib.Q_GEMM_FORM)) == 1
    rows = {k: [] for k in STAGES + ["tail"]}
    for g in range(1, total):
        j = (g - 1) % per
        kind = "tail" if j == per - 1 else STAGES[j % 7]
        prev_done = float(torch.nan_to_num(us[g - 1, :, 4], nan=-1.0).max())
        done = float(torch.nan_to_num(us[g, :, 4], nan=-1.0).max())
        act = ~torch.isnan(us[g, :, 0])
        if not bool(act.any()):
            continue
        wait_end = float(us[g, act, 0].max())
        rec = {"wait": wait_end - prev_done, "work": done - wait_end}
        if kind == "down":
            red = us[g, :, 7]
            red = red[~torch.isnan(red)]
            if red.numel():
                rec["reducers_done"] = float(red.max()) - prev_done
        if kind in GEMM and not rows_form:
            a = us[g, act]
            rec["first_operands"] = _nanmed((a[:, 1] - a[:, 0]).tolist())
            rec["mfma_and_sum"] = _nanmed((a[:, 2] - a[:, 1]).tolist())
            rec["epilogue"] = _nanmed((a[:, 3] - a[:, 2]).tolist())
            rec["publish"] = _nanmed((a[:, 4] - a[:, 3]).tolist())
        if kind in ATTN and not rows_form:
            a = us[g, act]
            for name, (s0, s1) in ATTN[kind].items():
                rec[name] = _nanmed((a[:, s1] - a[:, s0]).tolist())
        rows[kind].append(rec)
    out = {"workload": workload, "form": "row-wise" if rows_form else "passes",
           "launch_us": float(torch.nan_to_num(us[total - 1, :, 4], nan=-1.0).max()), "stages": {}}
    for k, v in rows.items():
        if v:
            keys = sorted({kk for r in v for kk in r})
            out["stages"][k] = {kk: round(_nanmed([r.get(kk, float("nan")) for r in v]), 3) for kk in keys}
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--build", action="store_true", help="compile libmkx_trace.so and exit")
    ap.add_argument("--workload", default="A")
    ap.add_argument("--out", default="")
    ap.add_argument("--raw", default="", help="also save every workgroup's raw stamps (torch.save)")
    a = ap.parse_args()
    if a.build:
        print(build())
        return 0
    res = trace(a.workload, a.raw)
    text = json.dumps(res, indent=1)
    if a.out:
        with open(a.out, "w") as f:
            f.write(text)
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
