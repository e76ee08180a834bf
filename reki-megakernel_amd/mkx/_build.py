"""Compile libmkx.so (the HIP megakernel + C ABI) for gfx950 with hipcc, in-tree.

The library is built from several translation units: the C ABI with the small kernels (mkx.hip) and one
unit per megakernel shape (mkx_mk768.hip, mkx_mk1024.hip, mkx_mk256.hip), so that each shape gets the
code-generation options measured best for it: the H = 768 megakernel is scheduled with LLVM's
max-memory-clause strategy (workload A 2.73 -> 2.70 ms, B 9.31 -> 9.24 ms, C 3.55 -> 3.49 ms); the same
strategy makes the H = 1024 fp8 megakernel 20 % slower, so the other shapes keep the default scheduler.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import tempfile

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
OUT = os.path.join(PKG, "libmkx.so")

# (translation unit, its extra hipcc options)
UNITS = (
    ("mkx.hip", ()),
    ("mkx_mk768.hip", ("-mllvm", "-amdgpu-sched-strategy=max-memory-clause")),
    ("mkx_mk1024.hip", ()),
    ("mkx_mk256.hip", ()),
    ("mkx_mk768r.hip", ()),
    ("mkx_mk1024r.hip", ()),
    ("mkx_mk256r.hip", ()),
    ("mkx_mk768p.hip", ()),
    ("mkx_mk1024p.hip", ()),
    ("mkx_mk256p.hip", ()),
    ("mkx_mk768l.hip", ("-mllvm", "-amdgpu-sched-strategy=max-memory-clause")),
    ("mkx_mk1024l.hip", ()),
    ("mkx_mk256l.hip", ()),
)
COMMON = ("--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
          # packed fp32 instructions stay off: every HIP source is compiled without them
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def _filter(text: str) -> list[str]:
    return [ln for ln in text.splitlines() if "packed-fp32-ops' is not a recognized" not in ln]


def build_library(verbose: bool = False, csrc: str = CSRC, out: str = OUT, extra: tuple = ()) -> str:
    """Compiles every translation unit (in parallel) and links them into `out`. `csrc` and `extra` (more
    hipcc options for every unit, e.g. -D defines) let a caller build a variant of the sources."""
    with tempfile.TemporaryDirectory(prefix="mkx_build_") as tmp:
        procs, objs = [], []
        for name, flags in UNITS:
            obj = os.path.join(tmp, name.replace(".hip", ".o"))
            cmd = [hipcc(), *COMMON, *extra, *flags, "-I", INCLUDE, "-I", csrc, "-c", os.path.join(csrc, name), "-o", obj]
            procs.append((name, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
            objs.append(obj)
        msgs, failed = [], []
        for name, p in procs:
            text, _ = p.communicate()
            msgs += _filter(text)
            if p.returncode != 0:
                failed.append(name)
        if failed:
            raise RuntimeError(f"hipcc failed on {', '.join(failed)}:\n" + "\n".join(msgs))
        r = subprocess.run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", out + ".tmp"],
                           capture_output=True, text=True)
        msgs += _filter(r.stdout + r.stderr)
        if r.returncode != 0:
            raise RuntimeError("link failed:\n" + "\n".join(msgs))
    if verbose and msgs:
        print("\n".join(msgs))
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build_library(verbose=True))
