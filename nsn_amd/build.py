"""Build libnsn_hip.so (gfx950) in-tree with hipcc.

    python -m nsn_amd.build

Flags: -O3; -ffp-contract=off (the codec must not contract multiply-adds that
torch rounds separately; fma is written explicitly where torch fuses); packed
fp32 VALU ops disabled (-Xclang -target-feature -Xclang -packed-fp32-ops).
fp32 division and square root keep hipcc's correctly rounded default.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
SRC = PKG / "csrc"
OUT_DIR = PKG / "_build"
LIB = OUT_DIR / "libnsn_hip.so"
SOURCES = ["nsn_codec.hip", "nsn_attn.hip", "nsn_fast.hip", "nsn_prefill.hip", "nsn_cache.hip", "nsn_kscore.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = ["-O3", "-fPIC", "-std=c++17", "-ffp-contract=off",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall"]


def sources():
    return [SRC / s for s in SOURCES if (SRC / s).exists()]


def build(verbose=False, jobs=None):
    """Compile each source to an object in parallel, then link the shared library."""
    OUT_DIR.mkdir(exist_ok=True)
    objs = []
    procs = []
    for s in sources():
        o = OUT_DIR / (s.stem + ".o")
        objs.append(o)
        cmd = [HIPCC, f"--offload-arch={ARCH}", *FLAGS, "-c", str(s), "-o", str(o)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((s, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = []
    for s, p in procs:
        out, _ = p.communicate()
        msgs = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
        if p.returncode != 0:
            failed.append(s.name)
            print("\n".join(msgs), file=sys.stderr)
        elif verbose and msgs:
            print("\n".join(msgs))
    if failed:
        raise RuntimeError(f"hipcc failed on {failed}")
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
