"""Build libnsn_hip.so (gfx950) in-tree with hipcc.

    python -m nsn_amd.build
    python -m nsn_amd.build --resource-usage [source.hip ...]   # compiler's per-kernel resource report

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


_RES_KEYS = (("VGPRs", "vgpr"), ("AGPRs", "agpr"), ("TotalSGPRs", "sgpr"), ("ScratchSize [bytes/lane]", "scratch"),
             ("Occupancy [waves/SIMD]", "occupancy"), ("SGPRs Spill", "sgpr_spill"), ("VGPRs Spill", "vgpr_spill"),
             ("LDS Size [bytes/block]", "lds"))


def resource_usage(source):
    """Per-kernel register, spill, scratch, LDS and occupancy figures of one
    source as the compiler reports them (-Rpass-analysis=kernel-resource-usage,
    device code only, same flags as the build).  Returns {mangled name: {key: int}}."""
    cmd = [HIPCC, f"--offload-arch={ARCH}", *FLAGS, "--cuda-device-only", "-c", str(SRC / source), "-o", os.devnull,
           "-Rpass-analysis=kernel-resource-usage"]
    out = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, check=True).stdout
    kernels, cur = {}, None
    for ln in out.splitlines():
        if "remark:" not in ln:
            continue
        msg = ln.split("remark:", 1)[1].split("[-Rpass", 1)[0].strip()
        if msg.startswith("Function Name:"):
            cur = kernels.setdefault(msg.split(":", 1)[1].strip(), {})
            continue
        for label, key in _RES_KEYS:
            if cur is not None and msg.startswith(label + ":"):
                cur[key] = int(msg.split(":", 1)[1].strip())
    return kernels


def _demangle(names):
    try:
        out = subprocess.run(["c++filt"], input="\n".join(names), stdout=subprocess.PIPE, text=True, check=True).stdout
        return out.splitlines()
    except (OSError, subprocess.CalledProcessError):
        return list(names)


def resource_table(sources=None):
    """Markdown table of resource_usage() over the given (default: all) sources."""
    rows = ["| kernel | VGPR | AGPR | SGPR | SGPR spill | VGPR spill | scratch B/lane | LDS B/workgroup | waves/SIMD |",
            "|---|---|---|---|---|---|---|---|---|"]
    for s in sources or SOURCES:
        ks = resource_usage(s)
        for name, pretty in zip(ks, _demangle(list(ks))):
            r = ks[name]
            short = pretty.replace("nsn::", "").split("(")[0]
            rows.append(f"| `{short}` ({s}) | " + " | ".join(
                str(r.get(k, "?")) for k in ("vgpr", "agpr", "sgpr", "sgpr_spill", "vgpr_spill", "scratch", "lds",
                                             "occupancy")) + " |")
    return "\n".join(rows)


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "--resource-usage":
        print(resource_table(sys.argv[2:] or None))
    else:
        print(build(verbose=True))
