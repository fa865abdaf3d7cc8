"""Benchmark of the NSN packed-KV decode hot path on one MI355X.

Workload ("C2"): batch 16, 32 query / 8 KV heads,
head_dim 128, bf16 queries N(0,1), ragged context lengths uniform in
[16384, 32768] (numpy default_rng(2)), K and V from the outlier-token
generator (lognormal norms, 2% x20), packed as INT3 blocks of 64 tokens plus
an fp16 tail of < 64 tokens.  Synthetic data generated on the GPU
(torch.Generator seed 2); inputs are resident in HBM before timing.

A step = one fused decode-attention call for the whole batch (split kernel +
merge).  Printed: one JSON line (driver contract) with ``value`` = us/step,
the roofline of the dominant (split) kernel, encode tokens/s, the on-GPU
bridge and fp16-KV comparators, and the CPU oracle baseline.

    python bench.py [--steps 20] [--warmup 5] [--kernel fast|reference]

Profiling (the commands behind the committed summaries under profiles/):

    rocprofv3 --kernel-trace --stats --output-format csv -d OUT/kt -o kt -- python3 bench.py --profile
    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/fetch -o fetch -- python3 bench.py --profile
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/write -o write -- python3 bench.py --profile
    rocprofv3 --pmc SQ_WAVES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_INSTS_LDS SQ_INSTS_SALU SQ_INSTS_MFMA GRBM_GUI_ACTIVE --output-format csv -d OUT/sq1 -o sq1 -- python3 bench.py --profile
    rocprofv3 --pmc SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY SQ_LDS_BANK_CONFLICT SQ_ACTIVE_INST_LDS SQ_VALU_MFMA_BUSY_CYCLES SQ_INST_LEVEL_VMEM SQ_LEVEL_WAVES --output-format csv -d OUT/sq2 -o sq2 -- python3 bench.py --profile
    python3 bench.py --summarize OUT      # writes profiles/attn_fast_c2.{md,json}, profiles/encode_c2.{md,json}

``--profile`` runs one 1 GiB device-to-device copy (the counter calibration:
a plain copy kernel of known size), 10 launches of the C2 encode, and then
the C2 decode steps as the benchmark issues them (C2Decode: back to back over
three cache copies in turn): a 200-step warm-up and 100 measured steps.  The
HBM traffic per split-kernel launch is FETCH_SIZE and WRITE_SIZE (KiB per
dispatch) scaled by bytes-moved / counter-reading of that copy.  The normal
run reports it as ``roofline.traffic`` when profiles/attn_fast_c2.json was
measured on the current kernel source (sha256 of nsn_amd/csrc/nsn_fast.hip).
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
B, HQ, HKV, D = 16, 32, 8, 128
LMIN, LMAX = 16384, 32768
METRIC = "fused INT3-KV decode-attn µs/step + HBM GB/s (B=16, ctx 32K); encode tok/s"


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=1000)
    p.add_argument("--kernel", default="fast", choices=["fast", "reference"])
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    p.add_argument("--no-baselines", action="store_true", help="skip the bridge / fp16 / dense SDPA comparators")
    p.add_argument("--c2-only", action="store_true", help="default run: skip the C3 and C4 figures")
    p.add_argument("--profile", action="store_true", help="calibration copy + --steps decode steps only")
    p.add_argument("--summarize", metavar="DIR", help="turn rocprofv3 CSV output under DIR into profiles/")
    p.add_argument("--workload", default="c2", choices=["c2", "c3", "c4", "k1c", "adapter"],
                   help="c2: the headline line (default); c3 / c4: the 5-bit and streaming-cache "
                        "configurations, one line each; k1c: the K-score grid against the reference's "
                        "published cells; adapter: a transformers model decoding through the packed cache")
    p.add_argument("--k1c-model", default="Qwen3-30B-A3B", choices=["Qwen3-30B-A3B", "Gemma4-26B-A4B"])
    p.add_argument("--k1c-quick", action="store_true", help="k1c: only ctx 32768 at B = 8 and 32")
    p.add_argument("--k1c-summary", metavar="DIR",
                   help="turn a rocprofv3 --kernel-trace run of `--workload k1c --k1c-quick` under DIR "
                        "into profiles/kscore_k1c.md")
    p.add_argument("--slots", type=int, default=2, help="c4: attention slots measured (each the same work)")
    p.add_argument("--stats-summary", metavar="DIR",
                   help="c3 / c4: turn a rocprofv3 --kernel-trace --stats run of that workload under DIR "
                        "into profiles/<workload>.md")
    p.add_argument("--decode-steps", type=int, default=64, help="c4: decode steps timed (of the 256)")
    p.add_argument("--adapter-arms", default="hf_dense,graph,PACKED_KV_FUSED,NATIVE",
                   help="adapter: the runs, in order (the first packed one that ran gives the value)")
    p.add_argument("--adapter-shape", default="c4", choices=["c4", "ac08"],
                   help="adapter: c4 = B=32, 8192-token prefill in chunks of 512 (default); ac08 = the reference's "
                        "published AC08 run shape: B=1, 768-token prefill (chunks of 256), so that decode steps attend "
                        "769..1023 tokens, with --adapter-loops 8 for its 192 slots (24 layers x 8)")
    p.add_argument("--adapter-loops", type=int, default=1,
                   help="adapter: apply the 24 layers this many times (Ouro-like looped model, 24*N slots); "
                        "above 1 only the packed runs (graph, PACKED_KV_FUSED) with the packed prefill route")
    p.add_argument("--adapter-summary", metavar="DIR",
                   help="turn a rocprofv3 --kernel-trace run of `--workload adapter --adapter-arms graph` under DIR "
                        "into profiles/adapter_decode_graph.md")
    return p.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed(fn, steps, warmup, stream):
    """Average ms per call of fn() over `steps` back-to-back calls (HIP events on `stream`)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def timed_median(fn, steps, stream, reps=5):
    """Median over `reps` repetitions of timed(fn, steps, ...): the split
    kernel's launch duration for the roofline, steadier than one short run."""
    vals = sorted(timed(fn, steps, 5 if i == 0 else 2, stream) for i in range(reps))
    return vals[len(vals) // 2]


def algorithmic_bytes(lengths, bits):
    """Bytes the split kernel must move per step: packed K and V (codes + fp16
    norm/min/scale = bits*16 + 10 B per token per kv-head), fp16 tails
    (256 B/token/kv-head) and the bf16 queries.  Headers are not read."""
    per_tok = bits * 16 + 10
    kv = 0
    for L in lengths:
        C = (L // 64) * 64
        kv += HKV * 2 * (C * per_tok + (L - C) * 256)
    q = B * HQ * D * 2
    return int(kv + q)


def _cpu_model():
    """The host CPU as `lscpu` names it: model name, vendor, family / model /
    stepping, sockets x cores x threads (a VM may report a generic model
    name; the family / model numbers still identify the part)."""
    import subprocess
    info = {}
    try:
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in text.splitlines():
            if ":" in line:
                key, val = line.split(":", 1)
                info[key.strip()] = val.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    if not info.get("Model name"):
        try:
            for line in open("/proc/cpuinfo"):
                if line.startswith("model name"):
                    info["Model name"] = line.split(":", 1)[1].strip()
                    break
        except OSError:
            pass
    keys = ("Model name", "Vendor ID", "CPU family", "Model", "Stepping", "Socket(s)", "Core(s) per socket",
            "Thread(s) per core", "CPU(s)", "Hypervisor vendor")
    return "lscpu: " + "; ".join(f"{k} {info[k]}" for k in keys if info.get(k)) if info else "unknown"


def _median_time(fn, reps, warm=3):
    """Median wall time (s) of fn() over `reps` calls after `warm` untimed ones."""
    for _ in range(warm):
        fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline(kk, vv, q, lengths, sample_tokens=8192, reps=10):
    """The reference's CPU path, restated on torch's CPU backend
    (oracle/torch_cpu.py, pinned to the golden vectors), timed on this host.

    C2 step: the bridge readout of a sample -- the first `sample_tokens` tokens
    of sequence 0 (packed blocks only), 8 kv / 32 q heads: unpack3 +
    nsn_decode of K and V, then softmax(q K^T / sqrt(128)) V in fp32 -- scaled
    to the whole batch by total / sample tokens.  Also, as extra keys, C0
    (nsn_int3_qdq of K and V [32, 64, 128] fp16) and C1 (the V readout of
    4096 packed + 37 tail tokens with given fp32 logits, 32 q / 8 kv heads).
    Each figure is the median of `reps` calls after 3 warmups, with every
    thread torch may use here and with one thread.
    """
    import numpy as np
    import torch
    from nsn_amd import synthetic
    from oracle import oracle as O
    from oracle import torch_cpu as T

    nb = min(int(lengths[0]) // 64, sample_tokens // 64)
    L0 = nb * 64
    kb = tuple(t[0, :, :nb].cpu() for t in (kk.codes, kk.norm, kk.min, kk.scale))
    vb = tuple(t[0, :, :nb].cpu() for t in (vv.codes, vv.norm, vv.min, vv.scale))
    empty = torch.zeros((HKV, 0, D), dtype=torch.float16)
    qh = q[0].float().cpu()
    c2 = lambda: T.bridge_readout(qh, kb, empty, vb, empty)
    k0, v0 = (torch.from_numpy(x) for x in synthetic.config0(0))
    c0 = lambda: (T.nsn_int3_qdq(k0), T.nsn_int3_qdq(v0))
    rng = np.random.default_rng(1)
    v1 = synthetic.kv_tokens(rng, (8,), 4133)                       # C1's V: 64 blocks + 37 tail
    qv, n16, m16, s16, err = O.nsn_encode(v1[:, :4096].astype(np.float32).reshape(8, 64, 64, 128), 3)
    v1b = (torch.from_numpy(O.pack_codes(qv.reshape(8 * 64, -1), 3).reshape(8, 64, 3072)),
           torch.from_numpy(n16.view(np.float16)), torch.from_numpy(m16.view(np.float16)),
           torch.from_numpy(s16.view(np.float16)))
    v1t = torch.from_numpy(v1[:, 4096:])
    logits = torch.from_numpy((rng.standard_normal((32, 4133)) * 4).astype(np.float32))
    c1 = lambda: T.softmax_readout(logits, torch.cat((T.restore_blocks(*v1b), v1t.float()), dim=1))

    all_threads = min(os.cpu_count() or 1, int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1)))
    prev = torch.get_num_threads()
    res = {}
    for label, nt in (("all", all_threads), ("single", 1)):
        torch.set_num_threads(nt)
        res[label] = {"c2": _median_time(c2, reps), "c0": _median_time(c0, reps), "c1": _median_time(c1, reps)}
    torch.set_num_threads(prev)
    scale = float(sum(lengths)) / L0
    return dict(value=round(res["all"]["c2"] * scale * 1e6, 1), unit="µs/step", cores=all_threads, kind="port",
                single_thread=round(res["single"]["c2"] * scale * 1e6, 1), os_cpu_count=os.cpu_count(),
                cpu_model=_cpu_model(),
                sample=f"PyTorch-CPU bridge readout (oracle/torch_cpu.py: unpack3 + nsn_decode of K and V, then "
                       f"fp32 softmax(qK^T/sqrt(128))V) of sequence 0's first {L0} tokens, 8 kv / 32 q heads; median "
                       f"of {reps} after 3 warmups ({res['all']['c2'] * 1e3:.1f} ms on {all_threads} threads, "
                       f"{res['single']['c2'] * 1e3:.1f} ms on 1), scaled by total/sample tokens = {scale:.2f}",
                c0_int3_qdq_us=round(res["all"]["c0"] * 1e6, 1), c0_int3_qdq_us_single=round(res["single"]["c0"] * 1e6, 1),
                c1_readout_us=round(res["all"]["c1"] * 1e6, 1), c1_readout_us_single=round(res["single"]["c1"] * 1e6, 1))


ROTATE = 3         # copies of the packed C2 cache, used in turn by consecutive steps
BATCH = 24         # launches per timed batch of the per-kernel rounds (fixed, whatever --steps)
ROUNDS = 5         # interleaved rounds of batches
WARM_STEPS = 200   # steps before the measured launches of --profile
SETTLE_STEPS = 1000   # steps before the per-kernel rounds and the timed region (the first few hundred
                      # steps after the set-up run several us slower)


def clone_packed(kv):
    """A copy of one side of a packed cache at new addresses (every tensor cloned)."""
    import dataclasses
    import torch
    return dataclasses.replace(kv, **{f.name: getattr(kv, f.name).clone() for f in dataclasses.fields(kv)
                                      if isinstance(getattr(kv, f.name), torch.Tensor)})


class C2Decode:
    """The C2 decode step as the benchmark runs it: ROTATE copies of the packed
    cache at separate addresses (3 x 365 MB, beyond the 256 MB Infinity
    Cache), consecutive steps using them in turn, preallocated workspace and
    outputs, launches with the host checks off (the first, checked call per
    copy validates the cache) from argument blocks built once per copy
    (kernels.prepare_decode), as a serving loop would.  split() is the split
    kernel alone, merge() the merge alone, step() both over the next copy,
    step_single() both over copy 0."""

    def __init__(self, dev, lengths, k, v, q, kernel="fast"):
        import torch
        from nsn_amd import _dev, _lib, cache, kernels
        kk, self.seq = cache.pack_sequences(k, lengths, bits=3, tail_dtype=torch.float16)
        vv, _ = cache.pack_sequences(v, lengths, bits=3, tail_dtype=torch.float16)
        self.kk, self.vv, self.q, self.kernel = kk, vv, q, kernel
        self.caches = [(kk, vv)] + [(clone_packed(kk), clone_packed(vv)) for _ in range(ROTATE - 1)]
        self.max_len = max(lengths)
        split, n_splits = kernels.default_split(B, HKV, self.max_len)
        self.split_tokens = split
        self.n_splits = max(2, n_splits) if kernel == "fast" else n_splits
        self.ws = torch.empty(kernels.workspace_floats(B, HQ, self.n_splits), dtype=torch.float32, device=dev)
        self.out = torch.empty((B, HQ, D), dtype=torch.bfloat16, device=dev)
        self.ctx = torch.empty((B, HQ, D), dtype=torch.float32, device=dev)
        self.status = _dev.new_status(dev)
        self.stream = torch.cuda.current_stream()
        ref = None
        for ck, cv in self.caches:   # validated, checked calls (sync, raise on any error)
            kernels.decode_attention(q, ck, cv, self.seq, max_seq_len=self.max_len, kernel=kernel, split_tokens=split,
                                     workspace=self.ws, out=self.out, ctx=self.ctx)
            if ref is None:
                ref = self.ctx.clone()
            assert torch.equal(self.ctx, ref), "the cache copies give different outputs"
        self.turn = 0
        self._split_launch = [kernels.prepare_decode(q, ck, cv, self.seq, max_seq_len=self.max_len, kernel=kernel,
                                                     split_tokens=split, workspace=self.ws, out=self.out,
                                                     ctx=self.ctx, status=self.status, merge=False)
                              for ck, cv in self.caches]
        self._lib = _lib
        self._merge_args = (self.ws.data_ptr(), B, HQ, self.n_splits, self.ctx.data_ptr(), self.out.data_ptr(),
                            _lib.DTYPE_BF16, self.status.data_ptr())

    def split(self, rotate=True):
        launch = self._split_launch[self.turn]
        if rotate:
            self.turn = (self.turn + 1) % ROTATE
        launch()

    def merge(self):
        self._lib.check(self._lib.lib().nsn_attention_merge(*self._merge_args, self.stream.cuda_stream),
                        "nsn_attention_merge")

    def step(self):
        self.split()
        self.merge()

    def step_single(self):
        self.split(rotate=False)
        self.merge()


PROFILE_JSON = ROOT / "profiles" / "attn_fast_c2.json"
PROFILE_MD = ROOT / "profiles" / "attn_fast_c2.md"
FAST_SOURCE = ROOT / "nsn_amd" / "csrc" / "nsn_fast.hip"
CALIB_BYTES = 1 << 30
SPLIT_KERNEL = "nsn::fast::attn_fast_kernel<3, 1, false, 4, false>"
MERGE_KERNEL = "nsn::attn_merge_kernel<1>"
CALIB_KERNEL = "__amd_rocclr_copyBuffer"
PROFILE_STEPS = 100   # decode steps of `--profile` (the first launch runs cold)
ENCODE_KERNEL = "nsn::encode_kernel<0, 3, 0>"
ENCODE_PROFILE_STEPS = 10   # C2 encode launches of `--profile`, before the cache is packed
ENCODE_JSON = ROOT / "profiles" / "encode_c2.json"
ENCODE_MD = ROOT / "profiles" / "encode_c2.md"
CODEC_SOURCE = ROOT / "nsn_amd" / "csrc" / "nsn_codec.hip"


def source_sha():
    return hashlib.sha256(FAST_SOURCE.read_bytes()).hexdigest()


def _rows(path_glob):
    files = sorted(Path(path_glob[0]).glob(path_glob[1]))
    if not files:
        raise SystemExit(f"no {path_glob[1]} under {path_glob[0]}")
    with open(files[0], newline="") as f:
        return list(csv.DictReader(f))


def _counter(dirname, counter):
    """Per-dispatch readings (KiB) of one counter for the split kernel, the
    merge kernel, the calibration copy (the first copy dispatch with a grid
    of 64K threads or more; the later ones copy the packed cache) and
    the C2 encode launches (the first ENCODE_PROFILE_STEPS encoder dispatches:
    `--profile` runs them before it packs the cache with the same kernel)."""
    out = {"split": [], "merge": [], "calib": [], "encode": []}
    enc, calib = [], []
    for r in _rows((dirname, "**/*counter_collection.csv")):
        if r["Counter_Name"] != counter:
            continue
        name, val = r["Kernel_Name"], float(r["Counter_Value"])
        if SPLIT_KERNEL in name:
            out["split"].append(val)
        elif MERGE_KERNEL in name:
            out["merge"].append(val)
        elif ENCODE_KERNEL in name:
            enc.append((int(r["Dispatch_Id"]), val))
        elif name.startswith(CALIB_KERNEL) and int(r["Grid_Size"]) >= 65536:
            calib.append((int(r["Dispatch_Id"]), val))
    out["encode"] = [v for _, v in sorted(enc)[:ENCODE_PROFILE_STEPS]]
    out["calib"] = [min(calib)[1]] if calib else []   # the run's first large copy (the later ones copy the cache)
    return out


SQ_NOTES = {
    "SQ_WAVES": "waves",
    "SQ_INSTS_VALU": "VALU instructions (MFMA included)",
    "SQ_INSTS_MFMA": "MFMA instructions",
    "SQ_INSTS_SALU": "SALU instructions",
    "SQ_INSTS_LDS": "LDS instructions",
    "SQ_WAVE_CYCLES": "wave-lifetime quad-cycles (sum over waves)",
    "SQ_ACTIVE_INST_VALU": "VALU-issue quad-cycles (sum over waves)",
    "SQ_ACTIVE_INST_ANY": "any-issue quad-cycles (sum over waves)",
    "SQ_WAIT_ANY": "quad-cycles waves wait on anything (counters, dependencies)",
    "SQ_WAIT_INST_ANY": "quad-cycles waves wait for an instruction dependency",
    "SQ_ACTIVE_INST_LDS": "LDS-issue quad-cycles",
    "SQ_LDS_BANK_CONFLICT": "LDS bank-conflict cycles (sum over CUs)",
    "SQ_VALU_MFMA_BUSY_CYCLES": "MFMA-busy cycles (sum over SIMDs)",
    "SQ_BUSY_CYCLES": "SQ-busy cycles (sum over SEs)",
    "GRBM_GUI_ACTIVE": "GPU-active cycles (sum over the 8 XCDs)",
}


def _sq(d, kernel, first=None, last=None):
    """Per-dispatch SQ/GRBM counter readings of one kernel from the sq1/sq2
    passes (median over its dispatches; `first` / `last` keep only the first
    or the last ones)."""
    vals = {}
    for sub in ("sq1", "sq2"):
        if not (Path(d) / sub).exists():
            return {}
        per = {}
        for r in _rows((Path(d) / sub, "**/*counter_collection.csv")):
            if kernel in r["Kernel_Name"]:
                per.setdefault(r["Counter_Name"], []).append((int(r["Dispatch_Id"]), float(r["Counter_Value"])))
        for c, v in per.items():
            v = sorted(v)
            v = v[:first] if first else (v[-last:] if last else v)
            xs = sorted(x for _, x in v)
            vals[c] = xs[len(xs) // 2]
    return vals


def _sq_lines(sq, blocks_per_wave=None):
    """Markdown rows of the counters and the ratios quoted in the notes."""
    if not sq:
        return []
    L = ["| counter | median per dispatch | meaning |", "|---|---|---|"]
    for c in SQ_NOTES:
        if c in sq:
            L.append(f"| {c} | {sq[c]:.4g} | {SQ_NOTES[c]} |")
    w = sq.get("SQ_WAVES", 0)
    if w:
        L += ["", "Derived (per wave; quad-cycles x 4 = cycles):", ""]
        valu = sq["SQ_INSTS_VALU"] - sq.get("SQ_INSTS_MFMA", 0)
        L.append(f"- VALU (without MFMA) {valu / w:.0f}, MFMA {sq.get('SQ_INSTS_MFMA', 0) / w:.0f}, "
                 f"SALU {sq['SQ_INSTS_SALU'] / w:.0f}, LDS {sq['SQ_INSTS_LDS'] / w:.0f} instructions per wave"
                 + (f" ({valu / w / blocks_per_wave:.0f} / {sq.get('SQ_INSTS_MFMA', 0) / w / blocks_per_wave:.0f} / "
                    f"{sq['SQ_INSTS_SALU'] / w / blocks_per_wave:.0f} / {sq['SQ_INSTS_LDS'] / w / blocks_per_wave:.0f} "
                    f"per 64-token block)" if blocks_per_wave else "") + ";")
        L.append(f"- wave lifetime {4 * sq['SQ_WAVE_CYCLES'] / w:.0f} cycles; of it VALU issue "
                 f"{sq['SQ_ACTIVE_INST_VALU'] / sq['SQ_WAVE_CYCLES']:.1%}, any issue "
                 f"{sq['SQ_ACTIVE_INST_ANY'] / sq['SQ_WAVE_CYCLES']:.1%}, waiting "
                 f"{sq['SQ_WAIT_ANY'] / sq['SQ_WAVE_CYCLES']:.1%};")
        if "GRBM_GUI_ACTIVE" in sq:
            gui = sq["GRBM_GUI_ACTIVE"] / 8   # cycles of the dispatch (per XCD)
            L.append(f"- GPU-active cycles per XCD {gui:.0f}"
                     + (f"; MFMA busy {sq['SQ_VALU_MFMA_BUSY_CYCLES'] / (gui * 1024):.1%} of the 1024 SIMDs' cycles"
                        if "SQ_VALU_MFMA_BUSY_CYCLES" in sq else "")
                     + (f"; LDS bank-conflict cycles {sq['SQ_LDS_BANK_CONFLICT'] / (gui * 256):.1%} of the 256 CUs' "
                        "cycles" if "SQ_LDS_BANK_CONFLICT" in sq else "") + ".")
    return L


def split_resource_lines():
    """The split kernel's registers, spills, scratch, LDS and occupancy as
    the compiler reports them for the current source (the build's flags)."""
    from nsn_amd import build
    ks = build.resource_usage("nsn_fast.hip")
    name = next((n for n in ks if "attn_fast_kernelILi3ELi1ELb0ELi4ELb0E" in n), None)
    if name is None:
        return []
    r = ks[name]
    return ["## Compiler resources of the split kernel (`python -m nsn_amd.build --resource-usage`)", "",
            "| VGPR | AGPR | SGPR | SGPR spill | VGPR spill | scratch B/lane | LDS B/workgroup | waves/SIMD |",
            "|---|---|---|---|---|---|---|---|",
            "| " + " | ".join(str(r.get(k, "?")) for k in ("vgpr", "agpr", "sgpr", "sgpr_spill", "vgpr_spill",
                                                        "scratch", "lds", "occupancy")) + " |", "",
            "Where the spills sit (outside the packed-block loop but for 6 SGPR reloads per two blocks): "
            "profiles/resource_usage.md.", ""]


def summarize(d):
    """Write profiles/attn_fast_c2.{md,json} from rocprofv3 CSV output under d
    (subdirectories kt/, fetch/, write/ made by the commands in the module docstring)."""
    d = Path(d)
    stats = _rows((d / "kt", "**/*kernel_stats.csv"))
    fetch = _counter(d / "fetch", "FETCH_SIZE")
    write = _counter(d / "write", "WRITE_SIZE")
    for nm, c in (("FETCH_SIZE", fetch), ("WRITE_SIZE", write)):
        if not (c["split"] and c["calib"]):
            raise SystemExit(f"{nm}: split kernel or calibration copy missing")
    mean = lambda xs: sum(xs) / len(xs)
    f_scale = CALIB_BYTES / (mean(fetch["calib"]) * 1024)   # bytes moved per counted byte, reads
    w_scale = CALIB_BYTES / (mean(write["calib"]) * 1024)   # the same for writes
    split_read = mean(fetch["split"]) * 1024 * f_scale
    split_write = mean(write["split"]) * 1024 * w_scale
    lens = [int(x) for x in __import__("nsn_amd.synthetic", fromlist=["x"]).ragged_lengths(2, B, LMIN, LMAX)]
    alg = algorithmic_bytes(lens, 3)
    top = sorted(stats, key=lambda r: -float(r["TotalDurationNs"]))[:8]
    top += [r for r in stats if (SPLIT_KERNEL in r["Name"] or MERGE_KERNEL in r["Name"]) and r not in top]
    all_avg = next(float(r["AverageNs"]) for r in stats if SPLIT_KERNEL in r["Name"]) / 1e3
    # the measured launches: the last PROFILE_STEPS, after the WARM_STEPS warm-up the benchmark also runs
    seq = [dur for _, dur in sorted((int(r["Start_Timestamp"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
                                    for r in _rows((d / "kt", "**/*kernel_trace.csv")) if SPLIT_KERNEL in r["Kernel_Name"])]
    last = seq[-PROFILE_STEPS:]
    split_avg = sum(last) / len(last)
    durs = sorted(last)
    split_med = durs[len(durs) // 2]
    fig = {"kernel": SPLIT_KERNEL, "source_sha256": source_sha(), "workload": "C2",
           "split_avg_us": round(split_avg, 2), "split_median_us": round(split_med, 2),
           "split_avg_us_all_launches": round(all_avg, 2), "launches": len(seq), "measured_launches": len(last),
           "fetch_kib": round(mean(fetch["split"]), 1),
           "write_kib": round(mean(write["split"]), 1), "fetch_scale": round(f_scale, 4),
           "write_scale": round(w_scale, 4), "read_bytes": int(split_read), "write_bytes": int(split_write),
           "traffic": int(split_read + split_write), "algorithmic_bytes": alg}
    PROFILE_JSON.write_text(json.dumps(fig, indent=1) + "\n")
    L = ["# attn_fast_kernel on C2 (B=16, 32q/8kv, ctx U[16K,32K], INT3 + fp16 tail)", "",
         "Commands (run from the repository root on one MI355X, `OUT` = an output folder):", "", "```"]
    L += [ln.strip() for ln in __doc__.split("Profiling")[1].split("``--profile``")[0].strip().splitlines()[1:] if ln.strip()]
    L += ["```", "", "`python3 bench.py --profile`: one 1 GiB copy (calibration), then "
          "decode steps over the C2 cache (split kernel + merge per step).", "",
          "## Kernel trace (rocprofv3 --kernel-trace --stats)", "",
          "Top kernels by total time (the set-up kernels generate and pack the synthetic cache), "
          "then the split and merge kernels of the decode step.", "",
          "| kernel | calls | avg us | min us | max us |", "|---|---|---|---|---|"]
    for r in top:
        L.append(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                 f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} |")
    L += ["", "## HBM traffic per dispatch (rocprofv3 --pmc, one counter per pass)", "",
          "| dispatch | FETCH_SIZE KiB | WRITE_SIZE KiB |", "|---|---|---|",
          f"| calibration copy, {CALIB_BYTES >> 20} MiB read + written | {mean(fetch['calib']):.0f} | {mean(write['calib']):.0f} |",
          f"| split kernel (mean of {len(fetch['split'])}) | {mean(fetch['split']):.0f} | {mean(write['split']):.0f} |"]
    if fetch["merge"]:
        L.append(f"| merge kernel | {mean(fetch['merge']):.0f} | {mean(write['merge']):.0f} |")
    L += ["", f"Scale factors from the copy (bytes moved per counted byte): reads x{f_scale:.3f}, "
          f"writes x{w_scale:.3f}.", "",
          f"Split kernel: {split_read / 1e6:.1f} MB read + {split_write / 1e6:.1f} MB written = "
          f"**{fig['traffic'] / 1e6:.1f} MB** per launch, against {alg / 1e6:.1f} MB algorithmic "
          f"(ratio {fig['traffic'] / alg:.3f}).", "",
          f"Duration under the profiler, over the last {len(last)} of the {len(seq)} split launches (the "
          f"{len(seq) - len(last)} before them are the warm-up the benchmark also runs, {WARM_STEPS} steps, plus "
          f"the checked calls): mean **{split_avg:.1f} us** -> {alg / split_avg / 1e3:.0f} GB/s algorithmic = "
          f"{alg / split_avg / 1e3 / HBM_PEAK_GBS:.1%} of 8 TB/s; median {split_med:.1f} us; min {durs[0]:.1f} us, "
          f"max {durs[-1]:.1f} us.  Over all {len(seq)} launches the mean is {all_avg:.1f} us: during the "
          "warm-up the engine clock dips for a stretch of launches before it settles.", "",
          f"Kernel source sha256: `{fig['source_sha256']}`", ""]
    sq = _sq(d, SPLIT_KERNEL)
    if sq:
        L += ["## SQ counters (rocprofv3 --pmc, the sq1 and sq2 passes above)", ""]
        L += _sq_lines(sq, blocks_per_wave=sum((x + 63) // 64 for x in lens) * HKV / sq["SQ_WAVES"])
        L += ["", f"With 2 waves per SIMD the SIMD's VALU port is busy about twice the per-wave VALU-issue "
              f"share while the waves live; the mean wave lifetime is {4 * sq['SQ_WAVE_CYCLES'] / sq['SQ_WAVES'] / (sq['GRBM_GUI_ACTIVE'] / 8) :.0%} of the "
              f"dispatch's GPU-active cycles (the dispatch ramp and the end-of-kernel imbalance; the same share "
              f"in every profile of this kernel so far).", ""]
    L += split_resource_lines()
    PROFILE_MD.write_text("\n".join(L))
    print("\n".join(L))
    if fetch["encode"] and write["encode"]:
        summarize_encode(d, fetch, write, f_scale, w_scale)
    elif fetch["encode"] or write["encode"]:
        raise SystemExit("encode counters incomplete")


def summarize_encode(d, fetch, write, f_scale, w_scale):
    """profiles/encode_c2.{md,json}: the C2 encode launches of the same runs."""
    mean = lambda xs: sum(xs) / len(xs)
    trace = sorted(((int(r["Start_Timestamp"]), int(r["End_Timestamp"]))
                    for r in _rows((d / "kt", "**/*kernel_trace.csv")) if ENCODE_KERNEL in r["Kernel_Name"]))
    seq = [(e - b) / 1e3 for b, e in trace[:ENCODE_PROFILE_STEPS]]
    durs = sorted(seq)
    med = durs[len(durs) // 2]
    avg = sum(durs) / len(durs)
    tokens = B * HKV * LMAX
    alg = tokens * 314
    rd = mean(fetch["encode"]) * 1024 * f_scale
    wr = mean(write["encode"]) * 1024 * w_scale
    fig = {"kernel": ENCODE_KERNEL, "source_sha256": hashlib.sha256(CODEC_SOURCE.read_bytes()).hexdigest(),
           "workload": "C2 K, 128 rows x 512 blocks, fp16 in, 3-bit codes + fp16 metadata + fp32 decode factors out",
           "token_heads": tokens, "median_us": round(med, 2), "mean_us": round(avg, 2), "min_us": round(durs[0], 2),
           "read_bytes": int(rd), "write_bytes": int(wr), "traffic": int(rd + wr), "algorithmic_bytes": alg}
    ENCODE_JSON.write_text(json.dumps(fig, indent=1) + "\n")
    L = ["# encode_kernel on C2 (all 64-token blocks of K: 128 rows x 512 blocks, fp16 -> INT3)", "",
         "Same rocprofv3 runs as profiles/attn_fast_c2.md (commands there): `bench.py --profile` runs "
         f"{ENCODE_PROFILE_STEPS} encode launches of the C2 bench's encode (codes, fp16 metadata and the "
         "fp32 decode factors; no headers) right after the calibration copy, before it packs the decode "
         "cache.", "",
         "| item | value |", "|---|---|",
         f"| launches | {len(durs)} |",
         f"| duration, median / mean / min | {med:.1f} / {avg:.1f} / {durs[0]:.1f} us |",
         f"| durations in launch order | {', '.join(f'{x:.0f}' for x in seq)} us |",
         f"| token-heads per launch | {tokens} |",
         f"| algorithmic bytes (256 in + 58 out per token-head; the 4-byte factors are not counted) | {alg / 1e6:.1f} MB |",
         f"| FETCH_SIZE / WRITE_SIZE per launch | {mean(fetch['encode']):.0f} / {mean(write['encode']):.0f} KiB |",
         f"| HBM traffic (scaled by the calibration copy) | {rd / 1e6:.1f} MB read + {wr / 1e6:.1f} MB written = "
         f"**{(rd + wr) / 1e6:.1f} MB** (ratio {(rd + wr) / alg:.3f} to algorithmic) |",
         f"| rate | {tokens / med / 1e3:.2f} G token-heads/s = {alg / med / 1e3:.0f} GB/s algorithmic "
         f"({alg / med / 1e3 / HBM_PEAK_GBS * 100:.1f} % of 8 TB/s) at the median; "
         f"{alg / avg / 1e3:.0f} GB/s at the mean |", "",
         "Back-to-back launches lengthen as the engine clock drops under the sustained load "
         "(durations in launch order above).", "",
         f"Kernel source sha256 (nsn_amd/csrc/nsn_codec.hip): `{fig['source_sha256']}`", ""]
    sq = _sq(d, ENCODE_KERNEL, first=ENCODE_PROFILE_STEPS)
    if sq:
        L += ["## SQ counters (the first launches of the sq1 and sq2 passes)", ""] + _sq_lines(sq) + [""]
    ENCODE_MD.write_text("\n".join(L))
    print("\n".join(L))


def measured_traffic():
    """HBM bytes per split-kernel launch from the committed profile, if it was
    measured on this kernel source; else None."""
    try:
        fig = json.loads(PROFILE_JSON.read_text())
    except (OSError, ValueError):
        return None
    return fig["traffic"] if fig.get("source_sha256") == source_sha() else None


def measured_encode_traffic():
    """HBM bytes per C2 encode launch from the committed profile, if it was
    measured on this codec source; else None."""
    try:
        fig = json.loads(ENCODE_JSON.read_text())
    except (OSError, ValueError):
        return None
    ok = fig.get("source_sha256") == hashlib.sha256(CODEC_SOURCE.read_bytes()).hexdigest()
    return fig["traffic"] if ok else None


def make_workload(dev):
    from nsn_amd import synthetic
    log(f"[bench] generating C2 K/V on the GPU: B={B} Hkv={HKV} Lmax={LMAX}")
    return synthetic.c2_workload(dev)


def c2_encoder(dev, k):
    """The C2 encode: every 64-token block of K (B*Hkv rows x 512 blocks, fp16)
    to 3-bit codes, fp16 metadata and the fp32 decode factors the fast decode
    reads, in one launch (headers off).  Returns the launch closure and its
    buffers (status last)."""
    import torch
    from nsn_amd import _dev, _lib
    nblk = LMAX // 64
    codes = torch.empty((B * HKV, nblk, 3072), dtype=torch.uint8, device=dev)
    nrm = torch.empty((B * HKV, nblk, 64), dtype=torch.float16, device=dev)
    mn = torch.empty((B * HKV, nblk, 128), dtype=torch.float16, device=dev)
    sc = torch.empty((B * HKV, nblk, 128), dtype=torch.float16, device=dev)
    fac = torch.empty((B * HKV, nblk, 64), dtype=torch.float32, device=dev)
    st = _dev.new_status(dev)
    lib = _lib.lib()
    stream = torch.cuda.current_stream()

    def encode_all():
        rc = lib.nsn_encode_blocks(k.data_ptr(), _lib.DTYPE_F16, B * HKV, nblk, LMAX * D, 0, 3, _lib.NORM_LANES8, 1,
                                   codes.data_ptr(), nrm.data_ptr(), mn.data_ptr(), sc.data_ptr(), None, fac.data_ptr(),
                                   nblk, 0, 0, None, st.data_ptr(), stream.cuda_stream)
        assert rc == 0
    return encode_all, (codes, nrm, mn, sc, fac, st)


def profile_run(args):
    """Calibration copy, the C2 encode launches, then WARM_STEPS + `steps`
    decode steps of the C2 workload, issued as the benchmark's timed batches
    issue them (C2Decode.step: back to back, the cache copies in turn)."""
    import torch
    dev = torch.device("cuda:0")
    lengths, k, v, q = make_workload(dev)
    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    encode_all, enc_bufs = c2_encoder(dev, k)
    for _ in range(ENCODE_PROFILE_STEPS):
        encode_all()
    torch.cuda.synchronize()
    del encode_all, enc_bufs
    dec = C2Decode(dev, lengths, k, v, q, kernel=args.kernel)
    del k, v
    steps = max(args.steps, PROFILE_STEPS)
    for _ in range(WARM_STEPS + steps):   # as the timed steps: back to back, the copies in turn, no host sync
        dec.step()
    torch.cuda.synchronize()
    log(f"[bench] profile run done: {WARM_STEPS} + {steps} steps over {ROTATE} cache copies")


def _arm_timing(fn, calls):
    """loop_kv_vf01.py:105-117's timing of one arm: HIP events around `calls`
    back-to-back calls (each allocates its own outputs and runs its host checks,
    status reads included); extra device memory = allocated peak during the
    calls - allocated before them.  Returns (ms per call, extra bytes)."""
    import torch
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    out = None
    for _ in range(calls):
        if out is not None:
            del out
        out = fn()
    b.record()
    b.synchronize()
    peak = torch.cuda.max_memory_allocated()
    del out
    return a.elapsed_time(b) / calls, peak - before


def _paired(times, rounds, arms, num, den):
    """Median over rounds of the per-round ratio num / den of per-call times."""
    r = sorted(times[num][i] / times[den][i] for i in range(rounds))
    return r[len(r) // 2]


def readout_arms(dev, rounds=5, calls=20, warm=20):
    """GPU timings of the reference's two published readout comparisons.

    c1: the score-input V readout of one decode
    query (AF01 FULL=False, experiments/ac08/source/loop_kv_af01_kernel.py:52-54),
    B=1, 32 q / 8 kv heads, 4096 packed + 37 fp16 tail tokens, logits
    N(0,1)*4, V from the config-0 generator (numpy rng 1): FUSED = the fast
    kernel reading packed V; BRIDGE = V restored to HBM
    (loop_kv_vf01_kernel.py:120-126) then the same kernel over dense V.
    Kernel level: batches of back-to-back launches into preallocated buffers
    (HIP events); call level: each call allocating its outputs and checking
    its status, as below.

    vf01: the shape of the reference's only published timings
    (reports/vf01-results-v0.1-2026-10-02.md:27-35,68-69), B=1, 16 MHA heads,
    896 packed + 127 bf16 tail tokens, packed K and V, through
    kernels.pipeline's three arms on the fast kernel: V_FUSED, TILE_MATERIALIZE
    (bridge) and RF01_MATERIALIZE.  Timed as loop_kv_vf01.py:105-117 times
    them (_arm_timing, `calls` calls), `rounds` rounds with the arms
    interleaved after `warm` warm-up calls each; per-arm medians, the median
    of the per-round paired ratios, and the extra device memory per call.
    """
    import numpy as np
    import torch
    from nsn_amd import _dev, _lib, cache, codec, kernels, synthetic
    stream = torch.cuda.current_stream()
    res = {}

    # ---- c1
    rng = np.random.default_rng(1)
    T1 = 4096 + 37
    v1 = synthetic.kv_tokens(rng, (1, 8), T1)
    sc1 = torch.from_numpy((rng.standard_normal((1, 32, T1)) * 4).astype(np.float32)).to(dev)
    vv, seq = cache.pack_sequences(torch.from_numpy(v1).to(dev), [T1])
    q1 = torch.zeros(1, 32, 128, dtype=torch.bfloat16, device=dev)
    vden = torch.empty((1, 8, T1, 128), dtype=torch.float16, device=dev)
    vd = kernels.PackedKV(None, None, None, None, None, None, vden, 3)
    split, n_splits = kernels.default_split(1, 8, T1)
    n_splits = max(2, n_splits)
    ws = torch.empty(kernels.workspace_floats(1, 32, n_splits), dtype=torch.float32, device=dev)
    out1 = torch.empty((1, 32, 128), dtype=torch.bfloat16, device=dev)
    ctx1 = torch.empty((1, 32, 128), dtype=torch.float32, device=dev)
    st = _dev.new_status(dev)
    lib = _lib.lib()
    nb1 = T1 // 64

    def restore1():
        rc = lib.nsn_restore_blocks(vv.codes.data_ptr(), 0, vv.norm.data_ptr(), vv.min.data_ptr(),
                                    vv.scale.data_ptr(), 8, nb1, vv.codes.shape[2], 3, vden.data_ptr(),
                                    _lib.DTYPE_F16, T1, vv.tail.data_ptr(), _lib.DTYPE_F16, T1 - nb1 * 64,
                                    vv.tail.shape[2], st.data_ptr(), stream.cuda_stream)
        assert rc == 0

    def readout(vside):
        kernels.decode_attention(q1, None, vside, seq, max_seq_len=T1, scores=sc1, kernel="fast",
                                 split_tokens=split, workspace=ws, out=out1, ctx=ctx1, status=st, check=False)

    def fused_k():
        readout(vv)

    def bridge_k():
        restore1()
        readout(vd)

    def fused_call():
        return kernels.decode_attention(q1, None, vv, seq, max_seq_len=T1, scores=sc1, kernel="fast")[0]

    def bridge_call():
        v = codec.restore(vv.codes[0], (vv.norm[0], vv.min[0], vv.scale[0]), 3, torch.float16,
                          tail=vv.tail[0, :, :T1 - nb1 * 64])
        side = kernels.PackedKV(None, None, None, None, None, None, v[None], 3)
        return kernels.decode_attention(q1, None, side, seq, max_seq_len=T1, scores=sc1, kernel="fast")[0]
    bridge_k()
    torch.cuda.synchronize()
    fused_out = fused_call().clone()
    assert torch.allclose(fused_out.float(), bridge_call().float(), atol=2e-3, rtol=1e-2)
    kt = {"fused": [], "bridge": []}
    ct = {"fused": [], "bridge": []}
    mem = {}
    for _ in range(warm):
        fused_k(), bridge_k(), fused_call(), bridge_call()
    for _ in range(rounds):
        kt["fused"].append(timed(fused_k, 50, 0, stream))
        kt["bridge"].append(timed(bridge_k, 50, 0, stream))
        for arm, fn in (("fused", fused_call), ("bridge", bridge_call)):
            ms, extra = _arm_timing(fn, calls)
            ct[arm].append(ms)
            mem[arm] = max(mem.get(arm, 0), extra)
    assert _dev.read_status(st) == 0
    med = lambda xs: sorted(xs)[len(xs) // 2]
    res["c1"] = {
        "workload": "C1: score-input V readout, B=1, 32q/8kv, d=128, 4096 packed INT3 + 37 fp16 tail, logits N(0,1)*4",
        "fused_kernel_us": round(med(kt["fused"]) * 1e3, 2), "bridge_kernel_us": round(med(kt["bridge"]) * 1e3, 2),
        "kernel_ratio_fused_over_bridge": round(_paired(kt, rounds, None, "fused", "bridge"), 4),
        "fused_call_us": round(med(ct["fused"]) * 1e3, 2), "bridge_call_us": round(med(ct["bridge"]) * 1e3, 2),
        "call_ratio_fused_over_bridge": round(_paired(ct, rounds, None, "fused", "bridge"), 4),
        "extra_device_bytes_per_call": mem,
        "timing": f"kernel: median of {rounds} rounds of 50 back-to-back launches into preallocated buffers; call: "
                  f"median of {rounds} rounds of {calls} calls allocating their outputs, status read each call",
    }
    log(f"[bench] C1 readout: fused {res['c1']['fused_kernel_us']} us, bridge {res['c1']['bridge_kernel_us']} us "
        f"(kernel level); per call {res['c1']['fused_call_us']} / {res['c1']['bridge_call_us']} us; "
        f"extra memory {mem}")
    del vv, vden, ws

    # ---- vf01
    rng = np.random.default_rng(5)
    H, NP, NT = 16, 896, 127
    kx = synthetic.kv_tokens(rng, (1, H), NP + NT)
    vx = synthetic.kv_tokens(rng, (1, H), NP + NT)

    def group(x):
        blocks = torch.from_numpy(x[:, :, :NP]).to(dev).reshape(1, H, NP // 64, 64, 128)
        return codec.encode_group(blocks, 0)
    g, vg = group(kx), group(vx)
    kt_ = torch.from_numpy(kx[:, :, NP:]).to(dev).to(torch.bfloat16).contiguous()
    vt_ = torch.from_numpy(vx[:, :, NP:]).to(dev).to(torch.bfloat16).contiguous()
    qv = torch.from_numpy(rng.standard_normal((1, H, 1, 128)).astype(np.float32)).to(dev).to(torch.bfloat16)
    data = (g, kt_, qv, vg, vt_)
    arms = ("V_FUSED", "TILE_MATERIALIZE", "RF01_MATERIALIZE")
    outs = [kernels.pipeline(arm, data, kernel="fast").float() for arm in arms]
    for o in outs[1:]:
        assert torch.allclose(o, outs[0], atol=2e-3, rtol=1e-2)
    for arm in arms:
        for _ in range(warm):
            kernels.pipeline(arm, data, kernel="fast")
    vt = {arm: [] for arm in arms}
    vmem = {}
    for _ in range(rounds):
        for arm in arms:
            ms, extra = _arm_timing(lambda: kernels.pipeline(arm, data, kernel="fast"), calls)
            vt[arm].append(ms)
            vmem[arm] = max(vmem.get(arm, 0), extra)
    res["vf01"] = {
        "workload": "VF01 published shape: B=1, 16 MHA heads, d=128, 896 packed INT3 + 127 bf16 tail tokens, "
                    "packed K and V, one decode query; kernels.pipeline arms on the fast kernel",
        "ms_per_call": {arm: round(med(vt[arm]), 6) for arm in arms},
        "paired_ratio_fused_over_bridge": round(_paired(vt, rounds, None, "V_FUSED", "TILE_MATERIALIZE"), 4),
        "paired_ratio_fused_over_rf01": round(_paired(vt, rounds, None, "V_FUSED", "RF01_MATERIALIZE"), 4),
        "extra_device_bytes_per_call": vmem,
        "reference_published_rtx_pro_6000": {"ms_per_call": {"V_FUSED": 0.174514, "TILE_MATERIALIZE": 0.243244,
                                                             "RF01_MATERIALIZE": 0.299447},
                                             "paired_ratio_fused_over_bridge": 0.717196,
                                             "paired_ratio_fused_over_rf01": 0.582795,
                                             "extra_device_bytes_per_call": {"V_FUSED": 551424,
                                                                             "TILE_MATERIALIZE": 14665728,
                                                                             "RF01_MATERIALIZE": 21028864},
                                             "source": "reports/vf01-results-v0.1-2026-10-02.md:27-35,68-69 "
                                                       "(context only: other hardware and host stack)"},
        "timing": f"loop_kv_vf01.py:105-117 protocol: {rounds} rounds, arms interleaved, {calls} checked calls "
                  f"per arm and round between HIP events after {warm} warm-up calls; medians",
    }
    log(f"[bench] VF01 shape, ms per call {res['vf01']['ms_per_call']}, fused/bridge "
        f"{res['vf01']['paired_ratio_fused_over_bridge']}, fused/RF01 {res['vf01']['paired_ratio_fused_over_rf01']}, "
        f"extra memory {vmem}")
    return res


C3 = dict(B=64, HQ=16, HKV=4, L=8192, bits=5)


def interleaved_rounds(step, split, merge, stream, rounds=ROUNDS, batch=BATCH, settle=SETTLE_STEPS):
    """Mean per-launch ms of a decode step, its split kernel alone and its
    merge alone, as C2's rounds measure them: after `settle` untimed steps,
    `rounds` rounds of back-to-back batches of `batch` launches of each kind,
    enqueued without a host synchronisation, with a HIP event between
    consecutive batches on the launch stream (so that all three run at one
    clock, and the figures do not depend on --steps).  Also returns the
    per-round split times (sorted) and the batch size."""
    import torch
    for _ in range(settle):
        step()
    kinds = (("step", step), ("split", split), ("merge", merge))
    marks = []
    for _ in range(rounds):
        for name, fn in kinds:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(stream)
            marks.append((name, ev))
            for _ in range(batch):
                fn()
    end = torch.cuda.Event(enable_timing=True)
    end.record(stream)
    torch.cuda.synchronize()
    per = {name: [] for name, _ in kinds}
    for i, (name, ev) in enumerate(marks):
        nxt = marks[i + 1][1] if i + 1 < len(marks) else end
        per[name].append(ev.elapsed_time(nxt) / batch)
    mean = lambda xs: sum(xs) / len(xs)
    return mean(per["step"]), mean(per["split"]), mean(per["merge"]), sorted(per["split"]), batch


def main_c3(args, emit=True):
    """C3: 5-bit codes, B=64, 16q/4kv heads, every
    sequence 8192 tokens (128 packed blocks, no tail), K and V heavy-tailed
    (per-channel Student-t df=3 x lognormal token norms; GPU generator seed 3).
    Measures the encode of every block of K and V (one launch over both) and
    one fused decode step; prints one JSON line of its own."""
    import torch
    from nsn_amd import _dev, _lib, cache, kernels, synthetic

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    b_, hq, hkv, L, bits = C3["B"], C3["HQ"], C3["HKV"], C3["L"], C3["bits"]
    log(f"[bench] generating C3 K/V on the GPU: B={b_} Hkv={hkv} L={L}, {bits}-bit")
    kv, q = synthetic.c3_workload(dev)     # [K | V]

    # ---- encode: all 64-token blocks of K and V, one launch
    rows, nblk = 2 * b_ * hkv, L // 64
    nb_bytes = 64 * D * bits // 8
    codes = torch.empty((rows, nblk, nb_bytes), dtype=torch.uint8, device=dev)
    nrm = torch.empty((rows, nblk, 64), dtype=torch.float16, device=dev)
    mn = torch.empty((rows, nblk, 128), dtype=torch.float16, device=dev)
    sc = torch.empty((rows, nblk, 128), dtype=torch.float16, device=dev)
    st = _dev.new_status(dev)
    lib = _lib.lib()

    def encode_all():
        rc = lib.nsn_encode_blocks(kv.data_ptr(), _lib.DTYPE_F16, rows, nblk, L * D, 0, bits, _lib.NORM_LANES8, 1,
                                   codes.data_ptr(), nrm.data_ptr(), mn.data_ptr(), sc.data_ptr(), None, None, nblk, 0, 0,
                                   None, st.data_ptr(), stream.cuda_stream)
        assert rc == 0
    enc_ms = timed(encode_all, 10, 2, stream)
    assert _dev.read_status(st) == 0
    per_tok = 256 + bits * 16 + 10
    enc_tokens = rows * L
    enc_gbs = enc_tokens * per_tok / (enc_ms * 1e-3) / 1e9
    log(f"[bench] C3 encode: {enc_ms * 1e3:.1f} us per launch ({enc_tokens} token-heads), "
        f"{enc_tokens / (enc_ms * 1e-3) / 1e9:.2f} G tok/s, {enc_gbs:.0f} GB/s algorithmic ({per_tok} B/token)")
    del codes, nrm, mn, sc

    # ---- one decode step over the packed cache
    lengths = [L] * b_
    kk, seq = cache.pack_sequences(kv[0], lengths, bits=bits, tail_dtype=torch.float16)
    vv, _ = cache.pack_sequences(kv[1], lengths, bits=bits, tail_dtype=torch.float16)
    del kv
    split, n_splits = kernels.default_split(b_, hkv, L)
    n_splits = max(2, n_splits)
    ws = torch.empty(kernels.workspace_floats(b_, hq, n_splits), dtype=torch.float32, device=dev)
    out = torch.empty((b_, hq, D), dtype=torch.bfloat16, device=dev)
    ctx = torch.empty((b_, hq, D), dtype=torch.float32, device=dev)
    status = _dev.new_status(dev)
    kernels.decode_attention(q, kk, vv, seq, max_seq_len=L, kernel=args.kernel, split_tokens=split,
                             workspace=ws, out=out, ctx=ctx)

    # launches from argument blocks built once (kernels.prepare_decode), as in C2
    launches = {m: kernels.prepare_decode(q, kk, vv, seq, max_seq_len=L, kernel=args.kernel, split_tokens=split,
                                          workspace=ws, out=out, ctx=ctx, status=status, merge=m)
                for m in (True, False)}

    def step(merge=True):
        launches[merge]()
    lib = _lib.lib()

    def merge_kernel():
        _lib.check(lib.nsn_attention_merge(ws.data_ptr(), b_, hq, n_splits, ctx.data_ptr(), out.data_ptr(),
                                           _lib.DTYPE_BF16, status.data_ptr(), stream.cuda_stream), "nsn_attention_merge")
    # per-kernel rounds first, then the timed steps (as in C2)
    _, ms_split, ms_merge, _, _ = interleaved_rounds(step, lambda: step(merge=False), merge_kernel, stream)
    ms_step = timed(step, args.steps, args.warmup, stream)
    assert _dev.read_status(status) == 0
    nbytes = b_ * hkv * 2 * L * (bits * 16 + 10) + 2 * b_ * hq * D * 2
    achieved = nbytes / (ms_split * 1e-3) / 1e9
    log(f"[bench] C3 decode step {ms_step * 1e3:.1f} us, split kernel {ms_split * 1e3:.1f} us, merge {ms_merge * 1e3:.1f} us, "
        f"{nbytes / 1e6:.1f} MB algorithmic -> {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%} of 8 TB/s)")
    _, ref_ctx = kernels.decode_attention(q, kk, vv, seq, max_seq_len=L, kernel="reference",
                                          kv_round_dtype=torch.float32)
    err = (ctx - ref_ctx).abs()
    ok = bool((err <= 2e-3 + 1e-2 * ref_ctx.abs()).all())
    log(f"[bench] C3 parity vs exact-order kernel: max abs {float(err.max()):.2e}, within tol: {ok}")
    result = {
        "metric": "C3 5-bit fused decode-attn µs/step (B=64, 16q/4kv, ctx 8192) + encode of all K/V blocks",
        "value": round(ms_step * 1e3, 2), "unit": "µs/step", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16x2/f32", "data": "synthetic (GPU torch.Generator seed 3)",
        "config": {"workload": "C3: 5-bit packed K+V, B=64, 16q/4kv heads, d=128, ctx 8192 (128 blocks, no tail)",
                   "batch": b_, "heads_q": hq, "heads_kv": hkv, "head_dim": D, "ctx": L, "bits": bits,
                   "kernel": args.kernel, "split_tokens": split, "n_splits": n_splits},
        "encode_us": round(enc_ms * 1e3, 1), "encode_gbs": round(enc_gbs, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_c3_traffic() if args.kernel == "fast" else None,
                     "kernel": f"attn split kernel ({args.kernel})", "algorithmic_bytes": nbytes,
                     "kernel_us": round(ms_split * 1e3, 2), "merge_us": round(ms_merge * 1e3, 2),
                     "timing": f"{SETTLE_STEPS} warm-up steps, then {ROUNDS} rounds of back-to-back batches of "
                               f"{BATCH} steps / split-only / merge-only launches, enqueued without a host sync, HIP "
                               "events between batches on the launch stream; one cache copy (378 MB, beyond the "
                               "256 MB Infinity Cache); value: the timed steps after the rounds"},
        "encode_roofline": {"bound": "hbm", "achieved": round(enc_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(enc_gbs / HBM_PEAK_GBS, 4)},
        "parity_ok": ok,
    }
    if emit:
        print(json.dumps(result), flush=True)
    return result


K1C_MODELS = {"Qwen3-30B-A3B": dict(n_kv=8, head_dim=128, n_q=32), "Gemma4-26B-A4B": dict(n_kv=8, head_dim=256, n_q=32)}
K1C_BATCH = [1, 8, 32, 64]
K1C_CTX = [2048, 8192, 32768, 65536]
K1C_RECIPES = [("nsn", 5, False), ("kivi", 5, False), ("kivi", 4, False), ("nsn", 4, False), ("fp16", 16, False),
               ("nsn", 5, True), ("nsn", 3, True)]   # (recipe, bits, bit-packed codes)
K1C_HEADLINE = (32, 32768, "nsn", 5)


def main_k1c(args):
    """The reference's K-score grid (experiments/kernels/phase_k1c_triton_fused_kernel.py:
    Qwen3-30B-A3B or Gemma4 shape, B in {1, 8, 32, 64}, ctx in {2K .. 64K}, recipes
    NSN5 / KIVI5 / KIVI4 / NSN4 / fp16 on u8 codes, plus NSN5 and NSN3 on
    bit-packed codes), timed as the reference times it (30 warm-up calls, then
    the median of 100 calls each bracketed by events), against the published
    latencies (tests/golden/k1c_published.json, RTX PRO 6000 Blackwell).  K is
    N(0,1) from a GPU generator (the reference draws the same distribution on
    the CPU); the store is built on the GPU.  One JSON line: value = the
    B=32 / 32K / NSN5 cell."""
    import torch
    from nsn_amd import kscore
    dev = torch.device("cuda:0")
    model = K1C_MODELS[args.k1c_model]
    n_kv, hd, n_q = model["n_kv"], model["head_dim"], model["n_q"]
    pub = json.loads((ROOT / "tests" / "golden" / "k1c_published.json").read_text())
    published = {(c["batch"], c["ctx"], c["recipe"], c["bits"]): c["latency_ms_median"]
                 for c in pub["cells"] if c["model"] == args.k1c_model}
    stream = torch.cuda.current_stream()
    cells = []
    for B in ([8, 32] if args.k1c_quick else K1C_BATCH):
        for T in ([32768] if args.k1c_quick else K1C_CTX):
            gen = torch.Generator(device=dev).manual_seed(20260510 + B * 131 + T)
            q = torch.randn((B, n_q, hd), generator=gen, device=dev).to(torch.float16)
            k = torch.randn((B, T, n_kv * hd), generator=gen, device=dev)
            for recipe, bits, packed in K1C_RECIPES:
                ref, ts = kscore.make_store(k, bits, recipe, n_kv, hd, dev)
                del ref
                if packed:
                    ts = kscore.pack_store(ts, bits)
                out = torch.empty((B, n_q, T), dtype=torch.float32, device=dev)
                fn = lambda: kscore.decode_scores(q, ts, n_q, n_kv, hd, out=out)
                for _ in range(30):
                    fn()
                torch.cuda.synchronize()
                samples = []
                for _ in range(100):
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    fn()
                    e1.record(stream)
                    torch.cuda.synchronize()
                    samples.append(e0.elapsed_time(e1))
                med = sorted(samples)[len(samples) // 2]
                nbytes = (ts["code"].numel() * ts["code"].element_size() + out.numel() * 4 + q.numel() * 2
                          + (0 if recipe == "fp16" else 2 * 2 * B * n_kv * hd)
                          + (2 * B * n_kv * T if recipe == "nsn" else 0))
                pm = None if packed else published.get((B, T, recipe, bits))
                cell = {"batch": B, "ctx": T, "recipe": recipe, "bits": bits, "codes": "packed" if packed else
                        ("fp16" if recipe == "fp16" else "u8"), "ms": round(med, 5), "gbs": round(nbytes / med / 1e6, 1),
                        "published_ms": pm, "ratio_vs_published": round(med / pm, 4) if pm else None}
                cells.append(cell)
                log(f"[bench] k1c B={B:>2} T={T:>5} {recipe}{bits}{'p' if packed else ' '}: {med * 1e3:8.1f} us "
                    f"{cell['gbs']:7.1f} GB/s" + (f"  published {pm * 1e3:8.1f} us  x{pm / med:5.2f}" if pm else ""))
                del ts, out
            del q, k
            torch.cuda.empty_cache()
    hb, ht, hr, hbits = K1C_HEADLINE
    head = next(c for c in cells if (c["batch"], c["ctx"], c["recipe"], c["bits"], c["codes"]) == (hb, ht, hr, hbits, "u8"))
    result = {
        "metric": f"K1c K-score ms/call ({args.k1c_model}: {n_q}q/{n_kv}kv, d={hd}; B={hb}, ctx {ht}, NSN{hbits} u8 codes)",
        "value": head["ms"], "unit": "ms", "n_gpus": 1, "steps": 100, "warmup": 30, "ms_per_step": head["ms"],
        "higher_is_better": False, "scaling": "weak", "vs_baseline": head["ratio_vs_published"],
        "baseline": {"value": head["published_ms"], "device": pub["device"], "source": pub["source"]},
        "dtype": "f16", "data": "synthetic (K ~ N(0,1), GPU generator; the store built on the GPU)",
        "config": {"workload": "K1c K-score grid", "model": args.k1c_model, "heads_q": n_q, "heads_kv": n_kv,
                   "head_dim": hd},
        "roofline": {"bound": "hbm", "achieved": head["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": None, "kernel": "kscore (u8 NSN5)"},
        "grid": cells,
    }
    print(json.dumps(result), flush=True)


def k1c_summary(d):
    """profiles/kscore_k1c.md from the kernel trace of `bench.py --workload k1c
    --k1c-quick`: the kernel's own duration per cell (its 130 launches in
    order: 30 warm-up, then the 100 timed ones, whose median is reported)."""
    rows = _rows((Path(d), "**/*kernel_trace.csv"))
    ks = sorted(((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]) for r in rows
                 if "kscore_kernel" in r["Kernel_Name"]))
    model = K1C_MODELS["Qwen3-30B-A3B"]
    pub = json.loads((ROOT / "tests" / "golden" / "k1c_published.json").read_text())
    published = {(c["batch"], c["ctx"], c["recipe"], c["bits"]): c["latency_ms_median"]
                 for c in pub["cells"] if c["model"] == "Qwen3-30B-A3B"}
    cells = [(B, 32768, r, b, pk) for B in (8, 32) for r, b, pk in K1C_RECIPES]
    if len(ks) != 130 * len(cells):
        raise SystemExit(f"expected {130 * len(cells)} kscore dispatches, found {len(ks)}")
    L = ["# kscore_kernel on the K1c grid (Qwen3-30B-A3B shape: 32q/8kv, d=128, ctx 32768)", "",
         "Command (repository root, one MI355X; `OUT` = an output folder):", "", "```",
         "rocprofv3 --kernel-trace --stats --output-format csv -d OUT/kt -o kt -- python3 bench.py --workload k1c --k1c-quick",
         "python3 bench.py --k1c-summary OUT      # writes this file", "```", "",
         "Kernel duration from the trace: the median of each cell's 100 timed launches (after 30 warm-up "
         "launches).  Bytes: codes + scores (fp32) + q + min/step + eff_norm.  Published: the reference's "
         f"Triton kernel on {pub['device']} (event-timed calls, median of 100).", "",
         "| B | recipe | codes | kernel | us (median) | GB/s | % of 8 TB/s | published us |", "|---|---|---|---|---|---|---|---|"]
    n_kv, hd, n_q = model["n_kv"], model["head_dim"], model["n_q"]
    for i, (B, T, recipe, bits, packed) in enumerate(cells):
        part = ks[130 * i + 30:130 * (i + 1)]
        durs = sorted((e - b0) / 1e3 for b0, e, _ in part)
        med = durs[len(durs) // 2]
        name = part[0][2]
        kern = name[name.index("<"):name.index(">") + 1] if "<" in name else name
        code_b = B * T * n_kv * hd * (2 if recipe == "fp16" else (bits / 8 if packed else 1))
        nbytes = code_b + B * n_q * T * 4 + B * n_q * hd * 2 + (0 if recipe == "fp16" else 4 * B * n_kv * hd) + \
            (2 * B * n_kv * T if recipe == "nsn" else 0)
        pm = None if packed else published.get((B, T, recipe, bits))
        L.append(f"| {B} | {recipe}{bits if recipe != 'fp16' else ''} | {'packed' if packed else ('fp16' if recipe == 'fp16' else 'u8')} "
                 f"| `{kern}` | {med:.1f} | {nbytes / med / 1e3:.0f} | {nbytes / med / 1e3 / HBM_PEAK_GBS * 100:.1f} | "
                 f"{pm * 1e3:.1f} |" if pm else
                 f"| {B} | {recipe}{bits if recipe != 'fp16' else ''} | {'packed' if packed else ('fp16' if recipe == 'fp16' else 'u8')} "
                 f"| `{kern}` | {med:.1f} | {nbytes / med / 1e3:.0f} | {nbytes / med / 1e3 / HBM_PEAK_GBS * 100:.1f} | -- |")
    L.append("")
    out = ROOT / "profiles" / "kscore_k1c.md"
    out.write_text("\n".join(L))
    print("\n".join(L))


C4 = dict(B=32, H=16, T=8192, chunk=512, steps=256)


def dense_sdpa_comparator(qc, T, stream):
    """torch's own flash attention on the last C4 chunk's shape with DENSE
    bf16 K/V: the chunk's 512 queries against all T keys, no mask (the
    packed prefill's causal last chunk computes ~3 % fewer pairs), each
    backend torch offers on this build (aotriton flash and memory-efficient).
    TFLOP/s on the pairs each computes.  A comparator only: it reads
    materialised K/V the packed path never holds."""
    import torch
    import torch.nn.functional as Fn
    from torch.nn.attention import SDPBackend, sdpa_kernel

    b_, h, nq, d = qc.shape
    gen = torch.Generator(device=qc.device).manual_seed(5)
    k = torch.randn((b_, h, T, d), generator=gen, device=qc.device, dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn((b_, h, T, d), generator=gen, device=qc.device, dtype=torch.bfloat16)
    flops = 4.0 * b_ * h * nq * T * d
    out = {"shape": f"B={b_} H={h} q={nq} keys={T} d={d} bf16, no mask", "flops": flops,
           "fa_library": str(torch.backends.cuda.preferred_rocm_fa_library())}
    for name, be in (("flash", SDPBackend.FLASH_ATTENTION), ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel(be):
                ms = timed(lambda: Fn.scaled_dot_product_attention(qc, k, v), 5, 2, stream)
        except RuntimeError as e:   # backend not built for this device
            out[name] = {"error": str(e)[:120]}
            continue
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"us": round(ms * 1e3, 1), "tflops": round(tf, 1), "frac": round(tf / 2500, 4)}
        log(f"[bench] C4 dense comparator: torch SDPA {name} ({out['fa_library']}) on dense bf16 K/V, "
            f"{nq} queries x {T} keys: {ms * 1e3:.0f} us, {tf:.0f} TFLOP/s ({tf / 2500:.1%})")
    del k, v
    torch.cuda.empty_cache()
    return out


def main_c4(args, emit=True):
    """C4: a streaming packed cache of Ouro-like
    slots (MHA, 16 kv heads, d=128, batch 32, N(0,1) bf16 activations, GPU
    generator seed 4, fp16 tails).  Per slot: an 8192-token chunked prefill
    (16 chunks of 512: bf16-MFMA prefill attention over packed context + tail
    + the chunk, append to the fp16 tail, compress), then decode steps that
    append one token, attend over packed + tail with the fast kernel and
    compress a block every 64 tokens.  The 96
    slots of the configuration do identical work; `--slots` of them are run
    and the figures are per slot, after one untimed warm-up prefill (of slot 0,
    which is then emptied)."""
    import torch
    from nsn_amd import _dev, kernels
    from nsn_amd.stream_cache import StreamingKVCache

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    b_, h, T, ch = C4["B"], C4["H"], C4["T"], C4["chunk"]
    S = max(1, args.slots)
    gen = torch.Generator(device=dev).manual_seed(4)
    nchunks = T // ch
    log(f"[bench] C4: {S} slots x B={b_} x {h} kv-heads, {T}-token chunked prefill (chunk {ch}), decode")
    # activations: one set of chunk K/V/Q shared by the slots (identical work per slot)
    acts = [tuple(torch.randn((b_, h, ch, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
                  for _ in range(3)) for _ in range(nchunks)]
    cache = StreamingKVCache(S, b_, h, T + C4["steps"] + 64, bits=3, dtype=torch.float16, max_append=ch, device=dev)

    def prefill_slot(s):
        for c in range(nchunks):
            qc, kc, vc = acts[c]
            cache.prefill(s, qc, kc, vc, check=False, append=True)   # attention + the chunk's append
            cache.compress_to(s, max(cache.compressed[s], ((cache.length[s] - 64) // 64) * 64))
    prefill_slot(0)   # untimed warm-up: one slot's whole prefill, then the slot is emptied again
    cache.reset(0)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for s in range(S):
        prefill_slot(s)
    e1.record(stream)
    torch.cuda.synchronize()
    pre_ms = e0.elapsed_time(e1) / S
    cache.post_prefill()
    cache.check_status()
    flops = 2.0 * b_ * h * T * T * D          # causal QK^T + PV (2 * B * H * T^2 * d)
    mfma = flops / (pre_ms * 1e-3) / 1e12
    log(f"[bench] C4 prefill: {pre_ms:.2f} ms per slot (16 chunks incl. append + in-place encode), "
        f"{mfma:.0f} TFLOP/s = {mfma / 2500:.1%} of 2.5 PFLOP/s dense bf16")
    # the prefill kernel alone, on the last chunk of one slot (context 7680 tokens)
    qc, kc, vc = acts[-1]
    saved = (list(cache.seq_length[0]), list(cache.seq_compressed[0]))
    cache.seq_length[0] = [T - ch] * b_                             # state before the last chunk
    cache.seq_compressed[0] = [((T - ch - 64) // 64) * 64] * b_
    for name in ("K", "V"):
        cache.side(0, name).blocks.fill_(cache.compressed[0] // 64)
    pk_ms = timed(lambda: cache.prefill(0, qc, kc, vc, check=False), 5, 2, stream)
    last_flops = 2.0 * 2 * b_ * h * ch * D * ((T - ch) + (ch + 1) / 2)
    log(f"[bench] C4 prefill kernel, last chunk (context {T - ch}): {pk_ms * 1e3:.0f} us, "
        f"{last_flops / (pk_ms * 1e-3) / 1e12:.0f} TFLOP/s")
    cache.seq_length[0], cache.seq_compressed[0] = saved
    for name in ("K", "V"):
        cache.side(0, name).blocks.fill_(cache.compressed[0] // 64)
    dense = None if args.no_baselines else dense_sdpa_comparator(qc, T, stream)

    # ---- decode steps: append, attend (fast kernel), compress every 64 tokens
    qd = torch.randn((b_, h, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
    tok = [torch.randn((b_, h, 1, D), generator=gen, device=dev, dtype=torch.float32).to(torch.float16)
           for _ in range(2)]
    ws = torch.empty(kernels.workspace_floats(b_, h, 64), dtype=torch.float32, device=dev)
    out = torch.empty((b_, h, D), dtype=torch.bfloat16, device=dev)
    ctx = torch.empty((b_, h, D), dtype=torch.float32, device=dev)
    status = _dev.new_status(dev)

    def decode_step():
        for s in range(S):
            cache.append(s, tok[0], tok[1])
            L = cache.length[s]
            kernels.decode_attention(qd, cache.side(s, "K"), cache.side(s, "V"), cache.lengths(s), max_seq_len=L,
                                     kernel="fast", split_tokens=256, workspace=ws, out=out, ctx=ctx,
                                     status=status, check=False)
        cache.post_decode()
    n_dec = max(1, min(args.decode_steps, C4["steps"] - 2))
    for L in range(cache.length[0], cache.length[0] + n_dec + 3):
        cache.length_tensor(L)          # the per-length int32 tensors exist before timing
    for _ in range(2):
        decode_step()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(n_dec):
        decode_step()
    e1.record(stream)
    torch.cuda.synchronize()
    dec_us = e0.elapsed_time(e1) * 1e3 / n_dec / S
    assert _dev.read_status(status) == 0
    cache.check_status()
    L = cache.length[0]
    C = cache.compressed[0]
    dec_bytes = b_ * h * 2 * (C * 58 + (L - C) * 256) + 2 * b_ * h * D * 2
    dec_gbs = dec_bytes / (dec_us * 1e-6) / 1e9
    log(f"[bench] C4 decode: {dec_us:.1f} us per slot per step (append + fast decode + policy; context {L}), "
        f"{dec_bytes / 1e6:.0f} MB -> {dec_gbs:.0f} GB/s ({dec_gbs / HBM_PEAK_GBS:.1%} of 8 TB/s)")
    result = {
        "metric": "C4 streaming cache: chunked-prefill ms/slot (MFMA %) + decode µs/slot/step",
        "value": round(dec_us, 2), "unit": "µs/slot/step", "n_gpus": 1, "steps": n_dec, "warmup": 2,
        "ms_per_step": round(dec_us * S / 1e3, 5), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16 prefill / f16x2 decode",
        "data": "synthetic N(0,1) (GPU torch.Generator seed 4)",
        "config": {"workload": "C4: Ouro-like streaming cache, MHA 16 kv heads, d=128, batch 32, 8192-token "
                               "chunked prefill (chunk 512) + decode over packed INT3 + fp16 tail",
                   "slots_run": S, "batch": b_, "heads": h, "head_dim": D, "prefill_tokens": T, "chunk": ch,
                   "bits": 3},
        "prefill_ms_per_slot": round(pre_ms, 3),
        "prefill_roofline": {"bound": "mfma", "achieved": round(mfma, 1), "peak": 2500.0, "unit": "TFLOP/s",
                             "frac": round(mfma / 2500, 4), "flops_per_slot": flops},
        "prefill_kernel_last_chunk_us": round(pk_ms * 1e3, 1),
        "prefill_kernel_last_chunk_tflops": round(last_flops / (pk_ms * 1e-3) / 1e12, 1),
        "dense_sdpa_comparator": dense,
        "roofline": {"bound": "hbm", "achieved": round(dec_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(dec_gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode step (append + fast decode + merge + policy)", "algorithmic_bytes": dec_bytes},
    }
    if emit:
        print(json.dumps(result), flush=True)
    return result


STATS_DOC = {
    "c3": ("attn_fast_c3", "C3: 5-bit packed K/V, B=64, 16q/4kv, ctx 8192 -- encode of all blocks + decode steps",
           "rocprofv3 --kernel-trace --stats --output-format csv -d OUT/kt -o kt -- python3 bench.py --workload c3 --no-cpu\n"
           "rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/fetch -o p -- python3 bench.py --workload c3 --no-cpu\n"
           "rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/write -o p -- python3 bench.py --workload c3 --no-cpu"),
    "c4": ("prefill_c4", "C4: streaming cache, MHA 16 kv-heads, batch 32 -- 8192-token chunked prefill + decode steps",
           "rocprofv3 --kernel-trace --stats --output-format csv -d OUT/kt -o kt -- python3 bench.py --workload c4 "
           "--slots 1 --decode-steps 16\n"
           "rocprofv3 --pmc SQ_WAVES SQ_BUSY_CYCLES SQ_WAVE_CYCLES SQ_INSTS_VALU SQ_ACTIVE_INST_VALU SQ_INSTS_LDS "
           "SQ_INSTS_SALU SQ_INSTS_MFMA GRBM_GUI_ACTIVE --output-format csv -d OUT/sq1 -o sq1 -- python3 bench.py "
           "--workload c4 --slots 1 --decode-steps 16\n"
           "rocprofv3 --pmc SQ_WAIT_ANY SQ_WAIT_INST_ANY SQ_ACTIVE_INST_ANY SQ_LDS_BANK_CONFLICT SQ_ACTIVE_INST_LDS "
           "SQ_VALU_MFMA_BUSY_CYCLES SQ_INST_LEVEL_VMEM SQ_LEVEL_WAVES --output-format csv -d OUT/sq2 -o sq2 -- "
           "python3 bench.py --workload c4 --slots 1 --decode-steps 16"),
}
PREFILL_KERNEL = "nsn::prefill::prefill_kernel"
PREFILL_LAST_CALLS = 7   # the last-chunk timing of main_c4: 2 warm-up + 5 timed prefill launches, the run's last


ADAPTER = dict(layers=24, hidden=2048, heads=16, inter=5632, vocab=49152, B=32, T=8192, chunk=512)


def _Looped(base, loops):
    """An Ouro-like looped model over a transformers Llama: the decoder
    layers applied `loops` times with shared weights, the attention of loop
    ut, layer i in cache slot ut * layers + i (it gets `current_ut`).  The
    attention mask is left to the packed routes (causal, no padding)."""
    import types

    import torch

    class Looped(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.base = base

        def forward(self, input_ids, position_ids=None, past_key_values=None, use_cache=True, logits_to_keep=1):
            mdl = self.base.model
            h = mdl.embed_tokens(input_ids)
            if position_ids is None:
                past = past_key_values.get_seq_length()
                position_ids = torch.arange(past, past + input_ids.shape[1], device=h.device)[None]
            pe = mdl.rotary_emb(h, position_ids=position_ids)
            for ut in range(loops):
                for layer in mdl.layers:
                    h = layer(h, attention_mask=None, position_ids=position_ids, past_key_values=past_key_values,
                              use_cache=use_cache, position_embeddings=pe, current_ut=ut)
            h = mdl.norm(h)
            return types.SimpleNamespace(logits=self.base.lm_head(h[:, -logits_to_keep:]))

    return Looped().eval()


def main_adapter(args):
    """The transformers connection (nsn_amd.adapter) on an Ouro-1.4B-shaped
    Llama with random-init bf16 weights (24 layers = one loop of the C4 slot
    map, 16 MHA heads, d=128, B=32; torch seed 5): an 8192-token chunked
    prefill (chunks of 512, compressed after each), then `--steps` decode
    steps (fixed synthetic tokens; the compression policy after each step).
    The same step four ways: the packed cache with the fused arm replayed as
    one HIP graph per step (the value), the same arm run eagerly, the NATIVE
    arm (dense restore + sdpa), and transformers' own DynamicCache (dense
    bf16 K/V).  One JSON line."""
    import gc
    import time

    import torch
    from transformers import LlamaConfig, LlamaForCausalLM
    from transformers.cache_utils import DynamicCache

    from nsn_amd import adapter

    a = dict(ADAPTER)
    if args.adapter_shape == "ac08":
        a.update(B=1, T=768, chunk=256)
        if args.warmup + args.steps > 255:
            raise SystemExit("--adapter-shape ac08: --warmup + --steps must stay within 255 decode steps "
                             "(the published run's 769..1023-token window)")
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    b_, T, ch = a["B"], a["T"], a["chunk"]
    steps, warm = args.steps, args.warmup
    cfg = LlamaConfig(vocab_size=a["vocab"], hidden_size=a["hidden"], intermediate_size=a["inter"],
                      num_hidden_layers=a["layers"], num_attention_heads=a["heads"], num_key_value_heads=a["heads"],
                      head_dim=D, max_position_embeddings=T + steps + warm + 64)
    torch.manual_seed(5)
    with torch.device(dev):
        m = LlamaForCausalLM(cfg)
    m = m.to(torch.bfloat16).eval()
    loops = max(1, args.adapter_loops)
    base = m
    if loops > 1:
        m = _Looped(base, loops)
    n_embed = a["vocab"] * a["hidden"]
    # the embedding is gathered, not read; a looped model reads the layers once per loop
    layer_params = sum(p.numel() for p in base.model.layers.parameters())
    weight_bytes = 2 * (sum(p.numel() for p in base.parameters()) - n_embed + (loops - 1) * layer_params)
    gen = torch.Generator(device=dev).manual_seed(5)
    ids = torch.randint(0, a["vocab"], (b_, T), generator=gen, device=dev)
    toks = torch.randint(0, a["vocab"], (b_, warm + steps), generator=gen, device=dev)
    log(f"[bench] adapter: {a['layers']} layers x {loops} loops, {a['heads']} heads, B={b_}, prefill {T} "
        f"(chunk {ch}), {steps} decode steps; weights {weight_bytes / 1e9:.2f} GB read per step")
    restore = adapter.install(base)

    def run(kind):
        packed = kind != "hf_dense"
        graph = kind == "graph"
        arm = "PACKED_KV_FUSED" if graph else kind
        # the graph run is the full packed path (prefill over the packed context
        # on the MFMA prefill kernel); the eager fused run keeps the native prefill
        cache = (adapter.PackedKVCache(cfg, b_, T + warm + steps + 64, loops=loops, arm=arm, max_prefill=ch,
                                       strict=False, prefill="packed" if graph or loops > 1 else "native", device=dev)
                 if packed else DynamicCache(config=cfg))
        with torch.no_grad():
            t0 = time.perf_counter()
            for c in range(T // ch):
                m(input_ids=ids[:, c * ch:(c + 1) * ch], past_key_values=cache, use_cache=True, logits_to_keep=1)
                if packed:
                    cache.post_prefill()
            torch.cuda.synchronize()
            pre_s = time.perf_counter() - t0
            i = [0]
            dg = adapter.DecodeGraph(m, cache) if graph else None

            def step():
                if graph:
                    dg.step(toks[:, i[0]:i[0] + 1])
                else:
                    m(input_ids=toks[:, i[0]:i[0] + 1], past_key_values=cache, use_cache=True, logits_to_keep=1)
                    if packed:
                        cache.post_decode()
                i[0] += 1
            for _ in range(warm):
                step()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            h0 = time.perf_counter()
            e0.record(stream)
            for _ in range(steps):
                step()
            e1.record(stream)
            host_ms = (time.perf_counter() - h0) * 1e3 / steps
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1) / steps
        kv_bytes = 0
        if packed:
            cache.check_status()
            st = cache.store
            L, C = st.length[0], st.compressed[0]
            kv_bytes = st.slots * b_ * a["heads"] * 2 * (C * 58 + (L - C) * 256)
        # the graph (and its memory pool) and the step closure hold the cache:
        # drop all of them before handing the memory back
        dg = None
        del cache, step
        gc.collect()
        torch.cuda.empty_cache()
        free = torch.cuda.mem_get_info()[0] / 2**30
        log(f"[bench] adapter {kind}: prefill {pre_s:.2f} s, decode {ms:.2f} ms/step (host issue {host_ms:.2f} "
            f"ms/step); {free:.0f} GiB free after release")
        return ms, host_ms, kv_bytes, pre_s

    arms = args.adapter_arms.split(",")
    if loops > 1:   # the dense comparators index caches by layer, not by (loop, layer)
        arms = [k for k in arms if k in ("graph", "PACKED_KV_FUSED")]
    require_arms = {"hf_dense", "graph", "PACKED_KV_FUSED", "NATIVE"}
    if not arms or not set(arms) <= require_arms or "graph" not in arms:
        raise SystemExit(f"--adapter-arms: a comma list of {sorted(require_arms)} that includes graph")
    res = {}
    try:
        for kind in arms:                          # hf_dense first by default: the largest footprint, fresh memory
            res[kind] = run(kind)
    finally:
        restore()
    graph_ms, graph_host, kv_bytes, graph_pre = res["graph"]
    fused_ms, fused_host, _, fused_pre = res.get("PACKED_KV_FUSED", (None, None, 0, None))
    native_ms = res.get("NATIVE", (None,))[0]
    dense_ms, _, _, dense_pre = res.get("hf_dense", (None, None, 0, None))
    nbytes = weight_bytes + kv_bytes
    achieved = nbytes / (graph_ms * 1e-3) / 1e9
    result = {
        "metric": (f"HF-connected decode ms/step (Ouro-1.4B-shaped Llama, 24 layers x {loops} loops, B={b_}, "
                   f"ctx {T}, INT3 packed K/V)"),
        "value": round(graph_ms, 3), "unit": "ms/step", "n_gpus": 1, "steps": steps, "warmup": warm,
        "ms_per_step": round(graph_ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (random-init weights, torch seed 5; tokens from GPU generator seed 5)",
        "config": {"workload": "transformers connection: whole-model decode step through the packed cache",
                   "layers": a["layers"], "loops": loops, "slots": a["layers"] * loops, "hidden": a["hidden"],
                   "heads_q": a["heads"], "heads_kv": a["heads"],
                   "head_dim": D, "batch": b_, "prefill": T, "chunk": ch, "bits": 3,
                   "arm": "PACKED_KV_FUSED, step replayed as a HIP graph; packed prefill route"},
        "comparators": {"fused_eager_ms": _r(fused_ms), "fused_eager_host_issue_ms": _r(fused_host),
                        "graph_host_issue_ms": _r(graph_host), "native_arm_ms": _r(native_ms),
                        "hf_dynamic_cache_ms": _r(dense_ms),
                        "prefill_s": {"packed_route": _r(graph_pre, 2), "native_route": _r(fused_pre, 2),
                                      "hf_dynamic_cache": _r(dense_pre, 2)}},
        "shape": args.adapter_shape,
        "reference_published": ({"ms_per_token_median": {"unquantized": 146.009, "current_packed": 164.651,
                                                         "v_fused": 154.411},
                                 "source": "reports/ac08-results-v0.1-2026-10-02.md:36-48 (Ouro-1.4B with its real "
                                           "weights, B=1, KV 769..1023, RTX PRO 6000; context only)"}
                                if args.adapter_shape == "ac08" else None),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": f"whole decode step (weights + packed K/V of {a['layers'] * loops} slots)",
                     "algorithmic_bytes": nbytes},
    }
    print(json.dumps(result), flush=True)


def _r(x, nd=3):
    return None if x is None else round(x, nd)


ADAPTER_DOC = ("rocprofv3 --kernel-trace --stats --output-format csv -d OUT/kt -o kt -- "
               "python3 bench.py --workload adapter --adapter-arms graph --steps 20 --warmup 5")


def adapter_summary(d):
    """profiles/adapter_decode_graph.md from the kernel trace of
    `bench.py --workload adapter --adapter-arms graph`: the kernels from the
    first fused rotary + append on (the decode phase: one eager warm-up step,
    then warmup + steps graph replays), grouped by name, per step."""
    rows = _rows((Path(d), "**/*kernel_trace.csv"))
    ks = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]) for r in rows)
    first = next(i for i, k in enumerate(ks) if "rope_append_kernel" in k[2])
    dec = ks[first:]
    n_append = sum("rope_append_kernel" in k[2] for k in dec)
    layers = ADAPTER["layers"]
    if n_append % layers:
        raise SystemExit(f"{n_append} tail appends is not a multiple of {layers} layers")
    nstep = n_append // layers
    agg = {}
    for s0, s1, name in dec:
        a = agg.setdefault(name, [0, 0])
        a[0] += 1
        a[1] += s1 - s0
    busy = sum(v[1] for v in agg.values())
    wall = dec[-1][1] - dec[0][0]
    L = ["# Transformers connection: one decode step as a HIP graph (adapter workload)", "",
         "Ouro-1.4B-shaped Llama (24 layers, 16 MHA heads, d=128), random-init bf16 weights; B=32, 8192-token "
         "context in the packed cache (INT3 blocks + fp16 tail); the fused arm, the step captured once and "
         "replayed.", "", "Command (from the repository root on one MI355X, `OUT` = an output folder), then "
         "`python3 bench.py --adapter-summary OUT/kt`:", "", "```", ADAPTER_DOC, "```", "",
         f"Decode phase: {nstep} steps ({len(dec)} kernels, {len(dec) / nstep:.0f} per step); kernel busy "
         f"{busy / nstep / 1e6:.3f} ms per step, first start to last end {wall / nstep / 1e6:.3f} ms per step "
         "(the gaps are dispatch between the graph's small kernels).", "",
         "| kernel | per step | avg us | us per step | share of busy |", "|---|---|---|---|---|"]
    for name, (cnt, tot) in sorted(agg.items(), key=lambda kv: -kv[1][1])[:16]:
        L.append(f"| `{name[:100]}` | {cnt / nstep:.0f} | {tot / cnt / 1e3:.1f} | {tot / nstep / 1e3:.1f} | "
                 f"{tot / busy:.1%} |")
    L.append("")
    (ROOT / "profiles" / "adapter_decode_graph.md").write_text("\n".join(L))
    print("\n".join(L))


C3_SPLIT_KERNEL = "nsn::fast::attn_fast_kernel<5, 1, false, 4, false>"
C3_ENCODE_KERNEL = "nsn::encode_kernel<0, 5, 0>"
C3_JSON = ROOT / "profiles" / "attn_fast_c3.json"


def c3_traffic_lines(d):
    """HBM traffic of the C3 split kernel and of the C3 encode launch (all K
    and V blocks) from the FETCH_SIZE / WRITE_SIZE passes under OUT/fetch and
    OUT/write, scaled by the factors the C2 profile's 1 GiB calibration copy
    measured on this GPU type; also writes profiles/attn_fast_c3.json, which
    the C3 line reads while the kernel source is unchanged."""
    import statistics
    c2 = json.loads(PROFILE_JSON.read_text())
    fs, ws = c2["fetch_scale"], c2["write_scale"]

    def per(counter, sub, kernel, largest=False):
        vals = [float(r["Counter_Value"]) for r in _rows((Path(d) / sub, "**/*counter_collection.csv"))
                if r["Counter_Name"] == counter and kernel in r["Kernel_Name"]]
        return max(vals) if largest else statistics.median(vals), len(vals)

    fk, n = per("FETCH_SIZE", "fetch", C3_SPLIT_KERNEL)
    wk, _ = per("WRITE_SIZE", "write", C3_SPLIT_KERNEL)
    efk, _ = per("FETCH_SIZE", "fetch", C3_ENCODE_KERNEL, largest=True)
    ewk, _ = per("WRITE_SIZE", "write", C3_ENCODE_KERNEL, largest=True)
    rd, wr = fk * 1024 * fs, wk * 1024 * ws
    erd, ewr = efk * 1024 * fs, ewk * 1024 * ws
    b_, hq, hkv, L, bits = C3["B"], C3["HQ"], C3["HKV"], C3["L"], C3["bits"]
    alg = b_ * hkv * 2 * L * (bits * 16 + 10) + 2 * b_ * hq * D * 2
    enc_alg = 2 * b_ * hkv * L * 346
    fig = {"kernel": C3_SPLIT_KERNEL, "source_sha256": source_sha(), "workload": "C3", "dispatches": n,
           "fetch_kib": fk, "write_kib": wk, "fetch_scale": fs, "write_scale": ws,
           "read_bytes": int(rd), "write_bytes": int(wr), "traffic": int(rd + wr), "algorithmic_bytes": alg,
           "encode_traffic": int(erd + ewr), "encode_algorithmic_bytes": enc_alg}
    C3_JSON.write_text(json.dumps(fig, indent=1) + "\n")
    return ["## HBM traffic per dispatch (the FETCH_SIZE and WRITE_SIZE passes above)", "",
            f"Scaled by the factors of the calibration copy in `profiles/attn_fast_c2.md` (same GPU type): reads "
            f"x{fs:.3f}, writes x{ws:.3f}.", "",
            "| dispatch | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes | algorithmic | ratio |", "|---|---|---|---|---|---|",
            f"| split kernel (median of {n}) | {fk:.0f} | {wk:.0f} | {(rd + wr) / 1e6:.1f} MB | {alg / 1e6:.1f} MB | "
            f"{(rd + wr) / alg:.3f} |",
            f"| encode of all K and V blocks (the largest encode dispatch) | {efk:.0f} | {ewk:.0f} | "
            f"{(erd + ewr) / 1e6:.1f} MB | {enc_alg / 1e6:.1f} MB | {(erd + ewr) / enc_alg:.3f} |", "",
            f"Kernel source sha256 (nsn_amd/csrc/nsn_fast.hip): `{source_sha()}`", ""]


def measured_c3_traffic():
    """HBM bytes per C3 split-kernel launch from the committed profile, if it
    was measured on this kernel source; else None."""
    try:
        fig = json.loads(C3_JSON.read_text())
    except (OSError, ValueError):
        return None
    return fig["traffic"] if fig.get("source_sha256") == source_sha() else None


def stats_summary(d, workload):
    """profiles/<name>.md from the kernel statistics of one rocprofv3 run."""
    name, title, cmd = STATS_DOC[workload]
    stats = _rows((Path(d) / "kt", "**/*kernel_stats.csv"))
    top = sorted(stats, key=lambda r: -float(r["TotalDurationNs"]))[:12]
    L = [f"# {title}", "", "Command (from the repository root on one MI355X, `OUT` = an output folder), then "
         f"`python3 bench.py --workload {workload} --stats-summary OUT`:", "", "```", cmd, "```", "",
         "Kernels by total time (the largest are the synthetic-data generators of the set-up):", "",
         "| kernel | calls | avg us | min us | max us | total ms |", "|---|---|---|---|---|---|"]
    for r in top:
        L.append(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                 f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                 f"{float(r['TotalDurationNs']) / 1e6:.2f} |")
    L.append("")
    if workload == "c3" and (Path(d) / "fetch").is_dir() and (Path(d) / "write").is_dir():
        L += c3_traffic_lines(d)
    sq = _sq(d, PREFILL_KERNEL, last=PREFILL_LAST_CALLS) if workload == "c4" else {}
    if sq:
        L += ["## SQ counters of the prefill kernel on the last chunk (the sq1 and sq2 passes above)", "",
              f"Median over the run's last {PREFILL_LAST_CALLS} prefill launches (context 7680 tokens + the 512-token "
              "chunk: 119 packed blocks, 1 tail block and 4 or 8 chunk blocks per workgroup, 126 on average).", ""]
        L += _sq_lines(sq, blocks_per_wave=126) + [""]
    (ROOT / "profiles" / f"{name}.md").write_text("\n".join(L))
    print("\n".join(L))


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): the path would shard by sequence "
              "and kv-head, each GPU running this kernel on its share; no figure at several GPUs is produced.",
              file=sys.stderr)
        sys.exit(2)
    if args.summarize:
        summarize(args.summarize)
        return
    if args.stats_summary:
        stats_summary(args.stats_summary, args.workload)
        return
    if args.adapter_summary:
        adapter_summary(args.adapter_summary)
        return
    if args.profile:
        profile_run(args)
        return
    if args.workload == "c3":
        main_c3(args)
        return
    if args.workload == "c4":
        main_c4(args)
        return
    if args.k1c_summary:
        k1c_summary(args.k1c_summary)
        return
    if args.workload == "k1c":
        main_k1c(args)
        return
    if args.workload == "adapter":
        main_adapter(args)
        return
    import numpy as np
    import torch
    from nsn_amd import _dev, _lib, cache, codec, kernels, synthetic

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    lengths, k, v, q = make_workload(dev)

    # ---- encode throughput: all 64-token blocks of K (B*Hkv rows x 512 blocks) in one launch,
    # with the decode factors; per-launch HIP events, median of the launches
    encode_all, enc_bufs = c2_encoder(dev, k)
    for _ in range(3):
        encode_all()
    enc_times = []
    for _ in range(20):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        encode_all()
        e1.record(stream)
        e1.synchronize()
        enc_times.append(e0.elapsed_time(e1))
    assert _dev.read_status(enc_bufs[-1]) == 0
    enc_ms = sorted(enc_times)[len(enc_times) // 2]
    enc_tokens = B * HKV * LMAX
    enc_tok_s = enc_tokens / (enc_ms * 1e-3)
    enc_gbs = enc_tokens * 314 / (enc_ms * 1e-3) / 1e9
    log(f"[bench] encode (+ decode factors): median {enc_ms * 1e3:.1f} us per launch ({enc_tokens} token-heads), "
        f"{enc_tok_s / 1e9:.2f} G tok/s, {enc_gbs:.0f} GB/s algorithmic (314 B/token)")
    del encode_all, enc_bufs

    # ---- packed ragged caches (setup, untimed): see C2Decode
    dec = C2Decode(dev, lengths, k, v, q, kernel=args.kernel)
    kk, vv, seq, max_len = dec.kk, dec.vv, dec.seq, dec.max_len
    split, n_splits, ws, out, ctx, status = dec.split_tokens, dec.n_splits, dec.ws, dec.out, dec.ctx, dec.status
    split_kernel, merge_kernel, step, step_single = dec.split, dec.merge, dec.step, dec.step_single

    log(f"[bench] decode: kernel={args.kernel} split={split} tokens x {n_splits} splits, "
        f"{B * HKV * n_splits} work units; {ROTATE} cache copies in turn; warmup {args.warmup}, steps {args.steps}")
    # Per-kernel durations, independent of --steps: after a fixed warm-up,
    # ROUNDS rounds of back-to-back batches of BATCH launches each -- steps,
    # split-only launches, merge-only launches, and steps over one cache copy
    # -- all enqueued without a host synchronisation, with a HIP event on the
    # launch stream between consecutive batches.  A split-only batch has no
    # merge between its launches, so its per-launch time is the split
    # kernel's own duration plus the dispatch gap; the interleaving keeps all
    # four at one clock.
    for _ in range(SETTLE_STEPS):
        step()
    kinds = (("step", step), ("split", split_kernel), ("merge", merge_kernel), ("single", step_single))
    marks = []
    for _ in range(ROUNDS):
        for name, fn in kinds:
            ev = torch.cuda.Event(enable_timing=True)
            ev.record(stream)
            marks.append((name, ev))
            for _ in range(BATCH):
                fn()
    end = torch.cuda.Event(enable_timing=True)
    end.record(stream)
    torch.cuda.synchronize()
    per = {name: [] for name, _ in kinds}
    for i, (name, ev) in enumerate(marks):
        nxt = marks[i + 1][1] if i + 1 < len(marks) else end
        per[name].append(ev.elapsed_time(nxt) / BATCH)
    # The timed region follows the rounds, so that it measures a decode loop
    # in service rather than the first steps after the set-up (5 warm-up
    # steps right after it measured 76 us per step against 70 in the
    # rounds): `warmup` steps, a synchronisation, then exactly `steps` steps,
    # nothing else on the stream.
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps
    mean = lambda xs: sum(xs) / len(xs)
    ms_split, ms_merge = mean(per["split"]), mean(per["merge"])
    ms_step_rounds, ms_single = mean(per["step"]), mean(per["single"])
    split_ts = sorted(per["split"])
    consistent = ms_split + ms_merge <= ms_step_rounds * 1.02
    st_val = _dev.read_status(status)
    assert st_val == 0, f"status word {st_val:#x}"
    nbytes = algorithmic_bytes(lengths, 3)
    achieved = nbytes / (ms_split * 1e-3) / 1e9
    log(f"[bench] step {ms_step * 1e3:.1f} us (timed region, {ROTATE} copies in turn); rounds of {BATCH}: "
        f"step {ms_step_rounds * 1e3:.1f} us, split {ms_split * 1e3:.1f} us (median of rounds "
        f"{split_ts[len(split_ts) // 2] * 1e3:.1f}), merge {ms_merge * 1e3:.1f} us, one-copy step "
        f"{ms_single * 1e3:.1f} us; split + merge <= step: {consistent}; {nbytes / 1e6:.1f} MB algorithmic -> "
        f"{achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%} of 8 TB/s)")

    # parity spot check of this step against the exact-order kernel (untimed)
    if args.kernel != "reference":
        # exact-order kernel with fp32 reconstructions (no rounding of K/V): the fp32 reference math
        _, ref_ctx = kernels.decode_attention(q, kk, vv, seq, max_seq_len=max_len, kernel="reference",
                                              kv_round_dtype=torch.float32)
        err = (ctx - ref_ctx).abs()
        tol = 2e-3 + 1e-2 * ref_ctx.abs()
        log(f"[bench] parity vs exact-order kernel: max abs {float(err.max()):.2e}, within tol: {bool((err <= tol).all())}")

    result = {
        "metric": METRIC, "value": round(ms_step * 1e3, 2), "unit": "µs/step", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": False, "scaling": "weak", "vs_baseline": None, "dtype": "f16x2/f32",
        "data": "synthetic (GPU torch.Generator seed 2; lengths numpy rng 2); 3 copies of the packed cache used in turn",
        "config": {"workload": "C2: fused packed-INT3 K+V decode attention, B=16, 32q/8kv heads, d=128, "
                               "ragged ctx U[16K,32K], fp16 tail < 64", "batch": B, "heads_q": HQ, "heads_kv": HKV,
                   "head_dim": D, "ctx_min": LMIN, "ctx_max": LMAX, "bits": 3, "kernel": args.kernel,
                   "split_tokens": split, "n_splits": n_splits},
        "hbm_gbs": round(achieved, 1),
        "encode_tok_s": round(enc_tok_s, 1),
        "encode_gbs": round(enc_gbs, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic() if args.kernel == "fast" else None,
                     "kernel": f"attn split kernel ({args.kernel})", "algorithmic_bytes": nbytes,
                     "kernel_us": round(ms_split * 1e3, 2), "kernel_us_median": round(split_ts[len(split_ts) // 2] * 1e3, 2),
                     "merge_us": round(ms_merge * 1e3, 2), "step_us_same_rounds": round(ms_step_rounds * 1e3, 2),
                     "split_plus_merge_le_step": consistent,
                     "timing": f"{SETTLE_STEPS} warm-up steps, then {ROUNDS} rounds of back-to-back batches of {BATCH} "
                               "steps / split-only / merge-only / one-copy steps, enqueued without a host sync, HIP "
                               f"events between batches on the launch stream; every batch but the one-copy one "
                               f"turns over {ROTATE} copies of the packed cache"},
        "value_timing": f"after the roofline rounds: {args.warmup} warm-up steps, a host synchronisation, then "
                        f"{args.steps} steps between HIP events on the launch stream, nothing else on it",
        "cache_rotation": {"copies": ROTATE, "bytes_per_copy": nbytes,
                           "note": "value and roofline turn over the copies (no step re-reads the previous step's "
                                   "bytes); single_copy_step_us re-reads one copy every step"},
        "single_copy_step_us": round(ms_single * 1e3, 2),
        "encode_roofline": {"bound": "hbm", "achieved": round(enc_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                            "frac": round(enc_gbs / HBM_PEAK_GBS, 4), "traffic": measured_encode_traffic(),
                            "kernel": "encode (C2 K, fp16 -> INT3 + fp16 metadata + fp32 decode factors)",
                            "algorithmic_bytes": enc_tokens * 314, "kernel_us": round(enc_ms * 1e3, 1)},
    }

    if not args.no_baselines:
        # bridge: V restored to HBM (fp16), then attention reading packed K + dense V
        vfull = torch.empty((B, HKV, max_len, D), dtype=torch.float16, device=dev)

        cap = vv.codes.shape[2]
        lib = _lib.lib()

        def restore_all():
            for b in range(B):
                L = int(lengths[b])
                nb = L // 64
                rc = lib.nsn_restore_blocks(
                    vv.codes[b].data_ptr(), 0, vv.norm[b].data_ptr(), vv.min[b].data_ptr(), vv.scale[b].data_ptr(),
                    HKV, nb, cap, 3, vfull[b].data_ptr(), _lib.DTYPE_F16, max_len, vv.tail[b].data_ptr(),
                    _lib.DTYPE_F16, L - nb * 64, vv.tail.shape[2], status.data_ptr(), stream.cuda_stream)
                assert rc == 0
        vd = kernels.PackedKV(None, None, None, None, None, None, vfull, 3)

        def bridge():
            restore_all()
            kernels.decode_attention(q, kk, vd, seq, max_seq_len=max_len, kernel=args.kernel, split_tokens=split,
                                     workspace=ws, out=out, ctx=ctx, status=status, check=False)
        ms_bridge = timed(bridge, 10, 2, stream)
        del vfull
        # fp16-KV decode: the same kernel over dense fp16 K and V
        kd = kernels.PackedKV(None, None, None, None, None, None, k, 3)
        vdn = kernels.PackedKV(None, None, None, None, None, None, v, 3)

        def dense():
            kernels.decode_attention(q, kd, vdn, seq, max_seq_len=max_len, kernel=args.kernel, split_tokens=split,
                                     workspace=ws, out=out, ctx=ctx, status=status, check=False)
        ms_dense = timed(dense, 20, 3, stream)
        result["comparators"] = {"bridge_us": round(ms_bridge * 1e3, 1), "fp16_kv_us": round(ms_dense * 1e3, 1)}
        log(f"[bench] bridge {ms_bridge * 1e3:.1f} us/step, fp16-KV {ms_dense * 1e3:.1f} us/step")
        result.update(readout_arms(dev))

    if not args.no_cpu:
        log("[bench] CPU baseline (PyTorch-CPU restatement, all threads and one) ...")
        result["cpu_baseline"] = cpu_baseline(kk, vv, q, lengths)
        log(f"[bench] CPU baseline {result['cpu_baseline']['value']:.0f} us/step (scaled)")
    if not args.c2_only:
        # the other BASELINE.json configs at their own shapes, reduced repeat counts
        # (C3: 60 steps; C4: one slot, 32 decode steps), as sub-objects of this line
        del kk, vv, q, ws, k, v, dec
        torch.cuda.empty_cache()
        sub = argparse.Namespace(**vars(args))
        sub.steps, sub.warmup, sub.slots, sub.decode_steps = 60, 500, 1, 32
        r3 = main_c3(sub, emit=False)
        result["c3"] = {"workload": r3["config"]["workload"], "step_us": r3["value"],
                        "split_kernel_us": r3["roofline"]["kernel_us"], "hbm_frac": r3["roofline"]["frac"],
                        "traffic": r3["roofline"]["traffic"],
                        "encode_us": r3["encode_us"], "encode_hbm_frac": r3["encode_roofline"]["frac"],
                        "parity_ok": r3["parity_ok"]}
        torch.cuda.empty_cache()
        r4 = main_c4(sub, emit=False)
        result["c4"] = {"workload": r4["config"]["workload"], "prefill_ms_per_slot": r4["prefill_ms_per_slot"],
                        "prefill_mfma_frac": r4["prefill_roofline"]["frac"],
                        "prefill_kernel_last_chunk_us": r4["prefill_kernel_last_chunk_us"],
                        "prefill_kernel_last_chunk_tflops": r4["prefill_kernel_last_chunk_tflops"],
                        "dense_sdpa_comparator": r4["dense_sdpa_comparator"],
                        "decode_us_per_slot_step": r4["value"], "decode_hbm_frac": r4["roofline"]["frac"]}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
