"""Seeded synthetic K/V/query generators for the benchmark configurations.

The reference publishes no K/V arrays for these shapes (its saved inputs are in
release ZIPs that are not available offline), so every configuration is built
from a stated generator:

* ``kv_tokens``: a unit direction drawn from N(0, I_128) and normalised, times a
  per-token norm drawn from lognormal(0, 1); ``round(0.02 * rows)`` rows chosen
  by the same generator are scaled by 20 (outlier tokens).
* ``heavy_tailed_tokens``: per-channel Student-t (df=3) values times lognormal
  token norms (the 5-bit configuration).

``numpy.random.default_rng(seed)`` drives the small CPU-sized cases.  The
full-size cases draw on the GPU from ``torch.Generator(device='cuda')`` with the
same seed (a different stream of numbers, same distribution), because
generating half a billion fp16 values through numpy would dominate the run.
"""
from __future__ import annotations

import numpy as np

DIM = 128


def kv_tokens(rng, prefix, ntok, dim=DIM, outlier_frac=0.02, outlier_scale=20.0):
    """fp16 array [*prefix, ntok, dim] (see module docstring)."""
    shape = tuple(prefix) + (ntok, dim)
    u = rng.standard_normal(shape)
    u /= np.linalg.norm(u, axis=-1, keepdims=True)
    nrm = rng.lognormal(0.0, 1.0, tuple(prefix) + (ntok, 1))
    rows = int(np.prod(tuple(prefix) + (ntok,)))
    k = int(round(outlier_frac * rows))
    if k:
        idx = rng.choice(rows, size=k, replace=False)
        nrm.reshape(-1)[idx] *= outlier_scale
    return (u * nrm).astype(np.float16)


def heavy_tailed_tokens(rng, prefix, ntok, dim=DIM, df=3.0):
    shape = tuple(prefix) + (ntok, dim)
    x = rng.standard_t(df, shape)
    x /= np.linalg.norm(x, axis=-1, keepdims=True)
    nrm = rng.lognormal(0.0, 1.0, tuple(prefix) + (ntok, 1))
    return (x * nrm).astype(np.float16)


def config0(seed=0):
    """C0: K and V fp16 [32 heads, 64 tokens, 128], seed 0 (K drawn first)."""
    rng = np.random.default_rng(seed)
    k = kv_tokens(rng, (32,), 64)
    v = kv_tokens(rng, (32,), 64)
    return k, v


def ragged_lengths(seed, batch, lo, hi):
    """Per-sequence context lengths uniform in [lo, hi] (inclusive)."""
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=batch).astype(np.int64)


# ------------------------------------------------------------- device side

def kv_tokens_torch(gen, shape, device, outlier_frac=0.02, outlier_scale=20.0, dtype=None):
    """GPU version of ``kv_tokens``: fp16 tensor of ``shape`` [..., T, 128]."""
    import torch
    dtype = dtype or torch.float16
    u = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    u = u / torch.linalg.vector_norm(u, dim=-1, keepdim=True)
    nrm = torch.empty(shape[:-1] + (1,), device=device, dtype=torch.float32)
    nrm.log_normal_(0.0, 1.0, generator=gen)
    rows = nrm.numel()
    k = int(round(outlier_frac * rows))
    if k:
        idx = torch.randperm(rows, generator=gen, device=device)[:k]
        nrm.view(-1)[idx] *= outlier_scale
    return (u * nrm).to(dtype)


def heavy_tailed_torch(gen, shape, device, df=3.0, dtype=None):
    """GPU Student-t(df) channels (as N / sqrt(chi2/df)) times lognormal norms."""
    import torch
    dtype = dtype or torch.float16
    z = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    g = torch.zeros(shape, device=device, dtype=torch.float32)
    for _ in range(int(df)):
        e = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
        g += e * e
    x = z / torch.sqrt(g / df)
    x = x / torch.linalg.vector_norm(x, dim=-1, keepdim=True)
    nrm = torch.empty(shape[:-1] + (1,), device=device, dtype=torch.float32)
    nrm.log_normal_(0.0, 1.0, generator=gen)
    return (x * nrm).to(dtype)


# ------------------------------------------------------ benchmark workloads

# BASELINE.json configs[2] (C2), configs[3] (C3), configs[4] (C4)
C2 = dict(B=16, HQ=32, HKV=8, LMIN=16384, LMAX=32768, bits=3, seed=2)
C3 = dict(B=64, HQ=16, HKV=4, L=8192, bits=5, seed=3)
C4 = dict(B=32, H=16, T=8192, chunk=512, steps=256, seed=4)


def c2_workload(device):
    """C2 on the GPU: ragged lengths (numpy rng 2), K and V [B, Hkv, LMAX, 128]
    fp16 from the outlier-token generator and bf16 queries [B, Hq, 128]
    (torch.Generator seed 2).  Returns (lengths, k, v, q)."""
    import torch
    c = C2
    lengths = [int(x) for x in ragged_lengths(c["seed"], c["B"], c["LMIN"], c["LMAX"])]
    gen = torch.Generator(device=device).manual_seed(c["seed"])
    k = kv_tokens_torch(gen, (c["B"], c["HKV"], c["LMAX"], DIM), device)
    v = kv_tokens_torch(gen, (c["B"], c["HKV"], c["LMAX"], DIM), device)
    q = torch.randn((c["B"], c["HQ"], DIM), generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
    return lengths, k, v, q


def c3_workload(device):
    """C3 on the GPU: K and V heavy-tailed [2, B, Hkv, L, 128] fp16 (K first)
    and bf16 queries [B, Hq, 128] (torch.Generator seed 3)."""
    import torch
    c = C3
    gen = torch.Generator(device=device).manual_seed(c["seed"])
    kv = heavy_tailed_torch(gen, (2, c["B"], c["HKV"], c["L"], DIM), device)
    q = torch.randn((c["B"], c["HQ"], DIM), generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16)
    return kv, q
