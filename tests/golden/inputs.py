"""Input constructions shared by the golden writer and the tests.

Each builder restates how one of the reference's fixtures makes its input
(the reference files are cited per function), so that tests can rebuild the
inputs on any machine and check them against the SHA-256 stored with the
golden outputs.
"""
from __future__ import annotations

import numpy as np
import torch

from nsn_amd import synthetic


def config0_inputs():
    """C0: K, V fp16 [32, 64, 128], numpy default_rng(0)."""
    return synthetic.config0(0)


def core_fixtures():
    """data/validation/qdq-core/check_core.py:24-29 (seed 2026100303)."""
    g = torch.Generator(device="cpu").manual_seed(2026100303)
    x = torch.randn(2, 64, 128, generator=g)
    strided = torch.randn(2, 64, 256, generator=g)[..., ::2]
    zero_rows = x.clone()
    zero_rows[:, ::4, :] = 0
    return {
        "normal": x,
        "zero": torch.zeros_like(x),
        "constant_across_tokens": torch.ones_like(x),
        "zero_rows": zero_rows,
        "norm_dispersion": x * torch.logspace(-3, 3, 64).reshape(1, 64, 1),
        "strided_input": strided,
        "shifted": x + 5,
        "multi_head": torch.randn(2, 3, 64, 128, generator=g),
    }


def pilot_fixture_tensors():
    """experiments/ac08/source/loop_kv_pilot.py:366-377 (torch seed 2026093001)."""
    g = torch.Generator(device="cpu").manual_seed(2026093001)
    out = {}
    for bits in (3, 4, 5):
        out[bits] = [torch.zeros(64, 128), torch.ones(64, 128),
                     torch.randn(128, 64, generator=g).T,
                     torch.randn(2, 64, 128, generator=g)]
    return out


def group_samples():
    """experiments/ac08/source/loop_kv_pk01_cache.py:180-186 (bf16 after .to)."""
    g = torch.Generator(device="cpu").manual_seed(2026093001)
    return [("zeros", torch.zeros(1, 2, 2, 64, 128)),
            ("ones", torch.ones(1, 2, 2, 64, 128)),
            ("transposed", torch.randn(1, 2, 2, 128, 64, generator=g).transpose(-1, -2))]


def heavy_tailed_blocks():
    """Eight 5-bit-config blocks: Student-t(3) channels x lognormal norms, rng(3)."""
    rng = np.random.default_rng(3)
    return synthetic.heavy_tailed_tokens(rng, (8,), 64)


# ---------------------------------------------------------------- VF01 fixtures

def _bf16_bits(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def query_bits(kind, h, index=0):
    """Decode queries of experiments/ac08/source/loop_kv_qk01_contract.py:31-40 (bf16 bits)."""
    shape = (1, h, 1, 128)
    if kind == "gaussian":
        a = np.random.default_rng(2026100104 + index).standard_normal(shape).astype(np.float32)
    elif kind == "one_hot":
        a = np.zeros(shape, np.float32)
        for head in range(h):
            a[0, head, 0, head % 128] = 1
    elif kind == "alternating":
        a = np.broadcast_to(np.where(np.arange(128) % 2 == 0, 1.0, -1.0), shape).astype(np.float32)
    elif kind == "zero":
        a = np.zeros(shape, np.float32)
    else:
        raise ValueError(kind)
    return np.ascontiguousarray(_bf16_bits(a))


def pack3_bits(codes):
    flat = np.asarray(codes, np.uint8).reshape(-1)
    b = ((flat[:, None] >> np.arange(3, dtype=np.uint8)) & 1).reshape(-1)
    return np.packbits(b, bitorder="little")


def vf01_fixture(compressed, length, pattern, h=2):
    """Normal fixtures of experiments/ac08/source/loop_kv_vf01_contract.py:81-96.

    Returns numpy arrays: q/k_tail/v_tail as bf16 bits (uint16), codes u8
    [1,h,n,3072], headers u8 [1,h,n,12], meta0 f16 [1,h,n,64,1], meta1/meta2
    f16 [1,h,n,1,128].
    """
    import struct
    c, total = compressed, length
    out = {"q": query_bits("one_hot" if pattern == "constant" else "alternating", h)}
    for side in ("k", "v"):
        tail = _bf16_bits(np.linspace(-0.5, 0.5, h * (total - c) * 128, dtype=np.float32)
                          .reshape(1, h, total - c, 128))
        if pattern == "zero":
            tail.fill(0)
        if pattern == "constant":
            tail = _bf16_bits(np.full(tail.shape, 0.5, np.float32))
        out[side + "_tail"] = tail
        if c:
            nb = c // 64
            codes = (np.arange(h * c * 128) % 8).astype(np.uint8)
            n = np.ones((1, h, nb, 64, 1), np.float16)
            m = np.full((1, h, nb, 1, 128), -3, np.float16)
            s = np.ones_like(m)
            if pattern == "zero":
                n.fill(0)
            if pattern == "constant":
                n.fill(4)
                m.fill(1)
                s.fill(0)
            if pattern == "partial_zero_norm":
                n.reshape(-1)[::2] = 0
            hdr = b"".join(struct.pack("<QHBB", i * 64, 64, 3, 0) for _ in range(h) for i in range(nb))
            out[side + "_codes"] = pack3_bits(codes).reshape(1, h, nb, 3072)
            out[side + "_headers"] = np.frombuffer(hdr, np.uint8).reshape(1, h, nb, 12).copy()
            out[side + "_meta0"] = n
            out[side + "_meta1"] = m
            out[side + "_meta2"] = s
    return out


def array_hash(a):
    """experiments/ac08/source/loop_kv_af01_contract.py:20."""
    import hashlib
    return hashlib.sha256(str((a.shape, str(a.dtype))).encode() + a.tobytes()).hexdigest()


# The reference's 24 rejection kinds, in its plan order
# (experiments/ac08/source/loop_kv_vf01_inputs.json "negative_fixtures").
NEGATIVE_KINDS = (
    "q_nan", "q_inf", "k_tail_nan", "v_tail_inf", "k_norm_nan", "k_min_nan", "k_scale_inf", "v_norm_nan",
    "v_min_nan", "v_scale_nan", "v_norm_inf", "v_zero_norm_nan_direction", "q_dtype", "q_shape", "k_codes_dtype",
    "v_codes_dtype", "v_codes_short", "v_meta_shape", "v_tail_noncontiguous", "kv_length_mismatch",
    "k_header_position", "v_header_position", "empty_sequence", "score_overflow")

# kind -> (field, value, flat position) for the one-value nonfinite defects
_NONFINITE = {
    "q_nan": ("q", np.nan, 0), "q_inf": ("q", np.inf, 0), "k_tail_nan": ("k_tail", np.nan, 0),
    "v_tail_inf": ("v_tail", np.inf, -1), "k_norm_nan": ("k_meta0", np.nan, 0), "k_min_nan": ("k_meta1", np.nan, 0),
    "k_scale_inf": ("k_meta2", np.inf, 0), "v_norm_nan": ("v_meta0", np.nan, -1),
    "v_min_nan": ("v_meta1", np.nan, 0), "v_scale_nan": ("v_meta2", np.nan, 0), "v_norm_inf": ("v_meta0", np.inf, 0),
}


def vf01_negative(kind):
    """One defect planted in the 64 + 1 token mixed-codes fixture
    (experiments/ac08/source/loop_kv_vf01_contract.py:98-120).

    Returns (arrays, mutation): ``mutation`` names a defect made after the
    transfer to the device (a noncontiguous V tail), else None.
    """
    a = vf01_fixture(64, 65, "mixed_codes")
    mutation = None
    if kind in _NONFINITE:
        field, value, pos = _NONFINITE[kind]
        x = a[field]
        x.reshape(-1)[pos] = _bf16_bits(np.array([value], np.float32))[0] if x.dtype == np.uint16 else value
    elif kind == "v_zero_norm_nan_direction":       # every norm zero, one direction component NaN
        a["v_meta0"].fill(0)
        a["v_meta1"].reshape(-1)[0] = np.nan
    elif kind == "q_dtype":                          # fp32 values instead of bf16 bit patterns
        a["q"] = (a["q"].astype(np.uint32) << 16).view(np.float32)
    elif kind == "q_shape":
        a["q"] = a["q"][..., :127].copy()
    elif kind in ("k_codes_dtype", "v_codes_dtype"):
        a[kind[0] + "_codes"] = a[kind[0] + "_codes"].astype(np.int16)
    elif kind == "v_codes_short":
        a["v_codes"] = a["v_codes"][..., :-1].copy()
    elif kind == "v_meta_shape":
        a["v_meta1"] = a["v_meta1"][..., :127].copy()
    elif kind == "v_tail_noncontiguous":
        mutation = kind
    elif kind == "kv_length_mismatch":
        a["v_tail"] = np.concatenate([a["v_tail"], a["v_tail"]], axis=2)
    elif kind in ("k_header_position", "v_header_position"):
        a[kind[0] + "_headers"].reshape(-1)[0] = 1
    elif kind == "empty_sequence":
        a = {"q": a["q"], "k_tail": a["k_tail"][:, :, :0].copy(), "v_tail": a["v_tail"][:, :, :0].copy()}
    elif kind == "score_overflow":                   # q . k = 128 * 2**240 overflows fp32
        a = vf01_fixture(0, 17, "tail_only")
        for name in ("q", "k_tail"):
            a[name] = np.full(a[name].shape, 0x7B80, np.uint16)      # bf16 2**120
    else:
        raise ValueError("unknown negative fixture " + kind)
    return a, mutation
