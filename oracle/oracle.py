"""CPU oracle for the NSN packed-KV hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import this module, and only as the checker: the product path
(``nsn_amd``) never imports it and has no CPU fallback.

Two layers:

* ``libnsn_oracle.so`` (``oracle/nsn_oracle.c``): bit-exact C restatement of
  the reference's torch-CPU arithmetic for ``nsn_encode`` / ``nsn_decode`` /
  ``nsn_int3_qdq`` and the LSB-first bitstream (reference
  ``experiments/ac08/source/loop_kv_pilot.py:171-225``,
  ``papers/nsn-integrated/code/nsn_int3_core.py:11-21``).
* numpy: the 3-bit ``pack3``/``unpack3`` restatement through ``np.packbits``
  (reference ``experiments/ac08/source/loop_kv_qk01_contract.py:129-136``),
  the 12-byte block headers (``loop_kv_pk01_cache.py:35``), and float64
  attention oracles (softmax readout ``loop_kv_af01_contract.py:28-29``;
  QK scores ``loop_kv_qk01_contract.py:41-44``; decode attention over the
  restored K/V ``loop_kv_vf01_kernel.py:56-113`` + ``loop_kv_af01_kernel.py:70-82``;
  GQA head map ``kh = h // G``, ``experiments/nb06/source/loop_kv_nb06_kernel.py:56``).

Pinning (what fixes each function; the tests live in tests/test_oracle.py):

* encode/decode/qdq: golden vectors written from the reference's own CPU
  functions (tests/golden/make_goldens.py), the encoder invariants (code range,
  per-channel min/max codes), and torch.linalg.vector_norm itself.
* pack/unpack: closed form (three independent constructions agree), the
  reference's KATs (``(arange(n)*5+3)%8``, exhaustive byte pairs) and the
  SHA-256 input hashes saved by the reference's VF01 run.
* attention oracles: closed-form fixtures (uniform / dominant / cancel / zero
  softmax, one-hot queries), split invariance of the merge, and the GQA
  repeat invariant.
* chunked-prefill oracle: row i equals the decode oracle over context +
  chunk[:i + 1]; constant keys give prefix means (closed form); planted
  off-by-one causal masks fail both.
"""
from __future__ import annotations

import ctypes
import os
import struct
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libnsn_oracle.so"
BLOCK = 64
DIM = 128
EPS = np.float32(1e-12)
SCALE = 0.08838834764831845  # 1/sqrt(128), loop_kv_vf01_kernel.py:90

ERR_NONFINITE_INPUT = 1
ERR_META_NONFINITE = 2
ERR_META_UNDERFLOW = 4

_lib = None


def build():
    """Compile the C oracle (gcc via oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.oracle_nsn_encode.argtypes = [P, I64, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P, P, P, P]
        L.oracle_nsn_encode.restype = ctypes.c_int
        L.oracle_nsn_decode.argtypes = [P, P, P, P, I64, P]
        L.oracle_nsn_decode.restype = None
        L.oracle_vector_norm.argtypes = [P, I64, ctypes.c_int, ctypes.c_int, P]
        L.oracle_vector_norm.restype = None
        L.oracle_pack_codes.argtypes = [P, I64, ctypes.c_int, P]
        L.oracle_pack_codes.restype = I64
        L.oracle_unpack_codes.argtypes = [P, I64, ctypes.c_int, P]
        L.oracle_unpack_codes.restype = None
        L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- dtype bits

def bf16_bits(x):
    """fp32 -> bf16 bit pattern, round to nearest even, NaN kept NaN."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    u = a.view(np.uint32)
    r = ((u.astype(np.uint64) + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(a)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def from_bf16_bits(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f16_bits(x):
    """fp32 -> fp16 bit pattern, round to nearest even (numpy's cast is RNE)."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def from_f16_bits(b):
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def cast_bits(y, dtype):
    """Round fp32 values to ``dtype`` ('float16'|'bfloat16'|'float32'); return raw bits."""
    if dtype == "float16":
        return f16_bits(y)
    if dtype == "bfloat16":
        return bf16_bits(y)
    if dtype == "float32":
        return np.ascontiguousarray(y, np.float32).view(np.uint32)
    raise ValueError(dtype)


# ----------------------------------------------------------------- NSN codec

NORM_LANES8 = 0      # contiguous rows: 8-lane fma accumulators, lanes summed in order
NORM_SEQUENTIAL = 1  # rows with last-dim stride != 1: one fma chain


def vector_norm(rows, order=NORM_LANES8):
    """torch-CPU ``vector_norm(dim=-1)`` over fp32 rows, in the given order."""
    r = np.ascontiguousarray(rows, np.float32)
    out = np.empty(r.shape[:-1], np.float32)
    lib().oracle_vector_norm(_ptr(r), r.size // r.shape[-1], r.shape[-1], order, _ptr(out))
    return out


def nsn_encode(x_f32, bits, zero_flat_scale=True, order=NORM_LANES8):
    """Restates ``nsn_encode`` (loop_kv_pilot.py:195-213).

    ``x_f32``: fp32 values of shape [..., 64, 128] (the ``x.float()`` of the
    reference).  Returns ``(q u8 [...,64,128], n16 [...,64,1], m16 [...,1,128],
    s16 [...,1,128], err)`` where the metadata are fp16 bit patterns (uint16)
    and ``err`` ORs ERR_* bits the reference would raise on.
    """
    a = np.ascontiguousarray(x_f32, np.float32)
    assert a.shape[-2:] == (BLOCK, DIM)
    lead = a.shape[:-2]
    nb = int(np.prod(lead)) if lead else 1
    q = np.empty(a.shape, np.uint8)
    n16 = np.empty(lead + (BLOCK, 1), np.uint16)
    m16 = np.empty(lead + (1, DIM), np.uint16)
    s16 = np.empty(lead + (1, DIM), np.uint16)
    err = lib().oracle_nsn_encode(_ptr(a), nb, bits, 1 if zero_flat_scale else 0, order,
                                  _ptr(q), _ptr(n16), _ptr(m16), _ptr(s16), None, None, None)
    return q, n16, m16, s16, err


def nsn_encode_f32_metas(x_f32, bits, order=NORM_LANES8):
    """As nsn_encode, also returning the unrounded fp32 n, m, s."""
    a = np.ascontiguousarray(x_f32, np.float32)
    lead = a.shape[:-2]
    nb = int(np.prod(lead)) if lead else 1
    q = np.empty(a.shape, np.uint8)
    n16 = np.empty(lead + (BLOCK, 1), np.uint16)
    m16 = np.empty(lead + (1, DIM), np.uint16)
    s16 = np.empty(lead + (1, DIM), np.uint16)
    n32 = np.empty(n16.shape, np.float32)
    m32 = np.empty(m16.shape, np.float32)
    s32 = np.empty(s16.shape, np.float32)
    err = lib().oracle_nsn_encode(_ptr(a), nb, bits, 1, order, _ptr(q), _ptr(n16), _ptr(m16), _ptr(s16),
                                  _ptr(n32), _ptr(m32), _ptr(s32))
    return q, (n16, m16, s16), (n32, m32, s32), err


def nsn_decode_f32(q, n16, m16, s16):
    """Restates ``nsn_decode`` before its final cast (loop_kv_pilot.py:216-225)."""
    q = np.ascontiguousarray(q, np.uint8)
    assert q.shape[-2:] == (BLOCK, DIM)
    nb = q.size // (BLOCK * DIM)
    n16 = np.ascontiguousarray(n16, np.uint16)
    m16 = np.ascontiguousarray(m16, np.uint16)
    s16 = np.ascontiguousarray(s16, np.uint16)
    assert n16.size == nb * BLOCK and m16.size == nb * DIM and s16.size == nb * DIM
    y = np.empty(q.shape, np.float32)
    lib().oracle_nsn_decode(_ptr(q), _ptr(n16), _ptr(m16), _ptr(s16), nb, _ptr(y))
    return y


def decode_factors(q, n16, m16, s16):
    """f_t = n_t / max(|m + s*q_t|, 1e-12) in fp32 (the norm in nsn_decode's
    order, unfused m + s*q, IEEE division; 0 where n == 0): the per-token factor
    that turns m + s*q_t into the row nsn_decode reconstructs (before rounding).
    Pinned by tests/test_oracle.py against nsn_decode itself."""
    q = np.ascontiguousarray(q, np.uint8)
    lead = q.shape[:-2]
    m = from_f16_bits(m16).reshape(lead + (1, DIM))
    s = from_f16_bits(s16).reshape(lead + (1, DIM))
    n = from_f16_bits(n16).reshape(lead + (BLOCK,))
    d = (m + (s * q.astype(np.float32)).astype(np.float32)).astype(np.float32)
    den = vector_norm(d)
    den = np.where(den > EPS, den, EPS).astype(np.float32)
    f = (n / den).astype(np.float32)
    return np.where(n == 0, np.float32(0), f).astype(np.float32)


def nsn_decode(q, n16, m16, s16, dtype):
    """``nsn_decode(q, metas, dtype)``; returns raw bits of ``dtype``."""
    return cast_bits(nsn_decode_f32(q, n16, m16, s16), dtype)


def nsn_int3_qdq(x_f32, dtype, order=NORM_LANES8):
    """``nsn_int3_qdq`` (nsn_int3_core.py:11-21): encode(3) -> fp16 metas -> decode -> cast."""
    q, n16, m16, s16, _ = nsn_encode(x_f32, 3, zero_flat_scale=False, order=order)
    return nsn_decode(q, n16, m16, s16, dtype)


def nsn_qdq(x_f32, bits, dtype, order=NORM_LANES8):
    q, n16, m16, s16, _ = nsn_encode(x_f32, bits, order=order)
    return nsn_decode(q, n16, m16, s16, dtype)


# ------------------------------------------------------------ bitstream/pack

def pack_codes(codes, bits):
    """LSB-first bitstream (pack_codes, loop_kv_pilot.py:171-181) -> uint8 array."""
    a = np.ascontiguousarray(codes, np.uint8).reshape(-1)
    assert np.all(a < (1 << bits))
    out = np.empty((a.size * bits + 7) // 8, np.uint8)
    lib().oracle_pack_codes(_ptr(a), a.size, bits, _ptr(out))
    return out


def unpack_codes(payload, count, bits):
    p = np.ascontiguousarray(payload, np.uint8).reshape(-1)
    assert p.size == (count * bits + 7) // 8
    out = np.empty(count, np.uint8)
    lib().oracle_unpack_codes(_ptr(p), count, bits, _ptr(out))
    return out


def pack_bits_numpy(codes, bits):
    """Independent construction via np.packbits(bitorder='little')."""
    flat = np.ascontiguousarray(codes, np.uint8).reshape(-1)
    b = ((flat[:, None] >> np.arange(bits, dtype=np.uint8)) & 1).reshape(-1)
    return np.packbits(b, bitorder="little")


def unpack_bits_numpy(payload, count, bits):
    b = np.unpackbits(np.asarray(payload, np.uint8).reshape(-1), bitorder="little")
    b = b[: count * bits].reshape(count, bits)
    return (b @ (1 << np.arange(bits))).astype(np.uint8)


def headers(outer, nblocks, start, bits):
    """12-byte ``<QHBB`` block headers (loop_kv_pk01_cache.py:35): [outer, nblocks, 12]."""
    one = b"".join(struct.pack("<QHBB", start + i * 64, 64, bits, 0) for i in range(nblocks))
    return np.frombuffer(one * outer, np.uint8).reshape(outer, nblocks, 12).copy()


# ------------------------------------------------------------ attention (f64)

def softmax64(x):
    x = np.asarray(x, np.float64)
    p = np.exp(x - x.max(-1, keepdims=True))
    return p / p.sum(-1, keepdims=True)


def decode_attention64(q, k, v, scale=SCALE):
    """fp64 single-query attention.

    q: [B, Hq, 128]; k, v: [B, Hkv, T, 128] (any float); Hq = G * Hkv, q-head h
    reads kv-head h // G.  Returns (ctx [B,Hq,128] float64, p [B,Hq,T]).
    One matrix product per (sequence, kv-head) serves its G query heads.
    """
    q = np.asarray(q, np.float64)
    B, Hq, D = q.shape
    Hkv, T = k.shape[1], k.shape[2]
    G = Hq // Hkv
    ctx = np.empty((B, Hq, D))
    p = np.empty((B, Hq, T))
    for b in range(B):
        for kv in range(Hkv):
            kk = np.asarray(k[b, kv], np.float64)
            vv = np.asarray(v[b, kv], np.float64)
            hs = slice(kv * G, (kv + 1) * G)
            pw = softmax64((q[b, hs] @ kk.T) * scale)            # [G, T]
            p[b, hs] = pw
            ctx[b, hs] = pw @ vv
    return ctx, p


def prefill_attention64(q, kctx, vctx, kch, vch, scale=SCALE, causal_shift=0):
    """fp64 chunked-prefill attention of one sequence.

    q [Hq, n, 128]; kctx / vctx [Hkv, L, 128] the context (packed blocks
    restored, then the tail); kch / vch [Hkv, n, 128] the chunk's own K/V.
    Chunk query i attends all L context tokens and chunk tokens 0 .. i
    (0 .. i + causal_shift: a nonzero shift exists only to plant an off-by-one
    mask in the oracle's own tests).  q-head h reads kv-head h // G.  Returns
    [Hq, n, 128] float64.  The reference attends a chunk over its
    materialised cache plus the chunk (loop_kv_pk01_cache.py:87-106) with the
    model's causal attention; row i is the single-query attention of q[:, i]
    over context + chunk[:i + 1] (decode_attention64), which
    tests/test_oracle.py checks row by row.
    """
    q = np.asarray(q, np.float64)
    Hq, n, D = q.shape
    Hkv, L = kctx.shape[0], kctx.shape[1]
    G = Hq // Hkv
    hidden = np.arange(n)[None, :] > np.arange(n)[:, None] + causal_shift   # [query i, chunk token j]
    out = np.empty((Hq, n, D))
    for kv in range(Hkv):
        k = np.concatenate([np.asarray(kctx[kv], np.float64), np.asarray(kch[kv], np.float64)])
        v = np.concatenate([np.asarray(vctx[kv], np.float64), np.asarray(vch[kv], np.float64)])
        for h in range(kv * G, (kv + 1) * G):
            s = (q[h] @ k.T) * scale                                         # [n, L + n]
            s[:, L:][hidden] = -np.inf
            out[h] = softmax64(s) @ v
    return out


def readout64(scores, v, groups=1):
    """Softmax-weighted V given fp32 logits (the AF01 FULL=False readout).

    scores: [B, Hq, T]; v: [B, Hkv, T, 128].
    """
    p = softmax64(scores)
    vv = np.repeat(np.asarray(v, np.float64), groups, axis=1)
    return np.einsum("bht,bhtd->bhd", p, vv)


def restore_blocks_f32(codes_packed, n16, m16, s16, bits):
    """Unpack + nsn_decode (before cast) of packed blocks [..., nbytes]."""
    cp = np.ascontiguousarray(codes_packed, np.uint8)
    lead = cp.shape[:-1]
    nb = int(np.prod(lead)) if lead else 1
    q = unpack_codes(cp.reshape(-1), nb * BLOCK * DIM, bits).reshape(lead + (BLOCK, DIM))
    return nsn_decode_f32(q, n16.reshape(lead + (BLOCK, 1)), m16.reshape(lead + (1, DIM)),
                          s16.reshape(lead + (1, DIM)))


def kscore64(q, code, mins, steps, eff_norm, n_kv, head_dim):
    """fp64 K-score oracle of the K1c component (reference
    ``experiments/kernels/phase_k1c_triton_fused_kernel.py``: dequant
    ``code * step + min`` (:112-113, :240-241), per-token ``eff_norm`` (:104-108,
    :244-247), scores ``q . k / sqrt(D)`` with the GQA map ``hkv = h // (Hq/Hkv)``
    (:150-164, :230)).

    q [B, Hq, D]; code [B, T, Hkv*D] (codes, or K itself with mins = None);
    mins / steps [B, Hkv*D] or None; eff_norm [B, Hkv, T] or None.
    Returns float64 scores [B, Hq, T].  Pinned in tests/test_oracle.py by
    brute-force loops, closed forms (zero codes, one-hot queries) and the GQA
    repeat invariant."""
    q = np.asarray(q, np.float64)
    B, Hq, D = q.shape
    c = np.asarray(code, np.float64)
    T = c.shape[1]
    k = c if mins is None else c * np.asarray(steps, np.float64)[:, None, :] + np.asarray(mins, np.float64)[:, None, :]
    k = k.reshape(B, T, n_kv, head_dim)
    G = Hq // n_kv
    qx = q.reshape(B, n_kv, G, D)
    s = np.einsum("bngd,btnd->bngt", qx, k) / np.sqrt(head_dim)
    if eff_norm is not None:
        s = s * np.asarray(eff_norm, np.float64)[:, :, None, :]
    return s.reshape(B, Hq, T)
