"""Pins the CPU oracle (oracle/) before anything is checked against it.

Every oracle function is checked against at least one of: golden vectors
written from the reference's own functions (tests/golden/), the reference's
KATs and saved input hashes, torch itself, or a closed form -- chosen so a
plausible mistake (wrong norm order, MSB-first packing, a dropped fp16 round,
a transposed GQA map) fails.  CPU only.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.golden import inputs as gi

GOLDEN = Path(__file__).resolve().parent / "golden"


def sha(b):
    return hashlib.sha256(b).hexdigest()


def order_of(stride_last):
    return O.NORM_LANES8 if int(stride_last) == 1 else O.NORM_SEQUENTIAL


# ------------------------------------------------------------- torch's norm

def test_vector_norm_matches_torch_contiguous_rows():
    g = torch.Generator().manual_seed(11)
    a = torch.randn(20000, 128, generator=g) * torch.exp(torch.randn(20000, 1, generator=g) * 3)
    ref = torch.linalg.vector_norm(a, dim=-1).numpy()
    got = O.vector_norm(a.numpy(), O.NORM_LANES8)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))
    # the other order disagrees on a large fraction of rows: the test discriminates
    other = O.vector_norm(a.numpy(), O.NORM_SEQUENTIAL)
    assert (other != ref).mean() > 0.1


def test_vector_norm_matches_torch_strided_rows():
    g = torch.Generator().manual_seed(12)
    a = torch.randn(300, 128, 64, generator=g).transpose(-1, -2)   # last-dim stride 64
    ref = torch.linalg.vector_norm(a, dim=-1).numpy()
    got = O.vector_norm(a.contiguous().numpy(), O.NORM_SEQUENTIAL)
    assert np.array_equal(ref.view(np.uint32), got.view(np.uint32))


def test_f16_conversion_matches_numpy_everywhere_interesting():
    lib = O.lib()
    vals = np.concatenate([
        np.array([0.0, -0.0, 1e-8, 2.98e-8, 5.96e-8, 6.1e-5, 65504.0, 65519.99, 65520.0, 1e5, np.inf, -np.inf], np.float32),
        np.random.default_rng(0).standard_normal(20000).astype(np.float32) * np.float32(1e-3),
        (np.arange(1 << 16, dtype=np.uint32) << 13).view(np.float32)[:60000] * np.float32(1.0000001),
    ])
    with np.errstate(over="ignore"):
        want = vals.astype(np.float16).view(np.uint16)
    got = np.array([lib.oracle_f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, want)


# ------------------------------------------------------------- golden: C0

def test_c0_golden_encode_and_qdq(golden):
    G = golden("c0.npz")
    k, v = gi.config0_inputs()
    assert sha(k.tobytes()) == str(G["k_sha256"]) and sha(v.tobytes()) == str(G["v_sha256"])
    for name, x in (("k", k), ("v", v)):
        q, n16, m16, s16, err = O.nsn_encode(x.astype(np.float32), 3)
        assert err == 0
        assert np.array_equal(O.pack_codes(q, 3).reshape(32, 3072), G[name + "_codes"])
        assert np.array_equal(n16.reshape(32, 64), G[name + "_norm"])
        assert np.array_equal(m16.reshape(32, 128), G[name + "_min"])
        assert np.array_equal(s16.reshape(32, 128), G[name + "_scale"])
        assert np.array_equal(O.headers(32, 1, 0, 3).reshape(32, 12), G[name + "_headers"])
        y = O.nsn_int3_qdq(x.astype(np.float32), "float16")
        assert np.array_equal(y, G[name + "_qdq"])


def test_c0_golden_discriminates_a_wrong_norm_order(golden):
    """Planted mistake: the sequential order must NOT reproduce contiguous goldens."""
    G = golden("c0.npz")
    k, _ = gi.config0_inputs()
    y = O.nsn_int3_qdq(k.astype(np.float32), "float16", order=O.NORM_SEQUENTIAL)
    assert not np.array_equal(y, G["k_qdq"])


# --------------------------------------------------- golden: qdq-core fixtures

@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_core_fixtures(golden, dtype):
    G = golden("core.npz")
    for name, x in gi.core_fixtures().items():
        a = x.to(getattr(torch, dtype))
        key = f"{name}|{dtype}|"
        raw = a.contiguous().view(torch.uint8).numpy().tobytes()
        assert sha(raw) == str(G[key + "in_sha256"]), name
        order = order_of(G[key + "in_stride_last"])
        xf = a.float().contiguous().numpy()
        q, n16, m16, s16, err = O.nsn_encode(xf, 3, order=order)
        assert err == 0
        assert np.array_equal(O.pack_codes(q, 3), G[key + "codes"]), name
        assert np.array_equal(n16.reshape(-1), G[key + "norm"].reshape(-1)), name
        assert np.array_equal(m16.reshape(-1), G[key + "min"].reshape(-1)), name
        assert np.array_equal(s16.reshape(-1), G[key + "scale"].reshape(-1)), name
        y = O.nsn_int3_qdq(xf, dtype, order=order)
        assert np.array_equal(y.view(np.uint8).reshape(-1), G[key + "out"].reshape(-1)), name


# ------------------------------------------- golden: codec fixtures, 3/4/5 bit

def test_pilot_codec_fixtures(golden):
    G = golden("codec.npz")
    for bits, tensors in gi.pilot_fixture_tensors().items():
        for i, t in enumerate(tensors):
            key = f"b{bits}|t{i}|"
            assert sha(t.contiguous().numpy().tobytes()) == str(G[key + "in_sha256"])
            order = order_of(G[key + "in_stride_last"])
            q, n16, m16, s16, err = O.nsn_encode(t.contiguous().numpy(), bits, order=order)
            assert err == 0
            assert np.array_equal(O.pack_codes(q, bits), G[key + "codes"]), key
            assert np.array_equal(n16.reshape(-1), G[key + "norm"].reshape(-1)), key
            assert np.array_equal(m16.reshape(-1), G[key + "min"].reshape(-1)), key
            assert np.array_equal(s16.reshape(-1), G[key + "scale"].reshape(-1)), key
            y = O.nsn_decode(q, n16, m16, s16, "float32")
            assert np.array_equal(y.reshape(-1), G[key + "decoded"].reshape(-1)), key


def test_heavy_tailed_4_and_5_bit(golden):
    G = golden("heavy.npz")
    x = gi.heavy_tailed_blocks()
    assert sha(x.tobytes()) == str(G["in_sha256"])
    for bits in (4, 5):
        q, n16, m16, s16, err = O.nsn_encode(x.astype(np.float32), bits)
        assert err == 0
        assert np.array_equal(O.pack_codes(q, bits), G[f"b{bits}|codes"])
        assert np.array_equal(n16.reshape(-1), G[f"b{bits}|norm"].reshape(-1))
        assert np.array_equal(m16.reshape(-1), G[f"b{bits}|min"].reshape(-1))
        assert np.array_equal(s16.reshape(-1), G[f"b{bits}|scale"].reshape(-1))
        assert np.array_equal(O.nsn_decode(q, n16, m16, s16, "float16").reshape(-1),
                              G[f"b{bits}|qdq"].reshape(-1))


def test_group_codec_and_real_blocks(golden):
    G = golden("group.npz")
    samples = dict(gi.group_samples())
    for name in ("K_00", "V_43"):
        bits = G[f"real|{name}|input"]
        samples["real_" + name] = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).reshape(1, 8, 1, 64, 128)
    for name, x in samples.items():
        x = x.to(torch.bfloat16)
        key = f"group|{name}|"
        assert sha(x.contiguous().view(torch.int16).numpy().tobytes()) == str(G[key + "in_sha256"])
        order = order_of(G[key + "in_stride_last"])
        xf = x.float().contiguous().numpy()
        q, n16, m16, s16, err = O.nsn_encode(xf, 3, order=order)
        assert err == 0
        lead = xf.shape[:-2]
        assert np.array_equal(O.pack_codes(q, 3).reshape(lead + (3072,)), G[key + "codes"]), name
        assert np.array_equal(n16.reshape(-1), G[key + "norm"].reshape(-1)), name
        assert np.array_equal(m16.reshape(-1), G[key + "min"].reshape(-1)), name
        assert np.array_equal(s16.reshape(-1), G[key + "scale"].reshape(-1)), name
        assert np.array_equal(O.headers(int(np.prod(lead[:-1])), lead[-1], 0, 3).reshape(-1),
                              G[key + "headers"].reshape(-1))
        y = O.nsn_decode(q, n16, m16, s16, "bfloat16")
        assert np.array_equal(y.reshape(-1), G[key + "restored"].reshape(-1)), name


def test_decode_factors_reproduce_nsn_decode():
    """f_t * (m + s*q) equals nsn_decode's n * ((m + s*q) / den) to within 2 ulp,
    and exactly where the reference's quotient is exact (zero rows, n == 0)."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((8, 64, 128)) * rng.lognormal(0, 1, (8, 64, 1))).astype(np.float32)
    x[0, 3] = 0.0
    q, n16, m16, s16, err = O.nsn_encode(x, 3)
    assert err == 0
    f = O.decode_factors(q, n16, m16, s16)
    assert f[0, 3] == 0.0
    y = O.nsn_decode_f32(q, n16, m16, s16)
    d = (O.from_f16_bits(m16) + (O.from_f16_bits(s16) * q.astype(np.float32)).astype(np.float32)).astype(np.float32)
    approx = (f[..., None] * d).astype(np.float32)
    ulp = np.spacing(np.abs(y).astype(np.float32))
    assert np.all(np.abs(approx - y) <= 2 * ulp + 1e-30)
    # planted mistake: dropping the norm (f = n) is far off
    assert not np.allclose(O.from_f16_bits(n16).reshape(8, 64, 1) * d, y, rtol=1e-3)


# ------------------------------------------------------------ encoder errors

def test_encode_error_conditions():
    x = np.full((64, 128), 1e5, np.float32)          # loop_kv_pilot.py:391-395
    assert O.nsn_encode(x, 3)[4] & O.ERR_META_NONFINITE
    x = np.random.default_rng(0).standard_normal((64, 128)).astype(np.float32)
    x[3, 4] = np.nan
    assert O.nsn_encode(x, 3)[4] & O.ERR_NONFINITE_INPUT
    x = np.zeros((64, 128), np.float32)
    x[:, 0] = 1e-9                                   # norm 1e-9 underflows fp16
    assert O.nsn_encode(x, 3)[4] & O.ERR_META_UNDERFLOW


def test_encoder_invariants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((16, 64, 128)).astype(np.float32) * rng.lognormal(0, 1, (16, 64, 1)).astype(np.float32)
    for bits in (3, 4, 5):
        q, (n16, m16, s16), (n32, m32, s32), err = O.nsn_encode_f32_metas(x, bits)
        assert err == 0 and q.max() == (1 << bits) - 1
        # with s > 0 every channel uses both extreme codes
        assert np.all(q.min(axis=1) == 0) and np.all(q.max(axis=1) == (1 << bits) - 1)
        d = x / np.maximum(n32, O.EPS)
        assert np.array_equal(m32.reshape(16, 128), d.min(axis=1))


# ------------------------------------------------------------- bitstream

@pytest.mark.parametrize("bits", [3, 4, 5])
def test_bitstream_golden_and_independent_constructions(golden, bits):
    G = golden("codec.npz")
    for count in (1, 7, 63, 64, 65, 127, 128, 129, 8192):
        codes = G[f"stream|b{bits}|n{count}|codes"]
        want = G[f"stream|b{bits}|n{count}|bytes"]
        assert np.array_equal(O.pack_codes(codes, bits), want)
        assert np.array_equal(O.pack_bits_numpy(codes, bits), want)
        assert np.array_equal(O.unpack_codes(want, count, bits), codes)
        assert np.array_equal(O.unpack_bits_numpy(want, count, bits), codes)


def test_pack3_kat_and_msb_first_is_rejected(golden):
    G = golden("codec.npz")
    for n in (1, 2, 3, 7, 8, 9, 63, 64, 65, 8192):
        a = ((np.arange(n) * 5 + 3) % 8).astype(np.uint8)      # loop_kv_pk01_cache.py:175
        assert np.array_equal(O.pack_codes(a, 3), G[f"pack3|n{n}"])
    # planted mistake: MSB-first bit order fails the KAT
    a = ((np.arange(64) * 5 + 3) % 8).astype(np.uint8)
    b = ((a[:, None] >> np.arange(2, -1, -1)) & 1).reshape(-1)
    assert not np.array_equal(np.packbits(b, bitorder="little"), G["pack3|n64"])


def test_exhaustive_byte_pairs_roundtrip():
    """loop_kv_pu01_kernel.py:78-81: every (a, b, a^b) byte triple."""
    a = np.repeat(np.arange(256, dtype=np.uint8), 256)
    b = np.tile(np.arange(256, dtype=np.uint8), 256)
    packed = np.stack((a, b, a ^ b), -1).reshape(-1)
    n = 65536 * 8
    codes = O.unpack_codes(packed, n, 3)
    assert np.array_equal(codes, O.unpack_bits_numpy(packed, n, 3))
    assert np.array_equal(O.pack_codes(codes, 3), packed)


def test_vf01_fixture_input_hashes():
    """Rebuilt VF01 fixtures hash to what the reference's run recorded."""
    rec = json.loads((GOLDEN / "vf01_input_hashes.json").read_text())
    for f in rec["fixtures"]:
        arrays = gi.vf01_fixture(f["compressed"], f["length"], f["pattern"])
        for name, want in f["input_hashes"].items():
            key = name.replace("meta", "meta")
            assert gi.array_hash(arrays[key]) == want, (f["id"], name)
        # and the packed codes are the oracle's LSB-first stream
        if f["compressed"]:
            codes = (np.arange(2 * f["compressed"] * 128) % 8).astype(np.uint8)
            assert np.array_equal(O.pack_codes(codes, 3), arrays["k_codes"].reshape(-1))


# ------------------------------------------------------------- attention

def test_attention_oracle_closed_forms():
    rng = np.random.default_rng(0)
    T = 833
    v = rng.standard_normal((1, 2, T, 128))
    # uniform scores -> mean of V
    ctx = O.readout64(np.zeros((1, 2, T)), v)
    assert np.allclose(ctx, v.mean(axis=2), atol=1e-12)
    # dominant score: the mass 0.9999 on one token (loop_kv_af01_contract.py:83)
    s = np.zeros((1, 2, T))
    s[:, :, T // 2] = np.log((T - 1) * 0.9999 / 0.0001)
    p = O.softmax64(s)
    assert abs(p[0, 0, T // 2] - 0.9999) < 1e-12
    # alternating +-1 V with uniform weights over an even count cancels
    vc = np.where(np.arange(834)[None, None, :, None] % 2 == 0, 1.0, -1.0) * np.ones((1, 1, 834, 128))
    assert np.allclose(O.readout64(np.zeros((1, 1, 834)), vc), 0, atol=1e-15)
    # a one-hot query selects one channel of K into the scores
    k = rng.standard_normal((1, 1, 9, 128))
    q = np.zeros((1, 1, 128))
    q[0, 0, 5] = 1
    ctx, p = O.decode_attention64(q, k, k)
    want = O.softmax64(k[0, 0, :, 5] * O.SCALE)
    assert np.allclose(p[0, 0], want, atol=1e-15)


def test_gqa_head_map_and_split_invariance():
    rng = np.random.default_rng(1)
    q = rng.standard_normal((2, 8, 128))
    k = rng.standard_normal((2, 2, 50, 128))
    v = rng.standard_normal((2, 2, 50, 128))
    ctx, _ = O.decode_attention64(q, k, v)
    for h in range(8):
        c1, _ = O.decode_attention64(q[:, h:h + 1], k[:, h // 4:h // 4 + 1], v[:, h // 4:h // 4 + 1])
        assert np.allclose(ctx[:, h], c1[:, 0], atol=1e-13)
    # planted mistake: h % Hkv instead of h // G gives a different result
    bad, _ = O.decode_attention64(q[:, 1:2], k[:, 1:2], v[:, 1:2])
    assert not np.allclose(ctx[:, 1], bad[:, 0])
    # split-softmax merge (loop_kv_af01_kernel.py:70-82) equals one pass
    s = rng.standard_normal(50) * 3
    vv = rng.standard_normal((50, 128))
    parts = [(s[a:b], vv[a:b]) for a, b in ((0, 7), (7, 30), (30, 50))]
    m = np.array([x.max() for x, _ in parts])
    z = np.array([np.exp(x - x.max()).sum() for x, _ in parts])
    u = np.stack([(np.exp(x - x.max())[:, None] * y).sum(0) for x, y in parts])
    a = np.exp(m - m.max())
    merged = (u * a[:, None]).sum(0) / (z * a).sum()
    assert np.allclose(merged, O.readout64(s[None, None], vv[None, None])[0, 0], atol=1e-13)


# ------------------------------------------------------------- chunked prefill

def _prefill_case(seed, Hq=4, Hkv=2, L=37, n=9):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((Hq, n, 128)) * 2
    kc, vc = rng.standard_normal((2, Hkv, L, 128))
    kn, vn = rng.standard_normal((2, Hkv, n, 128))
    return q, kc, vc, kn, vn


def _rows_match_decode(out, q, kc, vc, kn, vn):
    """Row i of the prefill == decode attention of q[:, i] over context + chunk[:i+1]."""
    n = q.shape[1]
    for i in range(n):
        k = np.concatenate([kc, kn[:, :i + 1]], axis=1)[None]
        v = np.concatenate([vc, vn[:, :i + 1]], axis=1)[None]
        ctx, _ = O.decode_attention64(q[None, :, i], k, v)
        if not np.allclose(out[:, i], ctx[0], rtol=0, atol=1e-12):
            return False
    return True


@pytest.mark.parametrize("L", [0, 37])
def test_prefill_oracle_rows_are_decode_attention(L):
    q, kc, vc, kn, vn = _prefill_case(7, L=L)
    out = O.prefill_attention64(q, kc, vc, kn, vn)
    assert _rows_match_decode(out, q, kc, vc, kn, vn)
    # planted mistakes: a causal mask off by one either way fails the row check
    for shift in (-1, 1):
        with np.errstate(invalid="ignore"):     # (shift -1 with no context leaves row 0 nothing to attend)
            bad = O.prefill_attention64(q, kc, vc, kn, vn, causal_shift=shift)
        assert not _rows_match_decode(bad, q, kc, vc, kn, vn)


def test_prefill_oracle_constant_keys_give_prefix_means():
    """Equal keys -> uniform weights over every visible token: row i is the
    mean of the L context values and chunk values 0..i (closed form)."""
    rng = np.random.default_rng(8)
    Hq, Hkv, L, n = 2, 1, 5, 7
    q = rng.standard_normal((Hq, n, 128))
    key = rng.standard_normal(128)
    kc = np.broadcast_to(key, (Hkv, L, 128)).copy()
    kn = np.broadcast_to(key, (Hkv, n, 128)).copy()
    vc = rng.standard_normal((Hkv, L, 128))
    vn = rng.standard_normal((Hkv, n, 128))
    out = O.prefill_attention64(q, kc, vc, kn, vn)
    allv = np.concatenate([vc[0], vn[0]])
    want = np.stack([allv[:L + i + 1].mean(0) for i in range(n)])
    assert np.allclose(out[0], want, atol=1e-12) and np.allclose(out[1], want, atol=1e-12)
    bad = O.prefill_attention64(q, kc, vc, kn, vn, causal_shift=1)
    assert not np.allclose(bad[0], want, atol=1e-6)


# --------------------------------------------- PyTorch-CPU restatement (bench baseline)

def test_torch_cpu_restatement_matches_goldens(golden):
    """oracle/torch_cpu.py (timed as bench.py's cpu_baseline) is pinned to the
    same goldens: unpack3 of the golden bitstream equals the C oracle's codes,
    nsn_int3_qdq and nsn_decode reproduce the golden outputs bit for bit."""
    from oracle import torch_cpu as T
    G = golden("c0.npz")
    k, v = gi.config0_inputs()
    for name, x in (("k", k), ("v", v)):
        q, n16, m16, s16, err = O.nsn_encode(x.astype(np.float32), 3)
        codes = T.unpack3(torch.from_numpy(G[name + "_codes"]), (32, 64, 128))
        assert np.array_equal(codes.numpy(), q.reshape(32, 64, 128))
        y = T.nsn_int3_qdq(torch.from_numpy(x))                      # fp16 in, fp16 out
        assert np.array_equal(y.view(torch.int16).numpy().view(np.uint16), G[name + "_qdq"])
        yd = T.nsn_decode(codes, torch.from_numpy(G[name + "_norm"].view(np.float16)).reshape(32, 64, 1),
                          torch.from_numpy(G[name + "_min"].view(np.float16)).reshape(32, 1, 128),
                          torch.from_numpy(G[name + "_scale"].view(np.float16)).reshape(32, 1, 128), torch.float16)
        assert np.array_equal(yd.view(torch.int16).numpy().view(np.uint16), G[name + "_qdq"])
    C = golden("codec.npz")
    for bits, tensors in gi.pilot_fixture_tensors().items():
        if bits != 3:
            continue
        for i, t in enumerate(tensors):
            key = f"b3|t{i}|"
            q = T.unpack3(torch.from_numpy(C[key + "codes"]), C[key + "decoded"].shape)
            y = T.nsn_decode(q, torch.from_numpy(C[key + "norm"].view(np.float16)),
                             torch.from_numpy(C[key + "min"].view(np.float16)),
                             torch.from_numpy(C[key + "scale"].view(np.float16)))
            assert np.array_equal(y.numpy().view(np.uint32), C[key + "decoded"]), key


def test_torch_cpu_unpack3_kat_and_bridge_vs_fp64():
    from oracle import torch_cpu as T
    # the reference's KAT (loop_kv_pk01_cache.py:175-179): codes (arange*5+3)%8 round-trip
    codes = ((np.arange(1000) * 5 + 3) % 8).astype(np.uint8)
    packed = O.pack_codes(codes, 3)
    assert np.array_equal(T.unpack3(torch.from_numpy(packed), (1000,)).numpy(), codes)
    # the bridge readout equals the fp64 oracle over the same restored K/V (GQA 4:1, blocks + tail)
    rng = np.random.default_rng(5)
    H, nb, tail = 2, 3, 37
    side = []
    for _ in range(2):
        x = rng.standard_normal((H, nb, 64, 128)).astype(np.float32)
        q_, n16, m16, s16, err = O.nsn_encode(x, 3)
        assert err == 0
        blocks = (torch.from_numpy(O.pack_codes(q_.reshape(H * nb, -1), 3).reshape(H, nb, 3072)),
                  torch.from_numpy(n16.view(np.float16)), torch.from_numpy(m16.view(np.float16)),
                  torch.from_numpy(s16.view(np.float16)))
        t = torch.from_numpy(rng.standard_normal((H, tail, 128)).astype(np.float16))
        full = np.concatenate([O.nsn_decode_f32(q_, n16, m16, s16).reshape(H, nb * 64, 128), t.float().numpy()], 1)
        side.append((blocks, t, full))
    q = torch.from_numpy(rng.standard_normal((8, 128)).astype(np.float32))
    got = T.bridge_readout(q, side[0][0], side[0][1], side[1][0], side[1][1]).numpy()
    ref, _ = O.decode_attention64(q.numpy()[None], side[0][2][None], side[1][2][None])
    assert np.allclose(got, ref[0], rtol=1e-4, atol=1e-5)
    # planted mistake: the head map h % Hkv instead of h // G is far off
    bad = T.bridge_readout(q[[0, 4, 1, 5, 2, 6, 3, 7]], side[0][0], side[0][1], side[1][0], side[1][1]).numpy()
    assert not np.allclose(bad[[0, 2, 4, 6, 1, 3, 5, 7]], ref[0], rtol=1e-4, atol=1e-5)
