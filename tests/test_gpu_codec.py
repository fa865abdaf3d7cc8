"""GPU parity of the codec through the C-ABI: bit-exact against the golden
vectors written from the reference and against the CPU oracle."""
import hashlib

import numpy as np
import pytest
import torch

from nsn_amd import codec, kernels, primitives
from nsn_amd.errors import IntegrityError, NumericalFailure
from oracle import oracle as O
from tests.golden import inputs as gi

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def u16(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)


def gpu_like(x):
    """Copy to the GPU keeping the exact strides (the norm order depends on them)."""
    return torch.empty_strided(x.size(), x.stride(), dtype=x.dtype, device=DEV).copy_(x)


def sha(b):
    return hashlib.sha256(b).hexdigest()


def test_c0_golden(golden):
    G = golden("c0.npz")
    k, v = gi.config0_inputs()
    for name, a in (("k", k), ("v", v)):
        x = torch.from_numpy(a).to(DEV)
        g = codec.encode_group(x.reshape(1, 32, 1, 64, 128), 0)
        assert np.array_equal(g["codes"].cpu().numpy().reshape(32, 3072), G[name + "_codes"])
        assert np.array_equal(u16(g["metas"][0]), G[name + "_norm"].reshape(-1))
        assert np.array_equal(u16(g["metas"][1]), G[name + "_min"].reshape(-1))
        assert np.array_equal(u16(g["metas"][2]), G[name + "_scale"].reshape(-1))
        assert np.array_equal(g["headers"].cpu().numpy().reshape(32, 12), G[name + "_headers"])
        assert np.array_equal(u16(primitives.nsn_int3_qdq(x)), G[name + "_qdq"].reshape(-1))
        assert np.array_equal(u16(codec.restore_group(g, torch.float16)), G[name + "_qdq"].reshape(-1))


@pytest.mark.parametrize("dtype", ["float32", "float16", "bfloat16"])
def test_core_fixtures(golden, dtype):
    G = golden("core.npz")
    for name, x in gi.core_fixtures().items():
        a = x.to(getattr(torch, dtype))
        key = f"{name}|{dtype}|"
        xg = gpu_like(a)
        q, metas = primitives.nsn_encode(xg, 3)
        assert np.array_equal(primitives.pack_codes(q, 3).cpu().numpy(), G[key + "codes"]), name
        for i, part in enumerate(("norm", "min", "scale")):
            assert np.array_equal(u16(metas[i]), G[key + part].reshape(-1)), (name, part)
        y = primitives.nsn_int3_qdq(xg)
        assert np.array_equal(y.cpu().contiguous().view(torch.uint8).numpy().reshape(-1), G[key + "out"].reshape(-1)), name


def test_pilot_codec_fixtures(golden):
    G = golden("codec.npz")
    for bits, tensors in gi.pilot_fixture_tensors().items():
        for i, t in enumerate(tensors):
            key = f"b{bits}|t{i}|"
            q, metas = primitives.nsn_encode(gpu_like(t), bits)
            assert np.array_equal(primitives.pack_codes(q, bits).cpu().numpy(), G[key + "codes"]), key
            for j, part in enumerate(("norm", "min", "scale")):
                assert np.array_equal(u16(metas[j]), G[key + part].reshape(-1)), (key, part)
            y = primitives.nsn_decode(q, metas, torch.float32)
            assert np.array_equal(y.cpu().numpy().view(np.uint32).reshape(-1), G[key + "decoded"].reshape(-1)), key


def test_heavy_tailed_4_and_5_bit(golden):
    G = golden("heavy.npz")
    x = torch.from_numpy(gi.heavy_tailed_blocks()).to(DEV)
    for bits in (4, 5):
        q, metas = primitives.nsn_encode(x, bits)
        assert np.array_equal(primitives.pack_codes(q, bits).cpu().numpy(), G[f"b{bits}|codes"])
        for j, part in enumerate(("norm", "min", "scale")):
            assert np.array_equal(u16(metas[j]), G[f"b{bits}|{part}"].reshape(-1))
        assert np.array_equal(u16(primitives.nsn_qdq(x, bits)), G[f"b{bits}|qdq"].reshape(-1))
        # the one-launch group encoder agrees with nsn_encode + pack
        g = codec.encode_group(x.reshape(1, 8, 1, 64, 128), 0, bits=bits)
        assert np.array_equal(g["codes"].cpu().numpy().reshape(-1), G[f"b{bits}|codes"])


def test_group_codec_and_real_blocks(golden):
    G = golden("group.npz")
    samples = dict(gi.group_samples())
    for name in ("K_00", "V_43"):
        raw = G[f"real|{name}|input"]
        samples["real_" + name] = torch.from_numpy(raw.view(np.int16)).view(torch.bfloat16).reshape(1, 8, 1, 64, 128)
    for name, x in samples.items():
        key = f"group|{name}|"
        xg = gpu_like(x.to(torch.bfloat16))
        g = codec.encode_group(xg, 0)
        assert np.array_equal(g["codes"].cpu().numpy(), G[key + "codes"]), name
        for j, part in enumerate(("norm", "min", "scale")):
            assert np.array_equal(u16(g["metas"][j]), G[key + part].reshape(-1)), (name, part)
        assert np.array_equal(g["headers"].cpu().numpy(), G[key + "headers"]), name
        assert np.array_equal(u16(codec.restore_group(g, torch.bfloat16)), G[key + "restored"].reshape(-1)), name


@pytest.mark.parametrize("src_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bits", [3, 4, 5])
def test_encode_restore_random_vs_oracle(src_dtype, bits):
    rng = np.random.default_rng(100 + bits)
    x = (rng.standard_normal((3, 40, 64, 128)) * rng.lognormal(0, 2, (3, 40, 64, 1))).astype(np.float32)
    x[0, 0, 5] = 0.0                                   # a zero-norm token
    x[1, 2, :, 7] = x[1, 2, 0, 7]                       # a flat channel: scale may be 0
    xt = torch.from_numpy(x).to(src_dtype)
    xf = xt.float().numpy()
    q_o, n_o, m_o, s_o, err = O.nsn_encode(xf, bits)
    assert err == 0
    g = codec.encode_group(xt.to(DEV).reshape(1, 3, 40, 64, 128), 0, bits=bits)
    assert np.array_equal(g["codes"].cpu().numpy().reshape(-1), O.pack_codes(q_o, bits))
    assert np.array_equal(u16(g["metas"][0]), n_o.reshape(-1))
    assert np.array_equal(u16(g["metas"][1]), m_o.reshape(-1))
    assert np.array_equal(u16(g["metas"][2]), s_o.reshape(-1))
    for out_dt, name in ((torch.float16, "float16"), (torch.bfloat16, "bfloat16"), (torch.float32, "float32")):
        r = codec.restore_group(g, out_dt).cpu().reshape(3, 40, 64, 128)
        want = O.nsn_decode(q_o, n_o, m_o, s_o, name)
        got = r.view(torch.int32 if name == "float32" else torch.int16).numpy()
        assert np.array_equal(got.view(np.uint32 if name == "float32" else np.uint16).reshape(-1), want.reshape(-1)), name


@pytest.mark.parametrize("bits", [3, 4, 5])
def test_pack_unpack_vs_oracle(bits):
    rng = np.random.default_rng(bits)
    for count in (1, 7, 31, 32, 33, 63, 65, 127, 8192, 100003):
        codes = rng.integers(0, 1 << bits, count, dtype=np.uint8)
        want = O.pack_codes(codes, bits)
        got = primitives.pack_codes(torch.from_numpy(codes).to(DEV), bits).cpu().numpy()
        assert np.array_equal(got, want), count
        back = primitives.unpack_codes(torch.from_numpy(want).to(DEV), count, bits).cpu().numpy()
        assert np.array_equal(back, codes), count
    # unaligned device views (storage offset 1) take the byte path
    codes = rng.integers(0, 1 << bits, 1001, dtype=np.uint8)
    buf = torch.zeros(1002, dtype=torch.uint8, device=DEV)
    buf[1:] = torch.from_numpy(codes).to(DEV)
    assert np.array_equal(primitives.pack_codes(buf[1:], bits).cpu().numpy(), O.pack_codes(codes, bits))


def test_pack3_kats_and_exhaustive_byte_pairs(golden):
    G = golden("codec.npz")
    for n in (1, 2, 3, 7, 8, 9, 63, 64, 65, 8192):
        a = ((np.arange(n) * 5 + 3) % 8).astype(np.uint8)
        p = codec.pack3(torch.from_numpy(a).to(DEV))
        assert np.array_equal(p.cpu().numpy(), G[f"pack3|n{n}"])
        assert np.array_equal(codec.unpack3(p, (n,)).cpu().numpy(), a)
    a = np.repeat(np.arange(256, dtype=np.uint8), 256)
    b = np.tile(np.arange(256, dtype=np.uint8), 256)
    packed = np.stack((a, b, a ^ b), -1).reshape(-1)
    n = 65536 * 8
    got = codec.unpack3(torch.from_numpy(packed).to(DEV), (n,)).cpu().numpy()
    assert np.array_equal(got, O.unpack_bits_numpy(packed, n, 3))


@pytest.mark.parametrize("bits", [3, 5])
def test_decode_factors_vs_oracle(bits):
    from nsn_amd import cache
    rng = np.random.default_rng(40 + bits)
    x = (rng.standard_normal((2, 3, 320, 128)) * rng.lognormal(0, 1, (2, 3, 320, 1))).astype(np.float16)
    x[0, 1, 70] = 0
    kv, _ = cache.pack_sequences(torch.from_numpy(x).to(DEV), [320, 300], bits=bits)
    for b, L in enumerate((320, 300)):
        nb = L // 64
        q_o, n_o, m_o, s_o, _ = O.nsn_encode(x[b, :, :nb * 64].astype(np.float32).reshape(3, nb, 64, 128), bits)
        want = O.decode_factors(q_o, n_o, m_o, s_o)
        got = kv.factor[b, :, :nb].cpu().numpy()
        # the encoder sums in its own order (8-channel fma chains + a 16-lane
        # tree) and finishes with the hardware root and reciprocal: a few ulps
        assert np.array_equal(got == 0, want == 0)
        assert np.all(np.abs(got.astype(np.float64) - want) <= 2.0 ** -20 * np.abs(want))
        # standalone factor kernel on the same packed blocks: the oracle's order, bitwise
        f2 = kernels.block_factors(kv.codes[b, :, :nb].contiguous(), kv.norm[b, :, :nb], kv.min[b, :, :nb],
                                   kv.scale[b, :, :nb], bits).cpu().numpy()
        assert np.array_equal(f2.view(np.uint32), want.view(np.uint32))


def test_code_range_rejected():
    with pytest.raises(IntegrityError):
        codec.pack3(torch.tensor([1, 2, 8], dtype=torch.uint8, device=DEV))


def test_encode_errors():
    with pytest.raises(NumericalFailure, match="overflow"):
        primitives.nsn_encode(torch.full((64, 128), 1e5, device=DEV), 3)
    x = torch.randn(2, 64, 128, device=DEV)
    x[1, 3, 4] = float("nan")
    with pytest.raises(NumericalFailure, match="Nonfinite input"):
        primitives.nsn_encode(x, 3)
    x = torch.zeros(64, 128, device=DEV)
    x[:, 0] = 1e-9
    with pytest.raises(NumericalFailure, match="underflow"):
        primitives.nsn_encode(x, 3)


def test_restore_v_with_tail_matches_oracle():
    rng = np.random.default_rng(7)
    H, n, L = 4, 3, 37
    x = (rng.standard_normal((1, H, n, 64, 128)) * rng.lognormal(0, 1, (1, H, n, 64, 1))).astype(np.float16)
    tail = (rng.standard_normal((1, H, L, 128))).astype(np.float16)
    g = codec.encode_group(torch.from_numpy(x).to(DEV), 0)
    vt = torch.from_numpy(tail).to(DEV)
    out = kernels.restore_v(g, vt)
    assert tuple(out.shape) == (1, H, n * 64 + L, 128) and out.dtype == torch.float16
    q_o, n_o, m_o, s_o, _ = O.nsn_encode(x.astype(np.float32), 3)
    want = np.concatenate([O.nsn_decode(q_o, n_o, m_o, s_o, "float16").reshape(1, H, n * 64, 128),
                           tail.view(np.uint16)], axis=2)
    assert np.array_equal(u16(out), want.reshape(-1))


def _edge_blocks():
    """Blocks that take the encoder's rare paths, as fp32 [n, 64, 128] arrays
    keyed by name, with the source dtypes each one is meaningful in."""
    rng = np.random.default_rng(7)
    out = {}
    # signed-zero ties: channel 3 has min 0 reached by both +0 and -0, channel 9 max 0
    x = np.abs(rng.standard_normal((64, 128))).astype(np.float32) + 0.25
    x[:, 3] = np.abs(rng.standard_normal(64)) + 0.5
    x[[5, 9, 40], 3] = 0.0
    x[[2, 17, 33], 3] = -0.0
    x[:, 9] = -np.abs(rng.standard_normal(64)) - 0.5
    x[[1, 30], 9] = -0.0
    x[[12, 50], 9] = 0.0
    out["zero_ties"] = (x[None], ("float16", "bfloat16", "float32"))
    z = np.zeros((2, 64, 128), np.float32)
    z[1] = -0.0
    out["all_zero"] = (z, ("float16", "bfloat16", "float32"))
    # subnormal scale: quotients (d - m) / s past the top level, clamped
    t = np.arange(64)[:, None]
    c = np.arange(128)[None, :]
    sub = (((t * 7 + c) % 5) * 1e-38).astype(np.float32)
    sub[:, 0] = 1.0
    out["subnormal_scale"] = (sub[None], ("bfloat16", "float32"))
    # a row norm that overflows fp32 from finite inputs: not a nonfinite input
    ov = rng.standard_normal((64, 128)).astype(np.float32)
    ov[4, :2] = 2e38
    out["norm_overflow"] = (ov[None], ("bfloat16", "float32"))
    # nonfinite inputs
    nf = rng.standard_normal((3, 64, 128)).astype(np.float32)
    nf[0, 6, 77] = np.inf
    nf[1, 0, 0] = np.nan
    nf[2, 63, 127] = -np.inf
    out["nonfinite"] = (nf, ("float16", "bfloat16", "float32"))
    return out


@pytest.mark.parametrize("bits", [3, 4, 5])
def test_encode_edge_blocks_vs_oracle(bits):
    """Signed-zero ties, zero blocks, a subnormal scale (the clamped code
    path), a norm that overflows from finite inputs, and nonfinite inputs:
    metadata, codes and status bits against the oracle."""
    from nsn_amd import _dev
    for name, (x, dtypes) in _edge_blocks().items():
        for dt in dtypes:
            xt = torch.from_numpy(x).to(getattr(torch, dt))
            q_o, n_o, m_o, s_o, err = O.nsn_encode(xt.float().numpy(), bits)
            st = _dev.new_status(DEV)
            g = codec.encode_group(xt.to(DEV).reshape(1, 1, -1, 64, 128), 0, bits=bits, status=st, check=False)
            status = _dev.read_status(st)
            assert status == err, (name, dt, status, err)
            if err & O.ERR_NONFINITE_INPUT:
                continue   # outputs of a block with nonfinite input are unspecified (the reference raises)
            assert np.array_equal(u16(g["metas"][0]), n_o.reshape(-1)), (name, dt)
            assert np.array_equal(u16(g["metas"][1]), m_o.reshape(-1)), (name, dt)
            assert np.array_equal(u16(g["metas"][2]), s_o.reshape(-1)), (name, dt)
            assert np.array_equal(g["codes"].cpu().numpy().reshape(-1), O.pack_codes(q_o, bits)), (name, dt)
