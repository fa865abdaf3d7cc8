"""The registered operators (torch.ops.nsn.*) against the Python call surface
they wrap: every output bitwise equal on the same inputs (codec: C0-shaped
blocks in 3 and 5 bits; attention: a ragged packed cache with fp16 tails,
GQA 4:1, fast and exact-order kernels; chunked prefill over the same cache)."""
import numpy as np
import pytest
import torch

import nsn_amd  # noqa: F401  (registers the operators)
from nsn_amd import cache, codec, kernels, ops, primitives, synthetic

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def bits_equal(a, b):
    assert a.shape == b.shape and a.dtype == b.dtype
    assert torch.equal(a.contiguous().view(-1).view(torch.uint8), b.contiguous().view(-1).view(torch.uint8))


@pytest.mark.parametrize("bits", [3, 5])
def test_codec_operators_match_python_surface(bits):
    k, _ = synthetic.config0(0)
    x = torch.from_numpy(k).to(DEV)                                   # [32, 64, 128] fp16
    q, n, m, s = torch.ops.nsn.encode(x, bits)
    q2, (n2, m2, s2) = primitives.nsn_encode(x, bits)
    for a, b in ((q, q2), (n, n2), (m, m2), (s, s2)):
        bits_equal(a, b)
    bits_equal(torch.ops.nsn.decode(q, n, m, s, torch.bfloat16), primitives.nsn_decode(q2, (n2, m2, s2),
                                                                                       torch.bfloat16))
    bits_equal(torch.ops.nsn.int3_qdq(x), primitives.nsn_int3_qdq(x))
    p = torch.ops.nsn.pack_codes(q, bits)
    bits_equal(p, primitives.pack_codes(q2, bits))
    bits_equal(torch.ops.nsn.unpack_codes(p, q.numel(), bits), q.reshape(-1))
    g = torch.ops.nsn.encode_group(x.reshape(1, 8, 4, 64, 128), 128, bits)
    g2 = codec.encode_group(x.reshape(1, 8, 4, 64, 128), 128, bits)
    for a, b in zip(g, (g2["codes"], *g2["metas"], g2["headers"])):
        bits_equal(a, b)
    bits_equal(torch.ops.nsn.restore_group(*g[:4], torch.float16), codec.restore_group(g2, torch.float16))


@pytest.mark.parametrize("kernel", ["fast", "reference"])
def test_attention_operators_match_python_surface(kernel):
    rng = np.random.default_rng(5)
    B, Hkv, Hq = 3, 2, 8
    lengths = [700, 131, 64]
    L = max(lengths)
    x = torch.from_numpy(synthetic.kv_tokens(rng, (2, B, Hkv), L)).to(DEV)
    kk, seq = cache.pack_sequences(x[0], lengths, bits=3, tail_dtype=torch.float16)
    vv, _ = cache.pack_sequences(x[1], lengths, bits=3, tail_dtype=torch.float16)
    q = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(torch.bfloat16).to(DEV)
    out, ctx = torch.ops.nsn.decode_attention(q, *ops.side_tensors(kk), *ops.side_tensors(vv), seq, 3, L, kernel)
    out2, ctx2 = kernels.decode_attention(q, kk, vv, seq, max_seq_len=L, kernel=kernel)
    bits_equal(out, out2)
    bits_equal(ctx, ctx2)
    # chunked prefill of 40 new tokens over the same packed context
    qc = torch.from_numpy(rng.standard_normal((B, Hq, 40, 128)).astype(np.float16)).to(DEV)
    kc = torch.from_numpy(rng.standard_normal((B, Hkv, 40, 128)).astype(np.float16)).to(DEV)
    vc = torch.from_numpy(rng.standard_normal((B, Hkv, 40, 128)).astype(np.float16)).to(DEV)
    o = torch.ops.nsn.prefill_attention(qc, *ops.side_tensors(kk), *ops.side_tensors(vv), seq, kc, vc, 3)
    bits_equal(o, kernels.prefill_attention(qc, kk, vv, seq, kc, vc))
