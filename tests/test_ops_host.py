"""Host checks of the registered operators (nsn_amd.ops): every operator of
the call surface exists under torch.ops.nsn, its fake implementation gives the
shapes and dtypes of the Python function it wraps (meta tensors, no GPU), and
a CPU tensor has no kernel (the library has no CPU path).  The GPU test
tests/test_gpu_ops.py checks the operators bitwise against the Python surface."""
import pytest
import torch

import nsn_amd  # noqa: F401
from nsn_amd import ops

META = torch.device("meta")


def test_every_operator_is_registered():
    for name in ops.OPS:
        assert hasattr(torch.ops.nsn, name), name


def test_codec_fake_shapes():
    x = torch.empty(2, 3, 64, 128, dtype=torch.float16, device=META)
    q, n, m, s = torch.ops.nsn.encode(x, 5)
    assert q.shape == x.shape and q.dtype == torch.uint8
    assert n.shape == (2, 3, 64, 1) and m.shape == s.shape == (2, 3, 1, 128) and n.dtype == torch.float16
    assert torch.ops.nsn.decode(q, n, m, s, torch.bfloat16).dtype == torch.bfloat16
    assert torch.ops.nsn.int3_qdq(x).shape == x.shape
    p = torch.ops.nsn.pack_codes(torch.empty(1001, dtype=torch.uint8, device=META), 5)
    assert p.shape == ((1001 * 5 + 7) // 8,)
    assert torch.ops.nsn.unpack_codes(p, 1001, 5).shape == (1001,)
    g = torch.ops.nsn.encode_group(torch.empty(1, 8, 3, 64, 128, device=META), 64, 3)
    assert [tuple(t.shape) for t in g] == [(1, 8, 3, 3072), (1, 8, 3, 64, 1), (1, 8, 3, 1, 128), (1, 8, 3, 1, 128),
                                            (1, 8, 3, 12)]
    r = torch.ops.nsn.restore_group(*g[:4], torch.float16)
    assert r.shape == (1, 8, 192, 128) and r.dtype == torch.float16


def test_attention_fake_shapes():
    B, Hq, Hkv, cap = 2, 8, 2, 4
    q = torch.empty(B, Hq, 128, dtype=torch.bfloat16, device=META)
    side = [torch.empty(B, Hkv, cap, 3072, dtype=torch.uint8, device=META), None, None, None, None,
            torch.empty(B, dtype=torch.int32, device=META), torch.empty(B, Hkv, 64, 128, dtype=torch.float16,
                                                                          device=META)]
    out, ctx = torch.ops.nsn.decode_attention(q, *side, *side, torch.empty(B, dtype=torch.int32, device=META), 3, 300)
    assert out.shape == ctx.shape == (B, Hq, 128) and out.dtype == torch.bfloat16 and ctx.dtype == torch.float32
    qc = torch.empty(B, Hq, 40, 128, dtype=torch.bfloat16, device=META)
    kc = torch.empty(B, Hkv, 40, 128, dtype=torch.bfloat16, device=META)
    o = torch.ops.nsn.prefill_attention(qc, *side, *side, torch.empty(B, dtype=torch.int32, device=META), kc, kc, 3)
    assert o.shape == qc.shape and o.dtype == qc.dtype


def test_cpu_tensors_have_no_kernel():
    with pytest.raises(NotImplementedError):
        torch.ops.nsn.int3_qdq(torch.zeros(1, 64, 128))
