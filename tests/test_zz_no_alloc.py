"""The allocation-free decode entry point (nsn_decode_attention_static).

Two calls in a row, the second smaller, each compared bitwise with
nsn_decode_attention on a caller-allocated workspace (same kernels, same
partition, so the results must be identical), plus the fp64 oracle bound
of the decode tests.  An oversized shape is rejected before any launch.
"""
import numpy as np
import pytest
import torch

from nsn_amd import _lib, kernels
from tests.test_gpu_attention import make_case, oracle_ctx, within

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _run(kernel, static, q, kk, vv, seq, L):
    print(f"no-alloc case: kernel={kernel} static={static} lengths={L}", flush=True)
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=DEV)
    ctx = torch.empty(q.shape, dtype=torch.float32, device=DEV)
    st = torch.zeros(1, dtype=torch.int32, device=DEV)
    kernels.decode_attention(q, kk, vv, seq, max_seq_len=max(L), kernel=kernel, kv_round_dtype=torch.float16,
                             out=out, ctx=ctx, status=st, check=False, static_workspace=static)
    torch.cuda.synchronize()
    assert int(st.item()) == 0
    return out.cpu(), ctx.cpu()


@pytest.mark.parametrize("kernel", ["fast", "reference"])
def test_static_entry_matches_allocating_entry(kernel):
    cases = [(11, 3, 16, 4, [1500, 700, 931]), (12, 2, 8, 2, [300, 77])]   # the second call is smaller
    for seed, B, Hq, Hkv, L in cases:
        k, v, qb, kk, vv, seq = make_case(seed, B, Hq, Hkv, L)
        q = qb.to(DEV)
        out_s, ctx_s = _run(kernel, True, q, kk, vv, seq, L)
        out_a, ctx_a = _run(kernel, False, q, kk, vv, seq, L)
        assert torch.equal(out_s.view(torch.int16), out_a.view(torch.int16))
        assert torch.equal(ctx_s.view(torch.int32), ctx_a.view(torch.int32))
        ok, err = within(ctx_s.numpy(), oracle_ctx(k, v, qb, L, 3, "float32" if kernel == "fast" else "float16"))
        assert ok, err


def test_static_entry_rejects_oversized_workspace():
    """A workspace beyond the static maximum returns NSN_ENOSPC before any
    pointer is used or kernel launched (the argument block is otherwise empty)."""
    import ctypes
    a = _lib.AttnArgs()
    a.batch, a.heads_q, a.heads_kv = 1, 4, 1
    a.n_splits = _lib.STATIC_SCRATCH_FLOATS // (4 * kernels.PART_STRIDE) + 2
    a.split_tokens = 64
    assert kernels.workspace_floats(1, 4, a.n_splits) > _lib.STATIC_SCRATCH_FLOATS
    rc = _lib.lib().nsn_decode_attention_static(ctypes.byref(a), None)
    assert rc == _lib.NSN_ENOSPC
    with pytest.raises(RuntimeError, match="static scratch"):
        _lib.check(rc, "nsn_decode_attention_static")
