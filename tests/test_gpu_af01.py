"""The AF01 closed-form fixtures and input rejections through the attention
kernels.  The fixtures are those of
experiments/ac08/source/loop_kv_af01_contract.py:74-89, run as
loop_kv_ac08_diagnostics.py:71-95 runs them and checked as
loop_kv_ac08_audit.py:30-47 checks them:

- finish-T{17,769,833} x {uniform, dominant, cancel, zero}: the softmax
  readout of given fp32 logits over bf16 V (uniform logits: the mean of V;
  dominant: 0.9999 of the mass on the middle token; cancel: alternating +-1
  V; zero: V = 0);
- full-T{17,65,769,833}: the logits from the query and a dense bf16 K, then
  the readout.

Each runs through the exact-order kernel, held to the reference's context
budget 2e-6 + 2e-6 * sum_t |p_t v_t| against the fp64 readout
(loop_kv_af01_contract.py:66-72), and through the fast kernel, held to its
own 2e-3 + 1e-2 * |ref|.  The bf16 output must be the context rounded, and
every input must be bitwise unchanged.  The six AF01 input rejections
(loop_kv_af01_contract.py:91) stop on the host before any launch.
"""
import math

import numpy as np
import pytest
import torch

from nsn_amd import kernels
from nsn_amd.errors import IntegrityError, NumericalFailure
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
H = 2

FIXTURES = [("finish", n, pat) for n in (17, 769, 833) for pat in ("uniform", "dominant", "cancel", "zero")] + \
           [("full", n, "native") for n in (17, 65, 769, 833)]


def fixture(T, pattern):
    """q [1,H,1,128], K [1,H,T,128], V [1,H,T,128] (bf16, rounded from the
    fp32 values) and the fp32 logits [1,H,T] of one fixture."""
    q = np.sin(np.arange(H * 128).reshape(1, H, 1, 128) * 0.03) * 0.2
    k = np.cos(np.arange(H * T * 128).reshape(1, H, T, 128) * 0.007) * 0.5
    v = np.sin(np.arange(H * T * 128).reshape(1, H, T, 128) * 0.011) * 0.25
    logits = np.zeros((1, H, T))
    if pattern == "dominant":
        logits[:, :, T // 2] = math.log((T - 1) * 0.9999 / 0.0001)
    elif pattern == "cancel":
        v = np.broadcast_to(np.where(np.arange(T)[None, None, :, None] % 2 == 0, 1.0, -1.0), v.shape)
    elif pattern == "zero":
        v = np.zeros_like(v)

    def bf16(x):
        return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(DEV).to(torch.bfloat16)
    return bf16(q), bf16(k), bf16(v), torch.from_numpy(logits.astype(np.float32)).to(DEV)


def bits(x):
    return x.view(torch.int32 if x.dtype == torch.float32 else torch.int16).clone()


@pytest.mark.parametrize("kernel", ["reference", "fast"])
@pytest.mark.parametrize("kind,T,pattern", FIXTURES, ids=[f"{k}-T{n}-{p}" for k, n, p in FIXTURES])
def test_af01_fixture_through_kernels(kind, T, pattern, kernel):
    q, k, v, logits = fixture(T, pattern)
    before = [bits(x) for x in (q, k, v, logits)]
    kernels.af_validate(None, k, q)
    kernels.validate_v(v, q, T)
    if kind == "finish":
        kernels.validate_score(logits, v)
    out, ctx = kernels.af_launch(None, k, q, v, score=logits if kind == "finish" else None, full=kind == "full",
                                 kernel=kernel)
    torch.cuda.synchronize()
    for b0, x in zip(before, (q, k, v, logits)):
        assert torch.equal(b0, bits(x)), "input changed"
    assert torch.equal(bits(out.reshape(H, 128)), bits(ctx.reshape(H, 128).to(torch.bfloat16)))

    v64 = v.float().cpu().numpy().astype(np.float64)
    if kind == "finish":
        s = logits.cpu().numpy().astype(np.float64)
    else:
        q64 = q.float().cpu().numpy().astype(np.float64)[:, :, 0]
        s = np.einsum("bhd,bhtd->bht", q64, k.float().cpu().numpy().astype(np.float64)) * O.SCALE
    p = O.softmax64(s)
    prod = p[..., None] * v64[0][None]            # [1, H, T, 128]
    gold = prod.sum(-2)[0]                        # [H, 128]
    got = ctx.reshape(H, 128).cpu().numpy().astype(np.float64)
    assert np.isfinite(got).all()
    if kernel == "reference":
        budget = 2e-6 + 2e-6 * np.abs(prod).sum(-2)[0]
    else:
        budget = 2e-3 + 1e-2 * np.abs(gold)
    err = np.abs(got - gold)
    assert (err <= budget).all(), float((err - budget).max())
    if pattern == "zero":
        assert not got.any()
    if pattern == "uniform":   # the mean of V
        assert np.allclose(gold, v64[0].mean(axis=1), atol=1e-12)


@pytest.mark.parametrize("kind", ["q_nan", "v_nan", "score_nan", "score_dtype", "score_shape", "empty_tail"])
def test_af01_input_rejections_before_launch(kind):
    q, k, v, logits = fixture(17, "uniform")
    if kind == "q_nan":
        q.view(-1)[0] = float("nan")
    elif kind == "v_nan":
        v.view(-1)[0] = float("nan")
    elif kind == "score_nan":
        logits.view(-1)[0] = float("nan")
    elif kind == "score_dtype":
        logits = logits.double()
    elif kind == "score_shape":
        logits = logits[:, :, :-1].contiguous()
    elif kind == "empty_tail":
        k = k[:, :, :0].contiguous()
    with pytest.raises((IntegrityError, NumericalFailure)):
        kernels.af_validate(None, k, q)
        kernels.validate_v(v, q, 17)
        kernels.validate_score(logits, v)
