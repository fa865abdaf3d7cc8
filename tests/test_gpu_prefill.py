"""GPU parity of the chunked-prefill attention (nsn_prefill_attention) through the C-ABI.

Expected values: the context K/V restored by the oracle (C restatement of
nsn_encode + nsn_decode, fp32 reconstructions), the tail and the chunk K/V as
stored, then the oracle's float64 chunked-prefill attention
(oracle.prefill_attention64, pinned row by row against the decode oracle).
Tolerance (north star): |out - ref| <= 2e-3 + 1e-2 * |ref| elementwise, on
top of the output's own rounding (bf16/fp16).  K/V and queries are N(0,1)
activations, as in the chunked-prefill configuration: the kernel's MFMA
operands are fp16 (11-bit significands), so its absolute error grows with
the largest |v| a query attends to (about 2^-12 of it).
"""
import numpy as np
import pytest
import torch

from nsn_amd import cache, kernels
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ATOL, RTOL = 2e-3, 1e-2
SCALE = 0.08838834764831845


def normal_tokens(rng, prefix, ntok):
    """fp16 [*prefix, ntok, 128] N(0,1) activations (the C4 configuration's K/V)."""
    return rng.standard_normal(tuple(prefix) + (ntok, 128)).astype(np.float16)


def restore_ctx(x16, length, bits, dtype):
    """[H, T, 128] fp16 source -> fp32 [H, length, 128]: packed blocks restored
    (fp32), tail tokens as stored in `dtype`."""
    H = x16.shape[0]
    C = (length // 64) * 64
    parts = []
    if C:
        blocks = x16[:, :C].astype(np.float32).reshape(H, C // 64, 64, 128)
        q, n, m, s, err = O.nsn_encode(blocks, bits)
        assert err == 0
        parts.append(O.nsn_decode_f32(q, n, m, s).reshape(H, C, 128))
    if length > C:
        parts.append(torch.from_numpy(x16[:, C:length]).to(dtype).float().numpy())
    return np.concatenate(parts, axis=1) if parts else np.zeros((H, 0, 128), np.float32)


def run_case(seed, B, Hq, Hkv, ctx_lengths, n, bits, dtype):
    rng = np.random.default_rng(seed)
    T = max(max(ctx_lengths), 1)
    kx = normal_tokens(rng, (B, Hkv), T)
    vx = normal_tokens(rng, (B, Hkv), T)
    kch = torch.from_numpy(normal_tokens(rng, (B, Hkv), n)).to(dtype)
    vch = torch.from_numpy(normal_tokens(rng, (B, Hkv), n)).to(dtype)
    q = torch.from_numpy(rng.standard_normal((B, Hq, n, 128)).astype(np.float32)).to(dtype)
    if max(ctx_lengths) > 0:
        kk, seq = cache.pack_sequences(torch.from_numpy(kx).to(DEV), ctx_lengths, bits=bits, tail_dtype=dtype)
        vv, _ = cache.pack_sequences(torch.from_numpy(vx).to(DEV), ctx_lengths, bits=bits, tail_dtype=dtype)
    else:
        kk = vv = None
        seq = torch.zeros(B, dtype=torch.int32, device=DEV)
    out = kernels.prefill_attention(q.to(DEV), kk, vv, seq, kch.to(DEV), vch.to(DEV))
    got = out.float().cpu().numpy()
    for b in range(B):
        L = ctx_lengths[b]
        kc = restore_ctx(kx[b], L, bits, dtype)
        vc = restore_ctx(vx[b], L, bits, dtype)
        ref = O.prefill_attention64(q[b].float().numpy(), kc, vc, kch[b].float().numpy(), vch[b].float().numpy())
        ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11      # output rounding
        err = np.abs(got[b] - ref)
        bound = ATOL + (RTOL + ulp) * np.abs(ref)
        assert np.all(err <= bound), (b, float(err.max()), float((err / bound).max()))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_packed_context_tail_and_chunk(dtype):
    # sequence 0: 4 blocks + 44 tail tokens; sequence 1: 1 block + 13 tail; one query tile of 150
    run_case(21, 2, 4, 2, [300, 77], 150, 3, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_second_query_tile_ragged(dtype):
    """A workgroup covers 256 chunk queries: 520 queries take three tiles, the
    last with 8 rows, so the query offset, the end clamp and the causal mask
    of queries >= 256 against chunk blocks are all compared with the oracle."""
    run_case(25, 2, 4, 2, [300, 77], 520, 3, dtype)


def test_prefill_c4_chunk_of_512():
    # the C4 chunk size (two full query tiles) over a packed context + tail, GQA 2:1
    run_case(26, 2, 4, 2, [1000, 130], 512, 3, torch.float16)


def test_prefill_no_context_is_causal_attention():
    run_case(22, 1, 2, 2, [0], 200, 3, torch.bfloat16)


def test_prefill_block_aligned_context_gqa8():
    # context of whole blocks only (no tail); 8 q-heads per kv-head
    run_case(23, 1, 8, 1, [256], 64, 3, torch.bfloat16)


def test_prefill_5bit():
    run_case(24, 2, 2, 2, [192, 100], 70, 5, torch.float16)
