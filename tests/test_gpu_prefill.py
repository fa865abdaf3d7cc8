"""GPU parity of the chunked-prefill attention (nsn_prefill_attention) through the C-ABI.

Expected values: the context K/V restored by the oracle (C restatement of
nsn_encode + nsn_decode: fp32 reconstructions for fp16 data, rounded to bf16
for bf16 data as the reference's restore returns them), the tail and the
chunk K/V as stored, then the oracle's float64 chunked-prefill attention
(oracle.prefill_attention64, pinned row by row against the decode oracle).
Tolerance (north star): |out - ref| <= 2e-3 + 1e-2 * |ref| elementwise, plus
the output's own rounding (bf16: 2^-8, fp16: 2^-11 relative) and nothing
else.  K/V and queries are N(0,1) activations, as in the chunked-prefill
configuration, except where a test scales them.
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


def restore_ctx(x16, length, bits, dtype, packed_dtype=None):
    """[H, T, 128] fp16 source -> fp32 [H, length, 128]: packed blocks restored
    (fp32, rounded to ``packed_dtype`` when bf16), tail tokens as stored in `dtype`."""
    H = x16.shape[0]
    C = (length // 64) * 64
    parts = []
    if C:
        blocks = x16[:, :C].astype(np.float32).reshape(H, C // 64, 64, 128)
        q, n, m, s, err = O.nsn_encode(blocks, bits)
        assert err == 0
        y = O.nsn_decode_f32(q, n, m, s).reshape(H, C, 128)
        if packed_dtype == torch.bfloat16:
            y = O.from_bf16_bits(O.cast_bits(y, "bfloat16"))
        parts.append(y)
    if length > C:
        parts.append(torch.from_numpy(x16[:, C:length]).to(dtype).float().numpy())
    return np.concatenate(parts, axis=1) if parts else np.zeros((H, 0, 128), np.float32)


def run_case(seed, B, Hq, Hkv, ctx_lengths, n, bits, dtype, tail_dtype=None, chunk_scale=None, weighted=0.0,
             precise=None):
    """chunk_scale: optional [n] multipliers of the chunk's V rows (values past
    fp16's range).  weighted: a term added to the bound, times the attention
    over |V| (only the out-of-fp16-range case uses it; see there)."""
    rng = np.random.default_rng(seed)
    tail_dtype = tail_dtype or dtype
    T = max(max(ctx_lengths), 1)
    kx = normal_tokens(rng, (B, Hkv), T)
    vx = normal_tokens(rng, (B, Hkv), T)
    kch = torch.from_numpy(normal_tokens(rng, (B, Hkv), n)).to(dtype)
    vch = torch.from_numpy(normal_tokens(rng, (B, Hkv), n)).to(dtype)
    if chunk_scale is not None:
        vch = (vch.float() * torch.from_numpy(chunk_scale.astype(np.float32))[None, None, :, None]).to(dtype)
    q = torch.from_numpy(rng.standard_normal((B, Hq, n, 128)).astype(np.float32)).to(dtype)
    if max(ctx_lengths) > 0:
        kk, seq = cache.pack_sequences(torch.from_numpy(kx).to(DEV), ctx_lengths, bits=bits, tail_dtype=tail_dtype)
        vv, _ = cache.pack_sequences(torch.from_numpy(vx).to(DEV), ctx_lengths, bits=bits, tail_dtype=tail_dtype)
    else:
        kk = vv = None
        seq = torch.zeros(B, dtype=torch.int32, device=DEV)
    out = kernels.prefill_attention(q.to(DEV), kk, vv, seq, kch.to(DEV), vch.to(DEV), precise_weights=precise)
    got = out.float().cpu().numpy()
    for b in range(B):
        L = ctx_lengths[b]
        kc = restore_ctx(kx[b], L, bits, tail_dtype, dtype)
        vc = restore_ctx(vx[b], L, bits, tail_dtype, dtype)
        ref = O.prefill_attention64(q[b].float().numpy(), kc, vc, kch[b].float().numpy(), vch[b].float().numpy())
        ulp = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11      # the output's own rounding
        err = np.abs(got[b] - ref)
        bound = ATOL + (RTOL + ulp) * np.abs(ref)
        if weighted:
            bound = bound + weighted * O.prefill_attention64(q[b].float().numpy(), kc, np.abs(vc),
                                                             kch[b].float().numpy(), np.abs(vch[b].float().numpy()))
        ratio = float((err / bound).max())
        print(f"prefill case seed {seed} sequence {b}: max err {float(err.max()):.2e}, max err/bound {ratio:.3f}",
              flush=True)
        assert ratio <= 1.0, (b, float(err.max()), ratio)


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


@pytest.mark.parametrize("precise", [None, False])
def test_prefill_no_context_is_causal_attention(precise):
    """No context: by default (None) the bf16 weights carry their lo parts; the
    single-rounded form (False) is held to the same bound."""
    run_case(22, 1, 2, 2, [0], 200, 3, torch.bfloat16, precise=precise)


def test_prefill_block_aligned_context_gqa8():
    # context of whole blocks only (no tail); 8 q-heads per kv-head
    run_case(23, 1, 8, 1, [256], 64, 3, torch.bfloat16)


def test_prefill_5bit():
    run_case(24, 2, 2, 2, [192, 100], 70, 5, torch.float16)


@pytest.mark.parametrize("tail_dtype,precise", [(torch.bfloat16, None), (torch.float16, None),
                                                (torch.float16, True)])
def test_prefill_5bit_bf16_products(tail_dtype, precise):
    """5-bit packed context under bf16 queries and chunk (the bf16 MFMA form of
    the 5-bit kernel): over a bf16 or an fp16 tail, single-rounded or hi + lo
    weights, across two query tiles with a ragged second one."""
    run_case(29, 2, 4, 2, [300, 77], 300, 5, torch.bfloat16, tail_dtype=tail_dtype, precise=precise)


@pytest.mark.parametrize("precise", [None, True])
def test_prefill_bf16_products_with_an_fp16_tail(precise):
    """C4's mix: bf16 queries and chunk on the bf16 MFMA over an fp16 tail,
    with single-rounded weights (the default over a context) and with the
    weights as bf16 hi + lo (precise_weights=True)."""
    run_case(27, 2, 4, 2, [300, 77], 150, 3, torch.bfloat16, tail_dtype=torch.float16, precise=precise)


def test_prefill_bf16_values_beyond_fp16_range():
    """bf16 chunk values of order 1e6 compute on the bf16 products (fp16 would
    overflow).  This is a range test, not a precision test: with values of
    order 1e6 of both signs the output cancels to far below them, and no fp32
    computation meets an absolute 2e-3 there (fp32 softmax weights alone carry
    2^-24 of the attention-weighted |v|, ~0.06).  The bound therefore adds
    2^-8 of the attention-weighted |v| (the bf16 weights' rounding); every
    N(0,1) case above is held to the north-star bound alone."""
    scale = np.ones(200)
    scale[3::11] = 1e6
    run_case(28, 1, 2, 2, [130], 200, 3, torch.bfloat16, chunk_scale=scale, weighted=2.0 ** -8)
