"""GPU parity of the decode readout through the C-ABI.

Expected values come from the oracle: K/V restored by the C restatement of
nsn_decode, rounded to the attention dtype, then float64 softmax attention.
Tolerance (north star): |ctx - ref| <= 2e-3 + 1e-2 * |ref| elementwise.
"""
import math

import numpy as np
import pytest
import torch

from nsn_amd import cache, codec, kernels
from nsn_amd.errors import IntegrityError, NumericalFailure
from oracle import oracle as O
from tests.golden import inputs as gi

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ATOL, RTOL = 2e-3, 1e-2


def within(got, ref, atol=ATOL, rtol=RTOL):
    err = np.abs(np.asarray(got, np.float64) - ref)
    ok = np.all(err <= atol + rtol * np.abs(ref))
    return ok, float(err.max())


def oracle_restore(x16, length, bits, round_dtype, tail_dtype="float16"):
    """Oracle view of one sequence: x16 [H, T, 128] fp16 -> fp32 [H, length, 128]
    as the kernel sees it (packed prefix restored + rounded, tail as stored in
    ``tail_dtype``)."""
    H = x16.shape[0]
    C = (length // 64) * 64
    parts = []
    if C:
        blocks = x16[:, :C].astype(np.float32).reshape(H, C // 64, 64, 128)
        q, n, m, s, err = O.nsn_encode(blocks, bits)
        assert err == 0
        y = O.nsn_decode_f32(q, n, m, s).reshape(H, C, 128)
        if round_dtype == "float32":          # the fast kernel keeps fp32 reconstructions
            parts.append(y)
        else:
            bitsr = O.cast_bits(y, round_dtype)
            parts.append(O.from_bf16_bits(bitsr) if round_dtype == "bfloat16" else O.from_f16_bits(bitsr))
    if length > C:
        t = x16[:, C:length].astype(np.float32)
        if tail_dtype == "bfloat16":
            t = O.from_bf16_bits(O.cast_bits(t, "bfloat16"))
        parts.append(t)
    return np.concatenate(parts, axis=1)


def make_case(seed, B, Hq, Hkv, lengths, bits=3, gen="kv", tail_dtype=None):
    rng = np.random.default_rng(seed)
    T = max(lengths)
    if gen == "kv":
        from nsn_amd import synthetic
        k = synthetic.kv_tokens(rng, (B, Hkv), T)
        v = synthetic.kv_tokens(rng, (B, Hkv), T)
    else:
        from nsn_amd import synthetic
        k = synthetic.heavy_tailed_tokens(rng, (B, Hkv), T)
        v = synthetic.heavy_tailed_tokens(rng, (B, Hkv), T)
    q = rng.standard_normal((B, Hq, 128)).astype(np.float32)
    qb = torch.from_numpy(q).to(torch.bfloat16)
    kk, seq = cache.pack_sequences(torch.from_numpy(k).to(DEV), lengths, bits=bits, tail_dtype=tail_dtype)
    vv, _ = cache.pack_sequences(torch.from_numpy(v).to(DEV), lengths, bits=bits, tail_dtype=tail_dtype)
    return k, v, qb, kk, vv, seq


def oracle_ctx(k, v, qb, lengths, bits, round_dtype="float16", tail_dtype="float16"):
    B, Hq = qb.shape[:2]
    out = np.zeros((B, Hq, 128))
    q = qb.float().numpy()
    for b, L in enumerate(lengths):
        kr = oracle_restore(k[b], L, bits, round_dtype, tail_dtype)
        vr = oracle_restore(v[b], L, bits, round_dtype, tail_dtype)
        c, _ = O.decode_attention64(q[b:b + 1], kr[None], vr[None])
        out[b] = c[0]
    return out


@pytest.mark.parametrize("kernel", ["reference", "fast"])
@pytest.mark.parametrize("B,Hq,Hkv,lengths", [
    (1, 4, 4, [200]),              # MHA, 3 blocks + 8 tail
    (2, 8, 2, [1000, 333]),        # GQA 4:1, ragged
    (3, 6, 1, [64, 65, 17]),       # GQA 6:1, exact block / block+1 / tail only
    (2, 16, 2, [700, 130]),        # GQA 8:1
])
def test_decode_vs_oracle(kernel, B, Hq, Hkv, lengths):
    k, v, qb, kk, vv, seq = make_case(1, B, Hq, Hkv, lengths)
    out, ctx = kernels.decode_attention(qb.to(DEV), kk, vv, seq, kernel=kernel, kv_round_dtype=torch.float16)
    ref = oracle_ctx(k, v, qb, lengths, 3, "float16" if kernel == "reference" else "float32")
    ok, err = within(ctx.cpu().numpy(), ref)
    assert ok, err
    # the bf16 output is the RNE cast of the fp32 context
    assert torch.equal(out.cpu(), ctx.cpu().to(torch.bfloat16))


@pytest.mark.parametrize("kernel", ["reference", "fast"])
def test_5bit_decode_vs_oracle(kernel):
    lengths = [640, 200]
    k, v, qb, kk, vv, seq = make_case(3, 2, 8, 2, lengths, bits=5, gen="heavy")
    _, ctx = kernels.decode_attention(qb.to(DEV), kk, vv, seq, kernel=kernel, kv_round_dtype=torch.float16)
    ok, err = within(ctx.cpu().numpy(), oracle_ctx(k, v, qb, lengths, 5, "float16" if kernel == "reference" else "float32"))
    assert ok, err


@pytest.mark.parametrize("kernel", ["reference", "fast"])
@pytest.mark.parametrize("bits,Hq,Hkv", [(3, 8, 2), (3, 16, 2), (5, 16, 2)])
def test_decode_fp16_queries_vs_oracle(kernel, bits, Hq, Hkv):
    """fp16 queries (the fp16 query instantiations of both kernels; the fast
    kernel splits them hi + lo as it does bf16 ones), GQA 4:1 and 8:1, 3 and
    5 bits, fp16 tails."""
    lengths = [700, 130]
    k, v, _, kk, vv, seq = make_case(5, 2, Hq, Hkv, lengths, bits=bits)
    rng = np.random.default_rng(55)
    qh = torch.from_numpy(rng.standard_normal((2, Hq, 128)).astype(np.float32)).to(torch.float16)
    out, ctx = kernels.decode_attention(qh.to(DEV), kk, vv, seq, kernel=kernel, kv_round_dtype=torch.float16)
    ref = oracle_ctx(k, v, qh, lengths, bits, "float16" if kernel == "reference" else "float32")
    ok, err = within(ctx.cpu().numpy(), ref)
    assert ok, err
    assert torch.equal(out.cpu(), ctx.cpu().to(torch.bfloat16))


@pytest.mark.parametrize("split", [None, 512])
def test_fast_stream_k_partition_many_sequences(split):
    """More than 64 sequences: the fast kernel cuts the blocks of all streams,
    laid end to end, into equal ranges.  split=512 (>= every length) leaves two
    partial slots per stream, so each range is as long as the longest stream
    and most ranges cross stream boundaries."""
    rng = np.random.default_rng(11)
    lengths = [int(x) for x in rng.integers(1, 400, size=70)]
    lengths[:4] = [64, 128, 1, 399]
    k, v, qb, kk, vv, seq = make_case(11, 70, 8, 2, lengths)
    _, ctx = kernels.decode_attention(qb.to(DEV), kk, vv, seq, kernel="fast", split_tokens=split,
                                      kv_round_dtype=torch.float16)
    ok, err = within(ctx.cpu().numpy(), oracle_ctx(k, v, qb, lengths, 3, "float32"))
    assert ok, err


@pytest.mark.parametrize("kernel", ["reference", "fast"])
def test_merge_of_more_than_64_splits(kernel):
    """79 partial slots per (sequence, q-head) at split 64 over 5000 tokens:
    the merge's loop path (more than 64 slots) against the oracle, and
    against the merge's register path (16 slots at split 320)."""
    lengths = [5000, 300]
    k, v, qb, kk, vv, seq = make_case(6, 2, 8, 2, lengths)
    rnd = "float16" if kernel == "reference" else "float32"
    outs = []
    for split in (64, 320):
        _, ctx = kernels.decode_attention(qb.to(DEV), kk, vv, seq, split_tokens=split, kv_round_dtype=torch.float16,
                                          kernel=kernel)
        ok, err = within(ctx.cpu().numpy(), oracle_ctx(k, v, qb, lengths, 3, rnd))
        assert ok, (split, err)
        outs.append(ctx.cpu().numpy())
    atol, rtol = (1e-5, 1e-5) if kernel == "reference" else (2e-4, 2e-3)
    assert np.allclose(outs[0], outs[1], atol=atol, rtol=rtol)


@pytest.mark.parametrize("kernel", ["reference", "fast"])
def test_split_invariance(kernel):
    lengths = [1500, 900]
    k, v, qb, kk, vv, seq = make_case(5, 2, 8, 2, lengths)
    outs = []
    for split in (64, 256, 1536):
        _, ctx = kernels.decode_attention(qb.to(DEV), kk, vv, seq, split_tokens=split, kv_round_dtype=torch.float16,
                                          kernel=kernel)
        outs.append(ctx.cpu().numpy())
    # The fast kernel's MFMA products carry ~12-19 significant bits relative to
    # the largest term of each dot product (codes enter as fp16 subnormals),
    # and the terms change with the split's running max, so two layouts agree
    # to ~1e-4 there; a merge error would be orders of magnitude larger.
    atol, rtol = (1e-5, 1e-5) if kernel == "reference" else (2e-4, 2e-3)
    for o in outs[1:]:
        assert np.allclose(o, outs[0], atol=atol, rtol=rtol)



@pytest.mark.parametrize("kernel,static", [("reference", False), ("fast", False), ("fast", True)])
def test_prepared_decode_equals_decode_attention(kernel, static):
    """prepare_decode's launcher (argument block built once, as the C2 bench
    and a serving loop use it; with static=True over the library's static
    scratch, so that a launch allocates nothing) gives decode_attention's
    outputs bitwise, and reads the buffers' current contents at every
    launch."""
    lengths = [1500, 900, 64]
    k, v, qb, kk, vv, seq = make_case(8, 3, 8, 2, lengths)
    q = qb.to(DEV)
    kw = dict(max_seq_len=max(lengths), kernel=kernel, split_tokens=256)
    launch = kernels.prepare_decode(q, kk, vv, seq, static_workspace=static, **kw)
    for it in range(3):
        out, ctx = launch()
        torch.cuda.synchronize()
        got_out, got_ctx = out.clone(), ctx.clone()
        want_out, want_ctx = kernels.decode_attention(q, kk, vv, seq, **kw)
        assert torch.equal(got_ctx, want_ctx) and torch.equal(got_out, want_out)
        assert int(launch.status.item()) == 0
        q.mul_(-0.5)   # (new query values in the same storage)
    with pytest.raises(IntegrityError):
        kernels.prepare_decode(q, kk, vv, seq, check=True, **kw)
    with pytest.raises(TypeError):
        kernels.prepare_decode(q, kk, vv, seq, kernel=kernel)   # max_seq_len is required

def test_gqa_equals_repeated_mha():
    """Invariant: q-head h of a GQA call equals an MHA call on kv-head h // G."""
    lengths = [300]
    k, v, qb, kk, vv, seq = make_case(9, 1, 8, 2, lengths)
    _, ctx = kernels.decode_attention(qb.to(DEV), kk, vv, seq, kv_round_dtype=torch.float16)
    krep = np.repeat(k, 4, axis=1)
    vrep = np.repeat(v, 4, axis=1)
    km, _ = cache.pack_sequences(torch.from_numpy(krep).to(DEV), lengths)
    vm, _ = cache.pack_sequences(torch.from_numpy(vrep).to(DEV), lengths)
    _, ctx_m = kernels.decode_attention(qb.to(DEV), km, vm, seq, kv_round_dtype=torch.float16)
    assert torch.equal(ctx.cpu(), ctx_m.cpu())


def _fixture_data(f):
    a = gi.vf01_fixture(f["compressed"], f["length"], f["pattern"])
    bf = lambda x: torch.from_numpy(x.view(np.int16)).view(torch.bfloat16).to(DEV)
    g = vg = None
    if f["compressed"]:
        g = {"codes": torch.from_numpy(a["k_codes"]).to(DEV), "headers": torch.from_numpy(a["k_headers"]).to(DEV),
             "metas": tuple(torch.from_numpy(a[f"k_meta{i}"]).to(DEV) for i in range(3))}
        vg = {"codes": torch.from_numpy(a["v_codes"]).to(DEV), "headers": torch.from_numpy(a["v_headers"]).to(DEV),
              "metas": tuple(torch.from_numpy(a[f"v_meta{i}"]).to(DEV) for i in range(3))}
    return a, (g, bf(a["k_tail"]), bf(a["q"]), vg, bf(a["v_tail"]))


def _fixture_oracle(a, f, round_dtype="bfloat16"):
    """fp64 attention over the oracle-restored K/V of a VF01 fixture (packed
    tokens rounded to bf16, or kept in fp32 with round_dtype='float32')."""
    c, T = f["compressed"], f["length"]
    out = []
    for side in ("k", "v"):
        tail = O.from_bf16_bits(a[side + "_tail"])[0]
        if c:
            n = c // 64
            q = O.unpack_codes(a[side + "_codes"].reshape(-1), 2 * c * 128, 3).reshape(2, n, 64, 128)
            n16 = a[side + "_meta0"].view(np.uint16).reshape(2, n, 64, 1)
            m16 = a[side + "_meta1"].view(np.uint16).reshape(2, n, 1, 128)
            s16 = a[side + "_meta2"].view(np.uint16).reshape(2, n, 1, 128)
            if round_dtype == "float32":
                y = O.nsn_decode_f32(q, n16, m16, s16).reshape(2, c, 128)
            else:
                y = O.from_bf16_bits(O.nsn_decode(q, n16, m16, s16, "bfloat16")).reshape(2, c, 128)
            tail = np.concatenate([y, tail], axis=1)
        out.append(tail)
    q = O.from_bf16_bits(a["q"]).reshape(1, 2, 128)
    ctx, _ = O.decode_attention64(q, out[0][None], out[1][None])
    return ctx[0]


def test_vf01_normal_fixtures_fused_equals_bridge_and_oracle():
    """The reference's 16 normal fixtures (loop_kv_vf01_contract.py:81-96): the fused
    and bridge routes must be bitwise equal (AC/verify_loop_kv_vf01.py:41-50) and
    match the fp64 oracle."""
    import json
    from pathlib import Path
    rec = json.loads((Path(__file__).parent / "golden" / "vf01_input_hashes.json").read_text())
    for f in rec["fixtures"]:
        a, data = _fixture_data(f)
        out_f, ctx_f, _, v_f = kernels.pipeline("V_FUSED", data, trace=True)
        out_b, ctx_b, _, v_b = kernels.pipeline("TILE_MATERIALIZE", data, trace=True)
        out_r = kernels.pipeline("RF01_MATERIALIZE", data)
        assert torch.equal(out_f.view(torch.int16), out_b.view(torch.int16)), f["id"]
        assert torch.equal(ctx_f.view(torch.int32), ctx_b.view(torch.int32)), f["id"]
        assert torch.equal(out_f.view(torch.int16), out_r.view(torch.int16)), f["id"]
        assert torch.equal(v_f.view(torch.int16), v_b.view(torch.int16)), f["id"]
        ref = _fixture_oracle(a, f)
        ok, err = within(ctx_f.cpu().numpy().reshape(2, 128), ref, atol=1e-5, rtol=1e-5)
        assert ok, (f["id"], err)


def test_vf01_fused_trace_is_the_kernels_own():
    """The fused route's trace is what the exact-order kernel itself computed
    (the TRACE stores of loop_kv_vf01_kernel.py:104,113), over the 16 normal
    fixtures: the traced V rows equal the exact restore bitwise, the traced
    scores the fp64 q.k*scale of the restored K within fp32 rounding, and the
    context is the fp64 softmax readout of the traced scores and V within the
    reference's budget 2e-6 + 2e-6*sum_t|p_t v_t| (loop_kv_af01_contract.py:66-72,
    applied to its traces as loop_kv_ac08_audit.py:41 does)."""
    import json
    from pathlib import Path
    rec = json.loads((Path(__file__).parent / "golden" / "vf01_input_hashes.json").read_text())
    for f in rec["fixtures"]:
        a, data = _fixture_data(f)
        g, kt, q, vg, vt = data
        out, ctx, score, v = kernels.pipeline("V_FUSED", data, trace=True)
        T = f["length"]
        assert score.shape == (1, 2, T) and v.shape == (1, 2, T, 128)
        assert torch.equal(v.view(torch.int16), kernels.restore_v(vg, vt).view(torch.int16)), f["id"]
        k64 = kernels.restore_v(g, kt).float().cpu().numpy().astype(np.float64)[0]
        q64 = q.float().cpu().numpy().astype(np.float64).reshape(2, 128)
        gold_s = np.einsum("hd,htd->ht", q64, k64) * O.SCALE
        s = score.cpu().numpy().astype(np.float64)[0]
        s_scale = np.einsum("hd,htd->ht", np.abs(q64), np.abs(k64)) * O.SCALE
        assert (np.abs(s - gold_s) <= 4e-6 * s_scale + 1e-7).all(), f["id"]
        p = O.softmax64(s)
        prod = p[..., None] * v.float().cpu().numpy().astype(np.float64)[0]
        gold = prod.sum(-2)
        err = np.abs(ctx.cpu().numpy().astype(np.float64).reshape(2, 128) - gold)
        assert (err <= 2e-6 + 2e-6 * np.abs(prod).sum(-2)).all(), (f["id"], float(err.max()))


def test_trace_outputs_only_on_the_exact_order_kernel():
    """The fast kernel keeps no per-token scores: a trace request on it is an
    argument error (NSN_EINVAL from the library, IntegrityError here)."""
    from nsn_amd.errors import IntegrityError
    T = 100
    v = torch.randn(1, 1, T, 128, device=DEV).to(torch.float16)
    vv = kernels.PackedKV(None, None, None, None, None, None, v, 3)
    seq = torch.full((1,), T, dtype=torch.int32, device=DEV)
    q = torch.randn(1, 1, 128, device=DEV).to(torch.bfloat16)
    sc = torch.zeros(1, 1, T, device=DEV)
    tr = torch.empty(1, 1, T, device=DEV)
    with pytest.raises(IntegrityError):
        kernels.decode_attention(q, None, vv, seq, scores=sc, kernel="fast", trace_scores=tr)


@pytest.mark.parametrize("kernel", ["reference", "fast"])
def test_score_input_readout_config1(kernel):
    """C1: B=1, 32q/8kv, 64 packed blocks + 37-token fp16 tail; logits N(0,1)*4."""
    rng = np.random.default_rng(1)
    from nsn_amd import synthetic
    T = 4096 + 37
    v = synthetic.kv_tokens(rng, (1, 8), T)
    scores = (rng.standard_normal((1, 32, T)) * 4).astype(np.float32)
    vv, seq = cache.pack_sequences(torch.from_numpy(v).to(DEV), [T])
    qdummy = torch.zeros(1, 32, 128, dtype=torch.bfloat16, device=DEV)
    _, ctx = kernels.decode_attention(qdummy, None, vv, seq, scores=torch.from_numpy(scores).to(DEV),
                                      kv_round_dtype=torch.float16, kernel=kernel)
    vr = oracle_restore(v[0], T, 3, "float16" if kernel == "reference" else "float32")
    ref = O.readout64(scores, vr[None], groups=4)
    ok, err = within(ctx.cpu().numpy(), ref)
    assert ok, err
    # bridge: V restored to HBM, then the same readout -> bitwise equal
    vfull = codec.restore(vv.codes[0], (vv.norm[0], vv.min[0], vv.scale[0]), 3, torch.float16,
                          tail=vv.tail[0, :, :37])
    vd = kernels.PackedKV(None, None, None, None, None, None, vfull[None].contiguous(), 3)
    _, ctx_b = kernels.decode_attention(qdummy, None, vd, seq, scores=torch.from_numpy(scores).to(DEV),
                                        kv_round_dtype=torch.float16, kernel=kernel)
    if kernel == "reference":
        assert torch.equal(ctx.cpu(), ctx_b.cpu())
    else:
        ok, err = within(ctx_b.cpu().numpy(), ref)
        assert ok, err


@pytest.mark.parametrize("kernel", ["reference", "fast"])
@pytest.mark.parametrize("bits,Hq,Hkv,tail", [(5, 8, 2, "float16"), (3, 16, 2, "bfloat16"),
                                               (5, 16, 2, "bfloat16")])
def test_score_input_readout_ragged(kernel, bits, Hq, Hkv, tail):
    """Score-input readout beyond C1: two ragged sequences, 5-bit V, GQA 8:1,
    bf16 tails (the kernels' score-input instantiations past the C1 one)."""
    rng = np.random.default_rng(31)
    from nsn_amd import synthetic
    lengths = [700, 130]
    T = max(lengths)
    v = synthetic.kv_tokens(rng, (2, Hkv), T)
    scores = (rng.standard_normal((2, Hq, T)) * 4).astype(np.float32)
    tdt = torch.bfloat16 if tail == "bfloat16" else torch.float16
    vv, seq = cache.pack_sequences(torch.from_numpy(v).to(DEV), lengths, bits=bits, tail_dtype=tdt)
    qdummy = torch.zeros(2, Hq, 128, dtype=torch.bfloat16, device=DEV)
    _, ctx = kernels.decode_attention(qdummy, None, vv, seq, scores=torch.from_numpy(scores).to(DEV),
                                      kv_round_dtype=tdt, kernel=kernel)
    got = ctx.cpu().numpy()
    for b, L in enumerate(lengths):
        vr = oracle_restore(v[b], L, bits, tail if kernel == "reference" else "float32", tail)
        ref = O.readout64(scores[b:b + 1, :, :L], vr[None], groups=Hq // Hkv)
        ok, err = within(got[b:b + 1], ref)
        assert ok, (b, err)


@pytest.mark.parametrize("mode", ["dense", "bridge"])
def test_fast_dense_and_bridge_vs_oracle(mode):
    """fp16-KV baseline (no packed blocks) and the bridge (packed K, restored V)."""
    lengths = [1000, 333]
    k, v, qb, kk, vv, seq = make_case(11, 2, 8, 2, lengths)
    if mode == "dense":
        kd = kernels.PackedKV(None, None, None, None, None, None, torch.from_numpy(k).to(DEV), 3)
        vd = kernels.PackedKV(None, None, None, None, None, None, torch.from_numpy(v).to(DEV), 3)
        _, ctx = kernels.decode_attention(qb.to(DEV), kd, vd, seq, kernel="fast")
        ref = np.zeros((2, 8, 128))
        for b, L in enumerate(lengths):
            c, _ = O.decode_attention64(qb.float().numpy()[b:b + 1], k[b:b + 1, :, :L].astype(np.float32),
                                        v[b:b + 1, :, :L].astype(np.float32))
            ref[b] = c[0]
    else:
        vfull = torch.zeros((2, 2, 1000, 128), dtype=torch.float16, device=DEV)
        for b, L in enumerate(lengths):
            nb = L // 64
            vfull[b, :, :L] = codec.restore(vv.codes[b, :, :nb].contiguous(), (vv.norm[b, :, :nb], vv.min[b, :, :nb],
                                            vv.scale[b, :, :nb]), 3, torch.float16, tail=vv.tail[b, :, :L - nb * 64])
        vd = kernels.PackedKV(None, None, None, None, None, None, vfull, 3)
        _, ctx = kernels.decode_attention(qb.to(DEV), kk, vd, seq, kernel="fast")
        # K packed (fp32 reconstruction in-kernel) and V restored to fp16 in HBM
        ref = np.zeros((2, 8, 128))
        for b, L in enumerate(lengths):
            kr = oracle_restore(k[b], L, 3, "float32")
            vr = oracle_restore(v[b], L, 3, "float16")
            c, _ = O.decode_attention64(qb.float().numpy()[b:b + 1], kr[None], vr[None])
            ref[b] = c[0]
    ok, err = within(ctx.cpu().numpy(), ref)
    assert ok, err


def test_fast_matches_reference_launch_surface():
    """The reference-shaped launch() with the fast kernel (fp16 tails) agrees with the exact-order kernel."""
    rng = np.random.default_rng(12)
    from nsn_amd import synthetic
    x = synthetic.kv_tokens(rng, (2, 8), 64 * 5 + 21)
    k16 = torch.from_numpy(x[0]).to(DEV)[None]
    v16 = torch.from_numpy(x[1]).to(DEV)[None]
    g = codec.encode_group(k16[:, :, :320].reshape(1, 8, 5, 64, 128).contiguous(), 0)
    vg = codec.encode_group(v16[:, :, :320].reshape(1, 8, 5, 64, 128).contiguous(), 0)
    kt, vt = k16[:, :, 320:].contiguous(), v16[:, :, 320:].contiguous()
    q = torch.from_numpy(rng.standard_normal((1, 32, 1, 128)).astype(np.float32)).to(torch.bfloat16).to(DEV)
    _, c_ref, _, _ = kernels.launch(g, kt, q, vg, vt, kernel="reference")
    _, c_fast, _, _ = kernels.launch(g, kt, q, vg, vt, kernel="fast")
    ok, err = within(c_fast.cpu().numpy(), c_ref.cpu().numpy().astype(np.float64))
    assert ok, err


@pytest.mark.parametrize("kernel", ["reference", "fast"])
def test_batch1_routes_check_lengths_on_the_host(kernel):
    """launch() and af_launch() build the sequence length and block counts
    from the tensor shapes and check them on the host: K and V of different
    lengths, or an empty sequence, raise IntegrityError before any launch,
    and a consistent call still matches the checked general entry."""
    rng = np.random.default_rng(13)
    from nsn_amd import synthetic
    x = synthetic.kv_tokens(rng, (2, 4), 64 * 3 + 10)
    k16 = torch.from_numpy(x[0]).to(DEV)[None]
    v16 = torch.from_numpy(x[1]).to(DEV)[None]
    g = codec.encode_group(k16[:, :, :192].reshape(1, 4, 3, 64, 128).contiguous(), 0)
    vg = codec.encode_group(v16[:, :, :192].reshape(1, 4, 3, 64, 128).contiguous(), 0)
    kt, vt = k16[:, :, 192:].contiguous(), v16[:, :, 192:].contiguous()
    q = torch.from_numpy(rng.standard_normal((1, 8, 1, 128)).astype(np.float32)).to(torch.bfloat16).to(DEV)
    with pytest.raises(IntegrityError, match="K/V lengths differ"):
        kernels.launch(g, kt, q, vg, vt[:, :, :9].contiguous(), kernel=kernel)
    with pytest.raises(IntegrityError, match="Empty sequence"):
        kernels.launch(None, kt[:, :, :0].contiguous(), q, None, vt[:, :, :0].contiguous(), kernel=kernel)
    vdense = kernels.restore_v(vg, vt)
    with pytest.raises(IntegrityError, match="K/V lengths differ"):
        kernels.af_launch(g, kt, q, vdense[:, :, :200].contiguous(), full=True, kernel=kernel)
    # consistent: the same context as the general entry with its device-side length check
    _, c1, _, _ = kernels.launch(g, kt, q, vg, vt, kernel=kernel)
    ks, vs = kernels._fast_sides(((g, kt), (vg, vt)), kernel == "fast", None, DEV)
    seq = torch.full((1,), 202, dtype=torch.int32, device=DEV)
    _, c2 = kernels.decode_attention(q.reshape(1, 8, 128), ks, vs, seq, max_seq_len=202, kernel=kernel,
                                     kv_round_dtype=kt.dtype)
    assert torch.equal(c1.reshape(1, 8, 128), c2)


@pytest.mark.parametrize("fused", [True, False])
def test_negative_fixtures_rejected_at_reference_stage(fused, monkeypatch):
    """NaN/Inf inputs stop at 'input_finite'; overflowing scores at 'attention'
    (loop_kv_vf01_contract.py:98-120) -- with the finite check fused into the
    attention kernel (no separate scan is launched) and with the grouped scan."""
    monkeypatch.setattr(kernels, "FUSED_VALIDATION", fused)
    if fused:
        def no_scan(*a, **k):
            raise AssertionError("separate finite scan launched")
        monkeypatch.setattr(kernels, "finite", no_scan)
    f = {"compressed": 64, "length": 65, "pattern": "mixed_codes"}
    a, (g, kt, q, vg, vt) = _fixture_data(f)
    q2 = q.clone()
    q2.view(-1)[0] = float("nan")
    with pytest.raises(NumericalFailure):
        kernels.pipeline("V_FUSED", (g, kt, q2, vg, vt))
    assert kernels.LAST_STAGE == "input_finite"
    vg2 = dict(vg)
    m = vg["metas"][0].clone()
    m.view(-1)[-1] = float("inf")
    vg2["metas"] = (m, vg["metas"][1], vg["metas"][2])
    with pytest.raises(NumericalFailure):
        kernels.pipeline("V_FUSED", (g, kt, q, vg2, vt))
    assert kernels.LAST_STAGE == "input_finite"
    # score overflow: q = K tail = 2**120 (tail only, T=17)
    big = torch.full((1, 2, 1, 128), 2.0 ** 120, dtype=torch.bfloat16, device=DEV)
    tail = torch.full((1, 2, 17, 128), 2.0 ** 120, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(NumericalFailure):
        kernels.pipeline("V_FUSED", (None, tail, big, None, tail.clone()))
    assert kernels.LAST_STAGE == "attention"


def test_fast_kernel_flags_nonfinite_raw_input():
    """The fast kernel's fused finite check: a NaN query or tail token raises
    as a raw-input failure, not as an attention intermediate."""
    lengths = [200, 70]
    k, v, qb, kk, vv, seq = make_case(7, 2, 8, 2, lengths)
    q2 = qb.clone()
    q2[1, 3, 5] = float("nan")
    with pytest.raises(NumericalFailure, match="raw attention input"):
        kernels.decode_attention(q2.to(DEV), kk, vv, seq, kernel="fast")
    vv.tail[0, 1, 3, 7] = float("inf")          # token 64*3 + 3 of sequence 0 (tail)
    with pytest.raises(NumericalFailure, match="raw attention input"):
        kernels.decode_attention(qb.to(DEV), kk, vv, seq, kernel="fast")


def test_capacity_guard_with_device_lengths():
    """check=False (a graph replay's mode): a length past the cache's blocks +
    tail capacity is refused on the device -- nothing of that sequence is
    read and NSN_ST_CAPACITY is raised -- instead of reading past the tail.
    The prefill kernel refuses a block count past block_cap the same way."""
    from nsn_amd import _dev, _lib
    k, v, qb, kk, vv, seq = make_case(7, 2, 8, 2, [700, 300])
    assert kk.tail.shape[2] == 64 and int(kk.blocks[1]) == 4          # capacity of sequence 1: 4*64 + 64 tokens
    bad = torch.tensor([700, 300 + 640], dtype=torch.int32, device=DEV)
    print("capacity case: decode, seq_len [700, 940] against capacity 320", flush=True)
    st = _dev.new_status(DEV)
    kernels.decode_attention(qb.to(DEV), kk, vv, bad, max_seq_len=940, kernel="fast", check=False, status=st)
    assert _dev.read_status(st) & _lib.ST_CAPACITY
    with pytest.raises(Exception, match="capacity|Tail exceeds"):
        kernels.decode_attention(qb.to(DEV), kk, vv, bad, max_seq_len=940, kernel="fast")
    print("capacity case: prefill, blocks past block_cap", flush=True)
    kk.blocks[1] = kk.codes.shape[2] + 1
    vv.blocks[1] = kk.codes.shape[2] + 1
    ctx_len = torch.tensor([700, 64 * (kk.codes.shape[2] + 1)], dtype=torch.int32, device=DEV)
    q = torch.zeros((2, 8, 16, 128), dtype=torch.float16, device=DEV)
    ch = torch.zeros((2, 2, 16, 128), dtype=torch.float16, device=DEV)
    kk.tail, vv.tail = kk.tail.to(torch.float16), vv.tail.to(torch.float16)
    st = _dev.new_status(DEV)
    kernels.prefill_attention(q, kk, vv, ctx_len, ch, ch, check=False, status=st)
    assert _dev.read_status(st) & _lib.ST_CAPACITY


@pytest.mark.parametrize("kernel", ["fast", "reference"])
def test_empty_and_over_capacity_sequences_with_device_lengths(kernel):
    """check=False: a sequence of length 0, and one whose length lies past the
    cache's capacity, attend nothing -- both kernels write partial count 0,
    the merge writes a zero output and raises NSN_ST_EMPTY (the latter also
    NSN_ST_CAPACITY) -- while the other sequences still match the oracle.
    The merge never reads a slot the call did not write: the workspace is
    filled with NaN first, so a stale read would show as a nonfinite output."""
    from nsn_amd import _dev, _lib
    lengths = [700, 300, 130, 64]
    k, v, qb, kk, vv, seq = make_case(8, 4, 8, 2, lengths)
    split, n_splits = kernels.default_split(4, 2, 700)
    n_splits = max(2, n_splits)
    ws = torch.full((kernels.workspace_floats(4, 8, n_splits),), float("nan"), dtype=torch.float32, device=DEV)
    dev_len = torch.tensor([700, 0, 130, 64 * int(kk.blocks[3]) + kk.tail.shape[2] + 1], dtype=torch.int32,
                           device=DEV)
    print(f"empty/over-capacity case: kernel {kernel}, lengths {dev_len.tolist()}", flush=True)
    st = _dev.new_status(DEV)
    _, ctx = kernels.decode_attention(qb.to(DEV), kk, vv, dev_len, max_seq_len=700, kernel=kernel, check=False,
                                      status=st, split_tokens=split, workspace=ws)
    s = _dev.read_status(st)
    assert s & _lib.ST_EMPTY and s & _lib.ST_CAPACITY, hex(s)
    assert not s & (_lib.ST_NONFINITE_OUTPUT | _lib.ST_NONFINITE_ATTN), hex(s)
    got = ctx.cpu().numpy()
    assert np.all(got[1] == 0) and np.all(got[3] == 0)
    ref = oracle_ctx(k[[0, 2]], v[[0, 2]], qb[[0, 2]], [700, 130], 3, "float32" if kernel == "fast" else "float16")
    ok, err = within(got[[0, 2]], ref)
    assert ok, err


@pytest.mark.parametrize("Hq,Hkv,bits", [(8, 2, 3), (32, 4, 3), (8, 2, 5), (16, 8, 5), (16, 2, 5)])
def test_fast_bf16_tails_vs_oracle(Hq, Hkv, bits):
    """bf16 tails (the reference's dtype, loop_kv_qk01_kernel.py:66-69) on the
    fast kernel's bf16 MFMA path; packed tokens keep fp32 reconstructions."""
    lengths = [1000, 333, 320, 70]
    k, v, qb, kk, vv, seq = make_case(21, 4, Hq, Hkv, lengths, bits=bits, tail_dtype=torch.bfloat16)
    assert kk.tail.dtype == torch.bfloat16
    _, ctx = kernels.decode_attention(qb.to(DEV), kk, vv, seq, kernel="fast")
    ref = oracle_ctx(k, v, qb, lengths, bits, "float32", "bfloat16")
    ok, err = within(ctx.cpu().numpy(), ref)
    assert ok, err


def test_fast_bf16_dense_beyond_fp16_range():
    """A dense bf16 K/V (no packed blocks) holding values past fp16's range
    (|x| up to 3e6) computes on the bf16 path instead of overflowing."""
    rng = np.random.default_rng(22)
    B, Hq, Hkv, T = 2, 8, 2, 300
    k = rng.standard_normal((B, Hkv, T, 128)).astype(np.float32) * 0.05
    v = rng.standard_normal((B, Hkv, T, 128)).astype(np.float32)
    k[:, :, 17] *= 1e3          # large keys: scores of order 1e2
    v[:, :, 5::7] *= 3e6        # values beyond 65504
    kb = O.from_bf16_bits(O.cast_bits(k, "bfloat16"))
    vb = O.from_bf16_bits(O.cast_bits(v, "bfloat16"))
    qb = torch.from_numpy(rng.standard_normal((B, Hq, 128)).astype(np.float32)).to(torch.bfloat16)
    kd = kernels.PackedKV(None, None, None, None, None, None, torch.from_numpy(kb).to(torch.bfloat16).to(DEV), 3)
    vd = kernels.PackedKV(None, None, None, None, None, None, torch.from_numpy(vb).to(torch.bfloat16).to(DEV), 3)
    seq = torch.tensor([T, 251], dtype=torch.int32, device=DEV)
    _, ctx = kernels.decode_attention(qb.to(DEV), kd, vd, seq, kernel="fast")
    ref = np.zeros((B, Hq, 128))
    for b, L in enumerate([T, 251]):
        c, _ = O.decode_attention64(qb.float().numpy()[b:b + 1], kb[b:b + 1, :, :L], vb[b:b + 1, :, :L])
        ref[b] = c[0]
    scale = np.abs(ref).max(axis=-1, keepdims=True)     # (errors relative to each row's magnitude)
    ok, err = within(ctx.cpu().numpy() / scale, ref / scale)
    assert ok, err


@pytest.mark.parametrize("arm", ["V_FUSED", "TILE_MATERIALIZE", "RF01_MATERIALIZE"])
def test_vf01_normal_fixtures_on_the_fast_kernel(arm):
    """The 16 VF01 fixtures (bf16 tails and queries, the reference's dtypes)
    through every arm on the fast kernel, against the fp64 oracle over fp32
    reconstructions (fused arm) or the bf16-rounded restore (bridge arms)."""
    import json
    from pathlib import Path
    rec = json.loads((Path(__file__).parent / "golden" / "vf01_input_hashes.json").read_text())
    for f in rec["fixtures"]:
        a, data = _fixture_data(f)
        _, ctx, _, _ = kernels.pipeline(arm, data, trace=True, kernel="fast")
        assert kernels.LAST_STAGE == "returned"
        ref = _fixture_oracle(a, f, "float32" if arm == "V_FUSED" else "bfloat16")
        ok, err = within(ctx.cpu().numpy().reshape(2, 128), ref)
        assert ok, (f["id"], err)
