"""GPU parity at the full shapes of the benchmark configurations (BASELINE.json
configs[2], [3], [4]) against the oracle.

Each test builds its configuration exactly as bench.py does (the generators
of nsn_amd.synthetic, on the GPU), runs the HIP path through the C-ABI, and
then checks, on the host:

- every packed block (codes, fp16 norm / min / scale) bit-equal to the C
  oracle's encode of the same 64 tokens;
- attention outputs within 2e-3 + 1e-2*|ref| of the oracle's float64
  attention over the oracle-restored K/V (fp32 reconstructions, the tail as
  stored), plus the output's own rounding where the output is bf16/fp16
  (2^-8 relative for bf16) and nothing else.

C2: B=16, 32q/8kv, ragged 16K..32K, INT3 + fp16 tail (the headline step),
    the fast kernel, the exact-order kernel, and the fp16-KV baseline.
C3: 5-bit, B=64, 16q/4kv, 8192 tokens, heavy-tailed channels.
C4: the streaming cache (MHA 16 kv-heads, B=32): the 8,192-token chunked
    prefill in bf16 chunks of 512 over the fp16 tail, attention and append in
    one launch as bench.py times it (chunks 0, 1 and 15 compared: no context,
    one chunk of context, 119 packed blocks + 64 tail tokens), and the same
    prefill followed by 256 decode steps with the compression policy.  Attention is compared on a subset of sequences /
    heads (the float64 oracle of a full 512 x 8192 prefill is ~1 TFLOP);
    the packed state is compared on all of them.
"""
import numpy as np
import pytest
import torch

from nsn_amd import cache, kernels, synthetic
from nsn_amd.stream_cache import StreamingKVCache
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
ATOL, RTOL = 2e-3, 1e-2


def say(*a):
    print("[configs]", *a, flush=True)


def within(got, ref, ulp=0.0):
    err = np.abs(np.asarray(got, np.float64) - ref)
    return bool(np.all(err <= ATOL + (RTOL + ulp) * np.abs(ref))), float(err.max())


def ratio(got, ref, ulp=0.0):
    """max of |got - ref| / bound: <= 1 passes."""
    err = np.abs(np.asarray(got, np.float64) - ref)
    return float((err / (ATOL + (RTOL + ulp) * np.abs(ref))).max())


def oracle_history(x16, L, bits, side=None, row=None, packed=None):
    """One sequence's K or V as the kernels see it: x16 fp16 [H, >=L, 128] ->
    fp32 [H, L, 128] (the first `packed` tokens -- default all whole blocks --
    restored by the oracle, the rest as stored).  With `side` (a PackedKV) and
    `row` (its batch index), the GPU's packed blocks of that row are first
    checked bit for bit against the oracle's."""
    H = x16.shape[0]
    C = (L // 64) * 64 if packed is None else packed
    parts = []
    if C:
        nb = C // 64
        q, n, m, s, err = O.nsn_encode(x16[:, :C].astype(np.float32).reshape(H, nb, 64, 128), bits)
        assert err == 0
        if side is not None:
            assert int(side.blocks[row]) == nb
            codes = O.pack_codes(q.reshape(H * nb, -1), bits).reshape(H, nb, -1)
            assert np.array_equal(side.codes[row, :, :nb].cpu().numpy(), codes), "packed codes differ"
            assert np.array_equal(side.norm[row, :, :nb].cpu().numpy().view(np.uint16), n.reshape(H, nb, 64))
            assert np.array_equal(side.min[row, :, :nb].cpu().numpy().view(np.uint16), m.reshape(H, nb, 128))
            assert np.array_equal(side.scale[row, :, :nb].cpu().numpy().view(np.uint16), s.reshape(H, nb, 128))
        parts.append(O.nsn_decode_f32(q, n, m, s).reshape(H, C, 128))
    if L > C:
        parts.append(x16[:, C:L].astype(np.float32))
    return np.concatenate(parts, axis=1) if parts else np.zeros((H, 0, 128), np.float32)


# ------------------------------------------------------------------ C2

def test_c2_full_shape_decode_vs_oracle():
    lengths, k, v, q = synthetic.c2_workload(DEV)
    say(f"C2 lengths {lengths}")
    kk, seq = cache.pack_sequences(k, lengths, bits=3, tail_dtype=torch.float16)
    vv, _ = cache.pack_sequences(v, lengths, bits=3, tail_dtype=torch.float16)
    L = max(lengths)
    out_f, ctx_f = kernels.decode_attention(q, kk, vv, seq, max_seq_len=L, kernel="fast")
    _, ctx_r = kernels.decode_attention(q, kk, vv, seq, max_seq_len=L, kernel="reference",
                                        kv_round_dtype=torch.float32)
    dk = kernels.PackedKV(None, None, None, None, None, None, k, 3)
    dv = kernels.PackedKV(None, None, None, None, None, None, v, 3)
    _, ctx_d = kernels.decode_attention(q, dk, dv, seq, max_seq_len=L, kernel="fast")   # fp16-KV baseline
    torch.cuda.synchronize()
    assert torch.equal(out_f, ctx_f.to(torch.bfloat16))
    ctx_f, ctx_r, ctx_d = (c.cpu().numpy() for c in (ctx_f, ctx_r, ctx_d))
    qn = q.float().cpu().numpy()
    worst = [0.0, 0.0, 0.0]
    for b, Lb in enumerate(lengths):
        kx = k[b, :, :Lb].cpu().numpy()
        vx = v[b, :, :Lb].cpu().numpy()
        kr = oracle_history(kx, Lb, 3, kk, b)
        vr = oracle_history(vx, Lb, 3, vv, b)
        ref, _ = O.decode_attention64(qn[b:b + 1], kr[None], vr[None])
        dref, _ = O.decode_attention64(qn[b:b + 1], kx[None], vx[None])
        for i, (got, want) in enumerate(((ctx_f, ref), (ctx_r, ref), (ctx_d, dref))):
            ok, err = within(got[b], want[0])
            assert ok, ("fast", "exact-order", "fp16-KV")[i] + f" sequence {b}: max err {err}"
            worst[i] = max(worst[i], err)
        say(f"C2 sequence {b} ({Lb} tokens): blocks bit-exact, max err fast/exact/fp16 "
            f"{worst[0]:.2e}/{worst[1]:.2e}/{worst[2]:.2e}")


# ------------------------------------------------------------------ C3

def test_c3_full_shape_5bit_encode_and_decode_vs_oracle():
    c = synthetic.C3
    kv, q = synthetic.c3_workload(DEV)
    lengths = [c["L"]] * c["B"]
    kk, seq = cache.pack_sequences(kv[0], lengths, bits=5, tail_dtype=torch.float16)
    vv, _ = cache.pack_sequences(kv[1], lengths, bits=5, tail_dtype=torch.float16)
    _, ctx = kernels.decode_attention(q, kk, vv, seq, max_seq_len=c["L"], kernel="fast")
    ctx = ctx.cpu().numpy()
    qn = q.float().cpu().numpy()
    worst = 0.0
    for b in range(c["B"]):
        kr = oracle_history(kv[0, b].cpu().numpy(), c["L"], 5, kk, b)
        vr = oracle_history(kv[1, b].cpu().numpy(), c["L"], 5, vv, b)
        ref, _ = O.decode_attention64(qn[b:b + 1], kr[None], vr[None])
        ok, err = within(ctx[b], ref[0])
        assert ok, f"sequence {b}: max err {err}"
        worst = max(worst, err)
        if b % 16 == 15:
            say(f"C3 sequences 0..{b}: blocks bit-exact, max err {worst:.2e}")


# ------------------------------------------------------------------ C4

def _c4_tokens(gen, n, dtype=torch.float16):
    c = synthetic.C4
    return torch.randn((c["B"], c["H"], n, 128), generator=gen, device=DEV, dtype=torch.float32).to(dtype)


# the C4 rows whose attention is compared with the float64 oracle
C4_ROWS = [(0, 0), (0, 15), (13, 7), (31, 0), (31, 15)]


def _c4_check_chunk(out, qc, kc, vc, hist_k, hist_v, ctxlen, packed, side_k, side_v, label):
    """Rows C4_ROWS of a prefill chunk's bf16 output against the float64 oracle
    over the context as the cache holds it (packed blocks restored by the
    oracle -- and checked bit for bit against the GPU's -- then the fp16 tail)
    and the chunk's own bf16 K/V.  Bound: 2e-3 + 1e-2*|ref| plus the bf16
    output's own rounding (2^-8 relative)."""
    worst = worst_r = 0.0
    for b, h in C4_ROWS:
        kr = oracle_history(hist_k[b], ctxlen, 3, side_k, b, packed=packed)
        vr = oracle_history(hist_v[b], ctxlen, 3, side_v, b, packed=packed)
        ref = O.prefill_attention64(qc[b, h:h + 1].float().cpu().numpy(), kr[h:h + 1], vr[h:h + 1],
                                    kc[b, h:h + 1].float().cpu().numpy(), vc[b, h:h + 1].float().cpu().numpy())
        ok, err = within(out[b, h], ref[0], 2.0 ** -8)
        assert ok, f"{label} (b, h) = ({b}, {h}): max err {err}"
        worst = max(worst, err)
        worst_r = max(worst_r, ratio(out[b, h], ref[0], 2.0 ** -8))
    say(f"{label}: rows {C4_ROWS} within the bound, max err {worst:.2e}, max err/bound {worst_r:.3f}")


def test_c4_bf16_chunked_prefill_full_shape():
    """The C4 prefill exactly as bench.py times it: 16 chunks of 512 bf16
    queries / keys / values (N(0,1)) over the fp16 tail of a 3-bit streaming
    cache (B=32, 16 MHA heads), each through StreamingKVCache.prefill(...,
    append=True) -- the bf16-MFMA prefill kernel over packed context + tail +
    the chunk, with the chunk's append to the fp16 tail in the same launch --
    then the compression policy.  Chunk 0 (causal attention over the chunk
    alone: the first queries attend one or two tokens), chunk 1 and the last
    chunk (119 packed blocks + 64 tail tokens of context) are compared with
    the float64 oracle on rows C4_ROWS; after every append the new tail rows
    are bit-equal to the chunk rounded to fp16, and the final packed blocks of
    every row bit-equal to the oracle's encode of that history."""
    c = synthetic.C4
    B, H, T, ch = c["B"], c["H"], c["T"], c["chunk"]
    gen = torch.Generator(device=DEV).manual_seed(c["seed"])
    acts = [tuple(_c4_tokens(gen, ch, torch.bfloat16) for _ in range(3)) for _ in range(T // ch)]
    kh = torch.cat([a[1] for a in acts], 2).to(torch.float16)   # the history as the fp16 tail stores it
    vh = torch.cat([a[2] for a in acts], 2).to(torch.float16)
    khn, vhn = kh.cpu().numpy(), vh.cpu().numpy()
    sc = StreamingKVCache(1, B, H, T + 64, bits=3, dtype=torch.float16, max_append=ch, device=DEV)
    for i, (qc, kc, vc) in enumerate(acts):
        ctxlen, packed = sc.length[0], sc.compressed[0]
        out = sc.prefill(0, qc, kc, vc, append=True)
        assert sc.length[0] == ctxlen + ch
        tail = sc.side(0, "K").tail, sc.side(0, "V").tail
        t0 = ctxlen - packed
        for name, x, t in (("K", kh, tail[0]), ("V", vh, tail[1])):
            assert torch.equal(t[:, :, t0:t0 + ch].view(torch.int16), x[:, :, ctxlen:ctxlen + ch].view(torch.int16)), \
                f"chunk {i}: appended {name} rows differ from the chunk rounded to fp16"
        if i in (0, 1, T // ch - 1):
            _c4_check_chunk(out.float().cpu().numpy(), qc, kc, vc, khn, vhn, ctxlen, packed, sc.side(0, "K"),
                            sc.side(0, "V"), f"C4 chunk {i} (context {ctxlen}, {packed} packed)")
        sc.compress_to(0, max(sc.compressed[0], ((sc.length[0] - 64) // 64) * 64))
    sc.check_status()
    assert sc.length[0] == T and sc.compressed[0] == T - 64
    C = sc.compressed[0]
    for name, x in (("K", khn), ("V", vhn)):
        side = sc.side(0, name)
        for b in range(B):
            oracle_history(x[b], C, 3, side, b)
    say(f"C4 bf16 prefill: final state {C // 64} blocks per row bit-exact")


def test_c4_streaming_prefill_then_256_decode_steps():
    """One slot at the C4 shape: 16 bf16 prefill chunks of 512 (attend and
    append in one launch, then compress, as bench.py runs them), post_prefill,
    then 256 decode steps (append one fp16 token, fast decode over packed +
    tail, post_decode: a block every 64 tokens).  The tail stays 64..127
    tokens; decode outputs at steps around each compression are compared on
    sequences 0 and 31 (all 16 heads); the final packed state of every row is
    bit-equal to the oracle's encode."""
    c = synthetic.C4
    B, H, T, ch, steps = c["B"], c["H"], c["T"], c["chunk"], c["steps"]
    gen = torch.Generator(device=DEV).manual_seed(c["seed"] + 100)
    # bf16-representable history (the chunks are bf16; the decode tokens fp16 of the same values)
    kb, vb = _c4_tokens(gen, T + steps, torch.bfloat16), _c4_tokens(gen, T + steps, torch.bfloat16)
    kh, vh = kb.to(torch.float16), vb.to(torch.float16)
    sc = StreamingKVCache(1, B, H, T + steps + 64, bits=3, dtype=torch.float16, max_append=ch, device=DEV)
    for t0 in range(0, T, ch):
        qc = _c4_tokens(gen, ch, torch.bfloat16)
        sc.prefill(0, qc, kb[:, :, t0:t0 + ch].contiguous(), vb[:, :, t0:t0 + ch].contiguous(), append=True)
        sc.compress_to(0, max(sc.compressed[0], ((sc.length[0] - 64) // 64) * 64))
    sc.post_prefill()
    assert sc.length[0] == T and sc.compressed[0] == T - 64
    say("C4 prefill done")
    khn, vhn = kh.cpu().numpy(), vh.cpu().numpy()
    subset = (0, 31)
    full = {b: (oracle_history(khn[b], T + steps, 3), oracle_history(vhn[b], T + steps, 3)) for b in subset}
    check_at = {0, 1, 62, 63, 64, 65, 127, 128, 191, 192, 255}
    worst = 0.0
    for i in range(steps):
        t = T + i
        sc.append(0, kh[:, :, t:t + 1].contiguous(), vh[:, :, t:t + 1].contiguous())
        q = torch.randn((B, H, 128), generator=gen, device=DEV, dtype=torch.float32).to(torch.bfloat16)
        _, ctx = sc.decode(0, q, kernel="fast")
        if i in check_at:
            C, L = sc.compressed[0], sc.length[0]
            ctxn = ctx.cpu().numpy()
            qn = q.float().cpu().numpy()
            for b in subset:
                kr = np.concatenate([full[b][0][:, :C], khn[b][:, C:L].astype(np.float32)], 1)
                vr = np.concatenate([full[b][1][:, :C], vhn[b][:, C:L].astype(np.float32)], 1)
                ref, _ = O.decode_attention64(qn[b:b + 1], kr[None], vr[None])
                ok, err = within(ctxn[b], ref[0])
                assert ok, f"step {i} sequence {b}: max err {err}"
                worst = max(worst, err)
            say(f"C4 decode step {i}: context {L} ({C} packed), max err so far {worst:.2e}")
        sc.post_decode()
        assert 64 <= sc.tail_len(0) < 128
    sc.check_status()
    C, L = sc.compressed[0], sc.length[0]
    assert L == T + steps and 64 <= L - C < 128
    # the final packed state of every row, and the tail
    for name, x in (("K", khn), ("V", vhn)):
        side = sc.side(0, name)
        for b in range(B):
            oracle_history(x[b], C, 3, side, b)
        tail = side.tail[:, :, :L - C].cpu().numpy()
        assert np.array_equal(tail.view(np.uint16), x[:, :, C:L].view(np.uint16))
    say(f"C4 final state: {C // 64} blocks per row bit-exact, tail {L - C} tokens")
