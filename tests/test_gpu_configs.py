"""GPU parity at the full shapes of the benchmark configurations (BASELINE.json
configs[2], [3], [4]) against the oracle.

Each test builds its configuration exactly as bench.py does (the generators
of nsn_amd.synthetic, on the GPU), runs the HIP path through the C-ABI, and
then checks, on the host:

- every packed block (codes, fp16 norm / min / scale) bit-equal to the C
  oracle's encode of the same 64 tokens;
- attention outputs within 2e-3 + 1e-2*|ref| of the oracle's float64
  attention over the oracle-restored K/V (fp32 reconstructions, the tail as
  stored), plus the output's own rounding where the output is bf16/fp16.

C2: B=16, 32q/8kv, ragged 16K..32K, INT3 + fp16 tail (the headline step),
    the fast kernel, the exact-order kernel, and the fp16-KV baseline.
C3: 5-bit, B=64, 16q/4kv, 8192 tokens, heavy-tailed channels.
C4: the streaming cache (MHA 16 kv-heads, B=32): the chunk of 512 over a
    7,680-token context (119 packed blocks + 64 tail tokens), and an
    8,192-token chunked prefill followed by 256 decode steps with the
    compression policy.  Attention is compared on a subset of sequences /
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
    return np.concatenate(parts, axis=1)


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

def _c4_tokens(gen, n):
    c = synthetic.C4
    return torch.randn((c["B"], c["H"], n, 128), generator=gen, device=DEV, dtype=torch.float32).to(torch.float16)


def test_c4_last_chunk_prefill_full_shape():
    """The chunk of 512 after 7,680 tokens (state: 119 packed blocks + 64 tail
    tokens, as the streaming policy leaves it), all 32 x 16 rows computed,
    a subset compared with the float64 oracle."""
    c = synthetic.C4
    B, H, ch = c["B"], c["H"], c["chunk"]
    ctxlen = c["T"] - ch
    gen = torch.Generator(device=DEV).manual_seed(c["seed"])
    kh, vh = _c4_tokens(gen, ctxlen), _c4_tokens(gen, ctxlen)
    qc, kc, vc = _c4_tokens(gen, ch), _c4_tokens(gen, ch), _c4_tokens(gen, ch)
    sc = StreamingKVCache(1, B, H, c["T"] + 64, bits=3, dtype=torch.float16, max_append=ch, device=DEV)
    for t0 in range(0, ctxlen, ch):
        sc.append(0, kh[:, :, t0:t0 + ch].contiguous(), vh[:, :, t0:t0 + ch].contiguous())
        sc.compress_to(0, max(sc.compressed[0], ((sc.length[0] - 64) // 64) * 64))
    assert sc.compressed[0] == 7616 and sc.length[0] == ctxlen
    out = sc.prefill(0, qc, kc, vc).float().cpu().numpy()
    sc.check_status()
    khn, vhn = kh.cpu().numpy(), vh.cpu().numpy()
    rows = [(0, 0), (0, 15), (13, 7), (31, 0), (31, 15)]
    for b, h in rows:
        # (the packed blocks of the whole row b are checked bit for bit too)
        kr = oracle_history(khn[b], ctxlen, 3, sc.side(0, "K"), b, packed=7616)
        vr = oracle_history(vhn[b], ctxlen, 3, sc.side(0, "V"), b, packed=7616)
        ref = O.prefill_attention64(qc[b, h:h + 1].float().cpu().numpy(), kr[h:h + 1], vr[h:h + 1],
                                    kc[b, h:h + 1].float().cpu().numpy(), vc[b, h:h + 1].float().cpu().numpy())
        ok, err = within(out[b, h], ref[0], 2.0 ** -11)
        assert ok, f"(b, h) = ({b}, {h}): max err {err}"
        say(f"C4 last chunk (b, h) = ({b}, {h}): max err {err:.2e}")


def test_c4_streaming_prefill_then_256_decode_steps():
    """One slot at the C4 shape: 16 prefill chunks of 512 (attend, append,
    compress), post_prefill, then 256 decode steps (append one token, fast
    decode over packed + tail, post_decode: a block every 64 tokens).  The
    tail stays 64..127 tokens; decode outputs at steps around each
    compression are compared on sequences 0 and 31 (all 16 heads); the final
    packed state of every row is bit-equal to the oracle's encode."""
    c = synthetic.C4
    B, H, T, ch, steps = c["B"], c["H"], c["T"], c["chunk"], c["steps"]
    gen = torch.Generator(device=DEV).manual_seed(c["seed"] + 100)
    kh, vh = _c4_tokens(gen, T + steps), _c4_tokens(gen, T + steps)
    sc = StreamingKVCache(1, B, H, T + steps + 64, bits=3, dtype=torch.float16, max_append=ch, device=DEV)
    for t0 in range(0, T, ch):
        qc = _c4_tokens(gen, ch)
        kc, vc = kh[:, :, t0:t0 + ch].contiguous(), vh[:, :, t0:t0 + ch].contiguous()
        sc.prefill(0, qc, kc, vc)
        sc.append(0, kc, vc)
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
