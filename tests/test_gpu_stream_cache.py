"""GPU tests of the streaming packed cache (nsn_amd.stream_cache): chunked
prefill then token-by-token decode, against the oracle.

- the packed blocks, metadata and headers after every compression are
  bit-equal to the oracle's encode of the same 64-token blocks
  (nsn_encode + pack3 + '<QHBB' headers, loop_kv_pk01_cache.py:31-37);
- the tail holds the uncompressed tokens, 64..127 of them after every policy
  call (loop_kv_pk01_cache.py:122-127);
- prefill and decode attention over the cache agree with float64 attention
  over the oracle-restored history (tolerance 2e-3 + 1e-2*|ref|, plus the
  output's own rounding).
"""
import numpy as np
import pytest
import torch

from nsn_amd.stream_cache import StreamingKVCache
from oracle import oracle as O
from tests.test_gpu_prefill import normal_tokens, restore_ctx

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def check_blocks(cache, slot, hist_k, hist_v):
    """Packed state of `slot` == oracle encode of the compressed prefix."""
    C = cache.compressed[slot]
    nb = C // 64
    for name, x in (("K", hist_k), ("V", hist_v)):
        side = cache.side(slot, name)
        assert int(side.blocks[0]) == nb
        if not nb:
            continue
        B, H = x.shape[:2]
        blocks = x[:, :, :C].astype(np.float32).reshape(B * H, nb, 64, 128)
        q, n, m, s, err = O.nsn_encode(blocks, 3)
        assert err == 0
        codes = O.pack_codes(q.reshape(B * H * nb, -1), 3).reshape(B, H, nb, -1)
        assert np.array_equal(side.codes[:, :, :nb].cpu().numpy(), codes)
        assert np.array_equal(side.norm[:, :, :nb].cpu().numpy().view(np.uint16), n.reshape(B, H, nb, 64))
        assert np.array_equal(side.min[:, :, :nb].cpu().numpy().view(np.uint16), m.reshape(B, H, nb, 128))
        assert np.array_equal(side.scale[:, :, :nb].cpu().numpy().view(np.uint16), s.reshape(B, H, nb, 128))
        hdr = cache.headers(slot, name)[:, :, :nb].cpu().numpy()
        tok = hdr[..., :8].copy().view(np.uint64)[..., 0]
        assert np.array_equal(tok, np.broadcast_to(64 * np.arange(nb, dtype=np.uint64), (B, H, nb)))
        assert np.all(hdr[..., 8:10].copy().view(np.uint16)[..., 0] == 64)
        assert np.all(hdr[..., 10] == 3) and np.all(hdr[..., 11] == 0)
        # tail = the uncompressed tokens
        L = cache.length[slot]
        tail = side.tail[:, :, :L - C].cpu().numpy()
        assert np.array_equal(tail.view(np.uint16), x[:, :, C:L].view(np.uint16))


def within(got, ref, ulp):
    err = np.abs(got - ref)
    bound = 2e-3 + (1e-2 + ulp) * np.abs(ref)
    return bool(np.all(err <= bound)), float(err.max())


def test_stream_cache_prefill_then_decode():
    rng = np.random.default_rng(31)
    B, H, slots, T, chunk, steps = 2, 2, 2, 300, 128, 70
    k = normal_tokens(rng, (B, H), T + steps)       # fp16 history
    v = normal_tokens(rng, (B, H), T + steps)
    cache = StreamingKVCache(slots, B, H, 1024, bits=3, dtype=torch.float16, max_append=chunk, device=DEV)
    slot = 1
    # ---- chunked prefill: attend, append, compress (final state = one post_prefill)
    for c0 in range(0, T, chunk):
        n = min(chunk, T - c0)
        q = rng.standard_normal((B, H, n, 128)).astype(np.float16)
        kc = torch.from_numpy(k[:, :, c0:c0 + n].copy()).to(DEV)
        vc = torch.from_numpy(v[:, :, c0:c0 + n].copy()).to(DEV)
        out = cache.prefill(slot, torch.from_numpy(q).to(DEV), kc, vc).float().cpu().numpy()
        for b in range(B):
            # the cache's context: packed prefix (restored) + fp16 tail as stored
            C = cache.compressed[slot]
            kctx = np.concatenate([restore_ctx(k[b], C, 3, torch.float16)[:, :C], k[b][:, C:c0].astype(np.float32)], 1)
            vctx = np.concatenate([restore_ctx(v[b], C, 3, torch.float16)[:, :C], v[b][:, C:c0].astype(np.float32)], 1)
            ref = O.prefill_attention64(q[b].astype(np.float32), kctx, vctx, k[b][:, c0:c0 + n].astype(np.float32),
                                 v[b][:, c0:c0 + n].astype(np.float32))
            ok, err = within(out[b], ref, 2.0 ** -11)
            assert ok, (c0, b, err)
        cache.append(slot, kc, vc)
        cache.compress_to(slot, max(cache.compressed[slot], (max(0, cache.length[slot] - 64) // 64) * 64))
        check_blocks(cache, slot, k, v)
    cache.post_prefill()
    assert cache.compressed[slot] == 192 and cache.length[slot] == T      # 300 - 64 -> 236 -> 192
    assert cache.compressed[0] == 0 and cache.length[0] == 0              # the other slot is untouched
    # ---- decode: append one token, attend over the whole history, post_decode
    for i in range(steps):
        t = T + i
        cache.append(slot, torch.from_numpy(k[:, :, t:t + 1].copy()).to(DEV),
                     torch.from_numpy(v[:, :, t:t + 1].copy()).to(DEV))
        q = rng.standard_normal((B, 2 * H, 128)).astype(np.float32)
        qb = torch.from_numpy(q).to(torch.bfloat16)
        _, ctx = cache.decode(slot, qb.to(DEV), kernel="fast")
        C = cache.compressed[slot]
        L = t + 1
        for b in range(B):
            kr = np.concatenate([restore_ctx(k[b], C, 3, torch.float16)[:, :C], k[b][:, C:L].astype(np.float32)], 1)
            vr = np.concatenate([restore_ctx(v[b], C, 3, torch.float16)[:, :C], v[b][:, C:L].astype(np.float32)], 1)
            ref, _ = O.decode_attention64(qb[b:b + 1].float().numpy(), kr[None], vr[None])
            ok, err = within(ctx[b].cpu().numpy(), ref[0], 0.0)
            assert ok, (i, b, err)
        cache.post_decode()
        assert 64 <= cache.tail_len(slot) < 128
    check_blocks(cache, slot, k, v)
    assert cache.compressed[slot] == 256 and cache.encoded_blocks[slot] == 4
    cache.check_status()


def check_blocks_ragged(cache, slot, hist_k, hist_v):
    """Per sequence: packed prefix == oracle encode, headers, block count, tail."""
    for name, x in (("K", hist_k), ("V", hist_v)):
        side = cache.side(slot, name)
        blocks = side.blocks.cpu().numpy()
        for b in range(cache.batch):
            C, L = cache.seq_compressed[slot][b], cache.seq_length[slot][b]
            nb = C // 64
            assert blocks[b] == nb
            H = x.shape[1]
            if nb:
                q, n, m, s, err = O.nsn_encode(x[b, :, :C].astype(np.float32).reshape(H, nb, 64, 128), 3)
                assert err == 0
                codes = O.pack_codes(q.reshape(H * nb, -1), 3).reshape(H, nb, -1)
                assert np.array_equal(side.codes[b, :, :nb].cpu().numpy(), codes)
                assert np.array_equal(side.norm[b, :, :nb].cpu().numpy().view(np.uint16), n.reshape(H, nb, 64))
                assert np.array_equal(side.min[b, :, :nb].cpu().numpy().view(np.uint16), m.reshape(H, nb, 128))
                assert np.array_equal(side.scale[b, :, :nb].cpu().numpy().view(np.uint16), s.reshape(H, nb, 128))
                hdr = cache.headers(slot, name)[b, :, :nb].cpu().numpy()
                tok = hdr[..., :8].copy().view(np.uint64)[..., 0]
                assert np.array_equal(tok, np.broadcast_to(64 * np.arange(nb, dtype=np.uint64), (H, nb)))
            tail = side.tail[b, :, :L - C].cpu().numpy()
            assert np.array_equal(tail.view(np.uint16), x[b, :, C:L].view(np.uint16))


def test_stream_cache_ragged_lengths():
    """A ragged batch (prompts of 300, 171 and 69 tokens) streams through one
    slot: chunked prefill with per-sequence token counts, then 140 decode
    steps of one token each with the compression policy applied per sequence
    (each sequence compresses at its own steps); every packed block and tail
    checked against the oracle's encode, every attention output against
    float64 attention over that sequence's own restored history."""
    rng = np.random.default_rng(37)
    B, H, chunk, steps = 3, 2, 128, 140
    prompt = [300, 171, 69]
    T = max(prompt) + steps
    k = normal_tokens(rng, (B, H), T)
    v = normal_tokens(rng, (B, H), T)
    cache = StreamingKVCache(1, B, H, 1024, bits=3, dtype=torch.float16, max_append=chunk, device=DEV)
    slot = 0

    def hist(x, b, C, L):
        return np.concatenate([restore_ctx(x[b], C, 3, torch.float16)[:, :C], x[b][:, C:L].astype(np.float32)], 1)

    for c0 in range(0, max(prompt), chunk):
        counts = [max(0, min(chunk, P - c0)) for P in prompt]
        n = max(counts)
        q = rng.standard_normal((B, H, n, 128)).astype(np.float16)
        kc = torch.from_numpy(k[:, :, c0:c0 + n].copy()).to(DEV)
        vc = torch.from_numpy(v[:, :, c0:c0 + n].copy()).to(DEV)
        out = cache.prefill(slot, torch.from_numpy(q).to(DEV), kc, vc).float().cpu().numpy()
        for b in range(B):
            nb_q = counts[b]
            if not nb_q:
                continue
            C, L = cache.seq_compressed[slot][b], cache.seq_length[slot][b]
            assert L == c0
            ref = O.prefill_attention64(q[b, :, :nb_q].astype(np.float32), hist(k, b, C, L), hist(v, b, C, L),
                                        k[b][:, c0:c0 + nb_q].astype(np.float32),
                                        v[b][:, c0:c0 + nb_q].astype(np.float32))
            ok, err = within(out[b, :, :nb_q], ref, 2.0 ** -11)
            assert ok, (c0, b, err)
        cache.append(slot, kc, vc, counts=counts)
        cache.compress_to(slot, [max(C, (max(0, L - 64) // 64) * 64)
                                 for C, L in zip(cache.seq_compressed[slot], cache.seq_length[slot])])
        check_blocks_ragged(cache, slot, k, v)
    cache.post_prefill()
    assert cache.seq_length[slot] == prompt
    assert cache.seq_compressed[slot] == [192, 64, 0]
    assert not cache.uniform(slot)
    compressions = set()
    for i in range(steps):
        pos = list(cache.seq_length[slot])
        kt = torch.from_numpy(np.stack([k[b, :, pos[b]:pos[b] + 1] for b in range(B)])).to(DEV)
        vt = torch.from_numpy(np.stack([v[b, :, pos[b]:pos[b] + 1] for b in range(B)])).to(DEV)
        cache.append(slot, kt, vt)
        q = rng.standard_normal((B, 2 * H, 128)).astype(np.float32)
        qb = torch.from_numpy(q).to(torch.bfloat16)
        _, ctx = cache.decode(slot, qb.to(DEV), kernel="fast")
        for b in range(B):
            C, L = cache.seq_compressed[slot][b], cache.seq_length[slot][b]
            ref, _ = O.decode_attention64(qb[b:b + 1].float().numpy(), hist(k, b, C, L)[None], hist(v, b, C, L)[None])
            ok, err = within(ctx[b].cpu().numpy(), ref[0], 0.0)
            assert ok, (i, b, err)
        before = list(cache.seq_compressed[slot])
        cache.post_decode()
        compressions |= {(b, i) for b in range(B) if cache.seq_compressed[slot][b] != before[b]}
        for b in range(B):
            assert 64 <= cache.seq_tail_len(slot, b) < 128
    check_blocks_ragged(cache, slot, k, v)
    assert cache.seq_length[slot] == [P + steps for P in prompt]
    # each sequence compressed at its own steps (a uniform batch would share them)
    steps_of = [sorted(i for bb, i in compressions if bb == b) for b in range(B)]
    assert all(steps_of) and len({tuple(x) for x in steps_of}) == B
    cache.check_status()


def test_tail_append_cast_matches_torch_conversion():
    """nsn_tail_append_cast through the C ABI: every (source, tail) dtype pair
    writes, bit for bit, what torch's Tensor.to(tail dtype) + nsn_tail_append
    write (round to nearest even; values past fp16's range become inf,
    values below it subnormal or zero), and leaves the rest of the tail
    untouched."""
    from nsn_amd import _dev, _lib
    lib = _lib.lib()
    rows, n, cap, off = 5, 7, 24, 9
    g = torch.Generator(device=DEV).manual_seed(11)
    base = torch.randn((rows, n, 128), generator=g, device=DEV)
    base[0, 0, :8] = torch.tensor([7e4, -1e5, 3e-6, -6e-8, 1e-9, 65519.0, 65520.0, 0.0], device=DEV)
    stream = _dev.stream()
    for sdt in (torch.float16, torch.bfloat16, torch.float32):
        for ddt in (torch.float16, torch.bfloat16):
            k = base.to(sdt)
            v = (-2 * base).to(sdt)
            kt_a = torch.full((rows, cap, 128), 3.0, dtype=ddt, device=DEV)
            vt_a, kt_b, vt_b = kt_a.clone(), kt_a.clone(), kt_a.clone()
            assert lib.nsn_tail_append_cast(k.data_ptr(), v.data_ptr(), _dev.dtype_code(sdt), rows, n, n,
                                            kt_a.data_ptr(), vt_a.data_ptr(), cap, off, _dev.dtype_code(ddt),
                                            stream) == 0
            kc, vc = k.to(ddt), v.to(ddt)
            assert lib.nsn_tail_append(kc.data_ptr(), vc.data_ptr(), rows, n, n, kt_b.data_ptr(), vt_b.data_ptr(),
                                       cap, off, _dev.dtype_code(ddt), stream) == 0
            assert torch.equal(kt_a.view(torch.int16), kt_b.view(torch.int16)), (sdt, ddt)
            assert torch.equal(vt_a.view(torch.int16), vt_b.view(torch.int16)), (sdt, ddt)


def test_append_in_another_dtype_equals_append_of_converted_tokens():
    """StreamingKVCache.append of bf16 (or fp32) tokens into fp16 tails: the
    same tails, bit for bit, as appending the tokens converted first, for a
    uniform append and a ragged one (per-sequence counts)."""
    g = torch.Generator(device=DEV).manual_seed(12)
    B, H, n = 3, 2, 40
    for sdt in (torch.bfloat16, torch.float32):
        caches = [StreamingKVCache(1, B, H, 1024, dtype=torch.float16, max_append=64, device=DEV) for _ in range(2)]
        for counts in (None, [n, 5, 0]):
            k = torch.randn((B, H, n, 128), generator=g, device=DEV).to(sdt)
            v = torch.randn((B, H, n, 128), generator=g, device=DEV).to(sdt)
            caches[0].append(0, k, v, counts=counts)
            caches[1].append(0, k.to(torch.float16), v.to(torch.float16), counts=counts)
        for name in ("K", "V"):
            a, b = caches[0].side(0, name).tail, caches[1].side(0, name).tail
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), (sdt, name)
        assert caches[0].seq_length == caches[1].seq_length


F16, BF16 = torch.float16, torch.bfloat16


def _state(cache, slot=0):
    """The slot's meaningful state as raw bits: block counts, then per
    sequence its packed blocks (codes, metadata, decode factors) and its
    tail rows (storage past them is never read)."""
    def raw(t):
        t = t.contiguous()
        return t if t.dtype == torch.uint8 else t.view(torch.int8)
    out = []
    for name in ("K", "V"):
        kv = cache.side(slot, name)
        out.append(raw(kv.blocks))
        for b in range(cache.batch):
            L, C = cache.seq_length[slot][b], cache.seq_compressed[slot][b]
            for t in (kv.codes, kv.norm, kv.min, kv.scale, kv.factor):
                out.append(raw(t[b, :, :C // 64]))
            out.append(raw(kv.tail[b, :, :L - C]))
    return out


@pytest.mark.parametrize("dtype,tail_dtype,bits", [(BF16, F16, 3), (F16, F16, 3), (BF16, BF16, 3), (BF16, F16, 5)])
def test_prefill_with_append_equals_prefill_then_append(dtype, tail_dtype, bits):
    """prefill(append=True) writes the chunk to the tails inside the prefill
    launch: its outputs, lengths, tails and packed state are bit-identical to
    prefill() followed by append(), over three chunks of 300 (two query
    tiles) with compression between them, ragged context lengths and GQA
    2:1 (only one q-head's workgroup of each kv-head appends)."""
    B, Hq, H, n = 3, 4, 2, 300
    g = torch.Generator(device=DEV).manual_seed(31)
    caches = [StreamingKVCache(1, B, H, 2048, bits=bits, dtype=tail_dtype, max_append=n, device=DEV)
              for _ in range(2)]
    first = torch.randn((B, H, 100, 128), generator=g, device=DEV).to(dtype)
    for c in caches:
        c.append(0, first, first * 0.5, counts=[7, 47, 87])
    for step in range(3):
        q = torch.randn((B, Hq, n, 128), generator=g, device=DEV).to(dtype)
        k = torch.randn((B, H, n, 128), generator=g, device=DEV).to(dtype)
        v = torch.randn((B, H, n, 128), generator=g, device=DEV).to(dtype)
        want = caches[0].prefill(0, q, k, v)
        caches[0].append(0, k, v)
        got = caches[1].prefill(0, q, k, v, append=True)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), step
        assert caches[0].seq_length == caches[1].seq_length
        for a, b in zip(_state(caches[0]), _state(caches[1])):
            assert torch.equal(a, b), step
        for c in caches:
            c.post_prefill()
        assert caches[0].seq_compressed == caches[1].seq_compressed
    for a, b in zip(_state(caches[0]), _state(caches[1])):
        assert torch.equal(a, b)
    for c in caches:
        c.check_status()


def test_prefill_append_without_room():
    """A chunk that does not fit the tail: with check=True the host refuses it
    before the launch (nothing changes); with check=False the kernel's own
    bound raises the capacity flag, appends nothing and still computes the
    attention."""
    from nsn_amd import _dev, _lib, kernels
    from nsn_amd.errors import IntegrityError
    g = torch.Generator(device=DEV).manual_seed(32)
    c = StreamingKVCache(1, 1, 1, 1024, bits=3, dtype=F16, max_append=32, device=DEV)   # tail_cap 160
    x = torch.randn((1, 1, 150, 128), generator=g, device=DEV).to(F16)
    c.append(0, x, x)
    q, k, v = (torch.randn((1, 1, 64, 128), generator=g, device=DEV).to(F16) for _ in range(3))
    before = _state(c)
    with pytest.raises(IntegrityError):
        c.prefill(0, q, k, v, append=True)
    with pytest.raises(IntegrityError):
        kernels.prefill_attention(q, c.side(0, "K"), c.side(0, "V"), c.lengths(0), k, v, append=True)
    st = _dev.new_status(DEV)
    out = kernels.prefill_attention(q, c.side(0, "K"), c.side(0, "V"), c.lengths(0), k, v, append=True,
                                    check=False, status=st)
    want = kernels.prefill_attention(q, c.side(0, "K"), c.side(0, "V"), c.lengths(0), k, v)
    assert _dev.read_status(st) == _lib.ST_CAPACITY
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    for a, b in zip(before, _state(c)):
        assert torch.equal(a, b)
    assert c.seq_length[0] == [150]
