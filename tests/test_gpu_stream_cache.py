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
