"""GPU-resident streaming packed K/V cache (the reference's PackedCache, rebuilt).

The reference keeps, per slot (layer x loop) and side, a growing dict of
packed block groups joined with ``torch.cat`` on every compression and an
fp16/bf16 tail cut with ``clone`` (experiments/ac08/source/
loop_kv_pk01_cache.py:76-132).  Here every slot owns preallocated storage:

- packed blocks ``[B, Hkv, cap, ...]`` (codes, norm, min, scale, decode
  factors, 12-byte headers), written in place by one encoder launch per
  compression (``nsn_encode_blocks`` with a block offset);
- a tail buffer of ``tail_cap`` tokens, re-based after each compression
  (one device copy of the surviving tokens).

The policy is the reference's:

- ``post_prefill``: compress to ``max(0, ((L - 64) // 64) * 64)``
  (``loop_kv_pk01_cache.py:122-123``);
- ``post_decode``: once ``L - compressed >= 128``, compress one more block
  (``:124-127``);

so after either call the tail holds 64..127 tokens (fewer only for short
sequences).  Headers carry the token offset of each block ('<QHBB', as
``encode_group`` writes them, ``:31-37``).  Every sequence of the batch has
the same length (the reference runs batch 1; the C4 workload is uniform), so
lengths are host integers and nothing here synchronises with the device.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _dev, _lib
from .errors import IntegrityError, require
from .kernels import BLOCK, DIM, PackedKV

MIN_TAIL = 64


def prefill_target(length: int) -> int:
    """Compressed-token target after the prefill (loop_kv_pk01_cache.py:122-123)."""
    return max(0, ((length - MIN_TAIL) // BLOCK) * BLOCK)


def decode_target(length: int, compressed: int) -> int:
    """Compressed-token target after a decode step (loop_kv_pk01_cache.py:124-127)."""
    return compressed + BLOCK if length - compressed >= 2 * BLOCK else compressed


@dataclass
class _Side:
    kv: PackedKV
    headers: torch.Tensor   # u8 [B, H, cap, 12]


class StreamingKVCache:
    """Packed K/V of ``slots`` attention slots for ``batch`` sequences x ``heads`` kv-heads.

    max_tokens bounds the sequence length (block capacity = max_tokens // 64);
    max_append bounds the tokens appended between two compressions (a
    prefill chunk, or 1 per decode step).  ``dtype`` is the tail's dtype
    (fp16 or bf16; both kernels read either); appended K/V of another dtype
    are converted to it.
    """

    def __init__(self, slots, batch, heads, max_tokens, *, bits=3, dtype=torch.float16, max_append=512,
                 device=None):
        device = device or torch.device("cuda:0")
        require(bits in (3, 4, 5), "Bits")
        require(dtype in (torch.float16, torch.bfloat16), "Tail dtype")
        self.slots, self.batch, self.heads, self.bits, self.dtype = slots, batch, heads, bits, dtype
        self.block_cap = max(1, max_tokens // BLOCK)
        self.tail_cap = 2 * BLOCK + max_append
        self.device = device
        nbytes = BLOCK * DIM * bits // 8
        self._sides = {}
        for s in range(slots):
            for name in ("K", "V"):
                kv = PackedKV(
                    codes=torch.empty((batch, heads, self.block_cap, nbytes), dtype=torch.uint8, device=device),
                    norm=torch.empty((batch, heads, self.block_cap, BLOCK), dtype=torch.float16, device=device),
                    min=torch.empty((batch, heads, self.block_cap, DIM), dtype=torch.float16, device=device),
                    scale=torch.empty((batch, heads, self.block_cap, DIM), dtype=torch.float16, device=device),
                    factor=torch.empty((batch, heads, self.block_cap, BLOCK), dtype=torch.float32, device=device),
                    blocks=torch.zeros(batch, dtype=torch.int32, device=device),
                    tail=torch.zeros((batch, heads, self.tail_cap, DIM), dtype=dtype, device=device),
                    bits=bits)
                hdr = torch.zeros((batch, heads, self.block_cap, 12), dtype=torch.uint8, device=device)
                self._sides[(s, name)] = _Side(kv, hdr)
        self.length = [0] * slots        # tokens held per slot
        self.compressed = [0] * slots    # of which packed
        self._len_dev = {}               # cached int32 length tensors
        self.status = _dev.new_status(device)
        self.encoded_blocks = [0] * slots

    # ------------------------------------------------------------------ views
    def side(self, slot, name) -> PackedKV:
        return self._sides[(slot, name)].kv

    def headers(self, slot, name) -> torch.Tensor:
        return self._sides[(slot, name)].headers

    def lengths(self, slot) -> torch.Tensor:
        """int32 [B] device tensor of the slot's length (every sequence equal)."""
        return self.length_tensor(self.length[slot])

    def length_tensor(self, L) -> torch.Tensor:
        """int32 [B] device tensor filled with L (made once per L and kept)."""
        t = self._len_dev.get(L)
        if t is None:
            t = torch.full((self.batch,), L, dtype=torch.int32, device=self.device)
            self._len_dev[L] = t
        return t

    def tail_len(self, slot):
        return self.length[slot] - self.compressed[slot]

    # ------------------------------------------------------------------ updates
    def append(self, slot, k, v):
        """Append k, v [B, H, n, 128] to the slot's tail (converted to the tail dtype if needed)."""
        require(k.shape == v.shape and k.ndim == 4 and tuple(k.shape[:2]) == (self.batch, self.heads)
                and k.shape[3] == DIM, "Append shape")
        n = k.shape[2]
        t0 = self.tail_len(slot)
        if t0 + n > self.tail_cap:
            raise IntegrityError("Tail overflow: compress before appending more tokens")
        if self.length[slot] + n > self.block_cap * BLOCK + self.tail_cap:
            raise IntegrityError("Cache capacity exceeded")
        require(k.dtype in (torch.float16, torch.bfloat16, torch.float32) and v.dtype == k.dtype, "Append dtype")
        if k.dtype != self.dtype:
            k, v = k.to(self.dtype), v.to(self.dtype)
        k, v = k.contiguous(), v.contiguous()
        kt, vt = self._sides[(slot, "K")].kv.tail, self._sides[(slot, "V")].kv.tail
        rc = _lib.lib().nsn_tail_append(k.data_ptr(), v.data_ptr(), self.batch * self.heads, n, n, kt.data_ptr(),
                                        vt.data_ptr(), self.tail_cap, t0, _dev.dtype_code(self.dtype), _dev.stream())
        _lib.check(rc, "nsn_tail_append")
        self.length[slot] += n

    def compress_to(self, slot, target):
        """Encode tail tokens up to absolute position `target` (a multiple of
        64) into packed blocks, in place; the tail keeps the rest."""
        start = self.compressed[slot]
        if not (target >= start and (target - start) % BLOCK == 0):
            raise IntegrityError("Block overlap/ordering")
        if target == start:
            return
        if self.length[slot] < target + BLOCK:
            raise IntegrityError("Tail/compressed divergence")
        n = target - start
        nb = n // BLOCK
        if target // BLOCK > self.block_cap:
            raise IntegrityError("Cache capacity exceeded")
        lib = _lib.lib()
        rest = self.length[slot] - target
        for name in ("K", "V"):
            sd = self._sides[(slot, name)]
            kv = sd.kv
            rc = lib.nsn_encode_blocks(
                kv.tail.data_ptr(), _dev.dtype_code(self.dtype), self.batch * self.heads, nb,
                self.tail_cap * DIM, 0, self.bits, _lib.NORM_LANES8, 1,
                kv.codes.data_ptr(), kv.norm.data_ptr(), kv.min.data_ptr(), kv.scale.data_ptr(),
                sd.headers.data_ptr(), kv.factor.data_ptr(), self.block_cap, start // BLOCK, start,
                None, self.status.data_ptr(), _dev.stream())
            _lib.check(rc, "nsn_encode_blocks")
            # re-base the surviving tail tokens (source and target may overlap)
            src = kv.tail[:, :, n:n + rest]
            kv.tail[:, :, :rest] = src.clone() if rest > n else src
            kv.blocks.fill_(target // BLOCK)
        self.compressed[slot] = target
        self.encoded_blocks[slot] += nb

    def post_prefill(self):
        for s in range(self.slots):
            self.compress_to(s, prefill_target(self.length[s]))

    def post_decode(self):
        for s in range(self.slots):
            self.compress_to(s, decode_target(self.length[s], self.compressed[s]))

    def check_status(self):
        """Raise if any compression flagged nonfinite input or fp16 metadata trouble (syncs)."""
        s = _dev.read_status(self.status)
        if s:
            from .primitives import _encode_raise
            _encode_raise(s)

    # ------------------------------------------------------------------ attention
    def decode(self, slot, q, **kw):
        """Decode attention of q [B, Hq, 128] over the slot (packed blocks + tail)."""
        L = self.length[slot]
        return _attn().decode_attention(q, self.side(slot, "K"), self.side(slot, "V"), self.lengths(slot),
                                        max_seq_len=L, **kw)

    def prefill(self, slot, q, k_chunk, v_chunk, **kw):
        """Chunked-prefill attention of q [B, Hq, n, 128] over the slot's
        context plus the chunk's own K/V (not yet appended)."""
        has_ctx = self.length[slot] > 0
        return _attn().prefill_attention(q, self.side(slot, "K") if has_ctx else None,
                                         self.side(slot, "V") if has_ctx else None, self.lengths(slot),
                                         k_chunk, v_chunk, **kw)


def _attn():
    from . import kernels
    return kernels
