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
``encode_group`` writes them, ``:31-37``).

Sequences of a batch may have different lengths (the ragged decode batch of
the C2 workload): every sequence has its own length and compressed prefix,
the policy applies per sequence, and appends may carry a per-sequence token
count.  Lengths are host integers, so nothing here synchronises with the
device; while every sequence of a slot has the same state, each operation is
one launch for the whole batch, otherwise one per sequence that changes.
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

    ``seq_length[slot]`` / ``seq_compressed[slot]`` hold each sequence's token
    count and packed prefix; ``length[slot]`` / ``compressed[slot]`` are the
    longest sequence's length and the shortest packed prefix (the common
    values when the batch is uniform).
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
        # each slot's K and V packed-block counts: rows of one [2, batch]
        # tensor, set by one launch (or one upload) per compression
        self._blocks = [torch.zeros((2, batch), dtype=torch.int32, device=device) for _ in range(slots)]
        for s in range(slots):
            for i, name in enumerate(("K", "V")):
                kv = PackedKV(
                    codes=torch.empty((batch, heads, self.block_cap, nbytes), dtype=torch.uint8, device=device),
                    norm=torch.empty((batch, heads, self.block_cap, BLOCK), dtype=torch.float16, device=device),
                    min=torch.empty((batch, heads, self.block_cap, DIM), dtype=torch.float16, device=device),
                    scale=torch.empty((batch, heads, self.block_cap, DIM), dtype=torch.float16, device=device),
                    factor=torch.empty((batch, heads, self.block_cap, BLOCK), dtype=torch.float32, device=device),
                    blocks=self._blocks[s][i],
                    tail=torch.zeros((batch, heads, self.tail_cap, DIM), dtype=dtype, device=device),
                    bits=bits)
                hdr = torch.zeros((batch, heads, self.block_cap, 12), dtype=torch.uint8, device=device)
                self._sides[(s, name)] = _Side(kv, hdr)
        self.seq_length = [[0] * batch for _ in range(slots)]       # tokens held per slot and sequence
        self.seq_compressed = [[0] * batch for _ in range(slots)]   # of which packed
        self._len_dev = {}               # cached int32 length tensors
        self.status = _dev.new_status(device)
        self.encoded_blocks = [0] * slots
        self._side = None                # second stream of the compressions

    # ------------------------------------------------------------------ views
    def side(self, slot, name) -> PackedKV:
        return self._sides[(slot, name)].kv

    def headers(self, slot, name) -> torch.Tensor:
        return self._sides[(slot, name)].headers

    @property
    def length(self):
        """Per slot: the longest sequence's token count."""
        return [max(x) for x in self.seq_length]

    @property
    def compressed(self):
        """Per slot: the shortest packed prefix."""
        return [min(x) for x in self.seq_compressed]

    def uniform(self, slot) -> bool:
        """Every sequence of the slot holds the same tokens and packed prefix."""
        L, C = self.seq_length[slot], self.seq_compressed[slot]
        return min(L) == max(L) and min(C) == max(C)

    def lengths(self, slot) -> torch.Tensor:
        """int32 [B] device tensor of the slot's per-sequence lengths."""
        return self.length_tensor(self.seq_length[slot])

    def length_tensor(self, L) -> torch.Tensor:
        """int32 [B] device tensor of the lengths L (an int for every sequence, or
        one per sequence), made once per distinct value and kept."""
        key = tuple(L) if isinstance(L, (list, tuple)) else (int(L),) * self.batch
        t = self._len_dev.get(key)
        if t is None:
            # Uploaded from pinned memory without a host wait: a pageable copy
            # would drain the stream first, so every new length (each chunk,
            # each decode step) would leave the GPU idle while the host issues
            # the next launches.  The oldest entries are dropped (a dropped
            # tensor's memory is reused only by later work on the stream).
            gpu = torch.device(self.device).type == "cuda"
            t = torch.tensor(key, dtype=torch.int32, pin_memory=gpu).to(self.device, non_blocking=gpu)
            if len(self._len_dev) >= 256:
                self._len_dev.pop(next(iter(self._len_dev)))
            self._len_dev[key] = t
        return t

    def tail_len(self, slot):
        """Tail tokens of the slot (the batch must be uniform)."""
        if not self.uniform(slot):
            raise IntegrityError("Ragged slot: use seq_tail_len")
        return self.seq_length[slot][0] - self.seq_compressed[slot][0]

    def seq_tail_len(self, slot, b):
        return self.seq_length[slot][b] - self.seq_compressed[slot][b]

    def advance(self, slot, n=1):
        """Count n more tokens in every sequence of the slot: the host side of
        an append its caller made on the device (a device-position tail
        append, replayed from a HIP graph)."""
        L = self.seq_length[slot]
        for b in range(self.batch):
            L[b] += n

    def reset(self, slot):
        """Empty the slot for a new batch of sequences (its storage is kept;
        nothing past a sequence's length is ever read)."""
        for b in range(self.batch):
            self.seq_length[slot][b] = 0
            self.seq_compressed[slot][b] = 0
        self._blocks[slot].zero_()
        self.encoded_blocks[slot] = 0

    # ------------------------------------------------------------------ updates
    def append(self, slot, k, v, counts=None):
        """Append k, v [B, H, n, 128] to the slot's tails (converted to the tail
        dtype if needed).  ``counts`` (one int per sequence, each <= n) appends
        only sequence b's first counts[b] tokens; default n for every sequence."""
        require(k.shape == v.shape and k.ndim == 4 and tuple(k.shape[:2]) == (self.batch, self.heads)
                and k.shape[3] == DIM, "Append shape")
        n = k.shape[2]
        counts = [n] * self.batch if counts is None else [int(c) for c in counts]
        require(len(counts) == self.batch and all(0 <= c <= n for c in counts), "Append counts")
        L, C = self.seq_length[slot], self.seq_compressed[slot]
        for b in range(self.batch):
            if L[b] - C[b] + counts[b] > self.tail_cap:
                raise IntegrityError("Tail overflow: compress before appending more tokens")
            if L[b] + counts[b] > self.block_cap * BLOCK + self.tail_cap:
                raise IntegrityError("Cache capacity exceeded")
        require(k.dtype in (torch.float16, torch.bfloat16, torch.float32) and v.dtype == k.dtype, "Append dtype")
        k, v = k.contiguous(), v.contiguous()
        # another dtype converts inside the append kernel (no separate pass);
        # an fp32 tail takes the converted copy
        cast = k.dtype != self.dtype and self.dtype in (torch.float16, torch.bfloat16)
        if k.dtype != self.dtype and not cast:
            k, v = k.to(self.dtype), v.to(self.dtype)
        kt, vt = self._sides[(slot, "K")].kv.tail, self._sides[(slot, "V")].kv.tail
        lib = _lib.lib()
        dt = _dev.dtype_code(self.dtype)
        offs = [L[b] - C[b] for b in range(self.batch)]
        sdt = _dev.dtype_code(k.dtype)

        def launch(kp, vp, ktp, vtp, rows, cnt, off):
            if cast:
                rc = lib.nsn_tail_append_cast(kp, vp, sdt, rows, cnt, n, ktp, vtp, self.tail_cap, off, dt,
                                              _dev.stream())
                _lib.check(rc, "nsn_tail_append_cast")
            else:
                rc = lib.nsn_tail_append(kp, vp, rows, cnt, n, ktp, vtp, self.tail_cap, off, dt, _dev.stream())
                _lib.check(rc, "nsn_tail_append")
        if len(set(offs)) == 1 and len(set(counts)) == 1:
            if counts[0]:
                launch(k.data_ptr(), v.data_ptr(), kt.data_ptr(), vt.data_ptr(), self.batch * self.heads, counts[0],
                       offs[0])
        else:
            for b in range(self.batch):   # one launch per sequence: its own offset and count
                if counts[b]:
                    launch(k[b].data_ptr(), v[b].data_ptr(), kt[b].data_ptr(), vt[b].data_ptr(), self.heads,
                           counts[b], offs[b])
        for b in range(self.batch):
            L[b] += counts[b]

    def compress_to(self, slot, target):
        """Encode tail tokens up to absolute position `target` (a multiple of
        64; an int for every sequence or one per sequence) into packed
        blocks, in place; the tails keep the rest."""
        targets = [int(target)] * self.batch if not isinstance(target, (list, tuple)) else [int(t) for t in target]
        require(len(targets) == self.batch, "Compress targets")
        L, C = self.seq_length[slot], self.seq_compressed[slot]
        for b in range(self.batch):
            start, tgt = C[b], targets[b]
            if not (tgt >= start and (tgt - start) % BLOCK == 0):
                raise IntegrityError("Block overlap/ordering")
            if tgt == start:
                continue
            if L[b] < tgt + BLOCK:
                raise IntegrityError("Tail/compressed divergence")
            if tgt // BLOCK > self.block_cap:
                raise IntegrityError("Cache capacity exceeded")
        moving = [b for b in range(self.batch) if targets[b] != C[b]]
        if not moving:
            return
        if len(moving) == self.batch and len(set(C)) == 1 and len(set(targets)) == 1 and len(set(L)) == 1:
            self._encode_rows(slot, None, C[0], targets[0], L[0])   # the whole batch in one launch per side
        else:
            for b in moving:
                self._encode_rows(slot, b, C[b], targets[b], L[b])
        # blocks added per sequence (the most any sequence gained in this call)
        self.encoded_blocks[slot] += max((targets[b] - C[b]) // BLOCK for b in moving)
        for b in moving:
            C[b] = targets[b]
        nblocks = [c // BLOCK for c in C]
        if len(set(nblocks)) == 1:
            self._blocks[slot].fill_(nblocks[0])
        else:   # from pinned memory without a host wait, like the lengths
            gpu = self.device.type == "cuda"
            self._blocks[slot].copy_(torch.tensor([nblocks, nblocks], dtype=torch.int32, pin_memory=gpu),
                                     non_blocking=gpu)

    def _encode_rows(self, slot, b, start, target, length):
        """Encode tokens [start, target) of sequence b (or of every sequence,
        b None) from the tail into blocks start/64 .., then re-base the tail."""
        lib = _lib.lib()
        n = target - start
        nb = n // BLOCK
        rest = length - target
        rows = self.heads if b is not None else self.batch * self.heads
        sel = (lambda t: t[b]) if b is not None else (lambda t: t)

        def encode(name, stream):
            sd = self._sides[(slot, name)]
            kv = sd.kv
            rc = lib.nsn_encode_blocks(
                sel(kv.tail).data_ptr(), _dev.dtype_code(self.dtype), rows, nb,
                self.tail_cap * DIM, 0, self.bits, _lib.NORM_LANES8, 1,
                sel(kv.codes).data_ptr(), sel(kv.norm).data_ptr(), sel(kv.min).data_ptr(),
                sel(kv.scale).data_ptr(), sel(sd.headers).data_ptr(), sel(kv.factor).data_ptr(), self.block_cap,
                start // BLOCK, start, None, self.status.data_ptr(), stream)
            _lib.check(rc, "nsn_encode_blocks")
        # K and V are encoded side by side: V on a second stream forked from
        # and joined back into the current one (each launch alone is too
        # small to fill the GPU)
        cur = torch.cuda.current_stream(self.device)
        if self._side is None:
            self._side = torch.cuda.Stream(device=self.device)
        self._side.wait_stream(cur)
        encode("K", cur.cuda_stream)
        encode("V", self._side.cuda_stream)
        cur.wait_stream(self._side)
        # re-base the surviving tail tokens [n, n + rest) of every row to [0, rest)
        if rest <= 0:
            return
        kt, vt = sel(self._sides[(slot, "K")].kv.tail), sel(self._sides[(slot, "V")].kv.tail)
        if rest <= n:   # disjoint: one copy launch for both sides
            step = n * DIM * kt.element_size()
            rc = lib.nsn_tail_append(kt.data_ptr() + step, vt.data_ptr() + step, rows, rest, self.tail_cap,
                                     kt.data_ptr(), vt.data_ptr(), self.tail_cap, 0, _dev.dtype_code(self.dtype),
                                     _dev.stream())
            _lib.check(rc, "nsn_tail_append")
        else:           # overlapping rows: through a copy of the source
            for tail in (kt, vt):
                tail[..., :rest, :] = tail[..., n:n + rest, :].clone()

    def post_prefill(self):
        for s in range(self.slots):
            self.compress_to(s, [prefill_target(L) for L in self.seq_length[s]])

    def post_decode(self):
        for s in range(self.slots):
            self.compress_to(s, [decode_target(L, C) for L, C in zip(self.seq_length[s], self.seq_compressed[s])])

    def check_status(self):
        """Raise if any compression flagged nonfinite input or fp16 metadata trouble (syncs)."""
        s = _dev.read_status(self.status)
        if s:
            from .primitives import _encode_raise
            _encode_raise(s)

    # ------------------------------------------------------------------ attention
    def decode(self, slot, q, **kw):
        """Decode attention of q [B, Hq, 128] over the slot (packed blocks + tail;
        each sequence over its own length)."""
        L = max(self.seq_length[slot])
        return _attn().decode_attention(q, self.side(slot, "K"), self.side(slot, "V"), self.lengths(slot),
                                        max_seq_len=L, **kw)

    def prefill(self, slot, q, k_chunk, v_chunk, append=False, **kw):
        """Chunked-prefill attention of q [B, Hq, n, 128] over the slot's
        context plus the chunk's own K/V (not yet appended).  ``append=True``
        also appends the chunk to every sequence's tail in the same launch
        (k_chunk / v_chunk in the compute dtype; the tail rows get them
        rounded to the tail dtype, as ``append`` would).  bf16 chunks carry
        their softmax weights as bf16 hi + lo (``precise_weights``) while some
        sequence of the slot has less than one block of context: its first
        queries attend a handful of tokens."""
        kw.setdefault("precise_weights", min(self.seq_length[slot]) < BLOCK)
        if append:
            n = k_chunk.shape[2]
            L, C = self.seq_length[slot], self.seq_compressed[slot]
            for b in range(self.batch):
                if L[b] - C[b] + n > self.tail_cap:
                    raise IntegrityError("Tail overflow: compress before appending more tokens")
                if L[b] + n > self.block_cap * BLOCK + self.tail_cap:
                    raise IntegrityError("Cache capacity exceeded")
            out = _attn().prefill_attention(q, self.side(slot, "K"), self.side(slot, "V"), self.lengths(slot),
                                            k_chunk, v_chunk, append=True, **kw)
            for b in range(self.batch):
                L[b] += n
            return out
        has_ctx = max(self.seq_length[slot]) > 0
        return _attn().prefill_attention(q, self.side(slot, "K") if has_ctx else None,
                                         self.side(slot, "V") if has_ctx else None, self.lengths(slot),
                                         k_chunk, v_chunk, **kw)


def _attn():
    from . import kernels
    return kernels
