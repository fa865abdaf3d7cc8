"""Batched packed-KV construction on the GPU.

``pack_sequences`` turns dense K or V tokens of B ragged sequences into the
layout the decode kernels read (``kernels.PackedKV``): tokens
``0 .. 64*floor(L_b/64)-1`` of sequence b as packed blocks, the rest (< 64) as
an fp16/bf16 tail.  The reference builds the same state incrementally in its
``PackedCache.compress_to`` (experiments/ac08/source/loop_kv_pk01_cache.py:107-121)
with a ``torch.cat`` per block group; here every sequence is encoded by one
launch straight into preallocated storage.
"""
from __future__ import annotations

import torch

from . import _dev, _lib
from .errors import require
from .kernels import BLOCK, DIM, PackedKV


def alloc_packed(batch, heads, block_cap, tail_cap, bits, tail_dtype, device):
    nbytes = BLOCK * DIM * bits // 8
    return PackedKV(
        codes=torch.empty((batch, heads, block_cap, nbytes), dtype=torch.uint8, device=device),
        norm=torch.empty((batch, heads, block_cap, BLOCK), dtype=torch.float16, device=device),
        min=torch.empty((batch, heads, block_cap, DIM), dtype=torch.float16, device=device),
        scale=torch.empty((batch, heads, block_cap, DIM), dtype=torch.float16, device=device),
        factor=torch.zeros((batch, heads, block_cap, BLOCK), dtype=torch.float32, device=device),
        blocks=torch.zeros(batch, dtype=torch.int32, device=device),
        tail=torch.zeros((batch, heads, max(1, tail_cap), DIM), dtype=tail_dtype, device=device),
        bits=bits)


def pack_sequences(x, lengths, bits=3, tail_dtype=None, status=None):
    """Pack dense tokens x [B, H, Tcap, 128] (fp16/bf16/fp32) with per-sequence lengths.

    Returns (PackedKV, seq_len int32 device tensor).
    """
    _dev.require_gpu(x)
    require(x.ndim == 4 and x.shape[3] == DIM, "Dense KV shape")
    B, H, Tcap, _ = x.shape
    lengths = [int(v) for v in lengths]
    require(len(lengths) == B and all(0 < v <= Tcap for v in lengths), "Sequence lengths")
    tail_dtype = tail_dtype or (x.dtype if x.dtype != torch.float32 else torch.float16)
    nblk = [v // BLOCK for v in lengths]
    cap = max(1, max(nblk))
    kv = alloc_packed(B, H, cap, BLOCK, bits, tail_dtype, x.device)
    xc = x.contiguous()
    st = status if status is not None else _dev.new_status(x.device)
    lib = _lib.lib()
    order = _dev.norm_order(xc)
    for b in range(B):
        if nblk[b]:
            rc = lib.nsn_encode_blocks(
                xc[b].data_ptr(), _dev.dtype_code(xc.dtype), H, nblk[b], Tcap * DIM, 0, bits, order, 1,
                kv.codes[b].data_ptr(), kv.norm[b].data_ptr(), kv.min[b].data_ptr(), kv.scale[b].data_ptr(),
                None, kv.factor[b].data_ptr(), cap, 0, 0, None, st.data_ptr(), _dev.stream())
            _lib.check(rc, "nsn_encode_blocks")
        t0 = nblk[b] * BLOCK
        if lengths[b] > t0:
            kv.tail[b, :, : lengths[b] - t0] = x[b, :, t0:lengths[b]].to(tail_dtype)
    kv.blocks.copy_(torch.tensor(nblk, dtype=torch.int32))
    if status is None:
        s = _dev.read_status(st)
        if s:
            from .primitives import _encode_raise
            _encode_raise(s)
    seq = torch.tensor(lengths, dtype=torch.int32, device=x.device)
    return kv, seq
