"""Packed block codec on the GPU: the reference's L2 call surface.

Mirrors ``experiments/ac08/source/loop_kv_pk01_cache.py:7-50`` (``pack3``,
``unpack3``, ``encode_group``, ``restore_group``, ``append_group``).  A packed
group is the reference's dict ``{'codes': u8 [b,h,n,64*128*bits/8],
'metas': (norm f16 [b,h,n,64,1], min f16 [b,h,n,1,128], scale f16
[b,h,n,1,128]), 'headers': u8 [b,h,n,12]}``.  ``encode_group`` is one kernel
launch (encode + pack + metadata + headers); the reference runs ~25 eager ops
and builds the headers in a Python loop.
"""
from __future__ import annotations

import math

import torch

from . import _dev, _lib, primitives
from .errors import require

BLOCK, DIM = primitives.BLOCK, primitives.DIM


def pack3(q):
    """8 codes -> 3 bytes, LSB first (loop_kv_pk01_cache.py:7-16)."""
    require(q.dtype == torch.uint8, "3bit code range/dtype")
    return primitives.pack_codes(q, 3)


def unpack3(payload, shape):
    """Inverse of pack3 (loop_kv_pk01_cache.py:19-28)."""
    n = math.prod(shape)
    require(payload.dtype == torch.uint8 and payload.numel() == (n * 3 + 7) // 8, "3bit payload shape")
    return primitives.unpack_codes(payload, n, 3).reshape(tuple(shape))


def encode_group(x, start, bits=3, status=None, check=True):
    """Encode x [b,h,n,64,128] into a packed group (loop_kv_pk01_cache.py:31-37).

    One launch: rows (b, h) x blocks n; block i of every row gets header token
    offset ``start + 64*i``.
    """
    require(x.ndim == 5 and tuple(x.shape[-2:]) == (BLOCK, DIM), "Packed group input shape")
    require(bits in (3, 4, 5), "NSN bits must be 3, 4 or 5")
    _dev.require_gpu(x)
    b, h, n = x.shape[:3]
    rows = b * h
    order = _dev.norm_order(x)
    xc = primitives._as_encodable(x).contiguous()
    dev = x.device
    nbytes = BLOCK * DIM * bits // 8
    codes = torch.empty((b, h, n, nbytes), dtype=torch.uint8, device=dev)
    norm = torch.empty((b, h, n, BLOCK, 1), dtype=torch.float16, device=dev)
    mn = torch.empty((b, h, n, 1, DIM), dtype=torch.float16, device=dev)
    sc = torch.empty((b, h, n, 1, DIM), dtype=torch.float16, device=dev)
    hdr = torch.empty((b, h, n, 12), dtype=torch.uint8, device=dev)
    st = status if status is not None else _dev.new_status(dev)
    if rows and n:
        rc = _lib.lib().nsn_encode_blocks(
            xc.data_ptr(), _dev.dtype_code(xc.dtype), rows, n, n * BLOCK * DIM, 0, bits, order, 1,
            codes.data_ptr(), norm.data_ptr(), mn.data_ptr(), sc.data_ptr(), hdr.data_ptr(), None, n, 0, start,
            None, st.data_ptr(), _dev.stream())
        _lib.check(rc, "nsn_encode_blocks")
    if check and status is None:
        primitives._encode_raise(_dev.read_status(st))
    return dict(codes=codes, metas=(norm, mn, sc), headers=hdr)


def restore_group(g, dtype):
    """Exact reconstruction of a packed group -> [b, h, n*64, 128] (loop_kv_pk01_cache.py:40-42)."""
    codes = g["codes"]
    b, h, n, nbytes = codes.shape
    bits = nbytes * 8 // (BLOCK * DIM)
    return restore(codes.reshape(b * h, n, nbytes), g["metas"], bits, dtype).reshape(b, h, n * BLOCK, DIM)


def restore(codes, metas, bits, dtype, tail=None, out=None, status=None, check=True):
    """Restore packed blocks codes [rows, n, nbytes] and append ``tail`` [rows, L, 128].

    Returns [rows, n*64 + L, 128] of ``dtype``.
    """
    _dev.require_gpu(codes)
    rows, n, nbytes = codes.shape
    require(nbytes == BLOCK * DIM * bits // 8, "Packed code bytes per block")
    norm, mn, sc = (t.contiguous() for t in metas)
    require(norm.dtype == torch.float16 and mn.dtype == torch.float16 and sc.dtype == torch.float16, "Metadata dtype")
    require(norm.numel() == rows * n * BLOCK and mn.numel() == rows * n * DIM and sc.numel() == rows * n * DIM,
            "Metadata layout")
    L = 0 if tail is None else tail.shape[-2]
    if out is None:
        out = torch.empty((rows, n * BLOCK + L, DIM), dtype=dtype, device=codes.device)
    tl = None if tail is None else tail.contiguous()
    st = status if status is not None else _dev.new_status(codes.device)
    rc = _lib.lib().nsn_restore_blocks(
        codes.contiguous().data_ptr(), 0, norm.data_ptr(), mn.data_ptr(), sc.data_ptr(), rows, n, n, bits,
        out.data_ptr(), _dev.dtype_code(dtype), out.shape[1], _dev.ptr(tl),
        _dev.dtype_code(tl.dtype) if tl is not None else _lib.DTYPE_F16, L, L, st.data_ptr(), _dev.stream())
    _lib.check(rc, "nsn_restore_blocks")
    if check and status is None:
        primitives._restore_raise(_dev.read_status(st))
    return out


def append_group(old, new):
    """Concatenate two packed groups along blocks (loop_kv_pk01_cache.py:45-50)."""
    if old is None:
        return new
    return dict(codes=torch.cat((old["codes"], new["codes"]), 2),
                metas=tuple(torch.cat((a, b), 2) for a, b in zip(old["metas"], new["metas"])),
                headers=torch.cat((old["headers"], new["headers"]), 2))
