"""NSN arithmetic core on the GPU: the reference's L1 call surface.

Mirrors ``experiments/ac08/source/loop_kv_pilot.py:171-243``
(``pack_codes``, ``unpack_codes_reference``, ``nsn_encode``, ``nsn_decode``,
``nsn_qdq``, ``planned_bytes``) and ``papers/nsn-integrated/code/
nsn_int3_core.py:11-21`` (``nsn_int3_qdq``), with the same argument meaning,
output shapes/dtypes and exceptions.  Codes and fp16 metadata are bit-exact
with the reference's CPU functions; outputs are device tensors.
"""
from __future__ import annotations

import math

import torch

from . import _dev, _lib
from .errors import NumericalFailure, require

BLOCK = 64
DIM = 128
EPS = 1e-12


def _encode_raise(st):
    if st & _lib.ST_NONFINITE_INPUT:
        raise NumericalFailure("Nonfinite input to NSN")
    if st & _lib.ST_META_NONFINITE:
        raise NumericalFailure("FP16 metadata overflow/nonfinite")
    if st & _lib.ST_META_UNDERFLOW:
        raise NumericalFailure("Nonzero FP16 norm/step underflow")


def _as_encodable(x):
    return x if x.dtype in (torch.float16, torch.bfloat16, torch.float32) else x.float()


def encode_blocks(x, bits, *, zero_flat_scale=True, want_unpacked=True, want_headers=False, start=0,
                  status=None, check=True):
    """Encode every [64,128] block of ``x`` [..., 64, 128].

    Returns dict(codes [nb, 64*128*bits/8] u8, q [..., 64, 128] u8 | None,
    norm [..., 64, 1], min [..., 1, 128], scale [..., 1, 128] fp16,
    headers [nb, 12] | None).  ``check`` reads the status word and raises the
    reference's exceptions (a device sync).
    """
    require(x.ndim >= 2 and tuple(x.shape[-2:]) == (BLOCK, DIM), "NSN block shape")
    require(bits in (3, 4, 5), "NSN bits must be 3, 4 or 5")
    _dev.require_gpu(x)
    order = _dev.norm_order(x)
    xc = _as_encodable(x).contiguous()
    lead = tuple(x.shape[:-2])
    nb = math.prod(lead)
    dev = x.device
    codes = torch.empty((nb, BLOCK * DIM * bits // 8), dtype=torch.uint8, device=dev)
    q = torch.empty(x.shape, dtype=torch.uint8, device=dev) if want_unpacked else None
    n = torch.empty(lead + (BLOCK, 1), dtype=torch.float16, device=dev)
    m = torch.empty(lead + (1, DIM), dtype=torch.float16, device=dev)
    s = torch.empty(lead + (1, DIM), dtype=torch.float16, device=dev)
    hdr = torch.empty((nb, 12), dtype=torch.uint8, device=dev) if want_headers else None
    st = status if status is not None else _dev.new_status(dev)
    if nb:
        rc = _lib.lib().nsn_encode_blocks(
            xc.data_ptr(), _dev.dtype_code(xc.dtype), 1, nb, 0, 0, bits, order, 1 if zero_flat_scale else 0,
            codes.data_ptr(), n.data_ptr(), m.data_ptr(), s.data_ptr(), _dev.ptr(hdr), None, nb, 0, start,
            _dev.ptr(q), st.data_ptr(), _dev.stream())
        _lib.check(rc, "nsn_encode_blocks")
    if check and status is None:
        _encode_raise(_dev.read_status(st))
    return dict(codes=codes, q=q, norm=n, min=m, scale=s, headers=hdr)


def nsn_encode(x, bits):
    """``nsn_encode(x, bits)`` -> ``(q u8 [...,64,128], (n, m, s) fp16)`` (loop_kv_pilot.py:195-213)."""
    r = encode_blocks(x, bits)
    return r["q"], (r["norm"], r["min"], r["scale"])


def _restore_raise(st):
    if st & _lib.ST_NONFINITE_RESTORE:
        raise NumericalFailure("Nonfinite NSN reconstruction")


def nsn_decode(q, metas, dtype):
    """``nsn_decode(q, metas, dtype)`` (loop_kv_pilot.py:216-225): exact reconstruction."""
    n, m, s = metas
    require(q.dtype == torch.uint8 and q.ndim >= 2 and tuple(q.shape[-2:]) == (BLOCK, DIM), "NSN code shape")
    lead = tuple(q.shape[:-2])
    require(tuple(n.shape) == lead + (BLOCK, 1) and tuple(m.shape) == lead + (1, DIM) and tuple(s.shape) == lead + (1, DIM),
            "NSN metadata shape")
    _dev.require_gpu(q, n, m, s)
    nb = math.prod(lead)
    out = torch.empty(q.shape, dtype=dtype, device=q.device)
    if nb == 0:
        return out
    qc = q.contiguous()
    n16, m16, s16 = (t.to(torch.float16).contiguous() for t in (n, m, s))
    st = _dev.new_status(q.device)
    rc = _lib.lib().nsn_restore_blocks(
        qc.data_ptr(), 1, n16.data_ptr(), m16.data_ptr(), s16.data_ptr(), 1, nb, nb, 3,
        out.data_ptr(), _dev.dtype_code(dtype), nb * BLOCK, None, _lib.DTYPE_F16, 0, 0, st.data_ptr(), _dev.stream())
    _lib.check(rc, "nsn_restore_blocks")
    _restore_raise(_dev.read_status(st))
    return out


def nsn_qdq(x, bits):
    """``nsn_qdq(x, bits)`` = decode(encode(x)) in ``x.dtype`` (loop_kv_pilot.py:228-230)."""
    q, metas = nsn_encode(x, bits)
    return nsn_decode(q, metas, x.dtype)


def nsn_int3_qdq(x):
    """``nsn_int3_qdq(x)`` (papers/nsn-integrated/code/nsn_int3_core.py:11-21).

    Like the reference listing it runs no validity checks; for finite inputs
    its output equals ``nsn_qdq(x, 3)`` bit for bit.
    """
    r = encode_blocks(x, 3, zero_flat_scale=False, check=False)
    q, n, m, s = r["q"], r["norm"], r["min"], r["scale"]
    lead = tuple(q.shape[:-2])
    nb = math.prod(lead)
    out = torch.empty(q.shape, dtype=x.dtype if x.dtype in _dev.DTYPE_CODE else torch.float32, device=q.device)
    if nb:
        st = _dev.new_status(q.device)
        rc = _lib.lib().nsn_restore_blocks(
            q.data_ptr(), 1, n.data_ptr(), m.data_ptr(), s.data_ptr(), 1, nb, nb, 3, out.data_ptr(),
            _dev.dtype_code(out.dtype), nb * BLOCK, None, _lib.DTYPE_F16, 0, 0, st.data_ptr(), _dev.stream())
        _lib.check(rc, "nsn_restore_blocks")
    return out.to(x.dtype)


def pack_codes(codes, bits):
    """LSB-first bitstream (loop_kv_pilot.py:171-181) of a u8 code tensor -> u8 tensor."""
    _dev.require_gpu(codes)
    require(bits in (3, 4, 5) and codes.dtype == torch.uint8, "Invalid packed code")
    a = codes.contiguous().reshape(-1)
    out = torch.empty((a.numel() * bits + 7) // 8, dtype=torch.uint8, device=a.device)
    st = _dev.new_status(a.device)
    rc = _lib.lib().nsn_pack_codes(a.data_ptr(), a.numel(), bits, out.data_ptr(), st.data_ptr(), _dev.stream())
    _lib.check(rc, "nsn_pack_codes")
    require(not (_dev.read_status(st) & _lib.ST_CODE_RANGE), "Invalid packed code")
    return out


def unpack_codes(payload, count, bits):
    """Inverse of ``pack_codes`` (unpack_codes_reference, loop_kv_pilot.py:183-193)."""
    _dev.require_gpu(payload)
    require(bits in (3, 4, 5) and payload.dtype == torch.uint8 and payload.numel() == (count * bits + 7) // 8,
            "Packed payload shape")
    p = payload.contiguous().reshape(-1)
    out = torch.empty(count, dtype=torch.uint8, device=p.device)
    rc = _lib.lib().nsn_unpack_codes(p.data_ptr(), count, bits, out.data_ptr(), _dev.stream())
    _lib.check(rc, "nsn_unpack_codes")
    return out


unpack_codes_reference = unpack_codes


def planned_bytes(shape, compressed_tokens, bits):
    """Byte accounting of a packed cache (loop_kv_pilot.py:233-243)."""
    b, h, length, d = shape
    require(compressed_tokens % BLOCK == 0 and 0 <= compressed_tokens <= length, "Block accounting")
    if bits is None:
        return {"codes": 0, "metadata": 0, "native": b * h * length * d * 2, "block_headers": 0}
    blocks = b * h * (compressed_tokens // BLOCK)
    return {"codes": blocks * ((BLOCK * d * bits + 7) // 8),
            "metadata": blocks * (BLOCK * 2 + d * 4),
            "native": b * h * (length - compressed_tokens) * d * 2, "block_headers": blocks * 12}
