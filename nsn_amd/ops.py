"""The call surface as registered PyTorch operators: ``torch.ops.nsn.*``.

Each operator runs the same HIP path as the Python function it wraps (so its
results are bitwise those of that function) and has a fake implementation
that gives output shapes and dtypes without running anything, for tracing,
``torch.compile`` and meta tensors.  Only CUDA (HIP) tensors have a kernel:
CPU tensors raise, as the library has no CPU path.

======================================  =============================================
operator                                wraps (reference function it replaces)
======================================  =============================================
nsn::encode(x, bits)                    primitives.nsn_encode (loop_kv_pilot.py:195-213)
nsn::decode(q, n, m, s, dtype)          primitives.nsn_decode (loop_kv_pilot.py:216-225)
nsn::int3_qdq(x)                        primitives.nsn_int3_qdq (nsn_int3_core.py:11-21)
nsn::pack_codes(codes, bits)            primitives.pack_codes (loop_kv_pilot.py:171-181)
nsn::unpack_codes(payload, count, bits) primitives.unpack_codes (loop_kv_pilot.py:183-193)
nsn::encode_group(x, start, bits)       codec.encode_group (loop_kv_pk01_cache.py:31-37)
nsn::restore_group(codes, n, m, s, dt)  codec.restore_group (loop_kv_pk01_cache.py:40-42)
nsn::decode_attention(...)              kernels.decode_attention (loop_kv_vf01_kernel.py:128-139,
                                        loop_kv_nb06_kernel.py:54-154)
nsn::prefill_attention(...)             kernels.prefill_attention (loop_kv_pk01_cache.py:87-106)
======================================  =============================================

The attention operators take a packed side as its tensors -- codes, norm,
min, scale, decode factors, per-sequence block counts, tail -- in that order
(see ``kernels.PackedKV``); a side without packed blocks passes None for the
first six.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import codec, kernels, primitives

BLOCK, DIM = 64, 128
_DEV = "cuda"


def _side(codes, norm, mn, sc, factor, blocks, tail, bits):
    if codes is None and tail is None:
        return None
    return kernels.PackedKV(codes=codes, norm=norm, min=mn, scale=sc, factor=factor, blocks=blocks, tail=tail,
                            bits=bits)


# ---------------------------------------------------------------- codec

@torch.library.custom_op("nsn::encode", mutates_args=(), device_types=_DEV)
def encode(x: torch.Tensor, bits: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    q, (n, m, s) = primitives.nsn_encode(x, bits)
    return q, n, m, s


@encode.register_fake
def _(x, bits):
    lead = tuple(x.shape[:-2])
    return (x.new_empty(x.shape, dtype=torch.uint8), x.new_empty(lead + (BLOCK, 1), dtype=torch.float16),
            x.new_empty(lead + (1, DIM), dtype=torch.float16), x.new_empty(lead + (1, DIM), dtype=torch.float16))


@torch.library.custom_op("nsn::decode", mutates_args=(), device_types=_DEV)
def decode(q: torch.Tensor, n: torch.Tensor, m: torch.Tensor, s: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    return primitives.nsn_decode(q, (n, m, s), dtype)


@decode.register_fake
def _(q, n, m, s, dtype):
    return q.new_empty(q.shape, dtype=dtype)


@torch.library.custom_op("nsn::int3_qdq", mutates_args=(), device_types=_DEV)
def int3_qdq(x: torch.Tensor) -> torch.Tensor:
    return primitives.nsn_int3_qdq(x)


@int3_qdq.register_fake
def _(x):
    return torch.empty_like(x)


@torch.library.custom_op("nsn::pack_codes", mutates_args=(), device_types=_DEV)
def pack_codes(codes: torch.Tensor, bits: int) -> torch.Tensor:
    return primitives.pack_codes(codes, bits)


@pack_codes.register_fake
def _(codes, bits):
    return codes.new_empty(((codes.numel() * bits + 7) // 8,), dtype=torch.uint8)


@torch.library.custom_op("nsn::unpack_codes", mutates_args=(), device_types=_DEV)
def unpack_codes(payload: torch.Tensor, count: int, bits: int) -> torch.Tensor:
    return primitives.unpack_codes(payload, count, bits)


@unpack_codes.register_fake
def _(payload, count, bits):
    return payload.new_empty((count,), dtype=torch.uint8)


@torch.library.custom_op("nsn::encode_group", mutates_args=(), device_types=_DEV)
def encode_group(x: torch.Tensor, start: int, bits: int = 3) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                       torch.Tensor, torch.Tensor]:
    g = codec.encode_group(x, start, bits)
    n, m, s = g["metas"]
    return g["codes"], n, m, s, g["headers"]


@encode_group.register_fake
def _(x, start, bits=3):
    b, h, n = x.shape[:3]
    f16 = torch.float16
    return (x.new_empty((b, h, n, BLOCK * DIM * bits // 8), dtype=torch.uint8),
            x.new_empty((b, h, n, BLOCK, 1), dtype=f16), x.new_empty((b, h, n, 1, DIM), dtype=f16),
            x.new_empty((b, h, n, 1, DIM), dtype=f16), x.new_empty((b, h, n, 12), dtype=torch.uint8))


@torch.library.custom_op("nsn::restore_group", mutates_args=(), device_types=_DEV)
def restore_group(codes: torch.Tensor, n: torch.Tensor, m: torch.Tensor, s: torch.Tensor,
                  dtype: torch.dtype) -> torch.Tensor:
    return codec.restore_group({"codes": codes, "metas": (n, m, s)}, dtype)


@restore_group.register_fake
def _(codes, n, m, s, dtype):
    b, h, nb = codes.shape[:3]
    return codes.new_empty((b, h, nb * BLOCK, DIM), dtype=dtype)


# ---------------------------------------------------------------- attention

@torch.library.custom_op("nsn::decode_attention", mutates_args=(), device_types=_DEV)
def decode_attention(q: torch.Tensor,
                     k_codes: Optional[torch.Tensor], k_norm: Optional[torch.Tensor], k_min: Optional[torch.Tensor],
                     k_scale: Optional[torch.Tensor], k_factor: Optional[torch.Tensor],
                     k_blocks: Optional[torch.Tensor], k_tail: Optional[torch.Tensor],
                     v_codes: Optional[torch.Tensor], v_norm: Optional[torch.Tensor], v_min: Optional[torch.Tensor],
                     v_scale: Optional[torch.Tensor], v_factor: Optional[torch.Tensor],
                     v_blocks: Optional[torch.Tensor], v_tail: Optional[torch.Tensor],
                     seq_len: torch.Tensor, bits: int, max_seq_len: int,
                     kernel: str = "fast") -> Tuple[torch.Tensor, torch.Tensor]:
    k = _side(k_codes, k_norm, k_min, k_scale, k_factor, k_blocks, k_tail, bits)
    v = _side(v_codes, v_norm, v_min, v_scale, v_factor, v_blocks, v_tail, bits)
    out, ctx = kernels.decode_attention(q, k, v, seq_len, max_seq_len=max_seq_len, kernel=kernel)
    return out, ctx


@decode_attention.register_fake
def _(q, *args, **kw):
    return q.new_empty(q.shape, dtype=torch.bfloat16), q.new_empty(q.shape, dtype=torch.float32)


@torch.library.custom_op("nsn::prefill_attention", mutates_args=(), device_types=_DEV)
def prefill_attention(q: torch.Tensor,
                      k_codes: Optional[torch.Tensor], k_norm: Optional[torch.Tensor], k_min: Optional[torch.Tensor],
                      k_scale: Optional[torch.Tensor], k_factor: Optional[torch.Tensor],
                      k_blocks: Optional[torch.Tensor], k_tail: Optional[torch.Tensor],
                      v_codes: Optional[torch.Tensor], v_norm: Optional[torch.Tensor], v_min: Optional[torch.Tensor],
                      v_scale: Optional[torch.Tensor], v_factor: Optional[torch.Tensor],
                      v_blocks: Optional[torch.Tensor], v_tail: Optional[torch.Tensor],
                      ctx_len: torch.Tensor, k_chunk: torch.Tensor, v_chunk: torch.Tensor,
                      bits: int) -> torch.Tensor:
    k = _side(k_codes, k_norm, k_min, k_scale, k_factor, k_blocks, k_tail, bits)
    v = _side(v_codes, v_norm, v_min, v_scale, v_factor, v_blocks, v_tail, bits)
    return kernels.prefill_attention(q, k, v, ctx_len, k_chunk, v_chunk)


@prefill_attention.register_fake
def _(q, *args, **kw):
    return torch.empty_like(q)


def side_tensors(side: Optional[kernels.PackedKV]) -> List[Optional[torch.Tensor]]:
    """The seven tensors of a packed side in operator argument order (None: no side)."""
    if side is None:
        return [None] * 7
    return [side.codes, side.norm, side.min, side.scale, side.factor, side.blocks, side.tail]


OPS = ("encode", "decode", "int3_qdq", "pack_codes", "unpack_codes", "encode_group", "restore_group",
       "decode_attention", "prefill_attention")
