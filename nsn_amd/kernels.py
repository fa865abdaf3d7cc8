"""Decode-attention readout over packed K/V: the reference's L3 call surface.

Mirrors (paths relative to the reference root):
  * VF01 fused / bridge routes: ``restore_v``, ``launch``, ``pipeline``
    (experiments/ac08/source/loop_kv_vf01_kernel.py:117-158);
  * AF01 attention with materialised V or given scores: ``af_launch``
    (experiments/ac08/source/loop_kv_af01_kernel.py:100-111);
  * the grouped input checks ``structural`` / ``finite``
    (experiments/ac08/source/loop_kv_vf01_checks.py:5-63,
    loop_kv_qk01_kernel.py:66-78, loop_kv_rf01_kernel.py:49-58);
  * the GQA route (experiments/nb06/source/loop_kv_nb06_kernel.py:142-191):
    ``launch`` serves any Hq = G*Hkv -- query head h reads kv head h // G.
The reference requires batch 1; ``decode_attention`` is the batched, ragged
form the benchmark configurations need (one call for B sequences).
"""
from __future__ import annotations

import functools
import math
from dataclasses import dataclass
from typing import Optional

import numpy as np
import torch

from . import _dev, _lib, codec
from .errors import ContractError, IntegrityError, NumericalFailure, require

SCALE = 0.08838834764831845   # 1/sqrt(128), loop_kv_vf01_kernel.py:90
BLOCK, DIM = 64, 128
PART_STRIDE = 132
LAST_STAGE = "idle"

KERNELS = {"reference": _lib.ATTN_REFERENCE, "fast": _lib.ATTN_FAST}


@dataclass
class PackedKV:
    """One side (K or V) of a batched packed cache.

    codes  u8  [B, Hkv, cap, 64*128*bits/8]     norm f16 [B, Hkv, cap, 64(,1)]
    min    f16 [B, Hkv, cap, (1,)128]           scale f16 [B, Hkv, cap, (1,)128]
    factor f32 [B, Hkv, cap, 64]  decode factors n/|m+s*q| (fast kernel; see nsn_block_factors)
    blocks i32 [B]  packed blocks of each sequence (tokens 0 .. 64*blocks-1)
    tail   f16/bf16 [B, Hkv, tail_cap, 128]  tokens 64*blocks[b] .. seq_len[b]-1
    """
    codes: Optional[torch.Tensor]
    norm: Optional[torch.Tensor]
    min: Optional[torch.Tensor]
    scale: Optional[torch.Tensor]
    factor: Optional[torch.Tensor]
    blocks: Optional[torch.Tensor]
    tail: Optional[torch.Tensor]
    bits: int = 3

    @property
    def heads(self):
        return (self.codes if self.codes is not None else self.tail).shape[1]

    def side(self):
        s = _lib.KVSide()
        if self.codes is not None:
            s.codes = self.codes.data_ptr()
            s.norms = self.norm.data_ptr()
            s.mins = self.min.data_ptr()
            s.scales = self.scale.data_ptr()
            if self.factor is not None:
                s.factors = self.factor.data_ptr()
            s.blocks = self.blocks.data_ptr()
            s.block_cap = self.codes.shape[2]
        if self.tail is not None:
            s.tail = self.tail.data_ptr()
            s.tail_dtype = _dev.dtype_code(self.tail.dtype)
            s.tail_cap = self.tail.shape[2]
        else:
            s.tail_dtype = _lib.DTYPE_F16
        return s

    def validate(self, batch, heads):
        if self.codes is not None:
            nbytes = BLOCK * DIM * self.bits // 8
            require(self.codes.dtype == torch.uint8 and self.codes.is_contiguous() and self.codes.ndim == 4
                    and tuple(self.codes.shape[:2]) == (batch, heads) and self.codes.shape[3] == nbytes,
                    "Packed codes layout")
            cap = self.codes.shape[2]
            for t, last in ((self.norm, BLOCK), (self.min, DIM), (self.scale, DIM)):
                require(t.dtype == torch.float16 and t.is_contiguous() and t.numel() == batch * heads * cap * last,
                        "Packed metadata layout")
            require(self.blocks is not None and self.blocks.dtype == torch.int32 and self.blocks.numel() == batch,
                    "Packed block counts")
            if self.factor is not None:
                require(self.factor.dtype == torch.float32 and self.factor.is_contiguous()
                        and self.factor.numel() == batch * heads * cap * BLOCK, "Decode factor layout")
        if self.tail is not None:
            require(self.tail.dtype in (torch.float16, torch.bfloat16) and self.tail.is_contiguous()
                    and self.tail.ndim == 4 and tuple(self.tail.shape[:2]) == (batch, heads)
                    and self.tail.shape[3] == DIM, "Tail shape/type")


def workspace_floats(batch, heads_q, n_splits):
    """Workspace of nsn_decode_attention: [B, Hq, n_splits, 132] fp32 partials,
    then one int32 partial count per (b, hq)."""
    return batch * heads_q * (n_splits * PART_STRIDE + 1)


def default_split(batch, heads_kv, max_len, target_units=4096, min_split=256):
    """Split the context so that batch*heads_kv*splits covers the 256 CUs several times."""
    want = max(1, math.ceil(target_units / max(1, batch * heads_kv)))
    split = max(min_split, math.ceil(max_len / want / BLOCK) * BLOCK)
    split = min(split, math.ceil(max_len / BLOCK) * BLOCK)
    return max(BLOCK, split), max(1, math.ceil(max_len / max(BLOCK, split)))


def _decode_args(q, k: Optional[PackedKV], v: PackedKV, seq_len, *, max_seq_len=None, scores=None,
                     kernel="reference", kv_round_dtype=None, split_tokens=None, out_dtype=torch.bfloat16,
                     scale=SCALE, status=None, check=True, workspace=None, out=None, ctx=None, merge=True,
                     static_workspace=False, trace_scores=None, trace_v=None, validate_lengths=None):
    """decode_attention's checks and argument block: (entry point, args,
    status, out, ctx, workspace)."""
    _dev.require_gpu(q, seq_len)
    require(q.ndim == 3 and q.shape[2] == DIM and q.is_contiguous(), "Query shape/type")
    B, Hq = q.shape[:2]
    Hkv = v.heads
    require(Hq % Hkv == 0 and Hq // Hkv <= 16, "GQA group")
    require(seq_len.dtype == torch.int32 and seq_len.numel() == B and seq_len.is_cuda, "Sequence lengths")
    v.validate(B, Hkv)
    if kernel == "fast":
        for side in ((v,) if scores is not None else (k, v)):
            require(side.codes is None or side.factor is not None, "Fast kernel needs decode factors")
        require(v.bits in (3, 5), "Fast kernel supports 3- and 5-bit codes")
    if scores is None:
        require(k is not None, "K cache required")
        k.validate(B, Hkv)
        require(k.bits == v.bits, "K/V bit widths differ")
        if k.tail is not None and v.tail is not None:
            require(k.tail.dtype == v.tail.dtype, "K/V tail dtypes differ")
    else:
        require(scores.dtype == torch.float32 and scores.is_contiguous() and scores.ndim == 3
                and tuple(scores.shape[:2]) == (B, Hq), "Score shape/type")
    if validate_lengths is None:
        validate_lengths = max_seq_len is None or check
    if validate_lengths:
        _validate_lengths(seq_len, k if scores is None else None, v, scores, max_seq_len)
    if max_seq_len is None:
        max_seq_len = int(seq_len.max().item())
    if split_tokens is None:
        split_tokens, n_splits = default_split(B, Hkv, max_seq_len)
    else:
        n_splits = max(1, math.ceil(max_seq_len / split_tokens))
    if kernel == "fast":
        # the fast kernel balances blocks over a fixed grid; n_splits is its
        # partial-slot capacity per (b, hq) and must be at least 2
        n_splits = max(2, n_splits)
    if kv_round_dtype is None:
        tdt = v.tail.dtype if v.tail is not None else torch.bfloat16
        kv_round_dtype = tdt
    dev = q.device
    need = workspace_floats(B, Hq, n_splits)
    if static_workspace:
        require(need <= _lib.STATIC_SCRATCH_FLOATS,
                f"Decode workspace of {need} floats exceeds the static scratch ({_lib.STATIC_SCRATCH_FLOATS})")
    elif workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.float32, device=dev)
    if out is None:
        out = torch.empty((B, Hq, DIM), dtype=out_dtype, device=dev)
    if ctx is None:
        ctx = torch.empty((B, Hq, DIM), dtype=torch.float32, device=dev)
    st = status if status is not None else _dev.new_status(dev)
    a = _lib.AttnArgs()
    a.q = q.data_ptr()
    a.q_dtype = _dev.dtype_code(q.dtype)
    a.batch, a.heads_q, a.heads_kv = B, Hq, Hkv
    a.scale = scale
    a.seq_len = seq_len.data_ptr()
    a.max_seq_len = max_seq_len
    a.bits = v.bits
    a.k_mode = _lib.KV_SCORES if scores is not None else _lib.KV_PACKED
    if scores is None:
        a.k = k.side()
    else:
        a.scores = scores.data_ptr()
        a.scores_cap = scores.shape[2]
    a.v = v.side()
    a.kernel = KERNELS[kernel]
    a.kv_round_dtype = _dev.dtype_code(kv_round_dtype)
    a.split_tokens = split_tokens
    a.n_splits = n_splits
    a.partials = 0 if static_workspace else workspace.data_ptr()
    a.ctx = ctx.data_ptr()
    a.out = out.data_ptr()
    a.out_dtype = _dev.dtype_code(out_dtype)
    a.status = st.data_ptr()
    a.merge = 1 if merge else 0
    if trace_scores is not None or trace_v is not None:
        require(kernel == "reference", "Trace outputs come from the exact-order kernel")
        cap = (trace_scores if trace_scores is not None else trace_v).shape[2]
        if trace_scores is not None:
            require(trace_scores.dtype == torch.float32 and trace_scores.is_contiguous() and trace_scores.is_cuda
                    and tuple(trace_scores.shape) == (B, Hq, cap), "Trace score shape/type")
            a.trace_scores = trace_scores.data_ptr()
        if trace_v is not None:
            require(trace_v.dtype == torch.float32 and trace_v.is_contiguous() and trace_v.is_cuda
                    and tuple(trace_v.shape) == (B, Hkv, cap, DIM), "Trace V shape/type")
            a.trace_v = trace_v.data_ptr()
        require(cap >= max_seq_len, "Trace capacity below max_seq_len")
        a.trace_cap = cap
    entry = "nsn_decode_attention_static" if static_workspace else "nsn_decode_attention"
    return entry, a, st, out, ctx, workspace


def decode_attention(q, k: Optional[PackedKV], v: PackedKV, seq_len, *, max_seq_len=None, scores=None,
                     kernel="reference", kv_round_dtype=None, split_tokens=None, out_dtype=torch.bfloat16,
                     scale=SCALE, status=None, check=True, workspace=None, out=None, ctx=None, merge=True,
                     static_workspace=False, trace_scores=None, trace_v=None, validate_lengths=None):
    """Batched single-query decode attention.

    q [B, Hq, 128]; seq_len i32 [B] (device); returns (out [B,Hq,128] out_dtype,
    ctx [B,Hq,128] fp32).  ``scores`` [B, Hq, cap] fp32 replaces K (the AF01
    FULL=False readout).  ``check`` syncs and raises NumericalFailure on any
    nonfinite intermediate/output.  ``static_workspace`` runs through
    nsn_decode_attention_static: the partials live in the library's per-device
    scratch array (at most ``_lib.STATIC_SCRATCH_FLOATS`` floats), so with
    ``out``, ``ctx`` and ``status`` given the call allocates nothing.
    ``trace_scores`` [B, Hq, cap] and ``trace_v`` [B, Hkv, cap, 128] (fp32,
    cap >= max_seq_len; reference kernel only) receive what the kernel itself
    computed for every token t < seq_len[b]: its scores and the V rows it
    multiplied (the TRACE stores of loop_kv_vf01_kernel.py:104,113).
    ``validate_lengths`` (default: with ``check`` or without ``max_seq_len``)
    copies the lengths and block counts to the host and checks them against
    the buffers; callers that built them from tensor shapes pass False.
    """
    entry, a, st, out, ctx, _ = _decode_args(
        q, k, v, seq_len, max_seq_len=max_seq_len, scores=scores, kernel=kernel, kv_round_dtype=kv_round_dtype,
        split_tokens=split_tokens, out_dtype=out_dtype, scale=scale, status=status, check=check,
        workspace=workspace, out=out, ctx=ctx, merge=merge, static_workspace=static_workspace,
        trace_scores=trace_scores, trace_v=trace_v, validate_lengths=validate_lengths)
    rc = getattr(_lib.lib(), entry)(a, _dev.stream())
    _lib.check(rc, entry)
    if check and status is None:
        s = _dev.read_status(st)
        if s & _lib.ST_CAPACITY:
            raise IntegrityError("Sequence length past the cache's block / tail capacity")
        if s & _lib.ST_WORKSPACE:
            raise IntegrityError("Decode workspace too small: n_splits below the fast kernel's partial slots")
        if s & _lib.ST_EMPTY:
            raise IntegrityError("A sequence attended no token (zero length)")
        if s & _lib.ST_NONFINITE_ATTN_INPUT:
            raise NumericalFailure("Nonfinite raw attention input (q, tail or block metadata)")
        if s & (_lib.ST_NONFINITE_ATTN | _lib.ST_NONFINITE_RESTORE | _lib.ST_NONFINITE_OUTPUT):
            raise NumericalFailure("Nonfinite fused attention intermediate/output")
    return out, ctx


def prepare_decode(q, k: Optional[PackedKV], v: PackedKV, seq_len, *, max_seq_len, **kwargs):
    """decode_attention's checks and argument block, done once, for a loop
    that decodes over the same buffers again and again (a serving loop's
    fixed-shape steps; the C2 bench).  Takes decode_attention's arguments
    (``max_seq_len`` required, ``check`` off) and returns ``launch()``, which
    enqueues the same kernel launch(es) on the current stream with no other
    host work, and whose return value is (out, ctx).  Each launch reads the
    buffers' current contents (q, caches, lengths), so they may change
    between launches, but not their storage or shapes; nonfinite and
    capacity flags accumulate in ``status``, which the caller reads.
    """
    require(not kwargs.get("check", False), "prepare_decode launches without the host status check")
    require(kwargs.get("trace_scores") is None and kwargs.get("trace_v") is None, "No trace outputs in prepared launches")
    kwargs["check"] = False
    kwargs.setdefault("validate_lengths", True)
    if kwargs.get("status") is None:
        kwargs["status"] = _dev.new_status(q.device)
    entry, a, st, out, ctx, workspace = _decode_args(q, k, v, seq_len, max_seq_len=max_seq_len, **kwargs)
    fn = getattr(_lib.lib(), entry)
    keep = (q, k, v, seq_len, st, out, ctx, workspace)   # the storage the argument block points at

    def launch():
        _lib.check(fn(a, _dev.stream()), entry)
        return keep[5], keep[6]

    launch.status = st
    return launch


def prefill_attention(q, k: Optional[PackedKV], v: Optional[PackedKV], ctx_len, k_chunk, v_chunk, *, scale=SCALE,
                      status=None, check=True, out=None, append=False, precise_weights=None):
    """Chunked-prefill attention over a packed context (C4's prefill step).

    q [B, Hq, n, 128]; k_chunk, v_chunk [B, Hkv, n, 128] (the chunk's own K/V;
    one dtype, fp16 or bf16, for q, chunk and output, and the dtype of the
    MFMA products; the tails may hold either dtype).  Chunk query i
    attends the context -- ``blocks[b]`` packed blocks then ``ctx_len[b] -
    64*blocks[b]`` tail tokens of k/v (None: no context) -- and chunk tokens
    0..i.  Returns out [B, Hq, n, 128].  The reference materialises the
    packed blocks and runs dense attention instead
    (loop_kv_pk01_cache.py:87-106).  ``append=True`` also writes the
    chunk's K/V into the tails right after each sequence's context tokens
    (rounded to the tail dtype), in the same launch: the cache update
    (loop_kv_pk01_cache.py:101-102) that otherwise follows as a separate
    append; k and v must then carry tails with room for n more tokens.
    ``precise_weights`` (bf16 only): the softmax weights enter the PV product
    as bf16 hi + lo (~2^-17 relative) instead of one bf16 rounding, at ~24 %
    more kernel time; None = only when there is no context (k is None), where
    the first queries attend a handful of tokens.
    """
    _dev.require_gpu(q, k_chunk, v_chunk, ctx_len)
    require(q.ndim == 4 and q.shape[3] == DIM and q.is_contiguous(), "Query shape/type")
    B, Hq, n, _ = q.shape
    require(q.dtype in (torch.float16, torch.bfloat16), "Prefill dtype (fp16 or bf16)")
    require(k_chunk.dtype == q.dtype and v_chunk.dtype == q.dtype and k_chunk.shape == v_chunk.shape
            and k_chunk.ndim == 4 and k_chunk.shape[0] == B and k_chunk.shape[2] == n and k_chunk.shape[3] == DIM
            and k_chunk.is_contiguous() and v_chunk.is_contiguous(), "Chunk K/V shape/type")
    Hkv = k_chunk.shape[1]
    require(Hq % Hkv == 0, "GQA group")
    require(ctx_len.dtype == torch.int32 and ctx_len.numel() == B and ctx_len.is_cuda, "Context lengths")
    a = _lib.PrefillArgs()
    bits = 3
    if (k is None) != (v is None):
        raise ContractError("K and V context must both be given or both be None")
    if k is not None:
        for side in (k, v):
            side.validate(B, Hkv)
            require(side.codes is None or side.factor is not None, "Prefill needs decode factors")
            require(side.tail is None or side.tail.dtype in (torch.float16, torch.bfloat16), "Tail dtype (fp16 or bf16)")
        require(k.bits == v.bits and k.bits in (3, 5), "Prefill supports 3- and 5-bit codes")
        require(k.tail is None or v.tail is None or k.tail.dtype == v.tail.dtype, "K/V tail dtypes differ")
        require((k.codes is None) == (v.codes is None), "K/V packed layout differs")
        bits = k.bits
        if check:
            L = ctx_len.cpu().numpy().astype(np.int64)
            nk = k.blocks.cpu().numpy().astype(np.int64) if k.codes is not None else np.zeros_like(L)
            nv = v.blocks.cpu().numpy().astype(np.int64) if v.codes is not None else np.zeros_like(L)
            require(np.array_equal(nk, nv), "K/V packed block counts differ")
            tk = k.tail.shape[2] if k.tail is not None else 0
            tv = v.tail.shape[2] if v.tail is not None else 0
            rest = L - BLOCK * nk
            require(np.all(rest >= 0) and np.all(rest <= min(tk, tv)), "Context tail exceeds capacity")
            if k.codes is not None:
                require(np.all(nk <= k.codes.shape[2]), "Packed block count exceeds capacity")
        a.k = k.side()
        a.v = v.side()
    elif check:
        require(bool((ctx_len == 0).all()), "Context lengths without a context")
    if append:
        require(k is not None and k.tail is not None and v.tail is not None, "Append needs both tails")
        if check:
            L = ctx_len.cpu().numpy().astype(np.int64)
            nb = k.blocks.cpu().numpy().astype(np.int64) if k.codes is not None else np.zeros_like(L)
            require(np.all(L - BLOCK * nb + n <= min(k.tail.shape[2], v.tail.shape[2])),
                    "Tail overflow: compress before appending more tokens")
    if out is None:
        out = torch.empty_like(q)
    st = status if status is not None else _dev.new_status(q.device)
    a.q = q.data_ptr()
    a.dtype = _dev.dtype_code(q.dtype)
    a.batch, a.heads_q, a.heads_kv, a.n_q = B, Hq, Hkv, n
    a.scale = scale
    a.ctx_len = ctx_len.data_ptr()
    a.bits = bits
    a.k_chunk = k_chunk.data_ptr()
    a.v_chunk = v_chunk.data_ptr()
    a.out = out.data_ptr()
    a.status = st.data_ptr()
    a.append = 1 if append else 0
    a.precise_weights = 1 if (k is None if precise_weights is None else precise_weights) else 0
    rc = _lib.lib().nsn_prefill_attention(a, _dev.stream())
    _lib.check(rc, "nsn_prefill_attention")
    if check and status is None:
        s = _dev.read_status(st)
        if s & _lib.ST_CAPACITY:
            raise IntegrityError("Inconsistent cache: K/V block counts differ, the tail exceeds its capacity "
                                 "or lacks room for the append")
        if s & (_lib.ST_NONFINITE_ATTN | _lib.ST_NONFINITE_OUTPUT):
            raise NumericalFailure("Nonfinite prefill output")
    return out


def _validate_lengths(seq_len, k, v, scores, max_seq_len):
    """Host check (one device->host copy) that every token the kernels will
    touch lies inside the caller's buffers: 0 < seq_len[b] <= max_seq_len,
    blocks[b] <= block capacity, 0 <= seq_len[b] - 64*blocks[b] <= tail capacity,
    seq_len[b] <= score capacity."""
    L = seq_len.cpu().numpy().astype(np.int64)
    require(np.all(L > 0), "Empty sequence")
    if max_seq_len is not None:
        require(np.all(L <= max_seq_len), "Sequence longer than max_seq_len")
    for side in (k, v):
        if side is None:
            continue
        nb = side.blocks.cpu().numpy().astype(np.int64) if side.codes is not None else np.zeros_like(L)
        cap = side.codes.shape[2] if side.codes is not None else 0
        tcap = side.tail.shape[2] if side.tail is not None else 0
        require(np.all(nb >= 0) and np.all(nb <= cap), "Packed block count exceeds capacity")
        rest = L - BLOCK * nb
        require(np.all(rest >= 0) and np.all(rest <= tcap), "Tail exceeds capacity / packed past length")
    if scores is not None:
        require(np.all(L <= scores.shape[2]), "Score length")


# --------------------------------------------------- reference (b == 1) surface

def block_factors(codes, norm, mn, sc, bits, status=None):
    """Decode factors n/|m+s*q| of packed blocks codes [rows, n, nbytes] -> fp32 [rows, n, 64].
    ``status`` (int32 device word) receives NSN_ST_NONFINITE_ATTN_INPUT for nonfinite metadata."""
    rows, n, _ = codes.shape
    out = torch.empty((rows, n, BLOCK), dtype=torch.float32, device=codes.device)
    norm, mn, sc = (t.contiguous() for t in (norm, mn, sc))
    rc = _lib.lib().nsn_block_factors(codes.contiguous().data_ptr(), norm.data_ptr(), mn.data_ptr(), sc.data_ptr(),
                                      rows, n, n, bits, out.data_ptr(),
                                      None if status is None else status.data_ptr(), _dev.stream())
    _lib.check(rc, "nsn_block_factors")
    return out


def _group_side(g, tail, bits=None, factors=False, status=None):
    """Reference group dict (+ tail [1,H,L,128]) -> PackedKV for batch 1.  With
    ``factors`` the decode factors are computed (and the metadata checked into
    ``status``)."""
    dev = tail.device
    if g is None:
        return PackedKV(None, None, None, None, None, None, tail.contiguous(), bits or 3)
    codes = g["codes"]
    b_, h, n, nbytes = codes.shape
    b = (nbytes * 8) // (BLOCK * DIM)
    f = None
    if factors:
        f = block_factors(codes.reshape(b_ * h, n, nbytes), *g["metas"], b, status=status).reshape(b_, h, n, BLOCK)
    return PackedKV(codes, g["metas"][0], g["metas"][1], g["metas"][2], f, _length_tensor(n, dev),
                    tail.contiguous(), b)


@functools.lru_cache(maxsize=256)
def _length_tensor(T, device):
    """A [1] int32 device tensor holding T, made once per (T, device): the
    batch-1 routes read it (as a length or a block count) and never write
    it, so one fill per value serves every call."""
    return torch.full((1,), T, dtype=torch.int32, device=device)


def _length(g, tail):
    return (0 if g is None else g["codes"].shape[2] * BLOCK) + tail.shape[2]


def _shape_check(g, h):
    codes = g["codes"]
    require(codes.ndim == 4 and codes.dtype == torch.uint8 and codes.is_contiguous()
            and codes.shape[-1] in (3072, 4096, 5120), "RF01 packed layout")
    b, gh, n, _ = codes.shape
    require(b > 0 and gh > 0 and n > 0, "RF01 nonempty shape")
    shapes = [(b, gh, n, 64, 1), (b, gh, n, 1, 128), (b, gh, n, 1, 128)]
    require(len(g["metas"]) == 3 and all(tuple(a.shape) == sh and a.dtype == torch.float16 and a.is_contiguous()
                                         and a.device == codes.device for a, sh in zip(g["metas"], shapes)),
            "RF01 metadata layout")
    require(b == 1 and gh == h, "Packed head/device mismatch")
    return n


def _qshape(g, tail, q):
    require(tail.ndim == 4 and tail.shape[0] == 1 and tail.shape[-1] == 128
            and tail.dtype in (torch.bfloat16, torch.float16) and tail.is_contiguous(), "Tail shape/type")
    h = tail.shape[1]
    require(h > 0 and q.ndim == 4 and q.shape[0] == 1 and q.shape[2:] == (1, 128) and q.shape[1] % h == 0
            and q.dtype in (torch.bfloat16, torch.float16) and q.is_contiguous(), "Query shape/type")
    require(q.device == tail.device and tail.is_cuda, "CUDA only; no fallback")
    compressed = 0 if g is None else _shape_check(g, h) * 64
    require(tail.shape[-2] + compressed > 0, "Empty sequence")
    return h, compressed, compressed + tail.shape[-2]


def structural(g, kt, q, vg, vt):
    """Layout contract (loop_kv_vf01_checks.py:5-12): raises IntegrityError."""
    k = _qshape(g, kt, q)
    v = _qshape(vg, vt, q)
    require(k == v, "K/V lengths differ")
    for group in (g, vg):
        if group is not None:
            hd = group.get("headers")
            b, nh, n, _ = group["codes"].shape
            require(hd is not None and hd.dtype == torch.uint8 and hd.is_contiguous()
                    and tuple(hd.shape) == (b, nh, n, 12) and hd.device == q.device, "Header layout")
    return k[2]


def finite(g, kt, q, vg, vt):
    """One grouped NaN/Inf scan over q, tails and metadata (loop_kv_vf01_checks.py:55-63)."""
    arrays = [q, kt] + ([] if g is None else list(g["metas"])) + [vt] + ([] if vg is None else list(vg["metas"]))
    ptrs = (ctypes_array("c_void_p", [a.data_ptr() for a in arrays]))
    counts = ctypes_array("c_int64", [a.numel() for a in arrays])
    dts = ctypes_array("c_int", [_dev.dtype_code(a.dtype) for a in arrays])
    flags = torch.zeros(1, dtype=torch.int32, device=q.device)
    st = _dev.new_status(q.device)
    rc = _lib.lib().nsn_finite_scan(len(arrays), ptrs, counts, dts, flags.data_ptr(), st.data_ptr(), _dev.stream())
    _lib.check(rc, "nsn_finite_scan")
    if _dev.read_status(st):
        raise NumericalFailure("VF01 nonfinite raw input")


def ctypes_array(kind, values):
    import ctypes
    t = getattr(ctypes, kind) * len(values)
    return t(*values)


def restore_v(g, tail):
    """Bridge: write the full reconstructed V [1,H,T,128] to HBM (loop_kv_vf01_kernel.py:120-126)."""
    h = tail.shape[1]
    if g is None:
        return tail.contiguous().clone()
    codes = g["codes"]
    b, gh, n, nbytes = codes.shape
    bits = nbytes * 8 // (BLOCK * DIM)
    out = codec.restore(codes.reshape(b * gh, n, nbytes), g["metas"], bits, tail.dtype, tail=tail.reshape(h, -1, DIM))
    return out.reshape(1, h, -1, DIM)


def launch(g, kt, q, vg, vt, trace=False, kernel="reference", status=None):
    """Fused packed-K/V readout (loop_kv_vf01_kernel.py:128-139; GQA: loop_kv_nb06_kernel.py:142-154).

    Returns (out [1,1,Hq,128] bf16, context [1,Hq,1,128] fp32, score, v): score
    [1,Hq,T] fp32 and v [1,Hkv,T,128] are only produced with ``trace``; the
    exact-order kernel writes them itself (its scores and the V rows it
    multiplied, loop_kv_vf01_kernel.py:104,113), for the fast kernel, which
    keeps neither, they come from an exact restore.  With ``status`` (an
    int32 device word) nothing is raised: the caller reads the NSN_ST_* bits.
    """
    Hq = q.shape[1]
    T = _length(g, kt)
    # the lengths and block counts below are built from these shapes, so the
    # consistency check needs no device round trip
    require(T > 0, "Empty sequence")
    require(_length(vg, vt) == T, "K/V lengths differ")
    fast = kernel == "fast"
    ks, vs = _fast_sides(((g, kt), (vg, vt)), fast, status, q.device)
    seq = _length_tensor(T, q.device)
    Hkv = kt.shape[1]
    tr_s = tr_v = None
    if trace and not fast:
        tr_s = torch.empty((1, Hq, T), dtype=torch.float32, device=q.device)
        tr_v = torch.empty((1, Hkv, T, DIM), dtype=torch.float32, device=q.device)
    out, ctx = decode_attention(q.reshape(1, Hq, DIM), ks, vs, seq, max_seq_len=T, kernel=kernel,
                                kv_round_dtype=kt.dtype, status=status, trace_scores=tr_s, trace_v=tr_v,
                                validate_lengths=False)
    score = vtr = None
    if trace and not fast:   # what the exact-order kernel itself computed
        score, vtr = tr_s, tr_v.to(vt.dtype)
    elif trace:   # the fast kernel keeps neither: the scores and V of an exact restore
        kk = restore_v(g, kt).float()
        vtr = restore_v(vg, vt)
        G = Hq // Hkv
        score = (torch.einsum("hd,htd->ht", q.reshape(Hq, DIM).float(), kk[0].repeat_interleave(G, 0)) * SCALE)[None]
    return out.reshape(1, 1, Hq, DIM), ctx.reshape(1, Hq, 1, DIM), score, vtr


def _fast_sides(groups, fast, status, device):
    """PackedKV sides of (group, tail) pairs; for the fast kernel with their
    decode factors, whose computation also checks the raw block metadata:
    nonfinite metadata raises NumericalFailure, or with ``status`` given sets
    NSN_ST_NONFINITE_ATTN_INPUT there."""
    st = (status if status is not None else _dev.new_status(device)) if fast else None
    sides = [_group_side(g, t, factors=fast, status=st) for g, t in groups]
    if fast and status is None and any(g is not None for g, _ in groups) \
            and _dev.read_status(st) & _lib.ST_NONFINITE_ATTN_INPUT:
        raise NumericalFailure("Nonfinite raw attention input (block metadata)")
    return sides


def af_validate(g, tail, q):
    """AF01 input checks before any launch (loop_kv_qk01_kernel.py:66-77):
    tail [1,H,T,128] bf16 and query [1,H,1,128] bf16, contiguous, on the GPU,
    a nonempty sequence, and every raw value finite (NumericalFailure).
    Returns (heads, compressed tokens, total tokens)."""
    require(tail.ndim == 4 and tail.shape[0] == 1 and tail.shape[-1] == DIM and tail.dtype == torch.bfloat16
            and tail.is_contiguous(), "Tail shape/type")
    h = tail.shape[1]
    require(h > 0 and tuple(q.shape) == (1, h, 1, DIM) and q.dtype == torch.bfloat16 and q.is_contiguous(),
            "Query shape/type")
    _dev.require_gpu(q, tail)
    compressed = 0
    if g is not None:
        b, gh, n, _ = g["codes"].shape
        require(b == 1 and gh == h and g["codes"].device == tail.device, "Packed head/device mismatch")
        compressed = n * BLOCK
    require(tail.shape[-2] + compressed > 0, "Empty sequence")
    values = [q, tail] + ([] if g is None else list(g["metas"]))
    if not bool(torch.stack([torch.isfinite(x).all() for x in values]).all()):
        raise NumericalFailure("Nonfinite QK input")
    return h, compressed, compressed + tail.shape[-2]


def validate_v(v, q, total):
    """AF01 V check (loop_kv_af01_kernel.py:88-92): bf16 [1,H,total,128],
    contiguous, on the query's GPU, finite."""
    require(v.dtype == torch.bfloat16 and v.is_contiguous() and tuple(v.shape) == (1, q.shape[1], total, DIM),
            "V shape/type")
    _dev.require_gpu(v, q)
    if not bool(torch.isfinite(v).all()):
        raise NumericalFailure("Nonfinite V")


def validate_score(score, v):
    """AF01 score check (loop_kv_af01_kernel.py:94-98): fp32 [1,H,T] logits,
    contiguous, on V's GPU, finite."""
    require(score.dtype == torch.float32 and score.is_contiguous() and tuple(score.shape) == (1, v.shape[1], v.shape[2]),
            "Score shape/type")
    _dev.require_gpu(score, v)
    if not bool(torch.isfinite(score).all()):
        raise NumericalFailure("Nonfinite score")


def af_launch(g, tail, q, v, score=None, full=False, kernel="reference"):
    """AF01 attention (loop_kv_af01_kernel.py:100-111).

    full=True: K from the packed group + tail, V given dense [1,H,T,128];
    full=False: softmax readout of the given fp32 scores [1,Hq,T] over V.
    Returns (out [1,1,Hq,128], context [1,Hq,1,128]).
    """
    Hq = q.shape[1]
    T = v.shape[2]
    require(T > 0, "Empty sequence")
    vs = PackedKV(None, None, None, None, None, None, v.contiguous(), 3)
    seq = _length_tensor(T, v.device)
    # lengths and block counts from the shapes: checked here, on the host
    if full:
        require(_length(g, tail) == T, "K/V lengths differ")
        ks, = _fast_sides(((g, tail),), kernel == "fast", None, v.device)
        out, ctx = decode_attention(q.reshape(1, Hq, DIM), ks, vs, seq, max_seq_len=T, kernel=kernel,
                                    kv_round_dtype=v.dtype, validate_lengths=False)
    else:
        require(score is not None and tuple(score.shape) == (1, Hq, T), "Score shape/type")
        out, ctx = decode_attention(q.reshape(1, Hq, DIM), None, vs, seq, max_seq_len=T, scores=score.contiguous(),
                                    kernel=kernel, kv_round_dtype=v.dtype, validate_lengths=False)
    return out.reshape(1, 1, Hq, DIM), ctx.reshape(1, Hq, 1, DIM)


# The fused arms check their raw inputs inside the attention kernel instead of
# a separate grouped scan (loop_kv_vf01_checks.py:55-63) before it.
FUSED_VALIDATION = True


def pipeline(arm, data, trace=False, kernel="reference"):
    """Checked route selection (loop_kv_vf01_kernel.py:141-158, loop_kv_nb06_kernel.py:175-191).

    Arms: 'V_FUSED' / 'GQA_FUSED' (fused), 'TILE_MATERIALIZE' (bridge: V
    restored to HBM then attention), 'RF01_MATERIALIZE' (V from restore_group
    + cat).  Stages recorded in LAST_STAGE as the reference does.  ``kernel``
    picks the attention kernel: 'reference' (exact order, restored values
    rounded to the tail dtype) or 'fast' (MFMA, within the stated tolerance).
    """
    global LAST_STAGE
    g, kt, q, vg, vt = data
    LAST_STAGE = "structural"
    structural(g, kt, q, vg, vt)
    if arm in ("V_FUSED", "GQA_FUSED") and FUSED_VALIDATION:
        # the grouped finite check (q, tails, block metadata) runs inside the
        # attention kernel: one launch, one status read; a nonfinite raw input
        # still fails at the 'input_finite' stage
        LAST_STAGE = "attention"
        st = _dev.new_status(q.device)
        out, ctx, score, v = launch(g, kt, q, vg, vt, trace=trace, status=st, kernel=kernel)
        s = _dev.read_status(st)
        if s & _lib.ST_NONFINITE_ATTN_INPUT:
            LAST_STAGE = "input_finite"
            raise NumericalFailure("VF01 nonfinite raw input")
        if s & (_lib.ST_NONFINITE_ATTN | _lib.ST_NONFINITE_RESTORE):
            raise NumericalFailure("Nonfinite fused attention intermediate/output")
        # the output check: the merge flags a nonfinite output (fp32 context
        # or its rounded value) in the same status word, so the one read
        # above covers it without a second scan and synchronisation
        LAST_STAGE = "output"
        if s & _lib.ST_NONFINITE_OUTPUT:
            raise NumericalFailure("Nonfinite VF01 output")
        LAST_STAGE = "returned"
        return (out, ctx, score, v) if trace else out
    LAST_STAGE = "input_finite"
    finite(g, kt, q, vg, vt)
    if arm in ("V_FUSED", "GQA_FUSED"):
        LAST_STAGE = "attention"
        out, ctx, score, v = launch(g, kt, q, vg, vt, trace=trace, kernel=kernel)
    elif arm in ("TILE_MATERIALIZE", "RF01_MATERIALIZE"):
        LAST_STAGE = "restore"
        if arm == "TILE_MATERIALIZE":
            v = restore_v(vg, vt)
        else:
            v = vt if vg is None else torch.cat((codec.restore_group(vg, vt.dtype), vt), dim=-2)
        require(v.dtype == vt.dtype and v.is_contiguous() and tuple(v.shape) == (1, vt.shape[1], _length(vg, vt), 128),
                "V shape/type")
        if not bool(torch.isfinite(v).all()):
            raise NumericalFailure("Nonfinite V")
        LAST_STAGE = "attention"
        out, ctx = af_launch(g, kt, q, v, full=True, kernel=kernel)
        score = None
    else:
        raise IntegrityError("Unknown VF01 arm")
    LAST_STAGE = "output"
    if not bool(torch.isfinite(out).all()):
        raise NumericalFailure("Nonfinite VF01 output")
    LAST_STAGE = "returned"
    return (out, ctx, score, v) if trace else out
