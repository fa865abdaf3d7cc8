"""Decode-time connection of the packed K/V path into a Hugging Face
transformers model (the reference's AC08 connection, rebuilt).

The reference patches the attention modules of its Ouro model so that a
single-token decode step appends K/V to its packed cache and reads them back
through a fused kernel instead of a restored dense copy
(experiments/ac08/source/loop_kv_ac08_attention.py:46-96); prefill and every
call without the packed cache keep the original forward.  Here:

- ``PackedKVCache`` is a ``transformers.Cache`` whose per-slot layers are the
  GPU-resident ``StreamingKVCache`` (preallocated packed blocks + an fp16
  tail, compressed in place by the reference's policy:
  ``post_prefill`` / ``post_decode``, loop_kv_pk01_cache.py:122-127).
  ``update`` (the native route, used by prefill) appends and returns the
  exact dense reconstruction (restore of the packed blocks + the tail,
  loop_kv_pk01_cache.py:97-110); ``append_for_attention`` appends without
  it (loop_kv_ac08_attention.py:20-24).  With ``prefill="packed"`` a
  prefill chunk instead attends the packed context directly on the MFMA
  prefill kernel (no dense K/V; the reference has no such route).
- ``install(model)`` patches every ``model.model.layers[i].self_attn`` and
  returns a function that restores the original bound methods
  (loop_kv_ac08_attention.py:46-96).  Decode arms
  (loop_kv_ac08_attention.py:73-85):

  * ``NATIVE``: dense restore of K and V, then the model's own sdpa;
  * ``PACKED_GROUPED``: packed K, V restored dense (the bridge);
  * ``PACKED_KV_FUSED``: packed K and V read by the fused MFMA kernel;
  * ``PACKED_KV_EXACT``: packed K and V read by the exact-order kernel,
    reconstructions rounded to the query dtype as the reference's
    ``read_v`` does (loop_kv_vf01_kernel.py:15-44).

Unlike the reference (batch 1, MHA, explicit all-zero mask), any batch,
GQA group and the model's attention scale are taken; sliding-window
attention, training mode and beam reordering are refused.  Slots are
``current_ut * num_hidden_layers + layer_idx`` (looped models pass
``current_ut``; others use loop 0).

For Llama-family attention (``FUSED_ROPE_CLASSES``) the packed decode step
runs its q/k/v projections as one GEMM over weights concatenated at
``install`` and its rotary embedding + fp16 casts + tail append as one
launch (``nsn_rope_append``, bit-identical to ``apply_rotary_pos_emb``).
``DecodeGraph`` captures a whole decode step as one HIP graph.
``auto_policy=True`` runs the compression policy per slot for callers that
never call ``post_prefill`` / ``post_decode`` (transformers' ``generate``).

Nothing here synchronises with the device when ``strict=False``: the
position / mask checks (host syncs in the reference) are then skipped and
nonfinite flags accumulate in the cache's status word, read by
``check_status()``.
"""
from __future__ import annotations

import sys
import types
from collections import Counter

import torch

from . import _dev, _lib, kernels, primitives
from .errors import IntegrityError, NumericalFailure, require
from .kernels import BLOCK, DIM, PackedKV
from .stream_cache import StreamingKVCache

ARMS = ("NATIVE", "PACKED_GROUPED", "PACKED_KV_FUSED", "PACKED_KV_EXACT")
# attention classes whose rotary step is transformers' standard
# apply_rotary_pos_emb over the whole head (rotate_half form, no q/k norm):
# their decode step can run it fused with the tail append (nsn_rope_append)
FUSED_ROPE_CLASSES = ("LlamaAttention", "MistralAttention", "Qwen2Attention")

try:   # transformers is optional: only the adapter needs it
    from transformers.cache_utils import Cache, CacheLayerMixin
except ImportError:   # pragma: no cover - the image ships transformers
    Cache, CacheLayerMixin = object, object


def sliding_window(config, layer_idx):
    """The attention window of layer ``layer_idx`` under ``config`` (None: full
    attention).  transformers keeps it in the config, not the module:
    ``layer_types`` entries ``"sliding_attention"``, or ``sliding_window``
    unless ``use_sliding_window`` is set false (Qwen2's default)."""
    window = getattr(config, "sliding_window", None)
    types_ = getattr(config, "layer_types", None)
    if types_ is not None and layer_idx is not None and 0 <= layer_idx < len(types_):
        return window if "sliding" in str(types_[layer_idx]) else None
    if getattr(config, "use_sliding_window", True) is False:
        return None
    return window


def _refuse_window(config, layer_idx, capacity):
    """The packed decode attends every cached token: a window shorter than what
    the cache can hold would change the result, so it is refused."""
    window = sliding_window(config, layer_idx)
    require(window is None or window >= capacity,
            f"Packed decode refuses sliding-window attention (window {window} < cache capacity {capacity})")


class _PackedLayer(CacheLayerMixin):
    """One slot of the packed cache seen through transformers' layer API."""

    is_sliding = False
    is_compileable = False

    def __init__(self, owner, slot):
        super().__init__()
        self.owner, self.slot = owner, slot
        self.is_initialized = True

    def lazy_initialization(self, key_states, value_states):
        pass

    def update(self, key_states, value_states, *args, **kwargs):
        return self.owner.update_slot(self.slot, key_states, value_states, kwargs.get("cache_kwargs") or kwargs)

    def get_mask_sizes(self, query_length):
        return self.get_seq_length() + query_length, 0

    def get_seq_length(self):
        return self.owner.store.length[self.slot]

    def get_max_length(self):
        return self.owner.max_tokens

    def reset(self):
        raise IntegrityError("Packed cache reset not supported: build a new cache")

    def reorder_cache(self, beam_idx):
        raise IntegrityError("Packed cache beam reorder not supported")


class PackedKVCache(Cache):
    """Packed K/V for every (loop, layer) slot of ``config``'s attention layers.

    batch, max_tokens: sequences and the token capacity per slot;
    max_prefill: the longest single append (the prompt) before compression.
    The packed side is ``bits``-bit NSN codes; the tail holds ``tail_dtype``
    (fp16 or bf16; every kernel reads either).  fp16, the default, keeps 3
    more mantissa bits, and bf16 activations convert to it exactly inside
    fp16's normal range; a bf16 model whose keys or values can pass 65504
    (fp16's largest finite value) takes ``tail_dtype=torch.bfloat16``, with
    which appends, the packed prefill and the fused rotary append stay in
    bf16 end to end.
    """

    nsn_connection = True

    def __init__(self, config, batch, max_tokens, *, loops=1, bits=3, arm="PACKED_KV_FUSED", max_prefill=512,
                 strict=True, prefill="native", fused_rope=True, auto_policy=False, tail_dtype=torch.float16,
                 device=None):
        require(arm in ARMS, "Unknown connection arm")
        require(tail_dtype in (torch.float16, torch.bfloat16), "Tail dtype (fp16 or bf16)")
        require(prefill in ("native", "packed") and (prefill == "native" or arm != "NATIVE"), "Prefill route")
        heads_q = config.num_attention_heads
        heads = getattr(config, "num_key_value_heads", None) or heads_q
        head_dim = getattr(config, "head_dim", None) or config.hidden_size // heads_q
        require(head_dim == DIM, "Packed cache needs head_dim 128")
        require(heads_q % heads == 0, "GQA group")
        self.n_layers, self.loops = config.num_hidden_layers, loops
        self.heads_q, self.heads = heads_q, heads
        self.batch, self.max_tokens, self.arm, self.strict = batch, max_tokens, arm, strict
        self.prefill = prefill
        self.fused_rope = fused_rope
        # auto_policy: each slot runs the compression policy its previous
        # append left pending (prefill or decode target) right before its
        # next append -- the state post_prefill / post_decode would have
        # left, for callers that never call them (transformers' generate)
        self.auto_policy = auto_policy
        self._pending = [None] * (self.n_layers * loops)
        # refused here, before any append changes the cache
        for i in range(self.n_layers):
            _refuse_window(config, i, max_tokens)
        self.config = config
        self.tail_dtype = tail_dtype
        self.store = StreamingKVCache(self.n_layers * loops, batch, heads, max_tokens, bits=bits,
                                      dtype=tail_dtype, max_append=max(max_prefill, 1),
                                      device=device or torch.device("cuda:0"))
        super().__init__(layers=[_PackedLayer(self, s) for s in range(self.n_layers * loops)])
        self.status = _dev.new_status(self.store.device)   # attention flags (strict=False)
        self.connection_calls = Counter()
        self.capture = None
        self._ws = None
        # device-position mode (DecodeGraph): int32 [B sequence lengths | tail end],
        # shared by every slot (the policy keeps all slots at one length)
        self.graph_mode = False
        self.counters = torch.zeros(batch + 1, dtype=torch.int32, device=self.store.device)
        self.cap_len = self.store.block_cap * BLOCK + self.store.tail_cap

    # ------------------------------------------------------------------ lengths
    def get_seq_length(self, layer_idx=0):
        i = 0 if layer_idx is None else layer_idx
        return self.store.length[i] if 0 <= i < self.store.slots else 0

    def slot(self, layer_idx, current_ut=0):
        s = current_ut * self.n_layers + layer_idx
        require(0 <= layer_idx < self.n_layers and 0 <= s < self.store.slots, "Packed KV coordinates")
        return s

    # ------------------------------------------------------------------ appends
    def _policy(self, slot, n):
        """auto_policy: run the slot's pending policy, then note the one this
        append of n tokens leaves."""
        if not self.auto_policy:
            return
        from .stream_cache import decode_target, prefill_target
        st, kind = self.store, self._pending[slot]
        if kind == "prefill":
            st.compress_to(slot, max(st.compressed[slot], prefill_target(st.length[slot])))
        elif kind == "decode":
            st.compress_to(slot, decode_target(st.length[slot], st.compressed[slot]))
        self._pending[slot] = "prefill" if n > 1 else "decode"

    def _append(self, slot, key, value):
        require(key.shape == value.shape and key.ndim == 4 and tuple(key.shape[:2]) == (self.batch, self.heads)
                and key.shape[3] == DIM, "Packed KV coordinates")
        self._policy(slot, key.shape[2])
        # another 16-bit dtype converts inside the append kernel
        self.store.append(slot, key.contiguous(), value.contiguous())

    def _check_position(self, slot, n, kwargs):
        pos = kwargs.get("cache_position")
        if pos is None:
            pos = kwargs.get("position_ids")
        if pos is not None and self.strict:
            old = self.store.length[slot]
            want = torch.arange(old, old + n, device=pos.device)
            require(bool(torch.equal(pos.reshape(-1, n)[0].to(want.dtype), want)), "Packed append position")

    def update_slot(self, slot, key, value, kwargs=None):
        """The native route: append, then the dense K/V of the whole slot in
        the key's dtype (loop_kv_pk01_cache.py:97-110)."""
        self._check_position(slot, key.shape[2], kwargs or {})
        self._append(slot, key, value)
        return self.materialize(slot, "K", key.dtype), self.materialize(slot, "V", key.dtype)

    def prefill_slot(self, slot, q, key, value, scale, kwargs=None):
        """The packed prefill route: the chunk's queries attend the slot's
        packed blocks + tail and the chunk's own K/V causally on the MFMA
        prefill kernel (no dense K/V), then the chunk is appended.  Returns
        [B, Hq, n, 128] in q's dtype.  The caller compresses between chunks
        (post_prefill) so that every chunk fits the tail."""
        self._check_position(slot, key.shape[2], kwargs or {})
        require(key.shape == value.shape and key.ndim == 4 and tuple(key.shape[:2]) == (self.batch, self.heads)
                and key.shape[3] == DIM, "Packed KV coordinates")
        dt = self.tail_dtype
        q16 = q.to(dt).contiguous()
        k16, v16 = key.to(dt).contiguous(), value.to(dt).contiguous()
        self._policy(slot, key.shape[2])
        # the chunk's append to the tail happens inside the prefill launch
        out = self.store.prefill(slot, q16, k16, v16, append=True, scale=scale, check=self.strict,
                                 status=None if self.strict else self.status)
        return out.to(q.dtype)

    def rope_append(self, slot, q, key, value, cos, sin, kwargs=None):
        """The decode step's rotary embedding and tail append in one launch
        (nsn_rope_append): q [B, 1, Hq*128], key / value [B, 1, Hkv*128] (the
        projection outputs, model dtype; each row contiguous, rows of
        sequences at any stride -- slices of one fused QKV output), cos / sin
        [B or 1, 1, 128].  Returns
        the rotated q [B, Hq, 128]; the rotated key and the value go to the
        tail in the tail dtype -- at the device tail end in device-position
        mode, else at the host tail length (then counted)."""
        B, st = self.batch, self.store
        dt = q.dtype
        require(dt in (torch.bfloat16, torch.float16) and all(t.dtype == dt for t in (key, value, cos, sin)),
                "Rotary dtypes")
        require(tuple(q.shape) == (B, 1, self.heads_q * DIM) and tuple(key.shape) == (B, 1, self.heads * DIM)
                and key.shape == value.shape and all(t.stride(2) == 1 for t in (q, key, value))
                and key.stride(0) == value.stride(0) and cos.is_contiguous() and sin.is_contiguous(),
                "Decode projections")
        require(cos.shape == sin.shape and cos.shape[-1] == DIM and cos.numel() in (DIM, B * DIM), "Rotary rows")
        cs_stride = 0 if cos.numel() == DIM else DIM
        kt, vt = st.side(slot, "K").tail, st.side(slot, "V").tail
        q_out = torch.empty((B, self.heads_q, DIM), dtype=dt, device=q.device)
        if self.graph_mode:
            tail_end, offset = self.counters.data_ptr() + 4 * B, 0
        else:
            self._check_position(slot, 1, kwargs or {})
            self._policy(slot, 1)
            offset = st.tail_len(slot)
            require(offset + 1 <= st.tail_cap and st.length[slot] + 1 <= self.cap_len,
                    "Tail overflow: compress before appending more tokens")
            tail_end = None
        rc = _lib.lib().nsn_rope_append(q.data_ptr(), key.data_ptr(), value.data_ptr(), q.stride(0), key.stride(0),
                                        cos.data_ptr(), sin.data_ptr(), cs_stride, B, self.heads_q, self.heads, q_out.data_ptr(), kt.data_ptr(),
                                        vt.data_ptr(), st.tail_cap, tail_end, offset, _dev.dtype_code(dt),
                                        _dev.dtype_code(self.tail_dtype), self.status.data_ptr(), _dev.stream())
        _lib.check(rc, "nsn_rope_append")
        if not self.graph_mode:
            st.advance(slot)
        return q_out

    def append_for_attention(self, slot, key, value, kwargs=None):
        """Append the step's K/V without the dense restore (loop_kv_ac08_attention.py:20-24).
        In device-position mode the tokens go to [tail_end - n, tail_end) with
        tail_end read from ``counters`` on the device, and the host lengths
        are left to the caller (DecodeGraph)."""
        if not self.graph_mode:
            self._check_position(slot, key.shape[2], kwargs or {})
            self._append(slot, key, value)
            return
        require(key.shape == value.shape and key.ndim == 4 and tuple(key.shape[:2]) == (self.batch, self.heads)
                and key.shape[3] == DIM, "Packed KV coordinates")
        k16, v16 = key.to(self.tail_dtype).contiguous(), value.to(self.tail_dtype).contiguous()
        kt, vt = self.store.side(slot, "K").tail, self.store.side(slot, "V").tail
        n = key.shape[2]
        rc = _lib.lib().nsn_tail_append_to(k16.data_ptr(), v16.data_ptr(), self.batch * self.heads, n, n,
                                           kt.data_ptr(), vt.data_ptr(), self.store.tail_cap,
                                           self.counters.data_ptr() + 4 * self.batch, _dev.dtype_code(self.tail_dtype),
                                           self.status.data_ptr(), _dev.stream())
        _lib.check(rc, "nsn_tail_append_to")

    def materialize(self, slot, name, dtype):
        """Dense [B, H, L, 128] of one side: packed blocks restored exactly
        (nsn_decode, rounded to ``dtype``) followed by the tail."""
        kv = self.store.side(slot, name)
        L, C = self.store.length[slot], self.store.compressed[slot]
        out = torch.empty((self.batch, self.heads, L, DIM), dtype=dtype, device=self.store.device)
        st = _dev.new_status(self.store.device) if self.strict else self.status
        rc = _lib.lib().nsn_restore_blocks(
            kv.codes.data_ptr(), 0, kv.norm.data_ptr(), kv.min.data_ptr(), kv.scale.data_ptr(),
            self.batch * self.heads, C // BLOCK, self.store.block_cap, kv.bits, out.data_ptr(),
            _dev.dtype_code(dtype), L, kv.tail.data_ptr(), _dev.dtype_code(kv.tail.dtype), L - C,
            self.store.tail_cap, st.data_ptr(), _dev.stream())
        _lib.check(rc, "nsn_restore_blocks")
        if self.strict:
            primitives._restore_raise(_dev.read_status(st))
        return out

    # ------------------------------------------------------------------ policy
    def post_prefill(self):
        self.store.post_prefill()

    def post_decode(self):
        self.store.post_decode()

    def check_status(self):
        """Raise on any flag raised since the cache was built (syncs)."""
        self.store.check_status()
        s = _dev.read_status(self.status)
        if s & _lib.ST_TAIL_RANGE:
            raise IntegrityError("Tail append position out of range")
        if s & _lib.ST_CAPACITY:
            raise IntegrityError("Sequence length past the cache's block / tail capacity")
        if s & _lib.ST_EMPTY:
            raise IntegrityError("A sequence attended no token (zero length)")
        if s & _lib.ST_NONFINITE_ATTN_INPUT:
            raise NumericalFailure("Nonfinite raw attention input (q, tail or block metadata)")
        if s:
            raise NumericalFailure("Nonfinite attention intermediate/output")

    # ------------------------------------------------------------------ attention
    def attend(self, slot, q, scale):
        """Decode attention of q [B, Hq, 128] over the slot by the cache's arm
        (not NATIVE); returns the bf16 output [B, Hq, 128]."""
        L = self.store.length[slot]
        kside, vside = self.store.side(slot, "K"), self.store.side(slot, "V")
        seq = self.store.lengths(slot)
        if self.graph_mode:
            # lengths from the device counters, the capacity as the bound: no
            # launch argument changes from step to step
            require(self.arm == "PACKED_KV_FUSED" and not self.strict, "Device positions: fused arm, strict=False")
            L, seq = self.cap_len, self.counters[:self.batch]
        kw = dict(max_seq_len=L, scale=scale, check=self.strict, status=None if self.strict else self.status)
        if self.arm == "PACKED_GROUPED":
            vd = PackedKV(None, None, None, None, None, None, self.materialize(slot, "V", self.tail_dtype), kside.bits)
            kw.update(kernel="fast", workspace=self._workspace(L))
            out, _ = kernels.decode_attention(q, kside, vd, seq, **kw)
        elif self.arm == "PACKED_KV_FUSED":
            kw.update(kernel="fast", workspace=self._workspace(L))
            out, _ = kernels.decode_attention(q, kside, vside, seq, **kw)
        else:
            kw.update(kernel="reference", kv_round_dtype=q.dtype)
            out, _ = kernels.decode_attention(q, kside, vside, seq, **kw)
        return out

    def _workspace(self, L):
        _, n = kernels.default_split(self.batch, self.heads, L)
        need = kernels.workspace_floats(self.batch, self.heads_q, max(2, n))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(max(need, 2 * (0 if self._ws is None else self._ws.numel())),
                                   dtype=torch.float32, device=self.store.device)
        return self._ws


def check_decode(module, q, cache, slot, position, mask):
    """Preconditions of the packed decode route (loop_kv_ac08_attention.py:26-33):
    eval mode, no sliding window, q [B, Hq, 1, 128] bf16/fp16 (fp32 too on
    the NATIVE arm, which is dense sdpa), and (strict
    mode) the step's position equal to the last cached token and the mask
    allowing every cached token.  Returns the slot's length."""
    total = cache.store.length[slot]
    require(not module.training and getattr(module, "sliding_window", None) is None,
            "Packed decode requires eval and no sliding window")
    config = getattr(module, "config", None)
    if config is not None:
        _refuse_window(config, getattr(module, "layer_idx", None), getattr(cache, "max_tokens", 0))
    dtypes = (torch.bfloat16, torch.float16) + ((torch.float32,) if cache.arm == "NATIVE" else ())
    require(q.ndim == 4 and tuple(q.shape) == (cache.batch, cache.heads_q, 1, DIM) and q.dtype in dtypes,
            "Decode query shape/dtype")
    if cache.strict:
        if position is not None:
            require(position.numel() >= 1 and int(position.reshape(-1)[-1].item()) == total - 1,
                    "Decode must append at current last position")
        if mask is not None:
            require(mask.shape[-1] == total, "Decode mask length")
            m = mask[..., -1:, :]
            allowed = bool(m.all()) if m.dtype == torch.bool else bool((m == 0).all())
            require(allowed, "Packed decode requires an all-allowed decode mask")
    return total


def _require_causal(mask, n, past):
    """A prefill mask (if any) must be the plain causal one over past + n
    tokens: chunk query i sees tokens 0 .. past + i (synchronises)."""
    if mask is None:
        return
    require(mask.ndim == 4 and tuple(mask.shape[-2:]) == (n, past + n), "Prefill mask shape")
    i = torch.arange(n, device=mask.device)[:, None]
    j = torch.arange(past + n, device=mask.device)[None, :]
    want = j <= past + i
    allowed = mask if mask.dtype == torch.bool else mask == 0
    require(bool((allowed == want).all()), "Packed prefill requires a plain causal mask (no padding)")


def _modeling(attn):
    return sys.modules[type(attn).__module__]


def _qkv_sources(attn):
    ps = [attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight, attn.q_proj.bias, attn.k_proj.bias,
          attn.v_proj.bias]
    return tuple(None if t is None else (t.data_ptr(), t._version, t.dtype, t.device) for t in ps)


def _fused_qkv(attn):
    """The decode step's q, k and v projections as one GEMM: the three weights
    (and biases) concatenated, rebuilt whenever a source weight was replaced,
    moved, cast or written in place since the last build (restore() drops it)."""
    key = _qkv_sources(attn)
    cached = getattr(attn, "_nsn_qkv", None)
    if cached is None or getattr(attn, "_nsn_qkv_key", None) != key:
        with torch.no_grad():
            ws = [attn.q_proj.weight, attn.k_proj.weight, attn.v_proj.weight]
            bs = [attn.q_proj.bias, attn.k_proj.bias, attn.v_proj.bias]
            cached = (torch.cat(ws, 0).contiguous(), None if bs[0] is None else torch.cat(bs, 0).contiguous(),
                      ws[0].shape[0], ws[1].shape[0])
        attn._nsn_qkv, attn._nsn_qkv_key = cached, key
    return cached


def install(model, module=None):
    """Patch the attention of every decoder layer (instances only) and return
    ``restore()``, which puts every original bound method back
    (loop_kv_ac08_attention.py:46-96).  ``module`` is the model's modeling
    module (for ``apply_rotary_pos_emb``); by default the attention class's own."""
    changed = []
    for layer in model.model.layers:
        attn = layer.self_attn
        original = attn.forward
        mod = module if module is not None else _modeling(attn)

        def forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                    current_ut=0, _original=original, _mod=mod, **kwargs):
            cache = past_key_values
            if not getattr(cache, "nsn_connection", False):
                return _original(hidden_states, position_embeddings, attention_mask, past_key_values=past_key_values,
                                 **kwargs)
            input_shape = hidden_states.shape[:-1]
            hidden_shape = (*input_shape, -1, self.head_dim)
            slot = cache.slot(self.layer_idx, current_ut)
            if (hidden_states.shape[1] == 1 and cache.arm != "NATIVE" and cache.fused_rope
                    and type(self).__name__ in FUSED_ROPE_CLASSES):
                # decode step, fused: rotary + append in one launch, then the packed attention
                cos, sin = position_embeddings
                w, bias, nq, nk = _fused_qkv(self)
                qkv = torch.nn.functional.linear(hidden_states, w, bias)       # one GEMM for q, k and v
                q3 = cache.rope_append(slot, qkv[..., :nq], qkv[..., nq:nq + nk], qkv[..., nq + nk:], cos, sin,
                                       kwargs)
                total = check_decode(self, q3.unsqueeze(2), cache, slot, kwargs.get("position_ids"), attention_mask)
                out = cache.attend(slot, q3, self.scaling).to(q3.dtype).unsqueeze(1)   # [B, 1, Hq, 128]
                if not cache.graph_mode:
                    cache.connection_calls[slot] += 1
                if cache.capture is not None:
                    require(not cache.graph_mode, "No capture hook under device positions")
                    cache.capture(slot, total, q3, out[:, 0])
                return self.o_proj(out.reshape(*input_shape, -1)), None
            q = self.q_proj(hidden_states).view(hidden_shape)
            k = self.k_proj(hidden_states).view(hidden_shape)
            if hasattr(self, "q_norm"):
                q, k = self.q_norm(q), self.k_norm(k)
            q, k = q.transpose(1, 2), k.transpose(1, 2)
            v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
            cos, sin = position_embeddings
            q, k = _mod.apply_rotary_pos_emb(q, k, cos, sin)
            if hidden_states.shape[1] != 1 and cache.prefill == "packed":
                # prefill over the packed context on the MFMA prefill kernel,
                # which applies the causal mask itself (no padding)
                if cache.strict:
                    _require_causal(attention_mask, hidden_states.shape[1], cache.store.length[slot])
                out = cache.prefill_slot(slot, q, k, v, self.scaling, kwargs).transpose(1, 2)
            elif hidden_states.shape[1] != 1:
                # prefill: the native route over the slot's dense K/V
                kd, vd = cache.update_slot(slot, k, v, kwargs)
                fn = _mod.ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation,
                                                                _mod.eager_attention_forward)
                out, _ = fn(self, q, kd, vd, attention_mask, dropout=0.0, scaling=self.scaling, **kwargs)
            else:
                cache.append_for_attention(slot, k, v, kwargs)
                q = q.contiguous()
                total = check_decode(self, q, cache, slot, kwargs.get("position_ids"), attention_mask)
                if cache.arm == "NATIVE":
                    kd = cache.materialize(slot, "K", q.dtype)
                    vd = cache.materialize(slot, "V", q.dtype)
                    fn = _mod.ALL_ATTENTION_FUNCTIONS["sdpa"]
                    out, _ = fn(self, q, kd, vd, attention_mask, dropout=0.0, scaling=self.scaling, **kwargs)
                    if cache.strict and not bool(torch.isfinite(out).all()):
                        raise NumericalFailure("Nonfinite attention output")
                else:
                    o = cache.attend(slot, q[:, :, 0], self.scaling)           # [B, Hq, 128] bf16
                    out = o.to(q.dtype).unsqueeze(1)                          # [B, 1, Hq, 128]
                if not cache.graph_mode:
                    cache.connection_calls[slot] += 1
                if cache.capture is not None:
                    require(not cache.graph_mode, "No capture hook under device positions")
                    cache.capture(slot, total, q[:, :, 0], out[:, 0])
            out = out.reshape(*input_shape, -1).contiguous()
            return self.o_proj(out), None

        changed.append((attn, original))
        attn.forward = types.MethodType(forward, attn)
        if type(attn).__name__ in FUSED_ROPE_CLASSES:
            _fused_qkv(attn)

    def restore():
        for a, orig in changed:
            a.forward = orig
            for name in ("_nsn_qkv", "_nsn_qkv_key"):
                if hasattr(a, name):
                    delattr(a, name)
    return restore


class DecodeGraph:
    """One decode step of ``model`` through ``cache`` (fused arm, strict=False)
    captured as a HIP graph and replayed per step.  A looped model (cache
    ``loops`` > 1) passes ``current_ut`` to its attention itself; every slot
    shares the device counters.

    Every launch argument of the step is fixed: the token and position ids
    sit in static buffers, the tail append and the attention read the
    sequence lengths and the tail end from ``cache.counters`` (advanced by
    one device op at the start of the step), and the attention's length
    bound is the cache capacity.  Between replays the host advances its own
    lengths, runs the compression policy eagerly and, after a compression,
    reloads the counters.  The first call runs the step once eagerly on a
    side stream (library warm-up; its tail writes are the ones the real step
    repeats), rewinds the counters, captures, then replays.  With
    ``use_graph=False`` the same step runs eagerly each call (the reference
    the replays are tested against).  Not a counterpart of anything in the
    reference, whose decode step is eager Python (loop_kv_ac08_attention.py:46-96).
    """

    def __init__(self, model, cache, use_graph=True):
        require(cache.arm == "PACKED_KV_FUSED" and not cache.strict and cache.capture is None
                and not cache.auto_policy, "Decode graph: fused arm, strict=False, no capture hook, no auto_policy "
                "(the graph runs post_decode itself; call post_prefill before the first step)")
        self.model, self.cache, self.use_graph = model, cache, use_graph
        dev = cache.store.device
        self.ids = torch.zeros((cache.batch, 1), dtype=torch.long, device=dev)
        self.pos = torch.zeros((cache.batch, 1), dtype=torch.long, device=dev)
        self.graph = None
        self.logits = None
        self.replays = 0
        cache._workspace(cache.cap_len)
        self._reload = True
        self._failed = None   # set when the policy after a step raised: no further steps

    def _load_counters(self):
        st, B = self.cache.store, self.cache.batch
        L, C = st.length[0], st.compressed[0]
        require(all(x == L for x in st.length) and all(c == C for c in st.compressed), "Slots at one length")
        require(L - C + 1 <= st.tail_cap and L + 1 <= self.cache.cap_len, "Cache capacity exceeded")
        self.cache.counters[:B].fill_(L)
        self.cache.counters[B:].fill_(L - C)
        self.pos.fill_(L - 1)

    def _body(self):
        self.cache.counters.add_(1)
        self.pos.add_(1)
        out = self.model(input_ids=self.ids, position_ids=self.pos, past_key_values=self.cache, use_cache=True,
                         logits_to_keep=1)
        return out.logits

    def step(self, tokens):
        """Decode ``tokens`` [B, 1] (int64, on the device).  Returns the logits
        [B, 1, vocab]; under replay this is the graph's static output buffer,
        overwritten by the next step."""
        st = self.cache.store
        if self._failed is not None:
            raise IntegrityError(f"Decode graph stopped: {self._failed}")
        self.ids.copy_(tokens)
        if self._reload:
            self._load_counters()
            self._reload = False
        self.cache.graph_mode = True
        try:
            with torch.no_grad():
                if not self.use_graph:
                    logits = self._body()
                else:
                    if self.graph is None:
                        side = torch.cuda.Stream()
                        side.wait_stream(torch.cuda.current_stream())
                        with torch.cuda.stream(side):
                            self._body()
                        torch.cuda.current_stream().wait_stream(side)
                        self._load_counters()
                        self.graph = torch.cuda.CUDAGraph()
                        with torch.cuda.graph(self.graph):
                            self.logits = self._body()
                    self.graph.replay()
                    self.replays += 1
                    logits = self.logits
        finally:
            self.cache.graph_mode = False
        for s in range(st.slots):
            st.advance(s)
            self.cache.connection_calls[s] += 1
        before = st.compressed[0]
        try:
            self.cache.post_decode()
        except Exception as e:
            # the device counters have already advanced past what the host
            # tracks: refuse further replays rather than read past the cache
            self._failed = str(e)
            raise
        if st.length[0] + 1 > self.cache.cap_len or st.length[0] - st.compressed[0] + 1 > st.tail_cap:
            self._failed = "Cache capacity exceeded"   # the next step would append past it
        if st.compressed[0] != before:
            self._reload = True
        return logits


def greedy(model, cache, input_ids, steps):
    """Prefill ``input_ids`` [B, P], then ``steps`` greedy decode steps through
    ``cache``, running the compression policy after each forward.  Returns
    (tokens [B, steps], logits [steps, B, vocab] fp32)."""
    toks, logits = [], []
    with torch.no_grad():
        out = model(input_ids=input_ids, past_key_values=cache, use_cache=True)
        cache.post_prefill()
        for _ in range(steps):
            lg = out.logits[:, -1].float()
            nxt = lg.argmax(-1, keepdim=True)
            toks.append(nxt)
            logits.append(lg)
            out = model(input_ids=nxt, past_key_values=cache, use_cache=True)
            cache.post_decode()
    return torch.cat(toks, 1), torch.stack(logits)
