"""K-score decode over the K1c cache layout: the reference's fused
dequant-then-score component (the K side of one decode query), on the GPU.

Mirrors ``experiments/kernels/phase_k1c_triton_fused_kernel.py``:

- ``kivi_store`` / ``nsn_store`` (:87-111): per-channel quantisation over all
  tokens of a sequence (KIVI on K itself, NSN on its unit directions with a
  per-token ``eff_norm``), restated in torch on any device;
- ``make_store`` (:160-182): the kernel's store -- u8 codes ``[B, T, Hkv*D]``,
  fp16 ``min`` / ``step`` ``[B, Hkv*D]``, fp16 ``eff_norm`` ``[B, Hkv, T]``;
- ``decode_scores`` (:252-281, ``triton_decode_scores``): fp32 scores
  ``[B, Hq, T]`` from one HIP launch (``nsn_kscore``);
- ``pack_store``: the same codes bit-packed LSB-first along each token row
  (the refinement the reference names but does not build, :20-23).

Scores are the reference's ``score = eff_norm * sum_d q * (code * step + min)
/ sqrt(D)`` up to fp32 rounding (checked against the fp64 oracle).
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import _dev, _lib, primitives
from .errors import require

EPS = 1e-12          # clamp of norms and steps (phase_k1c:55)
RENORM_EPS = 1e-8    # clamp of the dequantised direction's norm (:56)


def _codes_over_tokens(x, bits):
    """Per-channel min / step over the token axis (dim 1) and round-half-even
    codes, in x's dtype (phase_k1c:62-68)."""
    levels = (1 << bits) - 1
    lo = x.amin(dim=1, keepdim=True)
    hi = x.amax(dim=1, keepdim=True)
    step = ((hi - lo).float() / levels).clamp(min=EPS).to(x.dtype)
    code = ((x - lo).float() / step.float()).round().clamp(0, levels).to(x.dtype)
    return code, lo, step


def kivi_store(k, bits):
    """KIVI K store: codes, min, step over the tokens of k [B, T, hidden] (phase_k1c:87-89)."""
    code, lo, step = _codes_over_tokens(k, bits)
    return {"code": code, "min": lo, "step": step}


def nsn_store(k, bits, n_kv, head_dim):
    """NSN K store (phase_k1c:92-103): unit directions per (token, kv-head)
    quantised over tokens; eff_norm = norm / |dequantised direction|."""
    B, T, hidden = k.shape
    x = k.reshape(B, T, n_kv, head_dim).float()
    norm = x.norm(dim=-1, keepdim=True).clamp(min=EPS)
    d = x / norm
    code, lo, step = _codes_over_tokens(d, bits)
    dq = code * step + lo
    eff = norm / dq.norm(dim=-1, keepdim=True).clamp(min=RENORM_EPS)
    return {"code": code.reshape(B, T, hidden), "min": lo.reshape(B, 1, hidden),
            "step": step.reshape(B, 1, hidden), "eff_norm": eff.reshape(B, T, n_kv),
            "n_kv": n_kv, "head_dim": head_dim}


def store_from_reference(ref_store, recipe, n_kv, head_dim, T, device=None):
    """The kernel's store from a materialised reference store (phase_k1c:166-181):
    u8 codes, min / step [B, hidden], eff_norm transposed to [B, n_kv, T]."""
    if recipe == "fp16":
        k = ref_store["kfp16"]
        return {"code": k.to(device).to(torch.float16).contiguous(), "is_fp16": True, "is_nsn": False,
                "T": T, "n_kv": n_kv, "head_dim": head_dim}
    code = ref_store["code"].round().clamp(0, 255).to(torch.uint8)
    st = {"code": code.to(device).contiguous(), "is_fp16": False, "is_nsn": recipe == "nsn",
          "min": ref_store["min"].squeeze(1).to(device, torch.float16).contiguous(),
          "step": ref_store["step"].squeeze(1).to(device, torch.float16).contiguous(),
          "T": T, "n_kv": n_kv, "head_dim": head_dim}
    if recipe == "nsn":
        st["eff_norm"] = ref_store["eff_norm"].transpose(1, 2).to(device, torch.float16).contiguous()
    return st


def make_store(k, bits, recipe, n_kv, head_dim, device):
    """Reference store (fp16, as the reference keeps it) and the kernel's store
    for K [B, T, hidden] (any device; the quantisation runs where k is)."""
    require(recipe in ("nsn", "kivi", "fp16"), "recipe must be nsn, kivi or fp16")
    T = k.shape[1]
    if recipe == "fp16":
        ref = {"kfp16": k.to(torch.float16), "n_kv": n_kv, "head_dim": head_dim}
    elif recipe == "kivi":
        ref = {kk: v.to(torch.float16) for kk, v in kivi_store(k, bits).items()}
    else:
        ref = {kk: (v.to(torch.float16) if torch.is_tensor(v) else v)
               for kk, v in nsn_store(k, bits, n_kv, head_dim).items()}
    return ref, store_from_reference(ref, recipe, n_kv, head_dim, T, device)


def pack_store(tstore, bits):
    """The store with its u8 codes bit-packed LSB-first along each token row
    ([B, T, hidden*bits/8]); every other field shared."""
    require(not tstore["is_fp16"], "fp16 stores have no codes to pack")
    code = tstore["code"]
    B, T, hidden = code.shape
    require(hidden * bits % 32 == 0, "token rows must pack to whole dwords")
    packed = primitives.pack_codes(code.reshape(-1), bits).reshape(B, T, hidden * bits // 8)
    out = dict(tstore)
    out["code"] = packed
    out["bits"] = bits
    return out


def decode_scores(q, tstore, n_q, n_kv, head_dim, out=None):
    """fp32 scores [B, n_q, T] of fp16 queries q [B, n_q, head_dim] over the
    store (phase_k1c:252-281): one kernel launch, no materialised K."""
    _dev.require_gpu(q, tstore["code"])
    B = q.shape[0]
    T = tstore["T"]
    require(q.dtype == torch.float16 and q.is_contiguous() and tuple(q.shape) == (B, n_q, head_dim),
            "q must be contiguous fp16 [B, n_q, head_dim]")
    require(n_q % n_kv == 0 and 1 <= n_q // n_kv <= 8, "GQA group must be 1..8")
    require(head_dim in (128, 256), "head_dim must be 128 or 256")
    code = tstore["code"]
    if tstore["is_fp16"]:
        mode, bits = _lib.KS_FP16, 16
        require(code.dtype == torch.float16 and tuple(code.shape) == (B, T, n_kv * head_dim), "fp16 K shape")
    elif "bits" in tstore:
        mode, bits = _lib.KS_PACKED, tstore["bits"]
        require(code.dtype == torch.uint8 and tuple(code.shape) == (B, T, n_kv * head_dim * bits // 8),
                "packed code shape")
    else:
        mode, bits = _lib.KS_U8, 8
        require(code.dtype == torch.uint8 and tuple(code.shape) == (B, T, n_kv * head_dim), "u8 code shape")
    require(code.is_contiguous(), "codes must be contiguous")
    mins = steps = en = None
    if mode != _lib.KS_FP16:
        mins, steps = tstore["min"], tstore["step"]
        for t in (mins, steps):
            require(t.dtype == torch.float16 and t.is_contiguous() and tuple(t.shape) == (B, n_kv * head_dim),
                    "min / step must be contiguous fp16 [B, hidden]")
        if tstore["is_nsn"]:
            en = tstore["eff_norm"]
            require(en.dtype == torch.float16 and en.is_contiguous() and tuple(en.shape) == (B, n_kv, T),
                    "eff_norm must be contiguous fp16 [B, n_kv, T]")
    if out is None:
        out = torch.empty((B, n_q, T), dtype=torch.float32, device=q.device)
    require(out.dtype == torch.float32 and out.is_contiguous() and tuple(out.shape) == (B, n_q, T), "out shape")
    a = _lib.KScoreArgs(q.data_ptr(), B, n_q, n_kv, head_dim, T, mode, bits, code.data_ptr(), _dev.ptr(mins),
                        _dev.ptr(steps), _dev.ptr(en), 1.0 / math.sqrt(head_dim), out.data_ptr())
    _lib.check(_lib.lib().nsn_kscore(ctypes.byref(a), _dev.stream()), "nsn_kscore")
    return out


def bytes_per_token_K(bits, n_kv, head_dim, T, is_nsn):
    """The reference's packed-size accounting per token of K (phase_k1c:120-129):
    bits + 32/T (min, step) + 16/head_dim (eff_norm, NSN) bits per value."""
    bpv = bits + 32.0 / T + (16.0 / head_dim if is_nsn else 0.0)
    return bpv * n_kv * head_dim / 8.0
