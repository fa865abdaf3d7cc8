"""ctypes binding of libnsn_hip.so (declared in include/nsn_hip.h).

There is no CPU fallback: if the library is missing or no GPU is visible, the
ops raise.  The library is built in-tree by ``python -m nsn_amd.build`` (or
``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_build" / "libnsn_hip.so"

# dtype / mode enums (include/nsn_hip.h)
DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2
NORM_LANES8, NORM_SEQUENTIAL = 0, 1
KV_PACKED, KV_SCORES = 0, 1
ATTN_REFERENCE, ATTN_FAST = 0, 1

ST_NONFINITE_INPUT = 0x01
ST_META_NONFINITE = 0x02
ST_META_UNDERFLOW = 0x04
ST_CODE_RANGE = 0x08
ST_NONFINITE_RESTORE = 0x10
ST_NONFINITE_ATTN = 0x20
ST_NONFINITE_OUTPUT = 0x40
ST_NONFINITE_SCAN = 0x80
ST_NONFINITE_ATTN_INPUT = 0x100
ST_TAIL_RANGE = 0x200
ST_WORKSPACE = 0x400
ST_CAPACITY = 0x800
ST_EMPTY = 0x1000

NSN_OK, NSN_EINVAL, NSN_ELAUNCH, NSN_ENOSPC = 0, -1, -2, -3
STATIC_SCRATCH_FLOATS = 4 * 1024 * 1024   # NSN_STATIC_SCRATCH_FLOATS

P = ctypes.c_void_p
I32 = ctypes.c_int
I64 = ctypes.c_int64


class KVSide(ctypes.Structure):
    _fields_ = [("codes", P), ("norms", P), ("mins", P), ("scales", P), ("factors", P), ("blocks", P),
                ("block_cap", I64), ("tail", P), ("tail_dtype", I32), ("tail_cap", I64)]


class AttnArgs(ctypes.Structure):
    _fields_ = [("q", P), ("q_dtype", I32), ("batch", I64), ("heads_q", I64), ("heads_kv", I64),
                ("scale", ctypes.c_float), ("seq_len", P), ("max_seq_len", I32), ("bits", I32),
                ("k_mode", I32), ("k", KVSide), ("v", KVSide), ("scores", P), ("scores_cap", I64),
                ("kernel", I32), ("kv_round_dtype", I32), ("split_tokens", I32), ("n_splits", I32),
                ("partials", P), ("ctx", P), ("out", P), ("out_dtype", I32), ("status", P),
                ("merge", I32), ("trace_scores", P), ("trace_v", P), ("trace_cap", I64)]


class PrefillArgs(ctypes.Structure):
    _fields_ = [("q", P), ("dtype", I32), ("batch", I64), ("heads_q", I64), ("heads_kv", I64), ("n_q", I64),
                ("scale", ctypes.c_float), ("ctx_len", P), ("bits", I32), ("k", KVSide), ("v", KVSide),
                ("k_chunk", P), ("v_chunk", P), ("out", P), ("status", P), ("append", I32),
                ("precise_weights", I32)]


class KScoreArgs(ctypes.Structure):
    _fields_ = [("q", P), ("batch", I64), ("heads_q", I64), ("heads_kv", I64), ("head_dim", I64), ("T", I64),
                ("mode", I32), ("bits", I32), ("codes", P), ("mins", P), ("steps", P), ("eff_norm", P),
                ("scale", ctypes.c_float), ("out", P)]


KS_U8, KS_PACKED, KS_FP16 = 0, 1, 2

# symbol -> (restype, argtypes); must cover every function include/nsn_hip.h declares
SIGNATURES = {
    "nsn_version": (ctypes.c_char_p, []),
    "nsn_abi_sizeof": (I64, [I32]),
    "nsn_encode_blocks": (I32, [P, I32, I64, I64, I64, I64, I32, I32, I32, P, P, P, P, P, P, I64, I64, I64, P, P, P]),
    "nsn_block_factors": (I32, [P, P, P, P, I64, I64, I64, I32, P, P, P]),
    "nsn_pack_codes": (I32, [P, I64, I32, P, P, P]),
    "nsn_unpack_codes": (I32, [P, I64, I32, P, P]),
    "nsn_restore_blocks": (I32, [P, I32, P, P, P, I64, I64, I64, I32, P, I32, I64, P, I32, I64, I64, P, P]),
    "nsn_decode_attention": (I32, [ctypes.POINTER(AttnArgs), P]),
    "nsn_decode_attention_static": (I32, [ctypes.POINTER(AttnArgs), P]),
    "nsn_attention_merge": (I32, [P, I64, I64, I32, P, P, I32, P, P]),
    "nsn_attention_workspace_floats": (I64, [I64, I64, I32]),
    "nsn_finite_scan": (I32, [I32, P, P, P, P, P, P]),
    "nsn_prefill_attention": (I32, [ctypes.POINTER(PrefillArgs), P]),
    "nsn_tail_append": (I32, [P, P, I64, I64, I64, P, P, I64, I64, I32, P]),
    "nsn_tail_append_cast": (I32, [P, P, I32, I64, I64, I64, P, P, I64, I64, I32, P]),
    "nsn_tail_append_to": (I32, [P, P, I64, I64, I64, P, P, I64, P, I32, P, P]),
    "nsn_rope_append": (I32, [P, P, P, I64, I64, P, P, I64, I64, I64, I64, P, P, P, I64, P, I64, I32, I32, P, P]),
    "nsn_kscore": (I32, [ctypes.POINTER(KScoreArgs), P]),
}

_lib = None


def lib():
    """Load the HIP library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"NSN HIP library not built ({LIB_PATH}); run `python -m nsn_amd.build`")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        # the argument structs are passed by pointer: a library built from other
        # headers than these mirrors would read past or misread them on the GPU
        for which, st in enumerate((KVSide, AttnArgs, PrefillArgs, KScoreArgs)):
            if L.nsn_abi_sizeof(which) != ctypes.sizeof(st):
                raise RuntimeError(f"{LIB_PATH}: {st.__name__} is {L.nsn_abi_sizeof(which)} bytes in the library, "
                                   f"{ctypes.sizeof(st)} in the bindings -- rebuild (python -m nsn_amd.build)")
        _lib = L
    return _lib


def check(rc, what):
    if rc != NSN_OK:
        kind = {NSN_EINVAL: "invalid arguments", NSN_ELAUNCH: "kernel launch failed",
                NSN_ENOSPC: f"workspace exceeds the static scratch ({STATIC_SCRATCH_FLOATS} floats)"}.get(rc, str(rc))
        raise RuntimeError(f"{what}: {kind}")
