"""Host-side input contract of the packed decode readout.

``cpu_structure`` checks a host-resident input set before anything is copied
to the GPU: the bf16 query and tails as uint16 bit patterns, the packed 3-bit
codes, the fp16 block metadata and the 12-byte block headers -- their
contents included (little-endian ``<QHBB``: first token 64*i, 64 tokens,
3 bits, flags 0).  ``inputs`` runs it and copies the arrays to the device in
the layout ``kernels.pipeline`` takes.

Follows experiments/ac08/source/loop_kv_vf01_contract.py:50-67 (the checks)
and experiments/ac08/source/loop_kv_vf01.py:24-29 (the transfer).  A failure
raises ContractError with the stage recorded as 'cpu_structure', as there;
later stages (device-side layout, raw-input finiteness, attention) belong to
``kernels.pipeline``.
"""
from __future__ import annotations

import struct

import numpy as np

from . import kernels
from .errors import ContractError

BLOCK = 64
DIM = 128
HEADER = struct.Struct("<QHBB")     # first token position, tokens, bits, flags
PACKED_BYTES = BLOCK * DIM * 3 // 8


def _need(ok, message):
    if not ok:
        raise ContractError(message)


def block_headers(heads, n, bits=3):
    """Headers of n consecutive full blocks, the same for every head: u8 [1, heads, n, 12]."""
    one = np.frombuffer(b"".join(HEADER.pack(i * BLOCK, BLOCK, bits, 0) for i in range(n)), np.uint8)
    return np.broadcast_to(one.reshape(n, 12), (1, heads, n, 12))


def _array(a, name):
    x = a.get(name)
    return x if isinstance(x, np.ndarray) else None


def cpu_structure(a):
    """Check a host input set {q, k_tail, v_tail[, k_/v_ codes, headers, meta0..2]}.

    Returns (heads, packed tokens, total tokens); raises ContractError.
    """
    kernels.LAST_STAGE = "cpu_structure"
    q = _array(a, "q")
    _need(q is not None and q.dtype == np.uint16 and q.ndim == 4 and q.shape[0] == 1 and q.shape[2:] == (1, DIM),
          "Query layout")
    h = q.shape[1]
    _need(h > 0, "Empty head count")
    fields = {"q"}
    spans = []
    for side in ("k", "v"):
        tail = _array(a, side + "_tail")
        _need(tail is not None and tail.dtype == np.uint16 and tail.ndim == 4 and tail.shape[:2] == (1, h)
              and tail.shape[3] == DIM, "Tail layout")
        fields.add(side + "_tail")
        packed = 0
        if side + "_codes" in a:
            codes = _array(a, side + "_codes")
            _need(codes is not None and codes.dtype == np.uint8 and codes.ndim == 4 and codes.shape[:2] == (1, h)
                  and codes.shape[2] > 0 and codes.shape[3] == PACKED_BYTES, "Codes layout")
            n = codes.shape[2]
            for key, shape, dtype in (("headers", (1, h, n, 12), np.uint8), ("meta0", (1, h, n, BLOCK, 1), np.float16),
                                      ("meta1", (1, h, n, 1, DIM), np.float16),
                                      ("meta2", (1, h, n, 1, DIM), np.float16)):
                x = _array(a, side + "_" + key)
                _need(x is not None and x.shape == shape and x.dtype == dtype, "Metadata/header layout")
                fields.add(side + "_" + key)
            fields.add(side + "_codes")
            _need(np.array_equal(a[side + "_headers"], block_headers(h, n)), "Header positions/format")
            packed = n * BLOCK
        total = packed + tail.shape[2]
        _need(total > 0, "Empty sequence")
        spans.append((packed, total))
    _need(spans[0] == spans[1], "K/V length mismatch")
    _need(set(a) == fields, "Unexpected input fields")
    return h, spans[0][0], spans[0][1]


def inputs(a, device=None):
    """cpu_structure, then copy to the device: (k group, k tail, q, v group, v tail).

    Groups are {'codes', 'headers', 'metas': (norms, mins, scales)} or None;
    q and tails become bf16 tensors.  The host arrays are left unchanged.
    """
    import torch
    cpu_structure(a)
    dev = torch.device(device) if device is not None else torch.device("cuda")

    def bf16(x):
        return torch.from_numpy(np.ascontiguousarray(x).view(np.int16)).to(dev).view(torch.bfloat16)

    def group(side):
        if side + "_codes" not in a:
            return None
        return {"codes": torch.from_numpy(a[side + "_codes"]).to(dev),
                "headers": torch.from_numpy(a[side + "_headers"]).to(dev),
                "metas": tuple(torch.from_numpy(a[f"{side}_meta{i}"]).to(dev) for i in range(3))}

    return group("k"), bf16(a["k_tail"]), bf16(a["q"]), group("v"), bf16(a["v_tail"])
