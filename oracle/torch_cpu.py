"""PyTorch-CPU restatement of the NSN decode path -- TEST INFRASTRUCTURE ONLY.

The reference runs these steps as torch eager ops (on the CPU in its fixture
and qdq-core paths).  This module restates them on torch's CPU backend so
that ``bench.py``'s ``cpu_baseline`` leg can time the reference's CPU path in
the reference's own arithmetic, and so the tests can check that restatement
against the golden vectors.  Only ``tests/`` and ``bench.py``'s
``cpu_baseline`` leg use it; the product path never imports it.

Functions and the reference code each follows (paths relative to the
reference root):

* ``unpack3`` -- 3 bytes -> 8 LSB-first 3-bit codes
  (experiments/ac08/source/loop_kv_pk01_cache.py:19-28);
* ``nsn_decode`` -- n * ((m + s*q) / max(|m + s*q|, 1e-12)), zero where
  n == 0, cast (experiments/ac08/source/loop_kv_pilot.py:216-225);
* ``nsn_int3_qdq`` -- encode to 3-bit codes with fp16 metadata and decode in
  one function (papers/nsn-integrated/code/nsn_int3_core.py:11-21);
* ``bridge_readout`` -- the bridge route: restore K and V in full, then
  softmax(q K^T * scale) V in fp32 (experiments/ac08/source/
  loop_kv_vf01_kernel.py:47-54,120-126 followed by the AF01 readout,
  loop_kv_af01_kernel.py:100-111), with the GQA head map h // G.

Pinned in tests/test_oracle.py: ``unpack3`` against the C oracle's bitstream
and the reference's KAT, ``nsn_decode`` / ``nsn_int3_qdq`` bit for bit
against the golden vectors written from the reference's own functions, and
``bridge_readout`` against the fp64 attention oracle.
"""
from __future__ import annotations

import torch

EPS = 1e-12
SCALE = 0.08838834764831845


def unpack3(payload, shape):
    """uint8 bitstream [..., nbytes] -> uint8 codes of ``shape`` (3 bits each, LSB-first)."""
    n = 1
    for x in shape:
        n *= x
    a = payload.reshape(-1)
    pad = (-a.numel()) % 3
    if pad:
        a = torch.cat((a, torch.zeros(pad, dtype=torch.uint8)))
    a = a.reshape(-1, 3).to(torch.int32)
    b0, b1, b2 = a[:, 0], a[:, 1], a[:, 2]
    word = b0 | (b1 << 8) | (b2 << 16)                        # 24 bits = 8 codes
    codes = torch.stack([(word >> (3 * i)) & 7 for i in range(8)], dim=-1)
    return codes.reshape(-1)[:n].to(torch.uint8).reshape(shape).contiguous()


def nsn_decode(q, n16, m16, s16, dtype=torch.float32):
    """codes q [..., 64, 128] uint8; n16 [..., 64, 1], m16 / s16 [..., 1, 128] fp16."""
    n, m, s = (t.float().contiguous() for t in (n16, m16, s16))
    d = (m + s * q.float().contiguous()).contiguous()
    den = torch.linalg.vector_norm(d, dim=-1, keepdim=True).clamp_min(EPS)
    y = n * (d / den)
    return torch.where(n == 0, torch.zeros_like(y), y).to(dtype)


def nsn_int3_qdq(x):
    """[..., 64, 128] float -> reconstruction in x.dtype (3-bit codes, fp16 metadata)."""
    a = x.float()
    n = torch.linalg.vector_norm(a, dim=-1, keepdim=True)
    d = a / n.clamp_min(EPS)
    lo = d.amin(dim=-2, keepdim=True)
    step = (d.amax(dim=-2, keepdim=True) - lo) / 7
    safe = torch.where(step == 0, torch.ones_like(step), step)
    q = ((d - lo) / safe).round().clamp(0, 7).to(torch.uint8)
    n16, m16, s16 = (t.half() for t in (n, lo, step))
    return nsn_decode(q, n16, m16, s16, x.dtype)


def restore_blocks(codes, n16, m16, s16):
    """Packed 3-bit blocks [H, nb, 3072] + metadata -> fp32 [H, nb*64, 128]."""
    H, nb, _ = codes.shape
    q = unpack3(codes, (H, nb, 64, 128))
    y = nsn_decode(q, n16.reshape(H, nb, 64, 1), m16.reshape(H, nb, 1, 128), s16.reshape(H, nb, 1, 128))
    return y.reshape(H, nb * 64, 128)


def bridge_readout(q, kblocks, ktail, vblocks, vtail, scale=SCALE):
    """One sequence through the bridge route on the CPU.

    q [Hq, 128]; kblocks / vblocks: (codes [Hkv, nb, 3072] u8, norms, mins,
    scales fp16) or None; ktail / vtail [Hkv, T - 64*nb, 128].  Restores K and
    V in full (fp32), then softmax(q K^T * scale) V per query head, q-head h
    reading kv-head h // G.  Returns fp32 [Hq, 128].
    """
    def full(blocks, tail):
        parts = [] if blocks is None else [restore_blocks(*blocks)]
        parts.append(tail.float())
        return torch.cat(parts, dim=1)
    k = full(kblocks, ktail)
    v = full(vblocks, vtail)
    Hq, Hkv = q.shape[0], k.shape[0]
    G = Hq // Hkv
    qf = q.float().reshape(Hkv, G, 128)
    s = torch.matmul(qf, k.transpose(1, 2)) * scale            # [Hkv, G, T]
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v).reshape(Hq, 128)


def softmax_readout(scores, v):
    """The AF01 score-input readout: softmax(scores) V.  scores [Hq, T], v [Hkv, T, 128] fp32."""
    Hq, Hkv = scores.shape[0], v.shape[0]
    p = torch.softmax(scores.float(), dim=-1).reshape(Hkv, Hq // Hkv, -1)
    return torch.matmul(p, v.float()).reshape(Hq, 128)
