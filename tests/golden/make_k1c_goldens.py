"""Write golden vectors for the K1c K-score component from the reference's own
CPU functions.

Run in the build container only (the reference tree is not present on the GPU
box):  ``python tests/golden/make_k1c_goldens.py``  -> ``tests/golden/k1c.npz``.

Why an import: the exact u8 codes, fp16 min / step / eff_norm of the K1c
stores (per-channel quantisation over all tokens, torch-CPU rounding) and the
reference's fp32 scores are fixed by the reference's torch code and by no
saved fixture; so its functions are called on their own seeded inputs and only
inputs and outputs are written.

Reference functions called (experiments/kernels/phase_k1c_triton_fused_kernel.py):
  _make_inputs (:132-147), make_triton_store (:160-182),
  _torch_decode_scores (:150-164)
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np
import torch

sys.dont_write_bytecode = True
REF = Path("/root/reference/experiments/kernels/phase_k1c_triton_fused_kernel.py")
OUT = Path(__file__).resolve().parent / "k1c.npz"
MODEL = {"name": "Qwen3-30B-A3B", "n_kv": 8, "head_dim": 128, "n_q": 32}
CELLS = [("nsn", 5), ("kivi", 4), ("fp16", 16)]
B, T = 2, 40


def bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def main():
    spec = importlib.util.spec_from_file_location("phase_k1c", REF)
    k1c = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(k1c)
    # the q and K tensors _make_inputs draws (q first, then k, from the seeded CPU
    # generator): the same for every cell
    g = torch.Generator(device="cpu").manual_seed(k1c.SEED)
    torch.randn(B, MODEL["n_q"], MODEL["head_dim"], generator=g, dtype=torch.float32)
    k = torch.randn(B, T, MODEL["n_kv"] * MODEL["head_dim"], generator=g, dtype=torch.float32)
    out = {"k": k.numpy()}
    for recipe, bits in CELLS:
        key = f"{recipe}{bits}|"
        q, ref_store, ts, n_q, n_kv, hd = k1c.make_triton_store(MODEL, B, T, bits, recipe, "cpu")
        ref32 = k1c._torch_decode_scores(
            q.float(), {kk: (v.float() if torch.is_tensor(v) else v) for kk, v in ref_store.items()},
            recipe, n_q, n_kv, hd)
        out[key + "q"] = bits16(q)
        out[key + "scores"] = ref32.numpy()
        if recipe == "fp16":
            out[key + "code"] = bits16(ts["code"])
        else:
            out[key + "code"] = ts["code"].numpy()
            out[key + "min"] = bits16(ts["min"])
            out[key + "step"] = bits16(ts["step"])
            if recipe == "nsn":
                out[key + "eff_norm"] = bits16(ts["eff_norm"])
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(out)} arrays)")


if __name__ == "__main__":
    main()
