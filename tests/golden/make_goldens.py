"""Write golden vectors for the NSN codec from the reference's own CPU functions.

Run in the build container only (the reference tree is not present on the GPU
box):  ``python tests/golden/make_goldens.py``.

Why an import: the exact codes and fp16 metadata bits of ``nsn_encode`` /
``nsn_int3_qdq`` and the exact output bits of ``nsn_decode`` on seeded random
inputs depend on torch-CPU's reduction order inside ``vector_norm`` and on its
rounding; no closed form or saved fixture of the reference pins them, so the
reference's functions themselves are called here and their outputs stored as
data.  Nothing of the reference is copied: only inputs and outputs are written.

Reference functions called (paths relative to the reference root):
  loop_kv_pilot.nsn_encode / nsn_decode / nsn_qdq / pack_codes
      experiments/ac08/source/loop_kv_pilot.py:171-230
  loop_kv_pk01_cache.pack3 / encode_group / restore_group
      experiments/ac08/source/loop_kv_pk01_cache.py:7-42
  nsn_int3_qdq    papers/nsn-integrated/code/nsn_int3_core.py:11-21
Input constructions restated from the reference's fixtures:
  check_core fixtures   data/validation/qdq-core/check_core.py:24-29
  codec fixtures        experiments/ac08/source/loop_kv_pilot.py:366-385
  group codec samples   experiments/ac08/source/loop_kv_pk01_cache.py:180-186
  real bf16 blocks      experiments/nb06/source/nb06_codec_fixture.json (data)
"""
from __future__ import annotations

import base64
import hashlib
import importlib.util
import json
import sys
from pathlib import Path

import numpy as np
import torch

sys.dont_write_bytecode = True
REF = Path("/root/reference")
HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

from tests.golden import inputs as gi  # noqa: E402  (shared input constructions)


def sha(b: bytes) -> str:
    return hashlib.sha256(b).hexdigest()


def bits16(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16).copy()


def load_reference():
    sys.path.insert(0, str(REF / "experiments/ac08/source"))
    import loop_kv_pilot as w  # noqa
    w.numeric_imports()
    import loop_kv_pk01_cache as c  # noqa
    spec = importlib.util.spec_from_file_location(
        "nsn_int3_core", REF / "papers/nsn-integrated/code/nsn_int3_core.py")
    core = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(core)
    return w, c, core


def encode_record(w, x, bits, prefix, out):
    q, metas = w.nsn_encode(x, bits)
    packed = np.frombuffer(w.pack_codes(q.numpy(), bits), np.uint8).copy()
    out[prefix + "codes"] = packed
    out[prefix + "norm"] = bits16(metas[0])
    out[prefix + "min"] = bits16(metas[1])
    out[prefix + "scale"] = bits16(metas[2])
    return q, metas


def main():
    w, c, core = load_reference()
    torch.set_num_threads(1)

    # --- C0: K and V fp16 [32, 64, 128] (seed 0) -------------------------
    k, v = gi.config0_inputs()
    rec = {"k_sha256": np.array(sha(k.tobytes())), "v_sha256": np.array(sha(v.tobytes()))}
    for name, a in (("k", k), ("v", v)):
        x = torch.from_numpy(a)                       # [32, 64, 128] fp16
        g = c.encode_group(x.reshape(1, 32, 1, 64, 128), 0)
        rec[name + "_codes"] = g["codes"].numpy().reshape(32, 3072)
        rec[name + "_norm"] = bits16(g["metas"][0]).reshape(32, 64)
        rec[name + "_min"] = bits16(g["metas"][1]).reshape(32, 128)
        rec[name + "_scale"] = bits16(g["metas"][2]).reshape(32, 128)
        rec[name + "_headers"] = g["headers"].numpy().reshape(32, 12)
        y = core.nsn_int3_qdq(x)
        assert torch.equal(y.view(torch.int16), w.nsn_qdq(x, 3).view(torch.int16))
        r = c.restore_group(g, torch.float16).reshape(32, 64, 128)
        assert torch.equal(r.view(torch.int16), y.view(torch.int16))
        rec[name + "_qdq"] = bits16(y)
    np.savez_compressed(HERE / "c0.npz", **rec)

    # --- qdq-core fixtures (8 x 3 dtypes) ------------------------------------
    rec = {}
    for name, x in gi.core_fixtures().items():
        for dt in (torch.float32, torch.float16, torch.bfloat16):
            a = x.to(dt)
            key = f"{name}|{str(dt).split('.')[-1]}|"
            rec[key + "in_sha256"] = np.array(sha(a.contiguous().view(torch.uint8).numpy().tobytes()))
            rec[key + "in_stride_last"] = np.array(a.float().stride(-1))
            y = core.nsn_int3_qdq(a)
            assert torch.equal(y.contiguous().view(torch.uint8), w.nsn_qdq(a, 3).contiguous().view(torch.uint8))
            encode_record(w, a, 3, key, rec)
            rec[key + "out"] = y.contiguous().view(torch.uint8).numpy().copy()
    np.savez_compressed(HERE / "core.npz", **rec)

    # --- codec fixtures, bits 3/4/5 (pilot cpu_fixtures tensors) --------------
    rec = {}
    for bits, tensors in gi.pilot_fixture_tensors().items():
        for i, t in enumerate(tensors):
            key = f"b{bits}|t{i}|"
            rec[key + "in_sha256"] = np.array(sha(t.contiguous().numpy().tobytes()))
            rec[key + "in_stride_last"] = np.array(t.stride(-1))
            q, metas = encode_record(w, t, bits, key, rec)
            y = w.nsn_decode(q, metas, t.dtype)
            rec[key + "decoded"] = y.contiguous().view(torch.int32).numpy().view(np.uint32).copy()
    for bits in (3, 4, 5):
        for count in (1, 7, 63, 64, 65, 127, 128, 129, 8192):
            codes = np.random.default_rng(2026093001 + count + bits).integers(0, 1 << bits, count, dtype=np.uint8)
            rec[f"stream|b{bits}|n{count}|codes"] = codes
            rec[f"stream|b{bits}|n{count}|bytes"] = np.frombuffer(w.pack_codes(codes, bits), np.uint8).copy()
    for n in (1, 2, 3, 7, 8, 9, 63, 64, 65, 8192):
        a = ((np.arange(n) * 5 + 3) % 8).astype(np.uint8)
        p = c.pack3(torch.from_numpy(a)).numpy()
        assert p.tobytes() == w.pack_codes(a, 3)
        rec[f"pack3|n{n}"] = p.copy()
    np.savez_compressed(HERE / "codec.npz", **rec)

    # --- 5-bit (and 4-bit) heavy-tailed blocks -------------------------------
    rec = {}
    x = gi.heavy_tailed_blocks()
    for bits in (4, 5):
        t = torch.from_numpy(x)
        q, metas = encode_record(w, t, bits, f"b{bits}|", rec)
        rec[f"b{bits}|qdq"] = bits16(w.nsn_qdq(t, bits))
    rec["in_sha256"] = np.array(sha(x.tobytes()))
    np.savez_compressed(HERE / "heavy.npz", **rec)

    # --- group codec: pk01 samples and the two real bf16 blocks --------------
    rec = {}
    fixture = json.loads((REF / "experiments/nb06/source/nb06_codec_fixture.json").read_text())
    for name, entry in fixture["blocks"].items():
        raw = base64.b64decode(entry["data_base64"], validate=True)
        assert sha(raw) == entry["sha256"]
        rec[f"real|{name}|input"] = np.frombuffer(raw, "<u2").copy().reshape(entry["shape"])
    samples = dict(gi.group_samples())
    for name in ("K_00", "V_43"):
        a = rec[f"real|{name}|input"]
        samples["real_" + name] = torch.from_numpy(a.view(np.int16)).view(torch.bfloat16).reshape(1, 8, 1, 64, 128)
    for name, x in samples.items():
        x = x.to(torch.bfloat16)
        key = f"group|{name}|"
        rec[key + "in_stride_last"] = np.array(x.float().stride(-1))
        rec[key + "in_sha256"] = np.array(sha(x.contiguous().view(torch.int16).numpy().tobytes()))
        g = c.encode_group(x, 0)
        rec[key + "codes"] = g["codes"].numpy().copy()
        rec[key + "norm"] = bits16(g["metas"][0])
        rec[key + "min"] = bits16(g["metas"][1])
        rec[key + "scale"] = bits16(g["metas"][2])
        rec[key + "headers"] = g["headers"].numpy().copy()
        y = c.restore_group(g, torch.bfloat16)
        assert torch.equal(y.reshape(x.shape).view(torch.int16), w.nsn_qdq(x, 3).view(torch.int16))
        rec[key + "restored"] = bits16(y)
    np.savez_compressed(HERE / "group.npz", **rec)
    print("goldens written:", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
