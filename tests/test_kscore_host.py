"""K-score component (reference experiments/kernels/phase_k1c_triton_fused_kernel.py)
on the CPU: the fp64 oracle pinned by brute force, closed forms and the GQA
invariant; the torch store builders against the reference's own self-tests
(:387-411); the packed-size accounting against the published cells."""
import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from nsn_amd import kscore
from nsn_amd.errors import IntegrityError
from oracle import oracle as O

GOLD = Path(__file__).resolve().parent / "golden" / "k1c_published.json"


def _rand_store(rng, B=2, T=5, n_kv=2, D=128, G=2):
    q = rng.standard_normal((B, n_kv * G, D)).astype(np.float16)
    code = rng.integers(0, 32, (B, T, n_kv * D)).astype(np.uint8)
    mn = (rng.standard_normal((B, n_kv * D)) * 0.1).astype(np.float16)
    st = (rng.random((B, n_kv * D)) * 0.07 + 0.01).astype(np.float16)
    en = (rng.lognormal(0, 1, (B, n_kv, T))).astype(np.float16)
    return q, code, mn, st, en


def test_oracle_brute_force():
    rng = np.random.default_rng(0)
    q, code, mn, st, en = _rand_store(rng)
    B, Hq, D = q.shape
    n_kv = 2
    got = O.kscore64(q, code, mn, st, en, n_kv, D)
    for b in range(B):
        for h in range(Hq):
            hkv = h // (Hq // n_kv)
            for t in range(code.shape[1]):
                acc = 0.0
                for d in range(D):
                    c = hkv * D + d
                    acc += float(q[b, h, d]) * (float(code[b, t, c]) * float(st[b, c]) + float(mn[b, c]))
                want = acc / math.sqrt(D) * float(en[b, hkv, t])
                assert abs(got[b, h, t] - want) <= 1e-12 * max(1.0, abs(want))


def test_oracle_closed_forms():
    rng = np.random.default_rng(1)
    q, code, mn, st, en = _rand_store(rng)
    D = q.shape[2]
    # zero codes: only the min term, the same for every token up to eff_norm
    z = np.zeros_like(code)
    s = O.kscore64(q, z, mn, st, en, 2, D)
    mrows = mn.astype(np.float64).reshape(2, 2, D)[:, [0, 0, 1, 1]]          # head h reads kv-head h // 2
    qm = (q.astype(np.float64) * mrows).sum(-1)
    assert np.allclose(s, qm[:, :, None] / math.sqrt(D) * np.repeat(en.astype(np.float64), 2, 1), rtol=1e-12)
    # one-hot query on channel 7: the dequantised value of that channel
    q1 = np.zeros_like(q)
    q1[:, :, 7] = 1
    s1 = O.kscore64(q1, code, mn, st, None, 2, D)
    want = (code[:, :, 7].astype(np.float64) * float(st[0, 7]) + float(mn[0, 7])) / math.sqrt(D)
    assert np.allclose(s1[0, 0], want[0], rtol=1e-12)
    # a planted mistake (no min term) fails the closed form
    s_bad = O.kscore64(q, z, np.zeros_like(mn), st, en, 2, D)
    assert not np.allclose(s_bad, s)


def test_oracle_gqa_repeat():
    rng = np.random.default_rng(2)
    q, code, mn, st, en = _rand_store(rng, n_kv=2, G=4)
    s = O.kscore64(q, code, mn, st, en, 2, 128)
    # MHA over repeated kv-heads (head h reads kv-head h // 4)
    code8 = np.repeat(code.reshape(2, 5, 2, 1, 128), 4, 3).reshape(2, 5, 8 * 128)
    mn8 = np.repeat(mn.reshape(2, 2, 1, 128), 4, 2).reshape(2, 8 * 128)
    st8 = np.repeat(st.reshape(2, 2, 1, 128), 4, 2).reshape(2, 8 * 128)
    en8 = np.repeat(en, 4, 1)
    s8 = O.kscore64(q, code8, mn8, st8, en8, 8, 128)
    assert np.allclose(s, s8, rtol=1e-13)


def test_store_nsn_folding_matches_unfolded_qdq():
    """The reference's self-test (phase_k1c:391-397): decoding the NSN store
    (eff_norm * (code*step + min)) equals the unfolded qdq
    (norm * dq / |dq|) within 1e-6 relative."""
    g = torch.Generator().manual_seed(20260510)
    for n_kv, D in ((4, 128), (8, 256)):
        k = torch.randn(2, 257, n_kv * D, generator=g)
        for bits in (4, 5):
            st = kscore.nsn_store(k, bits, n_kv, D)
            dq = (st["code"] * st["step"] + st["min"]).reshape(2, 257, n_kv, D)
            folded = (st["eff_norm"].unsqueeze(-1) * dq).reshape(2, 257, -1)
            x = k.reshape(2, 257, n_kv, D)
            norm = x.norm(dim=-1, keepdim=True).clamp(min=kscore.EPS)
            unf = (norm * dq / dq.norm(dim=-1, keepdim=True).clamp(min=kscore.RENORM_EPS)).reshape(2, 257, -1)
            rel = (folded - unf).abs().max() / unf.abs().max()
            assert rel < 1e-6


def test_store_codes_lossless_in_u8_and_packed_size():
    g = torch.Generator().manual_seed(5)
    k = torch.randn(2, 64, 8 * 128, generator=g)
    for recipe in ("kivi", "nsn"):
        ref, ts = kscore.make_store(k, 5, recipe, 8, 128, "cpu")
        assert torch.equal(ts["code"].float(), ref["code"].float())
        assert int(ts["code"].max()) <= 31
        assert ts["min"].shape == (2, 1024) and ts["step"].shape == (2, 1024)
    assert ts["eff_norm"].shape == (2, 8, 64)
    # memory delta NSN - KIVI = the norm only: 2*n_kv bytes per token (phase_k1c:406-409)
    for n_kv, D in ((4, 128), (8, 256)):
        d = kscore.bytes_per_token_K(5, n_kv, D, 32768, True) - kscore.bytes_per_token_K(5, n_kv, D, 32768, False)
        assert abs(d - 2.0 * n_kv) < 1e-9


def test_bytes_per_token_matches_published_cells():
    cells = json.loads(GOLD.read_text())["cells"]
    n = 0
    for c in cells:
        if c["recipe"] == "fp16":
            continue
        got = kscore.bytes_per_token_K(c["bits"], c["n_kv"], c["head_dim"], c["ctx"], c["recipe"] == "nsn")
        assert abs(got - c["bytes_per_token_K"]) < 1e-9, c
        n += 1
    assert n >= 100


def test_decode_scores_requires_gpu_tensors():
    q = torch.zeros(1, 32, 128, dtype=torch.float16)
    ts = {"code": torch.zeros(1, 4, 1024, dtype=torch.uint8), "is_fp16": False, "is_nsn": False,
          "min": torch.zeros(1, 1024, dtype=torch.float16), "step": torch.zeros(1, 1024, dtype=torch.float16),
          "T": 4, "n_kv": 8, "head_dim": 128}
    with pytest.raises(IntegrityError):
        kscore.decode_scores(q, ts, 32, 8, 128)


K1C = Path(__file__).resolve().parent / "golden" / "k1c.npz"
K1C_CELLS = [("nsn", 5), ("kivi", 4), ("fp16", 16)]


def _f16(bits):
    return np.asarray(bits, np.uint16).view(np.float16)


@pytest.mark.parametrize("recipe,bits", K1C_CELLS)
def test_store_matches_reference_goldens(recipe, bits):
    """The store builders reproduce the reference's make_triton_store bit for
    bit on its own seeded inputs (tests/golden/make_k1c_goldens.py)."""
    G = np.load(K1C)
    key = f"{recipe}{bits}|"
    k = torch.from_numpy(G["k"])
    _, ts = kscore.make_store(k, bits, recipe, 8, 128, "cpu")
    if recipe == "fp16":
        assert np.array_equal(ts["code"].view(torch.int16).numpy().view(np.uint16), G[key + "code"])
        return
    assert np.array_equal(ts["code"].numpy(), G[key + "code"])
    assert np.array_equal(ts["min"].view(torch.int16).numpy().view(np.uint16), G[key + "min"])
    assert np.array_equal(ts["step"].view(torch.int16).numpy().view(np.uint16), G[key + "step"])
    if recipe == "nsn":
        assert np.array_equal(ts["eff_norm"].view(torch.int16).numpy().view(np.uint16), G[key + "eff_norm"])


@pytest.mark.parametrize("recipe,bits", K1C_CELLS)
def test_oracle_matches_reference_scores(recipe, bits):
    """The fp64 oracle against the reference's own fp32 dequantise-then-score
    path (_torch_decode_scores) on the golden stores."""
    G = np.load(K1C)
    key = f"{recipe}{bits}|"
    q = _f16(G[key + "q"]).astype(np.float64)
    if recipe == "fp16":
        s = O.kscore64(q, _f16(G[key + "code"]), None, None, None, 8, 128)
    else:
        en = _f16(G[key + "eff_norm"]) if recipe == "nsn" else None
        s = O.kscore64(q, G[key + "code"], _f16(G[key + "min"]), _f16(G[key + "step"]), en, 8, 128)
    ref = G[key + "scores"].astype(np.float64)
    assert np.abs(s - ref).max() <= 1e-6 * np.abs(ref).max()
