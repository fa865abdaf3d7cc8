"""GPU parity of the K-score kernel (nsn_kscore) against the fp64 oracle, for
the reference's recipes (NSN, KIVI, fp16 K) on u8 codes and on bit-packed
codes (3, 4, 5 bits); ragged token counts, GQA 4 and 8, head_dim 128 and 256."""
import numpy as np
import pytest
import torch

from nsn_amd import kscore
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
# |got - ref| <= 2e-5 * max|ref| (the reference's gate is the same rel-max metric at 1e-2)
REL_MAX = 2e-5


def _case(B, T, n_kv, D, n_q, recipe, bits, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(B, n_q, D, generator=g).to(torch.float16)
    k = torch.randn(B, T, n_kv * D, generator=g) * torch.exp(torch.randn(B, T, 1, generator=g))
    ref, ts = kscore.make_store(k, bits, recipe, n_kv, D, DEV)
    return q, ref, ts


def _oracle(q, ts, n_kv, D):
    if ts["is_fp16"]:
        return O.kscore64(q.numpy(), ts["code"].cpu().float().numpy(), None, None, None, n_kv, D)
    en = ts["eff_norm"].cpu().float().numpy() if ts["is_nsn"] else None
    return O.kscore64(q.numpy(), ts["code"].cpu().numpy(), ts["min"].cpu().float().numpy(),
                      ts["step"].cpu().float().numpy(), en, n_kv, D)


def _check(got, want):
    err = np.abs(got.cpu().double().numpy() - want)
    assert err.max() <= REL_MAX * np.abs(want).max(), (err.max(), np.abs(want).max())


@pytest.mark.parametrize("recipe,bits", [("nsn", 5), ("kivi", 5), ("kivi", 4), ("nsn", 4), ("nsn", 3), ("fp16", 16)])
def test_kscore_qwen3_shape(recipe, bits):
    n_kv, D, n_q = 8, 128, 32
    for B, T in ((2, 300), (1, 17), (3, 64)):
        q, ref, ts = _case(B, T, n_kv, D, n_q, recipe, bits, 10 + B + T)
        got = kscore.decode_scores(q.to(DEV), ts, n_q, n_kv, D)
        want = _oracle(q, ts, n_kv, D)
        _check(got, want)
        if recipe != "fp16":
            # the same codes bit-packed (each code at a per-element bit position, its
            # coefficient scaled by 2^-k to match): the oracle's scores, and the u8
            # kernel's up to the order of the fp32 sums and the lo parts that the
            # 2^-k scaling moves into the fp16 subnormal range (~3e-6 of max|score|)
            gp = kscore.decode_scores(q.to(DEV), kscore.pack_store(ts, bits), n_q, n_kv, D)
            _check(gp, want)
            assert (gp - got).abs().max().item() <= 1e-5 * got.abs().max().item()


@pytest.mark.parametrize("recipe,bits", [("nsn", 5), ("kivi", 4), ("fp16", 16)])
def test_kscore_gqa8_and_head_dim_256(recipe, bits):
    for n_kv, D, n_q in ((2, 128, 16), (2, 256, 8), (1, 256, 8)):
        q, ref, ts = _case(2, 200, n_kv, D, n_q, recipe, bits, 7 + D + n_q)
        got = kscore.decode_scores(q.to(DEV), ts, n_q, n_kv, D)
        _check(got, _oracle(q, ts, n_kv, D))
        if recipe != "fp16":
            gp = kscore.decode_scores(q.to(DEV), kscore.pack_store(ts, bits), n_q, n_kv, D)
            _check(gp, _oracle(q, ts, n_kv, D))


def test_kscore_long_context():
    """One sequence of 65536 tokens (the largest published context): every
    token against the oracle."""
    n_kv, D, n_q = 8, 128, 32
    q, ref, ts = _case(1, 65536, n_kv, D, n_q, "nsn", 5, 3)
    got = kscore.decode_scores(q.to(DEV), ts, n_q, n_kv, D)
    _check(got, _oracle(q, ts, n_kv, D))


def test_kscore_matches_materialised_reference_scores():
    """The reference's gate (phase_k1c:304-311): kernel scores against the
    dequantise-then-score path in fp32 (here torch fp32 on the CPU over the
    stored fp16 values), rel-max far below its 1e-2."""
    n_kv, D, n_q = 8, 128, 32
    q, ref, ts = _case(2, 500, n_kv, D, n_q, "nsn", 5, 11)
    code = ref["code"].float()
    kdq = (code * ref["step"].float() + ref["min"].float()).reshape(2, 500, n_kv, D)
    kdq = ref["eff_norm"].float().unsqueeze(-1) * kdq
    qx = q.float().reshape(2, n_kv, 4, D)
    want = torch.einsum("bnrd,btnd->bnrt", qx, kdq).reshape(2, n_q, 500) / D ** 0.5
    got = kscore.decode_scores(q.to(DEV), ts, n_q, n_kv, D).cpu()
    rel = ((got - want).abs().max() / want.abs().max()).item()
    assert rel < 1e-4


@pytest.mark.parametrize("recipe,bits", [("nsn", 5), ("kivi", 4), ("fp16", 16)])
def test_kscore_reference_golden_scores(recipe, bits):
    """The kernel on the reference's own store (tests/golden/k1c.npz, written
    from phase_k1c_triton_fused_kernel.py) against the reference's fp32
    scores."""
    from pathlib import Path
    G = np.load(Path(__file__).resolve().parent / "golden" / "k1c.npz")
    key = f"{recipe}{bits}|"
    f16 = lambda a: torch.from_numpy(np.asarray(a, np.uint16).view(np.int16)).view(torch.float16).to(DEV)
    q = f16(G[key + "q"]).contiguous()
    B, n_q, D = q.shape
    T = G["k"].shape[1]
    if recipe == "fp16":
        ts = {"code": f16(G[key + "code"]).contiguous(), "is_fp16": True, "is_nsn": False, "T": T,
              "n_kv": 8, "head_dim": D}
    else:
        ts = {"code": torch.from_numpy(G[key + "code"]).to(DEV).contiguous(), "is_fp16": False,
              "is_nsn": recipe == "nsn", "min": f16(G[key + "min"]).contiguous(),
              "step": f16(G[key + "step"]).contiguous(), "T": T, "n_kv": 8, "head_dim": D}
        if recipe == "nsn":
            ts["eff_norm"] = f16(G[key + "eff_norm"]).contiguous()
    got = kscore.decode_scores(q, ts, n_q, 8, D).cpu().double().numpy()
    ref = G[key + "scores"].astype(np.float64)
    assert np.abs(got - ref).max() <= REL_MAX * np.abs(ref).max()
