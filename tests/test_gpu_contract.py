"""The reference's 24 negative fixtures through every arm on the GPU.

Each kind must be rejected at the stage the reference verifier assigns
(experiments/ac08/source/verify_loop_kv_vf01.py:73-88, recorded in
tests/golden/vf01_rejections.json), with the error type the reference
raised there, and every input -- host arrays and device tensors -- must be
bitwise unchanged afterwards (loop_kv_vf01.py:69-72,86-93 hash them before
and after each call).

v_tail_noncontiguous: the reference harness built its mutation as
transpose().contiguous().transpose() of a one-token tail, which torch still
reports as contiguous, so its own check raised at 'cpu_structure' and its
verifier marked the kind failed.  Here the V tail is a genuinely strided view
of the same values and must stop at the verifier's stage, 'structural'.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from nsn_amd import contract, kernels
from nsn_amd.errors import ContractError, IntegrityError, NumericalFailure
from tests.golden import inputs as gi

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
GOLDEN = Path(__file__).parent / "golden"
REJ = json.loads((GOLDEN / "vf01_rejections.json").read_text())["kinds"]
NORMAL = json.loads((GOLDEN / "vf01_input_hashes.json").read_text())["fixtures"]
ARMS = ("RF01_MATERIALIZE", "TILE_MATERIALIZE", "V_FUSED")
ERROR = {"cpu_structure": "ContractError", "structural": "IntegrityError", "input_finite": "NumericalFailure",
         "attention": "NumericalFailure"}


def host_hashes(a):
    return {n: gi.array_hash(x) for n, x in a.items()}


def device_hashes(data):
    """Hashes of every device input (loop_kv_vf01.py:30-35 input_arrays)."""
    g, kt, q, vg, vt = data
    out = {"q": q, "k_tail": kt, "v_tail": vt}
    for side, group in (("k", g), ("v", vg)):
        if group is not None:
            out[side + "_codes"] = group["codes"]
            out[side + "_headers"] = group["headers"]
            out.update({f"{side}_meta{i}": m for i, m in enumerate(group["metas"])})
    def host(t):
        t = t.detach().cpu().contiguous()
        return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()
    return {n: gi.array_hash(host(t)) for n, t in out.items()}


def strided_tail(vt):
    """The same values as a noncontiguous view (every other element of a wider buffer)."""
    buf = torch.zeros(vt.shape[:-1] + (2 * vt.shape[-1],), dtype=vt.dtype, device=vt.device)
    buf[..., ::2] = vt
    view = buf[..., ::2]
    assert not view.is_contiguous() and torch.equal(view, vt)
    return view


def run(kind, arm, kernel="reference"):
    a, mutation = gi.vf01_negative(kind)
    host_before = host_hashes(a)
    data = before = None
    kernels.LAST_STAGE = "cpu_structure"
    try:
        data = contract.inputs(a, DEV)
        if mutation:
            g, kt, q, vg, vt = data
            data = (g, kt, q, vg, strided_tail(vt))
        before = device_hashes(data)
        kernels.pipeline(arm, data, kernel=kernel)
        result = dict(rejected=False, stage=kernels.LAST_STAGE, error_type=None)
    except (ContractError, IntegrityError, NumericalFailure) as exc:
        result = dict(rejected=True, stage=kernels.LAST_STAGE, error_type=type(exc).__name__)
    torch.cuda.synchronize()
    result["input_unchanged"] = host_hashes(a) == host_before and (data is None or device_hashes(data) == before)
    return result


@pytest.mark.parametrize("kernel", ["reference", "fast"])
@pytest.mark.parametrize("arm", ARMS)
@pytest.mark.parametrize("kind", gi.NEGATIVE_KINDS)
def test_negative_fixture_rejected_at_reference_stage(kind, arm, kernel):
    """kernel: the attention kernel behind every arm (the fast one checks the
    raw block metadata while computing its decode factors)."""
    want = REJ[kind]
    r = run(kind, arm, kernel)
    assert r["rejected"], (kind, arm, r)
    assert r["stage"] == want["expected_stage"], (kind, arm, r)
    assert r["error_type"] == ERROR[want["expected_stage"]], (kind, arm, r)
    if want["reference_pass"]:       # the reference's own outcome, reproduced
        rec = want["recorded"][arm]
        assert (r["stage"], r["error_type"]) == (rec["stage"], rec["error_type"])
    assert r["input_unchanged"], (kind, arm)


def test_negative_fixtures_with_the_separate_finite_scan(monkeypatch):
    """The fused arm with the grouped scan before the kernel instead of inside it."""
    monkeypatch.setattr(kernels, "FUSED_VALIDATION", False)
    for kind in gi.NEGATIVE_KINDS:
        r = run(kind, "V_FUSED")
        assert r["rejected"] and r["stage"] == REJ[kind]["expected_stage"] and r["input_unchanged"], (kind, r)


@pytest.mark.parametrize("kernel", ["reference", "fast"])
@pytest.mark.parametrize("arm", ARMS)
def test_normal_fixtures_leave_inputs_unchanged(arm, kernel):
    for f in NORMAL:
        a = gi.vf01_fixture(f["compressed"], f["length"], f["pattern"])
        assert host_hashes(a) == f["input_hashes"]
        data = contract.inputs(a, DEV)
        before = device_hashes(data)
        assert before == f["input_hashes"], f["id"]
        out = kernels.pipeline(arm, data, kernel=kernel)
        torch.cuda.synchronize()
        assert bool(torch.isfinite(out).all()) and kernels.LAST_STAGE == "returned", f["id"]
        assert device_hashes(data) == before and host_hashes(a) == f["input_hashes"], f["id"]
