"""Host-side input contract (nsn_amd.contract) against the reference's records.

The stage each negative fixture must stop at comes from the reference
verifier's own table (tests/golden/vf01_rejections.json, written by
make_vf01_rejections.py from the reference run's summary.json and
rejections.jsonl); the fixtures follow loop_kv_vf01_contract.py:81-120.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from nsn_amd import contract
from nsn_amd.errors import ContractError
from tests.golden import inputs as gi

GOLDEN = Path(__file__).parent / "golden"
REJ = json.loads((GOLDEN / "vf01_rejections.json").read_text())["kinds"]
NORMAL = json.loads((GOLDEN / "vf01_input_hashes.json").read_text())["fixtures"]


def hashes(a):
    return {n: gi.array_hash(x) for n, x in a.items()}


def test_kind_list_matches_the_reference_records():
    assert tuple(REJ) == gi.NEGATIVE_KINDS


@pytest.mark.parametrize("f", NORMAL, ids=[f["id"] for f in NORMAL])
def test_normal_fixtures_pass_cpu_structure(f):
    a = gi.vf01_fixture(f["compressed"], f["length"], f["pattern"])
    assert hashes(a) == f["input_hashes"]
    assert contract.cpu_structure(a) == (2, f["compressed"], f["length"])


@pytest.mark.parametrize("kind", gi.NEGATIVE_KINDS)
def test_cpu_structure_rejects_exactly_the_cpu_stage_kinds(kind):
    a, mutation = gi.vf01_negative(kind)
    before = hashes(a)
    stage = REJ[kind]["expected_stage"]
    assert (mutation is not None) == (stage == "structural")
    if stage == "cpu_structure":
        with pytest.raises(ContractError):
            contract.cpu_structure(a)
    else:
        contract.cpu_structure(a)
    assert hashes(a) == before
    if stage == "input_finite":      # the verifier's precondition: some raw input is nonfinite
        def values(x):
            return (x.astype(np.uint32) << 16).view(np.float32) if x.dtype == np.uint16 else x
        assert not all(np.isfinite(values(x)).all() for n, x in a.items()
                       if n == "q" or n.endswith("_tail") or "_meta" in n)


@pytest.mark.parametrize("defect", ["bits", "shifted", "flags", "length"])
def test_header_contents_are_checked(defect):
    """Planted header defects other than the reference's position corruption."""
    a = gi.vf01_fixture(128, 130, "mixed_codes")
    h = a["v_headers"].reshape(2, 2, 12)
    if defect == "bits":
        h[1, 1, 10] = 5
    elif defect == "shifted":                      # positions 64, 128 instead of 0, 64
        h[:, :, :8] = contract.block_headers(2, 3)[0, :, 1:, :8]
    elif defect == "flags":
        h[0, 0, 11] = 1
    else:
        h[0, 1, 8] = 63
    with pytest.raises(ContractError, match="Header"):
        contract.cpu_structure(a)


def test_block_headers_layout():
    hd = contract.block_headers(2, 3)
    assert hd.shape == (1, 2, 3, 12)
    row = hd[0, 1, 2]
    assert int.from_bytes(row[:8].tobytes(), "little") == 128 and row[8] == 64 and row[9] == 0
    assert row[10] == 3 and row[11] == 0
