"""Write vf01_rejections.json: the reference's recorded rejection outcomes.

Reads the reference run's records (data files only, nothing executed):
  runs/loop-kv-vf01-20261002-072452-1d1c10c0/rejections.jsonl  (per kind and arm:
      rejected, stage, error type, inputs unchanged)
  runs/loop-kv-vf01-20261002-072452-1d1c10c0/summary.json      (the verifier's
      expected stage per kind, experiments/ac08/source/verify_loop_kv_vf01.py:73-88)
Run from the repository root: python -m tests.golden.make_vf01_rejections
"""
import json
import sys
from pathlib import Path

RUN = "runs/loop-kv-vf01-20261002-072452-1d1c10c0"


def main(ref="/root/reference"):
    run = Path(ref) / RUN
    summary = json.loads((run / "summary.json").read_text())
    expected = {r["kind"]: r for r in summary["rejections"]}
    kinds = {}
    for line in (run / "rejections.jsonl").read_text().splitlines():
        r = json.loads(line)
        e = expected[r["kind"]]
        kinds[r["kind"]] = {
            "expected_stage": e["expected_stage"],
            "reference_pass": e["pass_rejection"],
            "mutation": r["mutation"],
            "recorded": {x["arm"]: {"rejected": x["rejected"], "stage": x["stage"], "error_type": x["error_type"],
                                    "input_unchanged": x["input_unchanged"]} for x in r["results"]},
        }
    out = {"source": RUN + "/rejections.jsonl + summary.json['rejections']", "kinds": kinds}
    path = Path(__file__).with_name("vf01_rejections.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print("wrote", path, len(kinds), "kinds")


if __name__ == "__main__":
    main(*sys.argv[1:])
