"""Extract compact golden vectors from the reference's recorded result files (data only).

Reads, from a shell-term/vesper checkout (default /root/reference):
  results/2026-10-18-moe-arithmetic/moe-aggregation.json
      38 aggregation cases recorded from the official DeepSeek MoE.forward on CUDA:
      inputs are regenerable from seeds, and every FP32 stage + the BF16 output
      is recorded as SHA-256.
  results/2026-10-18-routing-ties/router-postprocessing.json -> selection_cases
      232 synthetic selection cases run through PyTorch-CUDA topk/gather/sum/x1.5,
      with input hashes, the reference indices and the weight bits.

Writes tests/golden/moe_aggregation.json and tests/golden/router_selection.json.
Only recorded numbers are kept; no reference source is read or copied. Run once
in a container that has the reference mounted; the outputs are committed.
"""

from __future__ import annotations

import argparse
import json
from pathlib import Path

HERE = Path(__file__).resolve().parent


def main():
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--reference", type=Path, default=Path("/root/reference"))
    args = parser.parse_args()
    results = args.reference / "results"

    report = json.loads((results / "2026-10-18-moe-arithmetic" / "moe-aggregation.json").read_text())
    assert report["probe"] == "moe_aggregation_parity" and report["status"] == "pass"
    cases = [{"input": c["input"], "indices": c["indices"], "expert_order": c["expert_order"],
              "contribution_sha256": c["contribution_sha256"], "shared_sha256": c["shared_sha256"],
              "expected_sha256": c["expected_sha256"]} for c in report["cases"]]
    (HERE / "moe_aggregation.json").write_text(json.dumps(
        {"source": "results/2026-10-18-moe-arithmetic/moe-aggregation.json",
         "reference_method": report["reference_method"], "torch_version": report["torch_version"],
         "negative_controls_detected": report["negative_controls_detected"], "cases": cases}, indent=1) + "\n")

    report = json.loads((results / "2026-10-18-routing-ties" / "router-postprocessing.json").read_text())
    assert report["probe"] == "router_postprocessing_parity" and report["status"] == "pass"
    keep = ("kind", "seed", "bins", "strictly_higher", "equal_to_boundary", "repeat")
    cases = [{**{k: c[k] for k in keep if k in c},
              "input_scores_sha256": c["input_scores_sha256"], "input_selection_sha256": c["input_selection_sha256"],
              "reference_indices": c["reference_indices"], "reference_weight_bits": c["reference_weight_bits"],
              "candidate_tie_flag": c["candidate_tie_flag"]}
             for c in report["selection_cases"]]
    (HERE / "router_selection.json").write_text(json.dumps(
        {"source": "results/2026-10-18-routing-ties/router-postprocessing.json#selection_cases",
         "config": report["config"], "tie_policy": report["tie_policy"],
         "torch_git_version": report["torch_git_version"], "cases": cases}, indent=1) + "\n")
    print("wrote", HERE / "moe_aggregation.json", HERE / "router_selection.json")


if __name__ == "__main__":
    main()
