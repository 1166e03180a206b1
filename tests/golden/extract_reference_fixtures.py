#!/usr/bin/env python3
"""Copy the reference's known-answer DATA for this hot path into tests/golden/.

Run in the build container (the reference checkout is not on the GPU box):

    python tests/golden/extract_reference_fixtures.py [/root/reference]

Only data is copied -- inputs, expected outputs, checksums and hashes that the
reference's own probe suites hold. No reference source is copied. What each file is:

  qkv_boundary.safetensors   byte copy of
      moa-dev/experiments/candidates/qkv-fullh-weight-switch/boundary-suite/fixtures/boundary.safetensors
      (QKV whole-op cancellation probe, 2 cases, pos 1763; expected q/k/v as f32, input
      checksums; construction in moa-dev/experiments/candidates/qkv-boundary-probe-e53/generate_suite.py:24-105)
  qkv_boundary_ranges.json   per-case intermediate ranges from qkv-boundary-probe-e53/cpu-references.json
  qkv_raw_truth.json         9 QKV raw-projection cases (input checksums/sha256, expected sha256 and
      samples) from qkv-fullh-weight-switch/boundary-suite/raw-truth-v1.json
      (construction: .../boundary-suite/raw-src/generate.py:14-54)
  o_raw_truth.json           8 O raw-projection cases from
      c09-output-first-npu/validation/probe-oracle.json (construction: .../probe-v1/generate.py:20-75)
  o_boundary.json            8 O whole-op cases (input sha256/checksums, intermediate ranges, expected
      first bits) from output-boundary-probe-e47/cpu-references.json
      (construction: output-boundary-probe-e47/generate_suite.py:37-108)
  ffn_stress_expected_bf16.bin + ffn_stress.json
      NVFP4 FFN known answer (3840 x 0x3ecf) and its recorded input hashes/intermediates from
      ffn-native-down-weighted-residual/full-ffn-stress/{expected-bf16.bin,reference.json}
      (construction: .../full-ffn-stress/generate_reference.py:34-92)
"""
import json
import shutil
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CAND = "moa-dev/experiments/candidates"


def main() -> None:
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    cand = ref / CAND

    shutil.copyfile(
        cand / "qkv-fullh-weight-switch/boundary-suite/fixtures/boundary.safetensors",
        HERE / "qkv_boundary.safetensors",
    )

    e53 = json.loads((cand / "qkv-boundary-probe-e53/cpu-references.json").read_text())
    (HERE / "qkv_boundary_ranges.json").write_text(json.dumps({
        "pos": e53["pos"], "slot": e53["slot"],
        "records": [{k: r[k] for k in ("case", "name", "checksums", "sha256", "ranges",
                                      "first_output_bf16_bits") if k in r}
                    for r in e53["records"]],
    }, indent=1) + "\n")

    raw = json.loads((cand / "qkv-fullh-weight-switch/boundary-suite/raw-truth-v1.json").read_text())
    (HERE / "qkv_raw_truth.json").write_text(json.dumps(
        {"oracle": raw["oracle"], "cases": raw["cases"]}, indent=1) + "\n")

    o_raw = json.loads((cand / "c09-output-first-npu/validation/probe-oracle.json").read_text())
    (HERE / "o_raw_truth.json").write_text(json.dumps(
        {"oracle": o_raw["oracle"], "cases": o_raw["cases"]}, indent=1) + "\n")

    e47 = json.loads((cand / "output-boundary-probe-e47/cpu-references.json").read_text())
    (HERE / "o_boundary.json").write_text(json.dumps({
        "atol": e47["atol"], "rtol": e47["rtol"], "weight_rule": e47.get("weight_rule"),
        "records": e47["records"],
    }, indent=1) + "\n")

    stress = cand / "ffn-native-down-weighted-residual/full-ffn-stress"
    shutil.copyfile(stress / "expected-bf16.bin", HERE / "ffn_stress_expected_bf16.bin")
    rj = json.loads((stress / "reference.json").read_text())
    (HERE / "ffn_stress.json").write_text(json.dumps({
        k: rj[k] for k in ("inputs", "intermediates", "post_rms", "expected", "unchanged_tolerance")
    }, indent=1) + "\n")
    print("wrote", sorted(p.name for p in HERE.iterdir() if p.suffix in (".json", ".bin", ".safetensors")))


if __name__ == "__main__":
    main()
