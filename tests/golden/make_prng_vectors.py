#!/usr/bin/env python3
"""Write golden vectors for the reference's name-addressed input synthesis.

The synthesis functions (FO/scripts/fixture_prng.py:94-166: bf16_uniform, f32_uniform,
bf16_signs, f8_banded, f4_nibbles) are integer/bit recipes with no published test
vector; the reference's own fixture of their checksums (ref/fixtures.safetensors) is
not in the tree. So this script imports the reference module itself, IN THE BUILD
CONTAINER ONLY, and records small input/output vectors under tests/golden/ so the
restatements (oracle/moa_oracle.c, moa_amd/prng.py) can be checked on any machine.

    python tests/golden/make_prng_vectors.py [/root/reference]
"""
import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent


def main() -> None:
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    sys.path.insert(0, str(ref / "furiosa-opt-gemma4-12B" / "scripts"))
    import fixture_prng as prng  # the reference module; build container only

    n = 257  # odd on purpose: exercises a partial last checksum word for u8 tensors
    out = {"count": n, "cases": []}

    def add(kind, name, args, data):
        arr = data.tolist()
        out["cases"].append({"kind": kind, "name": name, "args": args, "values": arr,
                             "checksum": int(prng.checksum(data))})

    for name, (lo, hi) in {
        "run0.sliding_project_qkv.input_rms_weight": (0.75, 1.25),
        "run1.sliding_attention_output.x": (-1.0, 1.0),
        "run2.decoder_feedforward.residual": (0.0, 1.0),
        "run0.sliding_project_qkv.q_weight_scale": (0.0, 1e-3),
    }.items():
        add("bf16_uniform", name, [lo, hi], prng.bf16_uniform(name, n, lo, hi))
    for run in range(3):
        for which in ("up", "gate", "down"):
            name = f"run{run}.global.{which}_global_scale"
            add("f32_uniform", name, [2048.0, 16384.0], prng.f32_uniform(name, 1, 2048.0, 16384.0))
    add("bf16_signs", "run0.sliding_project_qkv.x_signs", [1.0],
        prng.bf16_signs("run0.sliding_project_qkv.x_signs", n, 1.0))
    add("f8_banded", "run0.sliding_project_qkv.q_weight", [7, 14, True],
        prng.f8_banded("run0.sliding_project_qkv.q_weight", n, 7, 14, True))
    add("f8_banded", "run1.decoder_feedforward.up_weight_scale", [8, 10, False],
        prng.f8_banded("run1.decoder_feedforward.up_weight_scale", n, 8, 10, False))
    add("f4_nibbles", "run2.decoder_feedforward.down_weight_packed", [],
        prng.f4_nibbles("run2.decoder_feedforward.down_weight_packed", n + 1))
    out["name_hash"] = {s: int(prng.name_hash(s)) for s in ("", "a", "run0.global.pos", "run8.global.pos")}
    out["words"] = {s: [int(w) for w in prng.words(s, 4, 1000)] for s in ("run0.global.pos", "x")}
    (HERE / "prng_vectors.json").write_text(json.dumps(out) + "\n")
    print("wrote prng_vectors.json with", len(out["cases"]), "cases")


if __name__ == "__main__":
    main()
