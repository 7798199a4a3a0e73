"""Writes tests/golden/rope_gemma3_local.json: the unscaled case of the
reference's RoPE fixture (crates/reng-model/testdata/rope_reference.json, case
`gemma3-4b-local`: Gemma-3's sliding-layer table, head_dim 256, no rope_scaling,
theta = Gemma3TextConfig's default rope_local_base_freq 10000), the inverse
frequencies and cos / sin rows transformers 5.16.1 produced at six positions.
Data only: this script copies numbers out of the reference's JSON."""
import json
import os
import sys

SRC = "/root/reference/crates/reng-model/testdata/rope_reference.json"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "rope_gemma3_local.json")


def main():
    doc = json.load(open(sys.argv[1] if len(sys.argv) > 1 else SRC))
    c = next(c for c in doc["cases"] if c["name"] == "gemma3-4b-local")
    out = {"source": "crates/reng-model/testdata/rope_reference.json, case gemma3-4b-local",
           "generated_by": doc["generated_by"], "transformers": doc["transformers"], "torch": doc["torch"],
           "theta": 10000.0, "head_dim": c["head_dim"], "rotary_dim": c["rotary_dim"], "table_len": c["table_len"],
           "attention_factor": c["attention_factor"], "inv_freq": c["inv_freq"], "positions": c["positions"],
           "cos": c["cos"], "sin": c["sin"]}
    with open(OUT, "w") as f:
        json.dump(out, f, separators=(",", ":"))


if __name__ == "__main__":
    main()
