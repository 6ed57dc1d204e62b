"""Extracts the MoE layer of the reference's DeepSeek-V4 tiny oracle fixture
(tests/fixtures/deepseek_v4_tiny_oracle.json: one hash-routed MoE layer, hidden 2, 3 F32
experts, top-2, routed_scaling_factor 1.5, swiglu_limit 10) into deepseek_v4_tiny_moe.json.

The values are copied as they are (inputs and expected outputs); nothing is recomputed.  Run
from the repository root in a tree where the reference sits at /root/reference.
"""

import json
import os
import sys

SRC = "/root/reference/tests/fixtures/deepseek_v4_tiny_oracle.json"
DST = os.path.join(os.path.dirname(os.path.abspath(__file__)), "deepseek_v4_tiny_moe.json")

KEEP_GEOMETRY = ("hidden_size", "moe_intermediate_size", "n_routed_experts",
                 "num_experts_per_tok", "routed_scaling_factor", "swiglu_limit", "vocab_size")
KEEP_EXPECTED = ("ffn_input", "router_logits", "routes", "routed_experts", "shared_expert",
                 "moe_branch")


def main() -> int:
    with open(SRC) as f:
        src = json.load(f)
    weights = {name: value for name, value in src["weights"].items()
               if name.startswith("layers.0.ffn.")}
    out = {
        "source": "tests/fixtures/deepseek_v4_tiny_oracle.json (MoE layer subset)",
        "generator": src["generator"],
        "token": src["token"],
        "geometry": {k: src["geometry"][k] for k in KEEP_GEOMETRY},
        "weights": weights,
        "expected": {k: src["expected"][k] for k in KEEP_EXPECTED},
    }
    with open(DST, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(f"wrote {DST}: {len(weights)} tensors")
    return 0


if __name__ == "__main__":
    sys.exit(main())
