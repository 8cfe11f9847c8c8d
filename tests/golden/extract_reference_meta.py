"""Copies the reference's published known answers for this path into a fixture.

Run in the build container (reads /root/reference, which the GPU box lacks):

    python tests/golden/extract_reference_meta.py

Writes tests/golden/reference_meta.json with data only:
  * golden_8f_intra : per-frame mean/std of the fp32 golden attention of the
                      8-frame seed-42 synthetic trace, max softmax row-sum
                      error (reference: traces/golden_meta.json)
  * trace_8f        : seed, tile regime counts and first-vs-last cosine stats
                      of that trace (reference: traces/trace_meta_8f.json)
  * grounding       : budget / tile-size numbers of the capacity scenario
                      (reference: configs/grounding_config.json)
"""

import json
from pathlib import Path

REF = Path("/root/reference")
OUT = Path(__file__).with_name("reference_meta.json")


def main():
    golden = json.loads((REF / "traces" / "golden_meta.json").read_text())
    trace = json.loads((REF / "traces" / "trace_meta_8f.json").read_text())
    cfg = json.loads((REF / "configs" / "grounding_config.json").read_text())
    out = {
        "golden_8f_intra": {
            "source_seed": golden["source_seed"],
            "output_shape": golden["output_shape"],
            "max_softmax_rowsum_error": golden["max_softmax_rowsum_error"],
            "per_frame_stats": golden["per_frame_stats"],
        },
        "trace_8f": {
            "seed": trace["seed"],
            "frames": trace["frames"],
            "frac_static_requested": trace["frac_static_requested"],
            "tiles": trace["tiles"],
            "validation_cosine_first_vs_last": trace["validation_cosine_first_vs_last"],
        },
        "grounding": {
            "max_persisting_l2_bytes": cfg["persistence_budget"]["max_persisting_l2_bytes"],
            "kv_tile_bytes": cfg["persistence_budget"]["kv_tile_bytes"],
            "tiles_fully_persistable": cfg["persistence_budget"]["tiles_fully_persistable"],
            "access_policy_max_window_bytes": cfg["gpu"]["access_policy_max_window_bytes"],
            "tokens_per_frame": cfg["model"]["tokens_per_frame"],
            "tile_size_tokens": cfg["model"]["tile_size_tokens"],
            "hidden_dim": cfg["model"]["hidden_dim"],
            "heads": cfg["model"]["heads"],
            "head_dim": cfg["model"]["head_dim"],
            "tiles_per_frame": cfg["kv_derivation"]["tiles_per_frame"],
        },
    }
    OUT.write_text(json.dumps(out, indent=1))
    print(f"-> {OUT}")


if __name__ == "__main__":
    main()
