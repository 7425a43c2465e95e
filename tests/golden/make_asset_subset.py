"""Writes tests/golden/oal_qwen_asset_subset.json: layers 0, 7 and 12 of the
reference's released group asset (configs/oal_qwen_n4096.json), unchanged, as a
data fixture for the asset loader tests.

Layer 0 (max_groups 4) has 8 heads with non-zero entries past the active factor
length, layer 7 (max_groups 5) has group counts 2..5, layer 12 has max_groups 2.
Run in the build container only (the reference is not on the GPU box):
    python tests/golden/make_asset_subset.py /root/reference/configs/oal_qwen_n4096.json
"""

import json
import os
import sys

LAYERS = (0, 7, 12)


def main(src: str) -> None:
    with open(src) as fh:
        data = json.load(fh)
    out = {k: v for k, v in data.items() if k not in ("layers", "layer_ids_zero_based")}
    out["layer_ids_zero_based"] = list(LAYERS)
    out["layers"] = {str(i): data["layers"][str(i)] for i in LAYERS}
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "oal_qwen_asset_subset.json")
    with open(dst, "w") as fh:
        json.dump(out, fh, separators=(",", ":"))
    print(dst, os.path.getsize(dst))


if __name__ == "__main__":
    main(sys.argv[1])
