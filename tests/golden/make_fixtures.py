"""Regenerates the committed fixtures under tests/golden/.

1. Copies the reference's own golden data files for the path's two math
   primitives (tests/golden/rope_*.bin and softmax_*.bin of the reference,
   produced by HF transformers 4.44.2 / torch 2.2.2, consumed by
   tests/ops_test.cpp:31-53) and records their shapes and sha256 in
   manifest.json. These are data, not code.
2. Writes kv_ring_cases.json: the case matrix of tests/kv_ring_test.cpp:90-97.
3. Writes spec_merge_cases.json: the direct merge vectors of
   tests/speculative_test.cpp:104-133.
4. Writes argmax_cases.json: the greedy argmax vectors of
   tests/sample_test.cpp:38-50.

Run from the repository root with the reference checkout mounted:
    python tests/golden/make_fixtures.py [/root/reference]
"""
from __future__ import annotations

import hashlib
import json
import os
import shutil
import sys

HERE = os.path.dirname(os.path.abspath(__file__))

# name -> (shape, tolerance the reference test applies)
TENSORS = {
    "rope_q_in": [14, 6, 64],
    "rope_q_out": [14, 6, 64],
    "rope_k_in": [2, 6, 64],
    "rope_k_out": [2, 6, 64],
    "softmax_in": [8, 512],
    "softmax_out": [8, 512],
}

KV_RING_CASES = [  # (n_sink, window, n_seen), kv_ring_test.cpp:90-97
    [4, 8, 40], [4, 8, 12], [4, 8, 11], [0, 8, 40], [1, 4, 40], [4, 8, 4], [4, 8, 2], [4, 8, 100],
]

SPEC_MERGE_CASES = [  # speculative_test.cpp:104-133: draft, target, accepted, merged
    {"draft": [10, 20, 30], "target": [10, 20, 30, 40], "accepted": 3, "out": [10, 20, 30, 40]},
    {"draft": [10, 99, 30], "target": [10, 20, 30, 40], "accepted": 1, "out": [10, 20]},
    {"draft": [5, 6], "target": [9, 8, 7], "accepted": 0, "out": [9]},
]

ARGMAX_CASES = [  # sample_test.cpp:38-50: logits, expected index
    {"logits": [0.1, 0.9, 0.3, -1.0], "index": 1},
    {"logits": [5.0, 1.0, 5.0, 5.0], "index": 0},
    {"logits": [-3.0, -2.0, -2.0], "index": 1},
    {"logits": [42.0], "index": 0},
]


def main(ref: str) -> None:
    src = os.path.join(ref, "tests", "golden")
    ref_manifest = json.load(open(os.path.join(src, "manifest.json")))
    by_name = {t["name"]: t for t in ref_manifest["tensors"]}
    out = {"source": "reference tests/golden (HF transformers fp32 outputs)",
           "provenance": ref_manifest.get("provenance", {}), "tensors": []}
    for name, shape in TENSORS.items():
        entry = by_name[name]
        assert entry["shape"] == shape, (name, entry["shape"])
        dst = os.path.join(HERE, entry["file"])
        shutil.copyfile(os.path.join(src, entry["file"]), dst)
        digest = hashlib.sha256(open(dst, "rb").read()).hexdigest()
        assert digest == entry["sha256"], f"{name}: sha256 mismatch"
        out["tensors"].append({"name": name, "file": entry["file"], "shape": shape,
                               "dtype": "f32", "sha256": digest})
    json.dump(out, open(os.path.join(HERE, "manifest.json"), "w"), indent=1)
    json.dump({"cases": KV_RING_CASES}, open(os.path.join(HERE, "kv_ring_cases.json"), "w"))
    json.dump({"cases": SPEC_MERGE_CASES},
              open(os.path.join(HERE, "spec_merge_cases.json"), "w"), indent=1)
    json.dump({"cases": ARGMAX_CASES}, open(os.path.join(HERE, "argmax_cases.json"), "w"),
              indent=1)
    print("fixtures written to", HERE)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
