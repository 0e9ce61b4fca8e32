"""Writes tests/golden/golden.json: seeded GGUF blocks with their f32 decode
and small GEMVs with their f64 products, produced by the oracle (whose
correctness tests/test_oracle.py pins) so that device tests and later oracle
changes are checked against frozen vectors.

    python tests/golden/make_golden.py
"""
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from runtimed_amd import synth  # noqa: E402

DEQUANT = [  # (name, qtype, n, k)
    ("q8_0", 8, 2, 128), ("q4_0", 2, 2, 128), ("q5_0", 6, 2, 128),
    ("q4_k_k896", 12, 2, 896), ("q5_k", 13, 2, 512), ("q6_k_k384", 14, 2, 384),
]
GEMV = [("q8_0", 8, 16, 896), ("q4_k", 12, 6, 896), ("q6_k", 14, 8, 384)]


def hexs(a: np.ndarray) -> str:
    return np.ascontiguousarray(a).tobytes().hex()


def main():
    out = {"dequant": [], "gemv": []}
    for i, (name, qt, n, k) in enumerate(DEQUANT):
        blocks = synth.weight_blocks(qt, 4242 + i, n, k)
        rc, y = oracle.dequant_tensor(qt, blocks, n * k)
        assert rc == 0
        out["dequant"].append({"name": name, "qtype": qt, "n": n, "k": k, "blocks": hexs(blocks),
                               "out_f32": hexs(y)})
    for i, (name, qt, n, k) in enumerate(GEMV):
        blocks = synth.weight_blocks(qt, 777 + i, n, k)
        rc, wf = oracle.dequant_tensor(qt, blocks, n * k)
        x = synth.activations(900 + i, 1, k)
        y = oracle.linear_f64(x, wf.reshape(n, k))
        out["gemv"].append({"name": name, "qtype": qt, "n": n, "k": k, "blocks": hexs(blocks),
                            "x_f32": hexs(x), "y_f64": hexs(y)})
    path = Path(__file__).with_name("golden.json")
    path.write_text(json.dumps(out, indent=1) + "\n")
    print(f"wrote {path} ({path.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
