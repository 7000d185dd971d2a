"""Write tests/golden/golden.json from the pinned CPU oracle.

Run from the repo root after the oracle pins pass (tests/test_oracle_pins.py):
    python tests/golden/make_golden.py

For every benchmark configuration it records the SHA-256 of the generated
weights and activations (so generator drift is caught), the oracle's output
bits for the first rows, and the SHA-256 of the oracle's full output.  The
reference (Rust) cannot run here; the oracle is the fixture source.
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "vitni-tensor_amd")]

import oracle  # noqa: E402
from vtq import synth  # noqa: E402

HEAD_ROWS = 8


def sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    threads = min(os.cpu_count() or 1, 16)
    out = {"generator": "vtq_synth SplitMix64 v1", "configs": {}}
    for name, cfg in synth.CONFIGS.items():
        t0 = time.time()
        x, w = cfg.make()
        y = oracle.linear_dispatch(cfg.ggml_type, 0, x, w, cfg.batch, cfg.in_feat, cfg.out_feat, threads)
        y2 = y.reshape(cfg.batch, cfg.out_feat)
        out["configs"][name] = {
            "ggml_type": cfg.ggml_type,
            "out_feat": cfg.out_feat,
            "in_feat": cfg.in_feat,
            "batch": cfg.batch,
            "w_sha256": sha(w),
            "x_sha256": sha(x),
            "y_sha256": sha(y),
            "y_head_bits": [f"{v:08x}" for v in y2[0, :HEAD_ROWS].view(np.uint32).tolist()],
            "y_last_bits": [f"{v:08x}" for v in y2[-1, -HEAD_ROWS:].view(np.uint32).tolist()],
        }
        print(f"{name}: {time.time() - t0:.1f}s", flush=True)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print("wrote", path)


if __name__ == "__main__":
    main()
