"""Writes tests/golden/generator_hashes.json: sha256 of the first 4 KiB of
the synthetic quantized weights for a few small seeded shapes, so a change
in the generator or the quantizers is caught.  Run after an intended change:
    python tests/golden/make_generator_hashes.py
"""
import hashlib
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from conftest import load_pkg  # noqa: E402

ENTRIES = [
    (2, 0x5EED ^ (1 << 32) ^ 0, 0.02, 16, 4096),
    (2, 0x5EED ^ (2 << 32) ^ 3, 0.02, 8, 14336),
    (12, 0x5EED ^ (3 << 32) ^ 1, 0.02, 16, 4096),
    (8, 0x5EED ^ (3 << 32) ^ 4, 0.02, 16, 4096),
    (12, 0x5EED ^ (5 << 32) ^ 2, 0.015, 4, 8192),
    (14, 0x5EED ^ (7 << 32) ^ 5, 0.02, 16, 4096),
]


def main():
    pkg = load_pkg()
    out = []
    for dt, seed, sigma, rows, cols in ENTRIES:
        raw = pkg.synth_quantized(dt, seed, sigma, rows, cols)
        out.append({"dtype": dt, "seed": str(seed), "sigma": sigma, "rows": rows, "cols": cols,
                    "sha256": hashlib.sha256(raw[:4096].tobytes()).hexdigest()})
    with open(os.path.join(HERE, "generator_hashes.json"), "w") as f:
        json.dump({"entries": out}, f, indent=1)


if __name__ == "__main__":
    main()
