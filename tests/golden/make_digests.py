"""Writes tests/golden/config0_mlp_digests.json.

    python tests/golden/make_digests.py

configs[0]'s 1,863,690-element MLP partition (fp16, static loss scale
2^16, no clip, lr 1e-4, betas (0.9, 0.999), eps 1e-8, weight decay 0.01)
stepped ten times through the oracle from seeded inputs (tests/helpers.py
MLP_CASE), and the SHA-256 of master, exp_avg, exp_avg_sq and param16 after
every step. A regression anchor rather than an independent pin: the
oracle's element math is pinned against torch elsewhere
(tests/test_oracle_*.py); these digests then hold the oracle and the GPU
step (tests/test_gpu_parity.py::test_config1_mlp_ten_steps) to the same
bits from one change to the next.
"""
from __future__ import annotations

import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from helpers import MLP_CASE, mlp_case_oracle_digests  # noqa: E402
from oracle import oracle as O  # noqa: E402


def main() -> None:
    out = {"case": {k: v for k, v in MLP_CASE.items()}, "digests": mlp_case_oracle_digests(O)}
    path = os.path.join(HERE, "config0_mlp_digests.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
