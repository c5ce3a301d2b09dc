"""Writes tests/golden/adamw_torch_gpu.npz on a machine with an MI355X:

    python tests/golden/make_golden_gpu.py [--out PATH]

torch.optim.AdamW with torch's default dispatch -- on GPU tensors the
multi-tensor path, torch/optim/adam.py:554-800, which is what the reference's
stages get from optimizer.step() (Src/zero/stage1.py:522-525,
Src/zero/stage2.py:609-612) -- run on the GPU over the same parameters,
grads (exactly representable in bf16, with 0, -0, 1e-20 and 65504 among
them) and four hyper-parameter sets as adamw_torch_cpu.npz, 5 steps from
zero state. Records the torch version and the device name.
"""
from __future__ import annotations

import argparse
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from make_golden import adamw_fixture  # noqa: E402


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--out", default=os.path.join(HERE, "adamw_torch_gpu.npz"))
    a = ap.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("needs a GPU")
    np.savez_compressed(a.out, **adamw_fixture(device="cuda", foreach=None))
    print("wrote", a.out)


if __name__ == "__main__":
    main()
