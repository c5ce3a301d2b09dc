"""Build libdsx.so in-tree with hipcc for gfx950.

    python -m distributedspeed_amd.build

The flags that matter for correctness:
  -ffp-contract=off   no implicit fused multiply-adds: each operation rounds
                      where torch's kernels round (explicit fmaf only)
  -Xclang -target-feature -Xclang -packed-fp32-ops
                      no packed fp32 instructions (v_pk_*_f32)
HIP's defaults keep fp32 division and sqrt correctly rounded and fp32
denormals intact, which the element math relies on.
"""
from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SRC = os.path.join(HERE, "csrc", "dsx_step.hip")
INCLUDE = os.path.join(ROOT, "include")
OUT = os.path.join(HERE, "libdsx.so")
ARCH = os.environ.get("DSX_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc"), "hipcc"):
        if os.path.sep not in cand or os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def command(out: str = OUT, extra: list[str] | None = None) -> list[str]:
    return [hipcc(), f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared",
            "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wall", "-Wno-unused-function",
            f"-I{INCLUDE}", SRC, "-o", out] + list(extra or [])


def build(out: str = OUT, verbose: bool = False) -> str:
    cmd = command(out)
    tmp = out + ".tmp"
    cmd[cmd.index(out)] = tmp
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    noise = [ln for ln in (res.stderr or "").splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(noise))
    if verbose and noise:
        print("\n".join(noise), file=sys.stderr)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
