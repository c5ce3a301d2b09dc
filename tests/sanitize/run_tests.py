"""Runs CPU tests in this process against a sanitized build (run.sh preloads
the matching ASan runtime): `libdsx <path>` -> the ABI and host-logic tests
and the chunk-table fuzz with libdsx.so loaded from <path>; `oracle <path>` ->
the oracle tests with the C oracle loaded from <path>."""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
TESTS = os.path.join(ROOT, "tests")


def main() -> int:
    which, path = sys.argv[1], os.path.abspath(sys.argv[2])
    args = ["-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider"]
    if which == "libdsx":
        from distributedspeed_amd import _lib
        _lib.load(path)  # cached: every test's _lib.load() returns this build
        files = ["test_abi_cpu.py", "test_host_logic.py"]
    elif which == "oracle":
        from oracle import oracle as O
        O._LIB_PATH = path
        O.lib()
        files = ["test_oracle_adamw.py", "test_oracle_casts_norm.py", "test_oracle_scaler.py"]
    else:
        raise SystemExit(f"unknown target {which!r}")
    return pytest.main(args + [os.path.join(TESTS, f) for f in files])


if __name__ == "__main__":
    sys.exit(main())
