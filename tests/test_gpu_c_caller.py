"""The C ABI from a plain C program, with no Python or torch in its process.

tests/c_abi/dsx_c_caller.c (built by build(), `make -C tests/c_abi`) is what
a C or C++ host would write against include/dsx.h: hipMalloc'd buffers,
dsx_state_init, the bias-correction table computed on its own host in
double, one dsx_zero_step_flat per step on a stream it created, and the
same steps through dsx_zero_step_flat_noalloc on a second copy. It writes
its inputs and results; here they are compared with the oracle, step by
step for the state and bit for bit for master, exp_avg, exp_avg_sq and
param16 at the end, for each form dsx_zero_step_flat takes:
- two launches, K1 and K2 with K0's finalize folded in (fp16, dynamic loss
  scale, configs[0]'s size, below the fold's 3 * 2^23-element bound);
- fold-first (bf16, above that bound: K1, then K0 folded into the first of
  K2's parts, then the other parts);
- three launches, K1 -> K0 -> K2 (the same bf16 partition with the fold
  switched off through dsx_set_tuning_fold(0)).
Step 1 holds an inf (skipped, scale backed off); the window of 2 makes the
scale grow."""
from __future__ import annotations

import os
import subprocess
import sys

import numpy as np
import pytest

from helpers import BF16, F16

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "c_abi", "dsx_c_caller")
STEPS = 4


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


@pytest.mark.parametrize("n,dt,fold", [(1_863_690, F16, None), (26_000_003, BF16, None), (26_000_003, BF16, 0)],
                         ids=["fp16-two-launch", "bf16-fold-first", "bf16-three-launch"])
def test_c_program_matches_oracle(gpu, oracle, tmp_path, n, dt, fold):
    from distributedspeed_amd import _lib
    O = oracle
    if not os.path.exists(EXE):
        pytest.fail(f"{EXE} is not built: run build() (make -C tests/c_abi)")
    _say(f"C caller n={n} dt={dt} fold={fold}")
    args = [EXE, str(n), str(dt), str(STEPS), str(tmp_path)] + ([] if fold is None else [str(fold)])
    r = subprocess.run(args, capture_output=True, text=True, timeout=240)
    assert r.returncode == 0, f"status {r.returncode}: {r.stderr[-2000:]}"
    assert "noalloc identical" in r.stdout

    rd = lambda name, t: np.fromfile(os.path.join(tmp_path, name), dtype=t)  # noqa: E731
    master0 = rd("master0.f32", np.float32)
    grads = rd("grads.u16", np.uint16).reshape(STEPS, n)
    states = [_lib.DsxState.from_buffer_copy(b) for b in rd("states.bin", np.uint8).reshape(STEPS, 64)]
    fp16 = dt == F16
    p = master0.copy()
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    p16 = O.cast16(p, dt)
    orc = O.ZeroStepOracle(p, m, v, p16, dt, dt,
                           O.Hyper(lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, max_grad_norm=1.0),
                           O.LossScalerSpec(scale=4096.0, window=2, hysteresis=1) if fp16
                           else O.LossScalerSpec(scale=1.0, dynamic=False))
    for k in range(STEPS):
        res = orc.step(grads[k])
        st = states[k]
        assert bool(st.last_skip) == res.skipped == (k == 1), k
        assert st.scale == res.scale_next, (k, st.scale, res.scale_next)
        assert st.t == orc.t and st.error == 0, k
        assert abs(st.last_norm - res.norm) <= 1e-12 * res.norm or (res.skipped and not np.isfinite(st.last_norm))
    for name, suffix, ref in (("master", "f32", orc.p), ("exp_avg", "f32", orc.m), ("exp_avg_sq", "f32", orc.v)):
        got = rd(f"{name}.{suffix}", np.uint32)
        assert np.array_equal(got, ref.view(np.uint32)), f"{name}: {(got != ref.view(np.uint32)).sum()} differ"
    assert np.array_equal(rd("param16.u16", np.uint16), orc.p16)
    if fp16:  # backed off at the inf, then grew after two clean steps
        assert states[-1].scale == 4096.0
