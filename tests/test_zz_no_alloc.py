"""dsx_zero_step_flat_noalloc (the flat step with its scratch in the
library's static device array) against dsx_zero_step_flat (caller-supplied
scratch), both through the C ABI on the same inputs: master, exp_avg,
exp_avg_sq, param16, the device state and the step scalars bit-identical,
over consecutive calls whose second partition is smaller than the first (so
the scratch still holds the first call's larger set of partials), and a
third call whose grads hold an inf (the skip path)."""
from __future__ import annotations

import ctypes
import sys

import numpy as np
import pytest

from helpers import BF16, F16, f32_to_torch, make_state, np16_to_torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class _Side:
    """One copy of a partition and its device state."""

    def __init__(self, gpu, p, m, v, p16, g16, dt, scaler):
        import torch
        from distributedspeed_amd import ops
        self.p, self.m, self.v = (f32_to_torch(a, gpu) for a in (p, m, v))
        self.p16 = np16_to_torch(p16, dt, gpu)
        self.g = np16_to_torch(g16, dt, gpu)
        self.state = ops.new_state(gpu, scaler.init_scale if scaler.mode != "none" else 1.0,
                                   scaler.hysteresis if scaler.mode == "dynamic" else 1)
        self.out = torch.zeros(ops.SCALARS_BYTES, dtype=torch.uint8, device=gpu)

    def host(self, n):
        import torch
        return [self.p[:n].cpu().numpy().view(np.uint32), self.m[:n].cpu().numpy().view(np.uint32),
                self.v[:n].cpu().numpy().view(np.uint32),
                self.p16[:n].cpu().view(torch.int16).numpy(), self.state.cpu().numpy()]


def _args(side, n, dt, scaler, hyper, bc, stream):
    return (_ptr(side.p), _ptr(side.m), _ptr(side.v), _ptr(side.p16), dt, _ptr(side.g), dt, ctypes.c_int64(n),
            _ptr(side.state), scaler.to_c(), hyper.to_c(), _ptr(bc.table), bc.length)


@pytest.mark.parametrize("dt", [F16, BF16])
def test_noalloc_step_matches_caller_scratch_step(gpu, dt):
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    from oracle import oracle as O

    n1, n2 = 3_000_017, 1_200_003  # the second call's partition is smaller
    scale = 2.0 ** 16 if dt == F16 else 1.0
    scaler = (ScalerConfig(mode="dynamic", init_scale=scale, window=1000, hysteresis=1) if dt == F16
              else ScalerConfig(mode="none"))
    hyper = AdamWHyper(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    p, m, v, g16 = make_state(n1, seed=77 + dt, gdt=dt, g_sigma=1e-3, scale=scale)
    p16 = O.cast16(p, dt)
    a = _Side(gpu, p, m, v, p16, g16, dt, scaler)  # dsx_zero_step_flat
    b = _Side(gpu, p, m, v, p16, g16, dt, scaler)  # dsx_zero_step_flat_noalloc
    bc = BiasCorrectionTable(gpu, hyper.beta1, hyper.beta2)
    stream = ops.stream_of(gpu)

    calls = [(n1, False, False), (n2, True, False), (n2, True, True)]  # (n, pass out, inject inf)
    for k, (n, pass_out, inf) in enumerate(calls):
        if inf:
            for side in (a, b):
                side.g[n // 3] = float("inf")
        nparts = ops.suggest_partials(n)
        partials = torch.zeros(nparts, dtype=torch.float64, device=gpu)
        _say(f"noalloc dt={dt} call={k} n={n} nparts={nparts} out={'caller' if pass_out else 'scratch'} inf={inf}")
        _lib.call("dsx_zero_step_flat", *_args(a, n, dt, scaler, hyper, bc, stream), _ptr(partials), nparts,
                  _ptr(a.out), stream)
        _lib.call("dsx_zero_step_flat_noalloc", *_args(b, n, dt, scaler, hyper, bc, stream), nparts,
                  _ptr(b.out) if pass_out else None, stream)
        torch.cuda.synchronize()
        for name, x, y in zip(("master", "exp_avg", "exp_avg_sq", "param16", "state"), a.host(n1), b.host(n1)):
            assert np.array_equal(x, y), f"call {k}: {name} differs ({(x != y).sum()} elements)"
        if pass_out:
            assert np.array_equal(a.out.cpu().numpy(), b.out.cpu().numpy()), f"call {k}: step scalars differ"
        st = ops.read_state(b.state)
        assert st.error == 0
        assert st.last_skip == (1 if inf else 0)
    assert ops.read_state(b.state).t == 2


def test_noalloc_picks_partials_and_rejects_oversize(gpu):
    """nparts = 0 takes the library's partial count (the same bits as passing
    it); a count above the scratch is refused before anything is launched."""
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    from oracle import oracle as O

    n, dt = 500_001, BF16
    scaler = ScalerConfig(mode="none")
    hyper = AdamWHyper(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, max_grad_norm=0.0)
    p, m, v, g16 = make_state(n, seed=5, gdt=dt, g_sigma=1e-3)
    p16 = O.cast16(p, dt)
    a = _Side(gpu, p, m, v, p16, g16, dt, scaler)
    b = _Side(gpu, p, m, v, p16, g16, dt, scaler)
    bc = BiasCorrectionTable(gpu, hyper.beta1, hyper.beta2)
    stream = ops.stream_of(gpu)
    with pytest.raises(_lib.DsxError, match="exceeds the library scratch"):
        _lib.call("dsx_zero_step_flat_noalloc", *_args(b, n, dt, scaler, hyper, bc, stream),
                  _lib.DSX_NOALLOC_MAX_PARTIALS + 1, None, stream)
    _say(f"noalloc nparts=0 n={n}")
    _lib.call("dsx_zero_step_flat_noalloc", *_args(b, n, dt, scaler, hyper, bc, stream), 0, None, stream)
    nparts = ops.suggest_partials(n)
    partials = torch.zeros(nparts, dtype=torch.float64, device=gpu)
    _lib.call("dsx_zero_step_flat", *_args(a, n, dt, scaler, hyper, bc, stream), _ptr(partials), nparts,
              _ptr(a.out), stream)
    torch.cuda.synchronize()
    for name, x, y in zip(("master", "exp_avg", "exp_avg_sq", "param16", "state"), a.host(n), b.host(n)):
        assert np.array_equal(x, y), f"{name} differs"


def test_noalloc_step_matches_on_every_launch_form(gpu):
    """The same comparison over the step's three launch forms: above the
    fold's bound (K0 folded into the first of K2's two parts, the second part
    reading its records; once with an inf in the second part, so the skip is
    decided in the first part's launch), more partials than the fold takes
    (K1, K0, K2 as three launches, K0's scalars in the library scratch), and
    a partition the fold takes whole. fp16 grads with the dynamic scaler."""
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    from oracle import oracle as O

    dt = F16
    big, small = 70_000_001, 3_000_017  # big: two K2 parts of 2^26 elements at most
    scaler = ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, window=1000, hysteresis=1)
    hyper = AdamWHyper(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, max_grad_norm=1.0)
    p, m, v, g16 = make_state(big, seed=91, gdt=dt, g_sigma=1e-3, scale=2.0 ** 16)
    p16 = O.cast16(p, dt)
    a = _Side(gpu, p, m, v, p16, g16, dt, scaler)
    b = _Side(gpu, p, m, v, p16, g16, dt, scaler)
    del p, m, v, p16, g16
    bc = BiasCorrectionTable(gpu, hyper.beta1, hyper.beta2)
    stream = ops.stream_of(gpu)
    # (n, nparts (0: suggested), pass out, put an inf into the second part)
    calls = [(big, 0, True, False), (big, 0, False, True), (small, 1024, False, False), (small, 0, True, False)]
    skips = 0
    for k, (n, nparts, pass_out, inf) in enumerate(calls):
        if inf:
            for side in (a, b):
                side.g[3 * n // 4] = float("inf")
            skips += 1
        nparts = nparts or ops.suggest_partials(n)
        partials = torch.zeros(nparts, dtype=torch.float64, device=gpu)
        _say(f"noalloc forms call={k} n={n} nparts={nparts} out={'caller' if pass_out else 'scratch'} inf={inf}")
        _lib.call("dsx_zero_step_flat", *_args(a, n, dt, scaler, hyper, bc, stream), _ptr(partials), nparts,
                  _ptr(a.out), stream)
        _lib.call("dsx_zero_step_flat_noalloc", *_args(b, n, dt, scaler, hyper, bc, stream), nparts,
                  _ptr(b.out) if pass_out else None, stream)
        torch.cuda.synchronize()
        for name, x, y in zip(("master", "exp_avg", "exp_avg_sq", "param16", "state"), a.host(big), b.host(big)):
            assert np.array_equal(x, y), f"call {k}: {name} differs ({(x != y).sum()} elements)"
        if pass_out:
            assert np.array_equal(a.out.cpu().numpy(), b.out.cpu().numpy()), f"call {k}: step scalars differ"
        st = ops.read_state(b.state)
        assert st.error == 0
        assert st.last_skip == (1 if inf else 0)
    st = ops.read_state(b.state)
    assert st.t == len(calls) - skips
    assert st.scale == 2.0 ** 15  # halved once, by the skipped step
