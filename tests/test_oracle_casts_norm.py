"""Pins the oracle's 16-bit conversions and its norm / overflow detection.

Casts: numpy's float16 conversion (IEEE binary16, round to nearest even) and
torch's bfloat16 conversion (c10::BFloat16, round to nearest even, NaN ->
0x7FC0) over every 16-bit value, every rounding tie between neighbours and a
random sample of fp32 bit patterns.
Norm: an fp64 brute force with numpy, a second summation order, and
torch.linalg.vector_norm; found_inf against torch's
_amp_foreach_non_finite_check_and_unscale_ (the op GradScaler.unscale_ runs,
torch/amp/grad_scaler.py:235-286).
Clip: the closed form of Src/zero/utils.py:211-214.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch


def _all16():
    return np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)


def test_widen_f16_every_value(oracle):
    h = _all16()
    got = oracle.widen16(h, oracle.F16)
    ref = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_widen_bf16_every_value(oracle):
    h = _all16()
    got = oracle.widen16(h, oracle.BF16)
    ref = torch.from_numpy(h.view(np.int16)).view(torch.bfloat16).float().numpy()
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def _probe_f32_for(dt, oracle):
    """fp32 values at, just below and just above every midpoint between
    adjacent finite 16-bit values, plus every 16-bit value itself."""
    h = _all16()
    w = oracle.widen16(h, dt).astype(np.float64)
    fin = np.isfinite(w)
    vals = np.sort(np.unique(w[fin]))
    mids = (vals[:-1] + vals[1:]) / 2
    mids32 = mids.astype(np.float32)
    cand = [vals.astype(np.float32), mids32, np.nextafter(mids32, np.float32(np.inf)),
            np.nextafter(mids32, np.float32(-np.inf))]
    # around the overflow threshold and into fp32 subnormals / specials
    extra = np.array([65504.0, 65519.996, 65520.0, 65536.0, 1e30, 3.4e38, np.inf, -np.inf, np.nan, 0.0, -0.0,
                      1e-45, 2.98e-8, 2.9802322e-08, 5.96e-8, 1e-40, -1e-40], np.float32)
    rng = np.random.default_rng(0)
    rnd = rng.integers(0, 1 << 32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    return np.concatenate(cand + [extra, rnd])


def test_cast_f16_matches_numpy(oracle):
    x = _probe_f32_for(oracle.F16, oracle)
    got = oracle.cast16(x, oracle.F16)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert ((got[nan] & 0x7FFF) == 0x7E00).all()


def test_cast_bf16_matches_torch(oracle):
    x = _probe_f32_for(oracle.BF16, oracle)
    got = oracle.cast16(x, oracle.BF16)
    ref = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], ref[~nan])
    assert (got[nan] == 0x7FC0).all()


@pytest.mark.parametrize("dt", [1, 2])
def test_sumsq_against_fp64_brute_force(oracle, dt):
    rng = np.random.default_rng(5)
    n = 1_000_003
    scale = 2.0 ** 16 if dt == 1 else 1.0
    g16 = oracle.cast16((rng.standard_normal(n) * 1e-3 * scale).astype(np.float32), dt)
    inv = oracle.inv_scale_of(scale)
    g = oracle.widen16(g16, dt).astype(np.float64) * inv
    ref = math.fsum((g * g).tolist())  # correctly rounded sum of the exact squares
    got = oracle.sumsq(g16, dt, inv)
    assert got == pytest.approx(ref, rel=1e-15)
    assert oracle.sumsq(g16, dt, inv, blocks=1021) == pytest.approx(ref, rel=1e-13)
    tn = torch.linalg.vector_norm(torch.from_numpy(oracle.widen16(g16, dt) * np.float32(inv)).double())
    assert math.sqrt(got) == pytest.approx(float(tn), rel=1e-13)


@pytest.mark.parametrize("n,blocks", [(1_000_003, 1021), (5, 16), (0, 8), (4097, 4096), (70_001, 9000)])
def test_parallel_blocked_sumsq_is_the_blocked_sum(oracle, n, blocks):
    """The OpenMP form used for the CPU-baseline timing adds the same block
    sums in the same order as the serial blocked form (blocks past the end,
    and more blocks than its cap of 4096, included), so it returns the same
    bits; and a non-finite grad still makes it non-finite."""
    rng = np.random.default_rng(n)
    g16 = oracle.cast16((rng.standard_normal(n) * 5e-4).astype(np.float32), oracle.BF16)
    serial = oracle.sumsq(g16, oracle.BF16, 1.0, blocks=min(blocks, 4096))
    par = oracle.sumsq_parallel(g16, oracle.BF16, 1.0, blocks)
    assert np.float64(par).view(np.uint64) == np.float64(serial).view(np.uint64)
    if n:
        g16[n // 3] = 0x7F80  # +inf
        assert not math.isfinite(oracle.sumsq_parallel(g16, oracle.BF16, 1.0, blocks))


@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
@pytest.mark.parametrize("pos", [0, 5, 1023, 1024])
def test_nonfinite_detection_matches_torch_unscale(oracle, bad, pos):
    n = 1025
    rng = np.random.default_rng(pos)
    g = (rng.standard_normal(n) * 1e-3 * 2 ** 16).astype(np.float32)
    g[pos] = bad
    g16 = oracle.cast16(g, oracle.F16)
    ss = oracle.sumsq(g16, oracle.F16, oracle.inv_scale_of(2.0 ** 16))
    t = [torch.from_numpy(g16.view(np.int16)).view(torch.float16).float()]
    found = torch.zeros(1)
    torch._amp_foreach_non_finite_check_and_unscale_(t, found, torch.tensor([2.0 ** -16]))
    assert (not math.isfinite(ss)) == bool(found.item()) == True  # noqa: E712


def test_unscale_power_of_two_is_exact(oracle):
    h = _all16()
    w = oracle.widen16(h, oracle.F16)
    fin = np.isfinite(w)
    inv = np.float32(oracle.inv_scale_of(2.0 ** 16))
    assert inv == np.float32(2.0 ** -16)
    assert np.array_equal((w[fin] * inv).astype(np.float64), w[fin].astype(np.float64) / 65536.0)


def test_clip_coefficient_closed_form(oracle):
    assert oracle.clip_coef(0.5, 1.0) == 1.0            # below the threshold: no clipping
    assert oracle.clip_coef(1.0, 1.0) == 1.0            # equal: not clipped (strict >)
    assert oracle.clip_coef(4.0, 1.0) == float(np.float32(1.0 / (4.0 + 1e-6)))
    assert oracle.clip_coef(4.0, 0.0) == 1.0            # max_norm <= 0 disables clipping
    # the clipped grad has norm max_norm * norm / (norm + 1e-6)
    g = np.array([3.0, 4.0], np.float32)
    c = np.float32(oracle.clip_coef(5.0, 1.0))
    assert float(np.linalg.norm((g * c).astype(np.float64))) == pytest.approx(5.0 / (5.0 + 1e-6), rel=1e-7)


# ---- clip_grad_norm_'s norm types (Src/zero/utils.py:126-154) ----------------------------

NORM_TYPES = [1.0, 2.0, 3.0, 0.5, 7.5, math.inf]


def _grads(oracle, n, dt, seed, scale):
    rng = np.random.default_rng(seed)
    g = (rng.standard_normal(n) * 1e-3 * scale).astype(np.float32)
    return g if dt == 0 else oracle.cast16(g, dt)


@pytest.mark.parametrize("p", NORM_TYPES)
@pytest.mark.parametrize("dt", [0, 1, 2])
def test_norm_p_against_torch_fp64(oracle, dt, p):
    """norm_p equals torch.linalg.vector_norm(ord=p) in fp64 over the same
    unscaled fp32 values (inf exactly: a maximum has no rounding)."""
    scale = 2.0 ** 10 if dt == 1 else 1.0
    g = _grads(oracle, 100_003, dt, 11 + dt, scale)
    inv = oracle.inv_scale_of(scale)
    x = oracle.unscaled(g, dt, inv)
    ref = float(torch.linalg.vector_norm(torch.from_numpy(x).double(), ord=p))
    got = oracle.norm_p(g, dt, inv, p)
    if math.isinf(p):
        assert got == ref
    else:
        assert got == pytest.approx(ref, rel=1e-13)


@pytest.mark.parametrize("p", NORM_TYPES)
def test_norm_p_against_the_reference_formula(oracle, p):
    """The reference's compute_norm restated with torch (Src/zero/utils.py:
    141-152): per tensor t.norm(p, dtype=float32).item() ** p summed in
    Python, then ** (1/p); for inf the max of t.abs().max(). torch
    accumulates each tensor in fp32, so agreement is to fp32 accuracy."""
    x = oracle.unscaled(_grads(oracle, 300_007, 2, 3, 1.0), 2, 1.0)
    pieces = [torch.from_numpy(c.copy()) for c in np.array_split(x, 7)]
    if math.isinf(p):
        ref = max(t.abs().max().item() for t in pieces)
        assert oracle.norm_p(oracle.cast16(x, 2), 2, 1.0, p) == ref
        return
    total = 0.0
    for t in pieces:
        total += (t.norm(dtype=torch.float32).item() ** 2 if p == 2.0
                  else t.norm(p=p, dtype=torch.float32).item() ** p)
    ref = total ** (1.0 / p)
    # the fp32 sums' relative error is multiplied by 1/p in the root
    assert oracle.norm_p(oracle.cast16(x, 2), 2, 1.0, p) == pytest.approx(ref, rel=2e-5 * max(1.0, 1.0 / p))


@pytest.mark.parametrize("p", NORM_TYPES)
def test_norm_p_closed_forms(oracle, p):
    """n equal magnitudes c of mixed sign: n^(1/p) * c (c for inf); a single
    nonzero element: its magnitude for every p; an inf anywhere: inf; a NaN
    anywhere: NaN; no elements or all zeros: 0."""
    n, c = 4096, np.float32(0.375)
    x = np.full(n, c, np.float32)
    x[::3] = -c
    want = float(c) if math.isinf(p) else n ** (1.0 / p) * float(c)
    assert oracle.norm_p(x, 0, 1.0, p) == pytest.approx(want, rel=1e-14)
    one = np.zeros(1000, np.float32)
    one[617] = -2.5
    assert oracle.norm_p(one, 0, 1.0, p) == pytest.approx(2.5, rel=1e-15)
    for bad, want_nan in ((np.inf, False), (-np.inf, False), (np.nan, True)):
        y = x.copy()
        y[100] = bad
        r = oracle.norm_p(y, 0, 1.0, p)
        assert math.isnan(r) if want_nan else r == math.inf
    assert oracle.norm_p(np.zeros(0, np.float32), 0, 1.0, p) == 0.0
    assert oracle.norm_p(np.zeros(77, np.float32), 0, 1.0, p) == 0.0


def test_norm_p_planted_mistakes_fail_the_pins(oracle):
    """Variants of norm_p with a plausible mistake -- no absolute value for an
    odd p, the loss scale not removed, 1/p not applied -- miss torch's fp64
    norm by far more than the 1e-13 the real one meets."""
    scale = 2.0 ** 10
    g = _grads(oracle, 50_001, 1, 4, scale)
    inv = oracle.inv_scale_of(scale)
    x = oracle.unscaled(g, 1, inv).astype(np.float64)
    ref = float(torch.linalg.vector_norm(torch.from_numpy(x), ord=3.0))
    assert oracle.norm_p(g, 1, inv, 3.0) == pytest.approx(ref, rel=1e-13)
    no_abs = abs(math.fsum(x ** 3)) ** (1 / 3)
    scaled = math.fsum(np.abs(oracle.widen16(g, 1).astype(np.float64)) ** 3) ** (1 / 3)
    no_root = math.fsum(np.abs(x) ** 3)
    for bad in (no_abs, scaled, no_root):
        assert abs(bad - ref) > 1e-3 * ref


def test_clip_once_coefficient_closed_form(oracle):
    """The explicit call clips iff norm > max_norm, with no max_norm > 0
    condition (Src/zero/utils.py:209-214): max_norm = 0 gives coefficient 0."""
    assert oracle.clip_once_coef(0.5, 1.0) == 1.0
    assert oracle.clip_once_coef(1.0, 1.0) == 1.0
    assert oracle.clip_once_coef(4.0, 1.0) == float(np.float32(1.0 / (4.0 + 1e-6)))
    assert oracle.clip_once_coef(4.0, 0.0) == 0.0
    assert oracle.clip_once_coef(math.inf, 1.0) == 0.0
    assert oracle.clip_once_coef(math.nan, 1.0) == 1.0  # NaN > max is false, as in Python
