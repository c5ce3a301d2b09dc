"""CPU oracle for the ZeRO optimizer step -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker. The product (distributedspeed_amd) never
imports it.

Parts and what pins each (tests/test_oracle_*.py):
  * element math (dsx_oracle.c, dsxo_adamw): torch.optim.AdamW(foreach=False)
    on CPU -- exp_avg / exp_avg_sq bit-exact, master within 1 ulp (torch's CPU
    sqrt is not correctly rounded); closed form of the first step; golden
    vectors in tests/golden/.
  * fp16/bf16 casts: numpy float16 and torch bfloat16 conversion over every
    16-bit pattern, every tie and a random sample.
  * norm (dsxo_sumsq): numpy float64 brute force and torch.linalg.vector_norm.
  * norms of type p (norm_p, clip_grad_norm_'s norm_type): torch's fp64
    vector_norm, the reference's per-tensor formula restated in torch, closed
    forms, and planted mistakes that must fail.
  * clip coefficients: the closed form of Src/zero/utils.py:211-214, for the
    configured clip (clip_coef) and the explicit call (clip_once_coef).
  * loss scaler (LossScalerSpec): torch._amp_update_scale_ for hysteresis=1,
    hand-derived sequences for hysteresis > 1 and min_loss_scale.
  * skip semantics: state bit-identical after a skipped step, t not advanced.

Reference algorithm followed: Src/zero/optimizer.py:212-274 (step order),
Src/zero/utils.py:126-154, 187-216 (norm, clip), Src/config.py:93-109 and
Src/zero/__init__.py:103-109 (scaler keys), torch/optim/adam.py:347-552
(AdamW arithmetic), torch/amp/grad_scaler.py:469-538 (scale update).
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from dataclasses import dataclass, field

import numpy as np

F32 = 0
F16 = 1
BF16 = 2

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libdsx_oracle.so")
_lib = None


class _Scalars(ctypes.Structure):
    _fields_ = [(name, ctypes.c_float) for name in
                ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2", "eps", "bc2s", "nss")]


def build() -> str:
    """Compile the C oracle in place (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        L.dsxo_sumsq.restype = ctypes.c_double
        L.dsxo_sumsq.argtypes = [P, ctypes.c_int, ctypes.c_int64, ctypes.c_float]
        L.dsxo_sumsq_blocked.restype = ctypes.c_double
        L.dsxo_sumsq_blocked.argtypes = [P, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_int64]
        L.dsxo_sumsq_parallel.restype = ctypes.c_double
        L.dsxo_sumsq_parallel.argtypes = [P, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_int64]
        L.dsxo_adamw.restype = None
        L.dsxo_adamw.argtypes = [P, P, P, P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int64,
                                 ctypes.POINTER(_Scalars)]
        L.dsxo_cast_f32.restype = None
        L.dsxo_cast_f32.argtypes = [P, P, ctypes.c_int, ctypes.c_int64]
        L.dsxo_widen.restype = None
        L.dsxo_widen.argtypes = [P, P, ctypes.c_int, ctypes.c_int64]
        L.dsxo_num_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray | None):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def _check(a: np.ndarray, dtype, n: int | None = None) -> None:
    if a.dtype != dtype or not a.flags.c_contiguous:
        raise TypeError(f"expected contiguous {dtype}, got {a.dtype}")
    if n is not None and a.size != n:
        raise ValueError(f"expected {n} elements, got {a.size}")


# ---- conversions ------------------------------------------------------------

def cast16(x: np.ndarray, dt: int) -> np.ndarray:
    """fp32 -> 16-bit storage (uint16), round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().dsxo_cast_f32(_ptr(x), _ptr(out), dt, x.size)
    return out


def widen16(h: np.ndarray, dt: int) -> np.ndarray:
    """16-bit storage (uint16) -> fp32, exact."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().dsxo_widen(_ptr(h), _ptr(out), dt, h.size)
    return out


# ---- norm -----------------------------------------------------------------------

def inv_scale_of(scale: float) -> float:
    """f32(1 / double(scale)), as GradScaler computes inv_scale
    (torch/amp/grad_scaler.py:303) and the static path's 1/loss_scale
    (Src/zero/optimizer.py:255)."""
    return float(np.float32(1.0 / float(np.float32(scale))))


def _gdtype(dt: int):
    return np.float32 if dt == F32 else np.uint16


def sumsq(g16: np.ndarray, dt: int, inv_scale: float, blocks: int = 0) -> float:
    """Sum of (f32(g) * inv_scale)^2 in fp64; g16 is uint16 storage for
    F16/BF16 or a float32 array for F32."""
    _check(g16, _gdtype(dt))
    if blocks:
        return lib().dsxo_sumsq_blocked(_ptr(g16), dt, g16.size, inv_scale, blocks)
    return lib().dsxo_sumsq(_ptr(g16), dt, g16.size, inv_scale)


def sumsq_parallel(g16: np.ndarray, dt: int, inv_scale: float, blocks: int = 1024) -> float:
    """sumsq(..., blocks=blocks) with the blocks summed on all OpenMP threads
    (bit-identical to it); for timing the oracle as a CPU baseline."""
    _check(g16, _gdtype(dt))
    return lib().dsxo_sumsq_parallel(_ptr(g16), dt, g16.size, inv_scale, blocks)


# ---- hyper-parameters and per-step scalars ---------------------------------------

@dataclass
class Hyper:
    lr: float = 1e-3
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 0.01
    max_grad_norm: float = 0.0
    clip_eps: float = 1e-6


def bias_corrections(beta1: float, beta2: float, t: int) -> tuple[float, float]:
    """(1 - beta1**t, (1 - beta2**t)**0.5) with t a Python float, exactly as
    torch/optim/adam.py:529-535 evaluates them (step = step_t.item())."""
    step = float(t)
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    return bc1, bc2 ** 0.5


def clip_coef(norm: float, max_norm: float, clip_eps: float = 1e-6) -> float:
    """Src/zero/utils.py:211-214: coefficient applied iff norm > max_norm
    (the configured max_grad_norm; 0 disables it)."""
    if max_norm > 0 and norm > max_norm:
        return float(np.float32(max_norm / (norm + clip_eps)))
    return 1.0


def unscaled(g16: np.ndarray, dt: int, inv_scale: float) -> np.ndarray:
    """f32(g) * f32(inv_scale), elementwise in fp32 (the unscale of K1/K2)."""
    x = g16 if dt == F32 else widen16(g16, dt)
    return (np.ascontiguousarray(x, np.float32) * np.float32(inv_scale)).astype(np.float32)


def norm_p(g16: np.ndarray, dt: int, inv_scale: float, norm_type: float) -> float:
    """compute_norm (Src/zero/utils.py:126-154) of the unscaled grads, exact
    up to the final rounding: p = inf is max |x| (NaN if any x is NaN, as
    tensor.abs().max()); p = 2 is sqrt of the exactly rounded sum of x^2;
    other p > 0 is (sum |x|^p)^(1/p) with each |x|^p in fp64 and the sum
    exactly rounded (math.fsum). The reference holds no vectors for it (its
    arithmetic is torch's fp32 per-tensor norm); it is pinned against
    torch.linalg.vector_norm in fp64, the reference's per-tensor formula in
    torch, and closed forms (tests/test_oracle_casts_norm.py)."""
    p = float(norm_type)
    if not p > 0:
        raise ValueError(f"norm_type must be > 0 (finite or inf), got {norm_type}")
    x = unscaled(g16, dt, inv_scale).astype(np.float64)
    if x.size == 0:
        return 0.0
    a = np.abs(x)
    if np.isnan(a).any():
        return float("nan")
    if math.isinf(p):
        return float(a.max())
    if p == 2.0:
        return math.sqrt(math.fsum(a * a))
    if p == 1.0:
        return math.fsum(a)
    with np.errstate(over="ignore"):
        return math.fsum(a ** p) ** (1.0 / p)


def clip_once_coef(norm: float, max_norm: float, clip_eps: float = 1e-6) -> float:
    """The explicit clip_grad_norm_(max_norm) call, Src/zero/utils.py:209-214:
    max_norm / (norm + clip_eps) iff norm > max_norm (no other condition:
    max_norm = 0 zeroes the grads), applied as an fp32 scalar."""
    if norm > max_norm:
        return float(np.float32(max_norm / (norm + clip_eps)))
    return 1.0


def step_scalars(h: Hyper, t: int, inv_scale: float, coef: float) -> _Scalars:
    f = lambda x: float(np.float32(x))  # noqa: E731  (round a double to fp32)
    bc1, bc2s = bias_corrections(h.beta1, h.beta2, t)
    s = _Scalars()
    s.inv_scale = inv_scale
    s.clip_coef = coef
    s.decay = f(1 - h.lr * h.weight_decay) if h.weight_decay != 0 else 1.0
    s.w1 = f(1 - h.beta1)
    s.w1c = float(np.float32(1.0) - np.float32(s.w1))
    s.b2 = f(h.beta2)
    s.val2 = f(1 - h.beta2)
    s.eps = f(h.eps)
    s.bc2s = f(bc2s)
    s.nss = f(-(h.lr / bc1))
    return s


def adamw(p: np.ndarray, m: np.ndarray, v: np.ndarray, p16: np.ndarray | None, pdt: int,
          g16: np.ndarray, gdt: int, sc: _Scalars) -> None:
    """One AdamW step in place (fp32 p/m/v), writing the 16-bit cast to p16."""
    n = p.size
    for a in (p, m, v):
        _check(a, np.float32, n)
    _check(g16, _gdtype(gdt), n)
    if p16 is not None:
        _check(p16, np.uint16, n)
    lib().dsxo_adamw(_ptr(p), _ptr(m), _ptr(v), _ptr(p16), pdt, _ptr(g16), gdt, n, ctypes.byref(sc))


# ---- loss scaler ---------------------------------------------------------------------

@dataclass
class LossScalerSpec:
    """Dynamic loss scaler with hysteresis and a minimum scale.

    ds_config keys fp16.{initial_scale_power, loss_scale_window, hysteresis,
    min_loss_scale} (Src/config.py:93-102, Src/zero/__init__.py:103-109).
    The reference builds torch's GradScaler(init 2**power, growth 2, backoff
    0.5, interval window) at Src/zero/optimizer.py:102-110 and never consumes
    hysteresis or min_loss_scale; with hysteresis=1 and a reachable minimum
    this machine is exactly torch._amp_update_scale_
    (torch/amp/grad_scaler.py:469-538).

      overflow: if hysteresis == 1 or hyst_left <= 1:
                    scale = max(scale * backoff, min_scale)
                else: hyst_left -= 1
                good = 0
      clean:    good += 1
                if good == window: scale *= growth if that is finite;
                                   good = 0; hyst_left = hysteresis
    """
    scale: float = 2.0 ** 16
    window: int = 1000
    hysteresis: int = 2
    min_scale: float = 1.0
    growth: float = 2.0
    backoff: float = 0.5
    dynamic: bool = True
    good: int = 0
    hyst_left: int = field(default=-1)

    def __post_init__(self):
        if self.hyst_left < 0:
            self.hyst_left = self.hysteresis
        self.scale = float(np.float32(self.scale))

    def update(self, found_inf: bool) -> None:
        if not self.dynamic:
            return
        f32 = np.float32
        if found_inf:
            if self.hysteresis <= 1 or self.hyst_left <= 1:
                nxt = float(f32(self.scale) * f32(self.backoff))
                self.scale = max(nxt, float(f32(self.min_scale)))
            else:
                self.hyst_left -= 1
            self.good = 0
        else:
            self.good += 1
            if self.good >= self.window:
                with np.errstate(over="ignore"):
                    nxt = f32(self.scale) * f32(self.growth)
                if math.isfinite(float(nxt)):
                    self.scale = float(nxt)
                self.good = 0
                self.hyst_left = self.hysteresis


# ---- a whole step -------------------------------------------------------------------------

@dataclass
class StepResult:
    skipped: bool
    t: int
    sumsq: float
    norm: float
    clip_coef: float
    scale_used: float
    scale_next: float


class ZeroStepOracle:
    """ZeROOptimizer.step (Src/zero/optimizer.py:212-274) over one flat
    partition, in the order: overflow check / skip -> unscale -> norm -> clip
    -> AdamW -> cast -> scaler update. Arrays are updated in place.

    groups: optional [(start, end, Hyper)] ranges of the partition with their
    own hyper-parameters (torch param_groups stepped by one optimizer): the
    norm, skip decision and clip coefficient stay global, the clip threshold
    is `hyper`'s. blocked_norm: take the norm as sumsq(..., blocks=1024) on
    all cores (sumsq_parallel, the same bits) -- for partitions of billions
    of elements."""

    def __init__(self, master: np.ndarray, exp_avg: np.ndarray, exp_avg_sq: np.ndarray,
                 p16: np.ndarray | None, pdt: int, gdt: int, hyper: Hyper,
                 scaler: LossScalerSpec, groups: list | None = None, blocked_norm: bool = False):
        self.p, self.m, self.v, self.p16 = master, exp_avg, exp_avg_sq, p16
        self.pdt, self.gdt, self.h, self.scaler = pdt, gdt, hyper, scaler
        self.groups = list(groups) if groups else [(0, master.size, hyper)]
        self.blocked_norm = blocked_norm
        self.t = 0
        self.overflow_count = 0

    def step(self, g16: np.ndarray, clip_once: float | None = None) -> StepResult:
        """clip_once: the coefficient of a clip_grad_norm_ call made before
        this step (clip_once_coef); it replaces the configured clip for this
        step only."""
        scale = self.scaler.scale
        inv = inv_scale_of(scale)
        ss = sumsq_parallel(g16, self.gdt, inv, 1024) if self.blocked_norm else sumsq(g16, self.gdt, inv)
        norm = math.sqrt(ss) if math.isfinite(ss) else ss
        found_inf = not math.isfinite(ss)
        coef = 1.0
        if found_inf:
            self.overflow_count += 1
        else:
            self.t += 1
            coef = (clip_once if clip_once is not None
                    else clip_coef(norm, self.h.max_grad_norm, self.h.clip_eps))
            for a, b, h in self.groups:
                adamw(self.p[a:b], self.m[a:b], self.v[a:b], None if self.p16 is None else self.p16[a:b],
                      self.pdt, g16[a:b], self.gdt, step_scalars(h, self.t, inv, coef))
        self.scaler.update(found_inf)
        return StepResult(found_inf, self.t, ss, norm, coef, scale, self.scaler.scale)


def ulp_diff_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|a - b| in units in the last place of fp32 (monotone integer mapping;
    NaN == NaN counts as 0, NaN vs number as a huge distance)."""
    ai = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    bi = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    ai = np.where(ai < 0, -(ai & 0x7FFFFFFF), ai)
    bi = np.where(bi < 0, -(bi & 0x7FFFFFFF), bi)
    d = np.abs(ai - bi)
    an, bn = np.isnan(a), np.isnan(b)
    d = np.where(an & bn, 0, d)
    d = np.where(an ^ bn, 1 << 40, d)
    return d


def ulp_diff_16(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|a - b| in ulps of a 16-bit format given as uint16 storage."""
    ai = np.ascontiguousarray(a, np.uint16).astype(np.int64)
    bi = np.ascontiguousarray(b, np.uint16).astype(np.int64)
    ai = np.where(ai & 0x8000, -(ai & 0x7FFF), ai)
    bi = np.where(bi & 0x8000, -(bi & 0x7FFF), bi)
    return np.abs(ai - bi)
