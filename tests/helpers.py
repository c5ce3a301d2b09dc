"""Shared test helpers: seeded inputs, host<->device transfers of 16-bit
storage, and the tolerance used against torch's CPU AdamW."""
from __future__ import annotations

import hashlib

import numpy as np

F16, BF16 = 1, 2


def np16_to_torch(a: np.ndarray, dt: int, device=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).view(
        torch.float16 if dt == F16 else torch.bfloat16)
    return t.to(device) if device is not None else t


def torch16_to_np(t) -> np.ndarray:
    import torch
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def f32_to_torch(a: np.ndarray, device=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32))
    return t.to(device) if device is not None else t


def edge_grads(dt: int) -> np.ndarray:
    """16-bit grad patterns the step must handle: zeros of both signs, the
    smallest subnormal, the largest finite, values near 1, ties."""
    if dt == F16:
        vals = [0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x3C00, 0xBC00, 0x3C01, 0x1234,
                0x5555, 0xD555, 0x2E66]
    else:
        vals = [0x0000, 0x8000, 0x0001, 0x8001, 0x007F, 0x0080, 0x7F7F, 0xFF7F, 0x3F80, 0xBF80, 0x3F81, 0x1234,
                0x5555, 0xD555, 0x3A83]
    return np.array(vals, np.uint16)


def make_state(n: int, seed: int, gdt: int, g_sigma: float, scale: float = 1.0, edges: bool = True,
               p_sigma: float = 0.02, mv_warm: bool = True):
    """Seeded fp32 master/exp_avg/exp_avg_sq and 16-bit grads (grads scaled
    by `scale` before the cast, as a backward with loss scaling produces)."""
    from oracle import oracle as O
    rng = np.random.default_rng(seed)
    p = (rng.standard_normal(n) * p_sigma).astype(np.float32)
    if mv_warm:
        m = (rng.standard_normal(n) * g_sigma * 0.3).astype(np.float32)
        v = (np.abs(rng.standard_normal(n)) * g_sigma * g_sigma).astype(np.float32)
    else:
        m = np.zeros(n, np.float32)
        v = np.zeros(n, np.float32)
    g32 = (rng.standard_normal(n) * g_sigma * scale).astype(np.float32)
    g16 = O.cast16(g32, gdt)
    if edges and n >= 64:
        e = edge_grads(gdt)
        k = min(len(e), n // 4)
        g16[:k] = e[:k]
        g16[-k:] = e[:k][::-1]
        p[:4] = np.array([0.0, -0.0, 1e-30, -3.0], np.float32)
        v[4:6] = np.array([0.0, 1e-38], np.float32)
        m[6:8] = np.array([0.0, -1e-3], np.float32)
    return p, m, v, g16


def cancellation_ulp_ok(ours: np.ndarray, ref: np.ndarray, decayed: np.ndarray, k: float = 2.0) -> np.ndarray:
    """|ours - ref| <= k * spacing(max(|ours|, |decayed|, |ours - decayed|)).

    The master update is p_new = p_decayed + u. Where the add cancels
    (|p_new| << |u|), one ulp of u is many ulps of p_new, so the tolerance is
    taken in ulps of the largest operand or result of that final add."""
    upd = np.abs(ours.astype(np.float64) - decayed.astype(np.float64))
    scale = np.maximum(np.maximum(np.abs(ours), np.abs(decayed)), upd).astype(np.float32)
    tol = k * np.spacing(scale)
    diff = np.abs(ours.astype(np.float64) - ref.astype(np.float64))
    return (diff <= tol) | (np.isnan(ours) & np.isnan(ref))


# configs[0] (the 3-layer MLP partition) as the parity tests run it: fp16
# grads and params, static loss scale 2^16, no clip, ten steps from zero
# moments. Its per-step digests are committed (tests/golden/make_digests.py).
MLP_CASE = dict(n=1_863_690, gdt=F16, pdt=F16, seed=0, g_sigma=0.01, steps=10, scale=2.0 ** 16,
                hyper=dict(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, max_grad_norm=0.0))


def step_digests(p, m, v, p16) -> dict:
    """SHA-256 of each array's bit pattern (fp32 as uint32, 16-bit as uint16)."""
    def h(a, dt):
        return hashlib.sha256(np.ascontiguousarray(a).view(dt).tobytes()).hexdigest()
    return {"master": h(p, np.uint32), "exp_avg": h(m, np.uint32), "exp_avg_sq": h(v, np.uint32),
            "param16": h(p16, np.uint16)}


def mlp_case_inputs(O):
    """MLP_CASE's initial master / exp_avg / exp_avg_sq / param16 and its
    grads generator (one call per step), as _flat_run in the GPU parity
    tests draws them."""
    c = MLP_CASE
    p, m, v, _ = make_state(c["n"], c["seed"], c["gdt"], c["g_sigma"], edges=False, mv_warm=False, p_sigma=0.02)
    p16 = O.cast16(p, c["pdt"])
    rng = np.random.default_rng(c["seed"] + 1)

    def grads():
        return O.cast16((rng.standard_normal(c["n"]) * c["g_sigma"] * c["scale"]).astype(np.float32), c["gdt"])
    return p, m, v, p16, grads


def mlp_case_oracle_digests(O) -> list:
    """MLP_CASE through the oracle: the digests after every step."""
    c = MLP_CASE
    p, m, v, p16, grads = mlp_case_inputs(O)
    orc = O.ZeroStepOracle(p, m, v, p16, c["pdt"], c["gdt"], O.Hyper(**c["hyper"]),
                           O.LossScalerSpec(scale=c["scale"], dynamic=False))
    out = []
    for _ in range(c["steps"]):
        r = orc.step(grads())
        assert not r.skipped
        out.append(step_digests(orc.p, orc.m, orc.v, orc.p16))
    return out
