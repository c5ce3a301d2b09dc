"""The 16-bit cast inside K2 and K3 at its edge cases, on the GPU.

With lr = 0 the AdamW update is an exact no-op on the master (decay = 1,
step size -0, m = v = g = 0 so m / denom = 0 with eps > 0), so param16 is the
kernel's round-to-nearest-even cast of the chosen masters. The masters cover
every rounding boundary of both formats: each finite 16-bit value itself, the
exact midpoint between it and its successor (a tie), and one fp32 ulp on
either side of that midpoint; every fp32 value from the fp16 maximum 65504 up
to 65536 (65520 is the tie that rounds to inf) and every fp32 value whose
upper half is bf16's largest finite 0x7F7F (the tie 0x7F7F8000 rounds to
inf); fp16 subnormal ties; +-0; +-inf; NaNs of both signs, quiet and
signalling; fp32 subnormals and the fp32 maximum. param16 must equal the
oracle's cast bit for bit (the north star's "16-bit params within 1 ulp",
which the cast adds to Src/zero/optimizer.py:212-274; the oracle's cast is
pinned exhaustively on the CPU against numpy and torch). The ragged run puts
the same masters through K3's chunk table, with tensors at aligned and
misaligned addresses so that both its vector and its scalar loop cast."""
from __future__ import annotations

import sys

import numpy as np
import pytest

from helpers import BF16, F16, np16_to_torch, torch16_to_np

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _u2f(u) -> np.ndarray:
    return np.asarray(u, np.uint32).view(np.float32)


def edge_masters(O, dt: int) -> np.ndarray:
    h = np.arange(65536, dtype=np.uint32)
    w = O.widen16(h.astype(np.uint16), dt)
    out = [w[np.isfinite(w)]]
    if dt == BF16:
        fin = h[(h & 0x7FFF) < 0x7F80]
        mid = _u2f((fin << 16) | 0x8000)  # exactly halfway to the successor in magnitude
        top = np.arange(65536, dtype=np.uint32)
        out += [_u2f((0x7F7F << 16) | top), _u2f((0xFF7F << 16) | top)]
    else:
        fin = h[(h & 0x7FFF) < 0x7C00]
        mag = fin & 0x7FFF
        sign = np.where(fin & 0x8000, -1.0, 1.0)
        # fp16 value of magnitude k (subnormal: k * 2^-24) and its successor:
        # the midpoint is exact in fp32 for every finite k, including the
        # subnormal range and the top (65504 -> 65520).
        lo = np.abs(O.widen16(mag.astype(np.uint16), F16).astype(np.float64))
        nxt = np.where(mag == 0x7BFF, 65536.0,
                       np.abs(O.widen16(np.minimum(mag + 1, 0x7BFF).astype(np.uint16), F16).astype(np.float64)))
        mid = (sign * (lo + nxt) / 2).astype(np.float32)
        assert np.array_equal(mid.astype(np.float64), sign * (lo + nxt) / 2), "fp16 midpoints must be exact in fp32"
        span = np.arange(0x477FE000, 0x47800001, dtype=np.uint32)  # 65504 .. 65536
        out += [_u2f(span), -_u2f(span)]
    out += [mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(-np.inf))]
    specials = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000,          # zeros, infinities
                0x7FC00000, 0xFFC00000, 0x7F800001, 0xFF800001,          # quiet / signalling NaNs
                0x7FFFFFFF, 0xFFFFFFFF, 0x7FA00000, 0xFFA00000,
                0x00000001, 0x80000001, 0x007FFFFF, 0x807FFFFF,          # fp32 subnormals
                0x7F7FFFFF, 0xFF7FFFFF, 0x47800000, 0xC7800000]          # fp32 max, 65536
    out.append(_u2f(np.array(specials, np.uint32)))
    return np.ascontiguousarray(np.concatenate(out).astype(np.float32))


def _scalars(O, gpu, ngroups=1):
    import torch
    from distributedspeed_amd import _lib, ops
    h = O.Hyper(lr=0.0, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    sc = O.step_scalars(h, 1, 1.0, 1.0)
    c = _lib.DsxStepScalars()
    c.skip, c.t = 0, 1
    for k in ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2", "eps", "bc2s", "nss"):
        setattr(c, k, getattr(sc, k))
    assert c.decay == 1.0 and c.nss == 0.0
    one = ops.scalars_from_host(c, gpu)
    return sc, torch.cat([one] * ngroups)


def _oracle(O, master, dt, sc):
    n = master.size
    p, m, v = master.copy(), np.zeros(n, np.float32), np.zeros(n, np.float32)
    p16 = np.empty(n, np.uint16)
    O.adamw(p, m, v, p16, dt, np.zeros(n, np.uint16), dt, sc)
    return p, p16


def _check(O, master, dt, got_p, got_p16, ref_p, ref_p16, tag):
    nan = np.isnan(master)
    assert np.array_equal(np.isnan(got_p), nan), f"{tag}: NaN positions of the master changed"
    same = got_p.view(np.uint32)[~nan] == master.view(np.uint32)[~nan]
    assert same.all(), f"{tag}: lr = 0 changed {(~same).sum()} masters"
    bad = got_p16 != ref_p16
    if bad.any():
        i = np.flatnonzero(bad)[:8]
        pytest.fail(f"{tag}: {bad.sum()} param16 differ from the oracle, e.g. masters "
                    f"{[hex(x) for x in master.view(np.uint32)[i]]} -> {[hex(x) for x in got_p16[i]]} "
                    f"vs {[hex(x) for x in ref_p16[i]]}")
    direct = O.cast16(master, dt)
    assert np.array_equal(ref_p16[~nan], direct[~nan])
    if dt == F16:
        assert np.array_equal(got_p16[nan] & 0x7FFF, np.full(nan.sum(), 0x7E00, np.uint16))
    else:
        assert np.array_equal(got_p16[nan], np.full(nan.sum(), 0x7FC0, np.uint16))


@pytest.mark.parametrize("dt", [F16, BF16])
def test_cast_edges_through_k2(gpu, oracle, dt):
    import torch
    from distributedspeed_amd import ops
    O = oracle
    master = edge_masters(O, dt)
    n = master.size
    _say(f"cast edges K2 dt={dt} n={n}")
    sc, scal = _scalars(O, gpu)
    tp = torch.from_numpy(master.copy()).to(gpu)
    tm = torch.zeros(n, dtype=torch.float32, device=gpu)
    tv = torch.zeros(n, dtype=torch.float32, device=gpu)
    tg = np16_to_torch(np.zeros(n, np.uint16), dt, gpu)
    tp16 = torch.empty(n, dtype=tg.dtype, device=gpu)
    ops.adamw_flat(tp, tm, tv, tp16, tg, scal)
    torch.cuda.synchronize()
    ref_p, ref_p16 = _oracle(O, master, dt, sc)
    _check(O, master, dt, tp.cpu().numpy(), torch16_to_np(tp16), ref_p, ref_p16, "K2")
    assert not tm.any() and not tv.any()


@pytest.mark.parametrize("shift", [0, 1])
@pytest.mark.parametrize("dt", [F16, BF16])
def test_cast_edges_through_k3(gpu, oracle, dt, shift):
    """The same masters cut into four tensors carved from one allocation,
    with sizes that leave ragged chunk tails: every tensor 16-byte aligned
    (shift 0: K3's vector loop) or every tensor one element off (shift 1:
    its scalar loop)."""
    import torch
    from distributedspeed_amd import ops
    O = oracle
    master = edge_masters(O, dt)
    n = master.size
    sc, scal = _scalars(O, gpu)
    cuts = [0, 100_003, 100_004, 231_077, n]
    total = n + 4 * 4 + 8
    bp = torch.zeros(total, dtype=torch.float32, device=gpu)
    bm = torch.zeros(total, dtype=torch.float32, device=gpu)
    bv = torch.zeros(total, dtype=torch.float32, device=gpu)
    gdt = torch.float16 if dt == F16 else torch.bfloat16
    bg = torch.zeros(total, dtype=gdt, device=gpu)
    bo = torch.zeros(total, dtype=gdt, device=gpu)
    views, end = [], 0
    for k in range(4):
        a, b = cuts[k], cuts[k + 1]
        off = (end + 3) // 4 * 4 + shift
        sl = slice(off, off + (b - a))
        bp[sl].copy_(torch.from_numpy(master[a:b].copy()))
        views.append(tuple(t[sl] for t in (bp, bm, bv, bo, bg)))
        end = off + (b - a)
    for x in views:
        assert all((t.data_ptr() % 16 == 0) if t.element_size() == 4 else (t.data_ptr() % 8 == 0) for t in x) \
            == (shift == 0)
    _say(f"cast edges K3 dt={dt} shift={shift} n={n}")
    table = ops.ChunkTable([x[0] for x in views], [x[1] for x in views], [x[2] for x in views],
                           [x[3] for x in views], [x[4] for x in views], chunk_elems=4096)
    ops.adamw_multi(table, scal)
    torch.cuda.synchronize()
    got_p = np.concatenate([x[0].cpu().numpy() for x in views])
    got_p16 = np.concatenate([torch16_to_np(x[3]) for x in views])
    ref_p, ref_p16 = _oracle(O, master, dt, sc)
    _check(O, master, dt, got_p, got_p16, ref_p, ref_p16, f"K3 shift {shift}")
