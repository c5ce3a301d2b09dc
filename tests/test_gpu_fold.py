"""The two-launch step against the three-launch step, through the C ABI.

One-call steps (dsx_zero_step_flat, dsx_zero_step_plan) of at most 3 * 2^23
elements with at most 512 partials run as K1 followed by K2 with K0's
finalize folded in (every K2 block reduces the partials and decides the step
with K0's code; one block writes the state and the step records). With
dsx_set_tuning_fold(0) the same calls run K1, K0, K2. On the same inputs the
two must agree bit for bit, step after step: master, exp_avg, exp_avg_sq,
param16, the whole 64-byte device state and the step record. The steps cover
an overflow skip with a scale back-off, scale growth (window 2), a one-shot
clip armed by dsx_norm_partials + dsx_clip_prepare, partition tails (n = 4,
5, 1001, odd sizes), the largest partial count the fold takes (512) and the
first it does not, a grid that strides (the fold widened past K2's one-trip
grid), fp32 grads with bf16 params, and bf16 without a scaler. The mlp case
is also checked against the oracle (ZeroStepOracle) at every step."""
from __future__ import annotations

import ctypes
import math
import sys

import numpy as np
import pytest

from helpers import BF16, F16, torch16_to_np

pytestmark = pytest.mark.gpu

F32 = 0
FOLD_DEFAULT = 3 << 23  # the library's default bound

# (id, n, grad dtype, param dtype, scaler mode, nparts (None: the library's), fold bound)
CASES = [
    ("mlp-f16-dynamic", 1_863_690, F16, F16, "dynamic", None, FOLD_DEFAULT),
    ("tail-bf16", 1001, BF16, BF16, "none", None, FOLD_DEFAULT),
    ("n4", 4, F16, F16, "dynamic", 1, FOLD_DEFAULT),
    ("n5", 5, BF16, BF16, "none", 3, FOLD_DEFAULT),
    ("parts-512", 300_001, F16, F16, "dynamic", 512, FOLD_DEFAULT),
    ("parts-513", 300_001, F16, F16, "dynamic", 513, FOLD_DEFAULT),
    ("strided", 40_000_003, BF16, BF16, "none", None, 1 << 26),
    ("f32-grads", 123_457, F32, BF16, "none", None, FOLD_DEFAULT),
    # above the bound: K0 folded into K2's first part alone (one block per CU),
    # here the whole partition (one part) and the first of two parts
    ("first-part-whole", 3_000_007, F16, F16, "dynamic", None, 1 << 20),
    ("first-of-two-parts", 70_000_001, BF16, BF16, "none", None, FOLD_DEFAULT),
    # bounds under 4: 2 and 3 elements take three launches (the fold needs a
    # 4-element slot), 4 elements above a bound of 3 fold into the first part
    ("n2-bound1", 2, BF16, BF16, "none", 1, 1),
    ("n3-bound2", 3, F16, F16, "dynamic", 1, 2),
    ("n4-bound3", 4, F16, F16, "dynamic", 1, 3),
]


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _tdt(dt):
    import torch
    return {F32: torch.float32, F16: torch.float16, BF16: torch.bfloat16}[dt]


class _Side:
    def __init__(self, gpu, master, pdt, gdt, n, scaler):
        import torch
        from distributedspeed_amd import ops
        self.p = master.clone()
        self.m = torch.zeros_like(master)
        self.v = torch.zeros_like(master)
        self.p16 = master.to(_tdt(pdt))
        self.g = torch.zeros(n, dtype=_tdt(gdt), device=gpu)
        self.state = ops.new_state(gpu, scaler.init_scale if scaler.mode != "none" else 1.0,
                                   scaler.hysteresis if scaler.mode == "dynamic" else 1)
        self.out = torch.zeros(ops.SCALARS_BYTES, dtype=torch.uint8, device=gpu)

    def bits(self):
        import torch
        return {"master": self.p.view(torch.int32).cpu(), "exp_avg": self.m.view(torch.int32).cpu(),
                "exp_avg_sq": self.v.view(torch.int32).cpu(), "param16": self.p16.view(torch.int16).cpu(),
                "state": self.state.cpu(), "record": self.out.cpu()}


def _arm_clip(side, n, gdt, max_norm, partials, stream):
    """clip_grad_norm_(max_norm, 2) through the C ABI: norm partials, then
    the one-shot coefficient armed in the state."""
    import torch
    from distributedspeed_amd import _lib
    nparts = partials.numel()
    norm = torch.zeros(1, dtype=torch.float64, device=side.state.device)
    _lib.call("dsx_norm_partials", _ptr(side.g), gdt, ctypes.c_int64(n), _ptr(side.state), ctypes.c_double(2.0),
              _ptr(partials), nparts, stream)
    _lib.call("dsx_clip_prepare", _ptr(partials), nparts, ctypes.c_double(2.0), ctypes.c_double(max_norm),
              ctypes.c_double(1e-6), _ptr(side.state), _ptr(norm), stream)
    return norm


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_two_launch_step_matches_three_launches(gpu, case):
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    cid, n, gdt, pdt, mode, nparts, fold_max = case
    scale0 = 2.0 ** 12 if mode == "dynamic" else 1.0
    scaler = (ScalerConfig(mode="dynamic", init_scale=scale0, window=2, hysteresis=1) if mode == "dynamic"
              else ScalerConfig(mode="none"))
    hyper = AdamWHyper(lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    gen = torch.Generator(device=gpu).manual_seed(1000 + n % 997)
    master = (torch.randn(n, generator=gen, device=gpu) * 0.02).float()
    a = _Side(gpu, master, pdt, gdt, n, scaler)  # the library's choice (two launches where the fold applies)
    b = _Side(gpu, master, pdt, gdt, n, scaler)  # three launches
    bc = BiasCorrectionTable(gpu, hyper.beta1, hyper.beta2)
    stream = ops.stream_of(gpu)
    nparts = nparts or ops.suggest_partials(n)
    parts_a = torch.zeros(nparts, dtype=torch.float64, device=gpu)
    parts_b = torch.zeros(nparts, dtype=torch.float64, device=gpu)
    oracle_run = cid == "mlp-f16-dynamic"
    if oracle_run:
        from oracle import oracle as O
        orc = O.ZeroStepOracle(master.cpu().numpy().copy(), np.zeros(n, np.float32), np.zeros(n, np.float32),
                               torch16_to_np(a.p16).copy(), pdt, gdt,
                               O.Hyper(lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1,
                                       max_grad_norm=1.0),
                               O.LossScalerSpec(scale=scale0, window=2, hysteresis=1))
    try:
        for step in range(6):
            scale = float(ops.read_state(a.state).scale)
            g = (torch.randn(n, generator=gen, device=gpu) * 1e-3 * scale).to(_tdt(gdt))
            if step == 1:
                g[n // 2] = float("inf")
            a.g.copy_(g)
            b.g.copy_(g)
            clip = None
            if step == 3:  # a one-shot clip far below the norm
                na = _arm_clip(a, n, gdt, 1e-4, parts_a, stream)
                _arm_clip(b, n, gdt, 1e-4, parts_b, stream)
                clip = float(na.item())
            _say(f"fold case={cid} n={n} nparts={nparts} step={step}")
            _lib.call("dsx_set_tuning_fold", ctypes.c_int64(fold_max))
            _lib.call("dsx_zero_step_flat", _ptr(a.p), _ptr(a.m), _ptr(a.v), _ptr(a.p16), pdt, _ptr(a.g), gdt,
                      ctypes.c_int64(n), _ptr(a.state), scaler.to_c(), hyper.to_c(), _ptr(bc.table), bc.length,
                      _ptr(parts_a), nparts, _ptr(a.out), stream)
            _lib.call("dsx_set_tuning_fold", ctypes.c_int64(0))
            _lib.call("dsx_zero_step_flat", _ptr(b.p), _ptr(b.m), _ptr(b.v), _ptr(b.p16), pdt, _ptr(b.g), gdt,
                      ctypes.c_int64(n), _ptr(b.state), scaler.to_c(), hyper.to_c(), _ptr(bc.table), bc.length,
                      _ptr(parts_b), nparts, _ptr(b.out), stream)
            torch.cuda.synchronize()
            xa, xb = a.bits(), b.bits()
            for name in xa:
                assert torch.equal(xa[name], xb[name]), \
                    f"step {step}: {name} differs ({int((xa[name] != xb[name]).sum())} elements)"
            st = ops.read_state(a.state)
            assert st.error == 0 and st.clip_once == 0
            assert st.last_skip == (1 if step == 1 else 0), step
            if oracle_run:
                g16 = torch16_to_np(g)
                coef = None if clip is None else O.clip_once_coef(clip, 1e-4)
                r = orc.step(g16, clip_once=coef)
                assert r.skipped == (step == 1) and st.scale == r.scale_next
                assert np.array_equal(a.p.cpu().numpy().view(np.uint32), orc.p.view(np.uint32)), step
                assert np.array_equal(a.m.cpu().numpy().view(np.uint32), orc.m.view(np.uint32)), step
                assert np.array_equal(a.v.cpu().numpy().view(np.uint32), orc.v.view(np.uint32)), step
                assert np.array_equal(torch16_to_np(a.p16), orc.p16), step
        st = ops.read_state(a.state)
        assert st.t == 5 and st.overflow_count == 1
        if mode == "dynamic":  # back-off at step 1, growth after two clean steps, twice
            assert st.scale == scale0 / 2 * 4
    finally:
        _lib.call("dsx_set_tuning_fold", ctypes.c_int64(FOLD_DEFAULT))


def _plan_step(side, n, gdt, pdt, scaler, hypers, tables, ends, parts, stream):
    """dsx_zero_step_plan over `side` with groups ending at `ends`."""
    from distributedspeed_amd import _lib
    P = _lib.DsxFlatPlan()
    P.master, P.exp_avg, P.exp_avg_sq = side.p.data_ptr(), side.m.data_ptr(), side.v.data_ptr()
    P.param16, P.grad, P.n = side.p16.data_ptr(), side.g.data_ptr(), n
    P.param_dtype, P.grad_dtype = pdt, gdt
    P.state, P.partials, P.out = side.state.data_ptr(), parts.data_ptr(), side.out.data_ptr()
    P.nparts, P.ngroups, P.scaler = parts.numel(), len(ends), scaler.to_c()
    G = _lib.DsxGroupsDev()
    for k, (h, bc, e) in enumerate(zip(hypers, tables, ends)):
        P.group_end[k] = e
        G.hyper[k] = h.to_c()
        G.bc_table[k] = bc.table.data_ptr()
        G.t_offset[k] = 0
    G.ngroups, G.bc_len = len(ends), min(bc.length for bc in tables)
    _lib.call("dsx_zero_step_plan", ctypes.byref(P), ctypes.byref(G), stream)


# group ends: the last group of 3 elements is one the fold does not take
# (three launches on both sides); the others fold, with an empty group
# between two nonempty ones (the first nonempty group's K2 writes the state).
PLAN_CASES = [("fold", [1000, 1000, 2005]), ("tiny-last-group", [1000, 1000, 1003]), ("empty-first", [0, 2000]),
              # above the bound: the first nonempty group's first part decides
              ("first-part", [20_000_000, 20_000_104, 30_000_000]), ("first-part-empty-first", [0, 30_000_000])]


@pytest.mark.parametrize("pcase", PLAN_CASES, ids=[c[0] for c in PLAN_CASES])
def test_plan_two_launch_step_matches_three_launches(gpu, pcase):
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    cid, ends = pcase
    n, gdt, pdt = ends[-1], F16, F16
    scaler = ScalerConfig(mode="dynamic", init_scale=2.0 ** 10, window=3, hysteresis=2)
    hypers = [AdamWHyper(lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, max_grad_norm=0.5),
              AdamWHyper(lr=5e-3, beta1=0.8, beta2=0.99, eps=1e-6, weight_decay=0.0, max_grad_norm=0.5),
              AdamWHyper(lr=2e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, max_grad_norm=0.5)][:len(ends)]
    tables = [BiasCorrectionTable(gpu, h.beta1, h.beta2) for h in hypers]
    gen = torch.Generator(device=gpu).manual_seed(31)
    master = (torch.randn(n, generator=gen, device=gpu) * 0.05).float()
    a, b = _Side(gpu, master, pdt, gdt, n, scaler), _Side(gpu, master, pdt, gdt, n, scaler)
    a.out = torch.zeros(ops.SCALARS_BYTES * len(ends), dtype=torch.uint8, device=gpu)
    b.out = torch.zeros(ops.SCALARS_BYTES * len(ends), dtype=torch.uint8, device=gpu)
    stream = ops.stream_of(gpu)
    nparts = ops.suggest_partials(n)
    parts_a = torch.zeros(nparts, dtype=torch.float64, device=gpu)
    parts_b = torch.zeros(nparts, dtype=torch.float64, device=gpu)
    try:
        for step in range(10):
            scale = float(ops.read_state(a.state).scale)
            g = (torch.randn(n, generator=gen, device=gpu) * 1e-2 * scale).half()
            if step in (2, 3):  # two overflows: hysteresis 2 tolerates the first
                g[n - 1] = float("nan")
            a.g.copy_(g)
            b.g.copy_(g)
            if step == 6:
                _arm_clip(a, n, gdt, 0.01, parts_a, stream)
                _arm_clip(b, n, gdt, 0.01, parts_b, stream)
            _say(f"fold plan case={cid} ends={ends} step={step}")
            _lib.call("dsx_set_tuning_fold", ctypes.c_int64(FOLD_DEFAULT))
            _plan_step(a, n, gdt, pdt, scaler, hypers, tables, ends, parts_a, stream)
            _lib.call("dsx_set_tuning_fold", ctypes.c_int64(0))
            _plan_step(b, n, gdt, pdt, scaler, hypers, tables, ends, parts_b, stream)
            torch.cuda.synchronize()
            xa, xb = a.bits(), b.bits()
            for name in xa:
                assert torch.equal(xa[name], xb[name]), f"step {step}: {name} differs"
        st = ops.read_state(a.state)
        assert st.t == 8 and st.overflow_count == 2 and st.error == 0
    finally:
        _lib.call("dsx_set_tuning_fold", ctypes.c_int64(FOLD_DEFAULT))


def test_optimizer_with_empty_group_matches_three_launches(gpu):
    """The drop-in optimizer's one-call step with an empty parameter group
    between two others, against three launches (track_skips keeps them
    separate) over 12 steps with a NaN overflow and a one-shot clip."""
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer
    shapes = [(130, 7), (64, 33), (40, 9)]
    torch.manual_seed(5)
    init = [torch.randn(s) * 0.05 for s in shapes]

    def build(track):
        ps = [torch.nn.Parameter(t.clone().to(gpu)) for t in init]
        groups = [{"params": ps[:1]}, {"params": [], "lr": 5e-3}, {"params": ps[1:], "lr": 2e-3}]
        opt = AdamWOptimizer(groups, lr=1e-3, betas=(0.9, 0.95), weight_decay=0.1, max_grad_norm=0.5,
                             param_dtype=torch.float16, device=gpu,
                             loss_scaler=ScalerConfig(mode="dynamic", init_scale=2.0 ** 8, window=3, hysteresis=1))
        opt.track_skips(track)
        return opt

    a, b = build(False), build(True)
    assert a._plan is not None
    gen = torch.Generator(device=gpu).manual_seed(6)
    _say("fold: optimizer with an empty group")
    for step in range(12):
        g = (torch.randn(a.flat.numel, device=gpu, generator=gen) * 1e-2 * 256).half()
        if step == 4:
            g[7] = float("nan")
        a.flat.grad.copy_(g)
        b.flat.grad.copy_(g)
        if step == 8:
            assert torch.equal(a.clip_grad_norm_(0.01), b.clip_grad_norm_(0.01))
        a.step()
        b.step()
    torch.cuda.synchronize()
    for name in ("master", "exp_avg", "exp_avg_sq", "param16"):
        x, y = getattr(a.flat, name), getattr(b.flat, name)
        assert torch.equal(x.view(torch.int16 if x.element_size() == 2 else torch.int32),
                           y.view(torch.int16 if y.element_size() == 2 else torch.int32)), name
    sa, sb = a.read_state(), b.read_state()
    assert bytes(sa) == bytes(sb)
    assert sa.t == 11 and sa.overflow_count == 1 and sa.error == 0 and not math.isnan(sa.last_norm)


@pytest.mark.parametrize("case", ["ok", "ngroups", "lr", "ok_fewer", "ok_big", "lr_big"])
def test_dev_block_step_two_and_three_launches(gpu, case):
    """dsx_zero_step_dev (the group block in device memory, the graph form)
    with a block the device-side checks accept or reject: two launches and
    three give the same bits; a rejected block (ngroups above the plan's
    slots, a negative lr) skips the step in every slot and sets
    DSX_STATE_ERR_GROUPS; a block with fewer groups than the plan steps those
    and writes the other slots as skipped. ok_big, lr_big: 2.7e7 elements,
    above the fold's bound (K0 folded into the first part alone, whose records
    the later parts read)."""
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    big = case.endswith("_big")
    n, ends = (27_000_000, [9_000_000, 18_000_000, 27_000_000]) if big else (48, [16, 32, 48])
    scaler = ScalerConfig(mode="dynamic", init_scale=2.0 ** 6, window=2, hysteresis=1)
    tab = BiasCorrectionTable(gpu, 0.9, 0.999)
    h = [AdamWHyper(lr=1e-3 * (k + 1), weight_decay=0.01, max_grad_norm=1.0).to_c() for k in range(3)]
    g = _lib.DsxGroupsDev.from_buffer_copy(ops.pack_groups(h, [tab.table] * 3, [0, 0, 0], tab.length))
    if case == "ngroups":
        g.ngroups = 5
    elif case in ("lr", "lr_big"):
        g.hyper[1].lr = -1.0
    elif case == "ok_fewer":
        g.ngroups = 1
    gen = torch.Generator(device=gpu).manual_seed(3)
    master = (torch.randn(n, generator=gen, device=gpu) * 0.05).float()
    sides = []
    for fold in (FOLD_DEFAULT, 0):
        sd = _Side(gpu, master, F16, F16, n, scaler)
        sd.out = torch.full((ops.SCALARS_BYTES * 3,), 0x7F, dtype=torch.uint8, device=gpu)
        sd.groups = torch.frombuffer(bytearray(bytes(g)), dtype=torch.uint8).to(gpu)
        sd.parts = torch.zeros(4, dtype=torch.float64, device=gpu)
        sd.fold = fold
        sides.append(sd)
    stream = ops.stream_of(gpu)
    _say(f"dev block step case={case}")
    try:
        for step in range(3):
            gg = (torch.randn(n, generator=gen, device=gpu) * 1e-2 * 64).half()
            for sd in sides:
                sd.g.copy_(gg)
                P = _lib.DsxFlatPlan()
                P.master, P.exp_avg, P.exp_avg_sq = sd.p.data_ptr(), sd.m.data_ptr(), sd.v.data_ptr()
                P.param16, P.grad, P.n, P.param_dtype, P.grad_dtype = sd.p16.data_ptr(), sd.g.data_ptr(), n, F16, F16
                P.state, P.partials, P.out = sd.state.data_ptr(), sd.parts.data_ptr(), sd.out.data_ptr()
                P.nparts, P.ngroups, P.scaler = 4, 3, scaler.to_c()
                for k, e in enumerate(ends):
                    P.group_end[k] = e
                _lib.call("dsx_set_tuning_fold", ctypes.c_int64(sd.fold))
                _lib.call("dsx_zero_step_dev", ctypes.byref(P), _ptr(sd.groups), stream)
            torch.cuda.synchronize()
            xa, xb = sides[0].bits(), sides[1].bits()
            for name in xa:
                assert torch.equal(xa[name], xb[name]), f"{case} step {step}: {name} differs"
    finally:
        _lib.call("dsx_set_tuning_fold", ctypes.c_int64(FOLD_DEFAULT))
    a = sides[0]
    s = ops.read_state(a.state)
    sc = [ops.read_scalars(a.out[k * ops.SCALARS_BYTES:(k + 1) * ops.SCALARS_BYTES]) for k in range(3)]
    p = a.p.cpu()
    moved = [not torch.equal(p[b - 16:b], master[b - 16:b].cpu()) for b in ends]
    if case in ("ngroups", "lr", "lr_big"):
        assert s.error & _lib.DSX_STATE_ERR_GROUPS and s.t == 0 and s.last_skip == 1
        assert all(x.skip == 1 for x in sc) and not any(moved)
    elif case == "ok_fewer":
        assert s.error == 0 and s.t == 3
        assert sc[0].skip == 0 and sc[1].skip == 1 and sc[2].skip == 1
        assert moved == [True, False, False]
    else:  # ok, ok_big
        assert s.error == 0 and s.t == 3 and all(x.skip == 0 for x in sc) and all(moved)


@pytest.mark.parametrize("dtype_name", ["float16", "bfloat16"])
def test_ragged_two_launch_step_matches_three_launches(gpu, dtype_name):
    """The ragged form's one-call step (dsx_zero_step_multi): K1 over the
    list and K3 with K0 folded in, against the same call with the fold off
    (K1, K0, K3) and against separate launches (track_skips), bit for bit
    over 12 steps: three parameter groups, one of them empty, a tensor whose
    storage sits one element off 16-byte alignment (K3's element-wise path), a
    NaN overflow (fp16: a dynamic scale backing off), a one-shot clip, and
    the bias corrections of each group's betas."""
    import torch
    from distributedspeed_amd import _lib
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import MultiTensorAdamWOptimizer
    dt = getattr(torch, dtype_name)
    shapes = [(130, 7), (64, 33), (1000,), (5,), (40, 9)]
    torch.manual_seed(8)
    init = [torch.randn(s) * 0.05 for s in shapes]
    fp16 = dt == torch.float16

    def build(track):
        ps = []
        for k, t in enumerate(init):
            if k == 2:  # storage one element past a 16-byte boundary
                buf = torch.empty(t.numel() + 1, dtype=dt, device=gpu)
                v = buf[1:].view(t.shape)
                v.copy_(t)
                ps.append(torch.nn.Parameter(v))
            else:
                ps.append(torch.nn.Parameter(t.clone().to(gpu, dt)))
        groups = [{"params": ps[:2]}, {"params": [], "lr": 5e-3}, {"params": ps[2:], "lr": 2e-3, "betas": (0.8, 0.99)}]
        sc = (ScalerConfig(mode="dynamic", init_scale=2.0 ** 8, window=3, hysteresis=1) if fp16
              else ScalerConfig(mode="none"))
        opt = MultiTensorAdamWOptimizer(groups, lr=1e-3, betas=(0.9, 0.95), weight_decay=0.1, max_grad_norm=0.5,
                                        param_dtype=dt, device=gpu, loss_scaler=sc)
        opt.track_skips(track)
        return opt

    fold, three, split = build(False), build(False), build(True)
    gen = torch.Generator(device=gpu).manual_seed(9)
    _say(f"ragged fold vs three launches, {dtype_name}")
    try:
        for step in range(12):
            for k, opts in enumerate(zip(fold.dsx_params, three.dsx_params, split.dsx_params)):
                g = (torch.randn(opts[0].shape, device=gpu, generator=gen) * 1e-2 * (256 if fp16 else 1)).to(dt)
                if step == 4 and k == 1:
                    g.view(-1)[3] = float("nan")
                for p in opts:
                    p.grad = g.clone()
            if step == 8:
                na, nb, nc = (o.clip_grad_norm_(0.01) for o in (fold, three, split))
                assert torch.equal(na, nb) and torch.equal(na, nc)
            _lib.call("dsx_set_tuning_fold", ctypes.c_int64(FOLD_DEFAULT))
            fold.step()
            split.step()
            _lib.call("dsx_set_tuning_fold", ctypes.c_int64(0))
            three.step()
    finally:
        _lib.call("dsx_set_tuning_fold", ctypes.c_int64(FOLD_DEFAULT))
    torch.cuda.synchronize()
    for other, tag in ((three, "three launches"), (split, "separate launches")):
        for i in range(len(shapes)):
            a, b = fold.store.views_of(i), other.store.views_of(i)
            for name in ("master", "exp_avg", "exp_avg_sq"):
                assert torch.equal(a[name].view(torch.int32), b[name].view(torch.int32)), (tag, i, name)
            assert torch.equal(fold.dsx_params[i].detach().view(torch.int16),
                               other.dsx_params[i].detach().view(torch.int16)), (tag, i, "param16")
        assert bytes(fold.read_state()) == bytes(other.read_state()), tag
    st = fold.read_state()
    assert st.t == 11 and st.overflow_count == 1 and st.error == 0
