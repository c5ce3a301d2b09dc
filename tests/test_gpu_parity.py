"""GPU parity: the HIP kernels (through libdsx.so's C ABI) against the CPU
oracle on the same seeded inputs. Integer/byte results and fp32 state must be
bit-identical: the kernels follow the oracle's operation order and rounding
(IEEE division/sqrt, explicit fma only), so any difference is a bug."""
from __future__ import annotations

import json
import math
import os
import sys

import numpy as np
import pytest

from helpers import (BF16, F16, MLP_CASE, f32_to_torch, make_state, np16_to_torch, step_digests,
                     torch16_to_np)

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _run_k2(gpu, p, m, v, g16, gdt, pdt, sc_host, with_p16=True):
    import torch
    from distributedspeed_amd import _lib, ops
    n = p.size
    tp, tm, tv = (f32_to_torch(a, gpu) for a in (p, m, v))
    tg = np16_to_torch(g16, gdt, gpu)
    tp16 = torch.empty(n, dtype=torch.float16 if pdt == F16 else torch.bfloat16, device=gpu) if with_p16 else None
    c = _lib.DsxStepScalars()
    c.skip = 0
    c.t = 1
    for k in ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2", "eps", "bc2s", "nss"):
        setattr(c, k, getattr(sc_host, k))
    scal = ops.scalars_from_host(c, gpu)
    ops.adamw_flat(tp, tm, tv, tp16, tg, scal)
    torch.cuda.synchronize()
    return (tp.cpu().numpy(), tm.cpu().numpy(), tv.cpu().numpy(),
            torch16_to_np(tp16) if with_p16 else None)


HYPERS = [
    dict(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01),   # config 1 (MLP)
    dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1),     # config 3 (Llama-3-8B)
    dict(lr=1e-2, beta1=0.3, beta2=0.5, eps=1e-6, weight_decay=0.0),      # lerp's |w| >= 0.5 branch, wd = 0
]


@pytest.mark.parametrize("n", [1, 3, 4, 7, 8, 1000, 65537, 262147])
@pytest.mark.parametrize("gdt,pdt", [(F16, F16), (BF16, BF16), (BF16, F16)])
@pytest.mark.parametrize("hi", range(len(HYPERS)))
def test_k2_single_step_bit_exact(gpu, oracle, n, gdt, pdt, hi):
    O = oracle
    h = O.Hyper(**HYPERS[hi])
    scale = 2.0 ** 16 if gdt == F16 else 1.0
    p, m, v, g16 = make_state(n, seed=1000 + n + hi, gdt=gdt, g_sigma=1e-3, scale=scale)
    t = 1 + hi * 3
    coef = 0.37 if hi == 1 else 1.0
    sc = O.step_scalars(h, t, O.inv_scale_of(scale), coef)
    _say(f"k2 n={n} gdt={gdt} pdt={pdt} hyper={hi}")
    gp, gm, gv, gp16 = _run_k2(gpu, p, m, v, g16, gdt, pdt, sc)
    rp, rm, rv, rp16 = p.copy(), m.copy(), v.copy(), np.empty(n, np.uint16)
    O.adamw(rp, rm, rv, rp16, pdt, g16, gdt, sc)
    for name, a, b in (("master", gp, rp), ("exp_avg", gm, rm), ("exp_avg_sq", gv, rv)):
        bad = O.ulp_diff_f32(a, b) != 0
        assert not bad.any(), f"{name}: {bad.sum()} mismatches, first at {np.flatnonzero(bad)[:5]}"
    assert np.array_equal(gp16, rp16), f"param16: {(gp16 != rp16).sum()} mismatches"


def test_k2_without_param16(gpu, oracle):
    O = oracle
    n = 4099
    p, m, v, g16 = make_state(n, 5, BF16, 1e-3)
    sc = O.step_scalars(O.Hyper(), 2, 1.0, 1.0)
    gp, gm, gv, _ = _run_k2(gpu, p, m, v, g16, BF16, BF16, sc, with_p16=False)
    O.adamw(p, m, v, None, BF16, g16, BF16, sc)
    assert np.array_equal(gp.view(np.uint32), p.view(np.uint32))
    assert np.array_equal(gm.view(np.uint32), m.view(np.uint32))
    assert np.array_equal(gv.view(np.uint32), v.view(np.uint32))


@pytest.mark.parametrize("n", [0, 1, 9, 1000, 1 << 20, 3_000_017])
@pytest.mark.parametrize("gdt", [F16, BF16])
def test_k1_norm_matches_oracle(gpu, oracle, n, gdt):
    import torch
    from distributedspeed_amd import ops
    O = oracle
    scale = 2.0 ** 16 if gdt == F16 else 1.0
    _, _, _, g16 = make_state(max(n, 1), 77 + n, gdt, 1e-3, scale=scale)
    g16 = g16[:n]
    st = ops.new_state(gpu, scale, 1)
    nparts = ops.suggest_partials(n)
    parts = torch.zeros(nparts, dtype=torch.float64, device=gpu)
    tg = np16_to_torch(g16, gdt, gpu) if n else torch.empty(0, dtype=torch.float16 if gdt == F16 else torch.bfloat16,
                                                             device=gpu)
    ops.unscale_norm(tg, st, parts, nparts)
    got = float(parts.sum().item())
    ref = O.sumsq(g16, gdt, O.inv_scale_of(scale)) if n else 0.0
    assert math.isfinite(got)
    assert got == pytest.approx(ref, rel=1e-12, abs=0.0)


@pytest.mark.parametrize("pos", ["first", "middle", "last", "tail"])
@pytest.mark.parametrize("bad", ["+inf", "-inf", "nan"])
@pytest.mark.parametrize("gdt", [F16, BF16])
def test_k1_detects_nonfinite(gpu, oracle, pos, bad, gdt):
    import torch
    from distributedspeed_amd import ops
    n = 100_003
    _, _, _, g16 = make_state(n, 3, gdt, 1e-3, edges=False)
    code = {F16: {"+inf": 0x7C00, "-inf": 0xFC00, "nan": 0x7E00},
            BF16: {"+inf": 0x7F80, "-inf": 0xFF80, "nan": 0x7FC0}}[gdt][bad]
    idx = {"first": 0, "middle": n // 2, "last": n - 1, "tail": n - 2}[pos]
    g16[idx] = code
    st = ops.new_state(gpu, 1.0, 1)
    parts = torch.zeros(ops.suggest_partials(n), dtype=torch.float64, device=gpu)
    ops.unscale_norm(np16_to_torch(g16, gdt, gpu), st, parts)
    assert not math.isfinite(float(parts.sum().item()))
    assert not math.isfinite(oracle.sumsq(g16, gdt, 1.0))


def _flat_run(gpu, O, n, gdt, pdt, hyper, scaler_cfg, steps, seed, g_sigma, inject=None, p_sigma=0.02,
              digests=None):
    """Run `steps` full steps through FlatStep and the oracle side by side;
    compare every step bit-for-bit. inject(step) -> index to set to +inf.
    digests: per-step SHA-256 digests the GPU arrays must also match."""
    import torch
    from distributedspeed_amd import ops
    from distributedspeed_amd.flat_step import AdamWHyper, FlatStep, ScalerConfig

    p, m, v, _ = make_state(n, seed, gdt, g_sigma, edges=False, mv_warm=False, p_sigma=p_sigma)
    p16 = O.cast16(p, pdt)
    hp = AdamWHyper(**hyper)
    sc = ScalerConfig(**scaler_cfg)
    fs = FlatStep(n, gpu, hp, sc)
    tp, tm, tv = (f32_to_torch(a, gpu) for a in (p, m, v))
    tp16 = np16_to_torch(p16, pdt, gpu)
    ospec = O.LossScalerSpec(scale=sc.init_scale if sc.mode != "none" else 1.0, window=sc.window,
                             hysteresis=sc.hysteresis if sc.mode == "dynamic" else 1, min_scale=sc.min_scale,
                             dynamic=sc.mode == "dynamic")
    orc = O.ZeroStepOracle(p, m, v, p16, pdt, gdt, O.Hyper(**hyper), ospec)
    rng = np.random.default_rng(seed + 1)
    history = []
    for step in range(1, steps + 1):
        scale = ospec.scale
        g32 = (rng.standard_normal(n) * g_sigma * scale).astype(np.float32)
        g16 = O.cast16(g32, gdt)
        if inject is not None:
            idx = inject(step)
            if idx is not None:
                g16[idx] = 0x7C00 if gdt == F16 else 0x7F80
        fs.step(tp, tm, tv, tp16, np16_to_torch(g16, gdt, gpu))
        r = orc.step(g16)
        scal = fs.read_scalars()
        st = fs.read_state()
        history.append((bool(scal.skip), st.scale, st.t))
        assert bool(scal.skip) == r.skipped, f"step {step}: skip {scal.skip} vs {r.skipped}"
        assert st.scale == r.scale_next, f"step {step}: scale {st.scale} vs {r.scale_next}"
        assert st.t == r.t
        if not r.skipped:
            assert scal.norm == pytest.approx(r.norm, rel=1e-12)
            assert scal.clip_coef == np.float32(r.clip_coef)
        gp, gm, gv = tp.cpu().numpy(), tm.cpu().numpy(), tv.cpu().numpy()
        for name, a, b in (("master", gp, p), ("exp_avg", gm, m), ("exp_avg_sq", gv, v)):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {step} {name} differs"
        assert np.array_equal(torch16_to_np(tp16), p16), f"step {step} param16 differs"
        if digests is not None:
            got = step_digests(gp, gm, gv, torch16_to_np(tp16))
            assert got == digests[step - 1], f"step {step}: {[k for k in got if got[k] != digests[step - 1][k]]}"
    return history, fs


def test_config1_mlp_ten_steps(gpu, oracle):
    """3-layer MLP partition, fp16, static scale 2^16, 10 steps."""
    n = 784 * 1024 + 1024 + 1024 * 1024 + 1024 + 1024 * 10 + 10
    assert n == 1_863_690
    _say("config1 mlp 10 steps")
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "config0_mlp_digests.json")) as f:
        golden = json.load(f)
    c = MLP_CASE
    assert golden["case"]["n"] == n == c["n"] and golden["case"]["steps"] == c["steps"] == 10
    hist, _ = _flat_run(gpu, oracle, n, c["gdt"], c["pdt"], c["hyper"],
                        dict(mode="static", init_scale=c["scale"]), steps=c["steps"], seed=c["seed"],
                        g_sigma=c["g_sigma"], digests=golden["digests"])
    assert [h[2] for h in hist] == list(range(1, 11))


def test_config2_gpt2_overflow_at_step3(gpu, oracle):
    """configs[1] semantics at reduced size: fp16, dynamic scale 2^16,
    hysteresis 1, clip 1.0; step 3 carries one +inf -> skip and halve."""
    n = 2_000_003
    inj_rng = np.random.default_rng(1000 + 1)
    idx3 = int(inj_rng.integers(0, n))
    _say("config2 gpt2 overflow")
    hist, fs = _flat_run(gpu, oracle, n, F16, F16,
                         dict(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, max_grad_norm=1.0),
                         dict(mode="dynamic", init_scale=2.0 ** 16, window=1000, hysteresis=1, min_scale=1.0),
                         steps=20, seed=1, g_sigma=1e-3, inject=lambda s: idx3 if s == 3 else None)
    assert [h[0] for h in hist] == [False, False, True] + [False] * 17
    assert hist[1][1] == 2.0 ** 16 and hist[2][1] == 2.0 ** 15
    assert hist[-1][2] == 19
    assert fs.read_state().overflow_count == 1


def test_scaler_sequence_config4_semantics(gpu, oracle):
    """configs[3] scaler (init 2^16, window 1000, hysteresis 2, min 1) over
    2000 steps with Bernoulli(1e-3) overflows, plus a dense variant that
    reaches every branch (growth, hysteresis countdown, min clamp)."""
    for (steps, prob, window, hyst, min_scale, seed) in ((2000, 1e-3, 1000, 2, 1.0, 4),
                                                        (600, 0.3, 7, 3, 2.0 ** 13, 5)):
        rng = np.random.default_rng(seed + 1000)
        flags = rng.random(steps) < prob
        _say(f"scaler sequence steps={steps} p={prob}")
        hist, _ = _flat_run(gpu, oracle, 1024, F16, F16,
                            dict(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, max_grad_norm=0.0),
                            dict(mode="dynamic", init_scale=2.0 ** 16, window=window, hysteresis=hyst,
                                 min_scale=min_scale),
                            steps=steps, seed=seed, g_sigma=1e-3,
                            inject=lambda s: 5 if flags[s - 1] else None)
        assert sum(h[0] for h in hist) == int(flags.sum())


def test_llama8b_shard_full_size_one_step(gpu, oracle):
    """configs[2] at full size (1,003,782,656 elements): one step, bit-exact
    against the oracle, plus the step's norm against an fp64 brute force."""
    import torch
    from distributedspeed_amd.flat_step import AdamWHyper, FlatStep, ScalerConfig
    O = oracle
    n = 1_003_782_656
    _say("llama8b full-size step: generating")
    gen = torch.Generator(device=gpu)
    gen.manual_seed(3)
    tp = torch.empty(n, dtype=torch.float32, device=gpu).normal_(0.0, 0.02, generator=gen)
    tg = torch.empty(n, dtype=torch.bfloat16, device=gpu)
    for s in range(0, n, 1 << 27):
        e = min(n, s + (1 << 27))
        tg[s:e].copy_(torch.empty(e - s, device=gpu).normal_(0.0, 5e-4, generator=gen))
    tm = torch.zeros(n, dtype=torch.float32, device=gpu)
    tv = torch.zeros(n, dtype=torch.float32, device=gpu)
    tp16 = tp.to(torch.bfloat16)
    p = tp.cpu().numpy()
    g16 = torch16_to_np(tg)
    hyper = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, max_grad_norm=1.0)
    fs = FlatStep(n, gpu, AdamWHyper(**hyper), ScalerConfig(mode="none"))
    _say("llama8b full-size step: gpu step")
    fs.step(tp, tm, tv, tp16, tg)
    scal = fs.read_scalars()
    _say("llama8b full-size step: oracle step")
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    p16 = np.empty(n, np.uint16)
    ss = O.sumsq(g16, BF16, 1.0)
    assert scal.sumsq == pytest.approx(ss, rel=1e-12)
    coef = O.clip_coef(math.sqrt(ss), 1.0)
    assert coef < 1.0 and scal.clip_coef == np.float32(coef)
    O.adamw(p, m, v, p16, BF16, g16, BF16, O.step_scalars(O.Hyper(**hyper), 1, 1.0, coef))
    _say("llama8b full-size step: compare")
    assert np.array_equal(tp.cpu().numpy().view(np.uint32), p.view(np.uint32))
    assert np.array_equal(tm.cpu().numpy().view(np.uint32), m.view(np.uint32))
    assert np.array_equal(tv.cpu().numpy().view(np.uint32), v.view(np.uint32))
    assert np.array_equal(torch16_to_np(tp16), p16)


def test_multi_tensor_equals_flat(gpu, oracle):
    """K3 over a ragged list (including tensors at unaligned offsets) is
    bit-identical to K2 over the same elements; its norm matches K1's."""
    import torch
    from distributedspeed_amd import ops
    O = oracle
    sizes = [4096 * 3, 1, 7, 14336 + 3, 65536 * 2 + 5, 4096, 9]
    offs = []
    pos = 0
    for i, s in enumerate(sizes):
        pos += (i % 3)  # 0, 1 or 2 elements of padding -> some views are unaligned
        offs.append(pos)
        pos += s
    total = pos
    p, m, v, g16 = make_state(total, 11, F16, 1e-3, scale=2.0 ** 10)
    h = O.Hyper(lr=1e-3, weight_decay=0.05)
    sc = O.step_scalars(h, 3, O.inv_scale_of(2.0 ** 10), 0.5)
    # flat reference through K2 on the whole buffer
    gp, gm, gv, gp16 = _run_k2(gpu, p, m, v, g16, F16, F16, sc)
    # ragged list through K3
    tp, tm, tv = (f32_to_torch(a, gpu) for a in (p, m, v))
    tg = np16_to_torch(g16, F16, gpu)
    tp16 = torch.zeros(total, dtype=torch.float16, device=gpu)
    views = lambda t: [t[o:o + s] for o, s in zip(offs, sizes)]  # noqa: E731
    table = ops.ChunkTable(views(tp), views(tm), views(tv), views(tp16), views(tg), chunk_elems=4096)
    c = oracle  # noqa: F841
    from distributedspeed_amd import _lib
    hs = _lib.DsxStepScalars()
    for k in ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2", "eps", "bc2s", "nss"):
        setattr(hs, k, getattr(sc, k))
    scal = ops.scalars_from_host(hs, gpu)
    ops.adamw_multi(table, scal)
    st = ops.new_state(gpu, 2.0 ** 10, 1)
    parts = torch.zeros(64, dtype=torch.float64, device=gpu)
    ops.unscale_norm_multi(table, st, parts, 64)
    torch.cuda.synchronize()
    covered = np.zeros(total, bool)
    for o, s in zip(offs, sizes):
        covered[o:o + s] = True
    for name, a, b in (("master", tp.cpu().numpy(), gp), ("exp_avg", tm.cpu().numpy(), gm),
                       ("exp_avg_sq", tv.cpu().numpy(), gv)):
        assert np.array_equal(a[covered].view(np.uint32), b[covered].view(np.uint32)), name
        # padding elements are not part of any tensor and must be untouched
        orig = {"master": p, "exp_avg": m, "exp_avg_sq": v}[name]
        assert np.array_equal(a[~covered].view(np.uint32), orig[~covered].view(np.uint32)), name
    assert np.array_equal(torch16_to_np(tp16)[covered], gp16[covered])
    ref = sum(O.sumsq(np.ascontiguousarray(g16[o:o + s]), F16, O.inv_scale_of(2.0 ** 10)) for o, s in zip(offs, sizes))
    assert float(parts.sum().item()) == pytest.approx(ref, rel=1e-12)


def test_skip_leaves_state_bit_identical(gpu, oracle):
    import torch
    from distributedspeed_amd.flat_step import AdamWHyper, FlatStep, ScalerConfig
    n = 10_007
    p, m, v, g16 = make_state(n, 21, F16, 1e-3, scale=2.0 ** 16)
    g16[n - 1] = 0x7E00  # NaN in the tail
    tp, tm, tv = (f32_to_torch(a, gpu) for a in (p, m, v))
    tp16 = np16_to_torch(oracle.cast16(p, F16), F16, gpu)
    before = [t.clone() for t in (tp, tm, tv, tp16)]
    fs = FlatStep(n, gpu, AdamWHyper(max_grad_norm=1.0),
                  ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, hysteresis=2))
    fs.step(tp, tm, tv, tp16, np16_to_torch(g16, F16, gpu))
    st = fs.read_state()
    assert fs.read_scalars().skip == 1 and st.t == 0 and st.overflow_count == 1
    assert st.scale == 2.0 ** 16 and st.hyst_left == 1  # hysteresis absorbs the first overflow
    for a, b in zip(before, (tp, tm, tv, tp16)):
        assert torch.equal(a.view(torch.uint8) if a.dtype != torch.float32 else a.view(torch.int32),
                           b.view(torch.uint8) if b.dtype != torch.float32 else b.view(torch.int32))


def test_short_bias_table_flags_error_and_skips(gpu):
    """A bias-correction table shorter than t is reported through the state's
    error bits and the step is skipped; the kernel still exits normally."""
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, ScalerConfig
    n = 4096
    tp = torch.ones(n, device=gpu)
    tm, tv = torch.zeros(n, device=gpu), torch.zeros(n, device=gpu)
    tg = torch.full((n,), 0.5, dtype=torch.bfloat16, device=gpu)
    st = ops.new_state(gpu, 1.0, 1)
    sc = ops.new_scalars(gpu)
    parts = torch.zeros(8, dtype=torch.float64, device=gpu)
    bc = torch.zeros(2, dtype=torch.float64, device=gpu)
    ops.zero_step_flat(tp, tm, tv, None, tg, st, ScalerConfig().to_c(), AdamWHyper().to_c(), bc, 0, parts, 8, sc)
    s = ops.read_state(st)
    assert s.error & _lib.DSX_STATE_ERR_BC_TABLE
    assert ops.read_scalars(sc).skip == 1
    assert torch.equal(tp, torch.ones(n, device=gpu))


def test_host_rejects_bad_arguments(gpu):
    import torch
    from distributedspeed_amd import _lib, ops
    n = 1024
    buf = torch.zeros(n + 4, device=gpu)
    tm, tv = torch.zeros(n, device=gpu), torch.zeros(n, device=gpu)
    tg = torch.zeros(n, dtype=torch.bfloat16, device=gpu)
    sc = ops.new_scalars(gpu)
    with pytest.raises(ValueError):  # master view 4 bytes off alignment
        ops.adamw_flat(buf[1:n + 1], tm, tv, None, tg, sc)
    with pytest.raises(ValueError):
        ops.adamw_flat(torch.zeros(n + 1, device=gpu), tm, tv, None, tg, sc)
    with pytest.raises(TypeError):
        ops.adamw_flat(buf[:n], tm, tv, None, tg.to(torch.int16), sc)
    with pytest.raises(_lib.DsxError):  # the C layer's own check, reached directly
        _lib.call("dsx_adamw_flat", buf[1:].data_ptr(), tm.data_ptr(), tv.data_ptr(), None, 2, tg.data_ptr(), 2,
                  n, sc.data_ptr(), None)


def test_k2_fp32_grads_bit_exact(gpu, oracle):
    """fp32 training: fp32 grads, no 16-bit cast (the master is the param)."""
    import torch
    O = oracle
    n = 100_003
    rng = np.random.default_rng(31)
    p = (rng.standard_normal(n) * 0.02).astype(np.float32)
    m = (rng.standard_normal(n) * 1e-4).astype(np.float32)
    v = (np.abs(rng.standard_normal(n)) * 1e-6).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    g[:4] = [0.0, -0.0, 1e-40, 3.0e38]
    sc = O.step_scalars(O.Hyper(lr=1e-3, weight_decay=0.02), 4, 1.0, 0.25)
    from distributedspeed_amd import _lib, ops
    c = _lib.DsxStepScalars()
    for k in ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2", "eps", "bc2s", "nss"):
        setattr(c, k, getattr(sc, k))
    tp, tm, tv, tg = (f32_to_torch(a, gpu) for a in (p, m, v, g))
    ops.adamw_flat(tp, tm, tv, None, tg, ops.scalars_from_host(c, gpu))
    st = ops.new_state(gpu, 1.0, 1)
    parts = torch.zeros(ops.suggest_partials(n), dtype=torch.float64, device=gpu)
    ops.unscale_norm(tg, st, parts)
    O.adamw(p, m, v, None, F16, g, O.F32, sc)
    for a, b in ((tp, p), (tm, m), (tv, v)):
        assert np.array_equal(a.cpu().numpy().view(np.uint32), b.view(np.uint32))
    assert float(parts.sum().item()) == pytest.approx(O.sumsq(g, O.F32, 1.0), rel=1e-12)


def test_finalize_groups_matches_oracle(gpu, oracle):
    """Per-group scalars (lr, betas, eps, weight decay, t offset) from one
    K0 launch; global norm, clip and scaler. Group 2 joined after step 2, so
    it steps with t - 2."""
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import BiasCorrectionTable, ScalerConfig
    O = oracle
    hyps = [O.Hyper(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.1, max_grad_norm=1.0),
            O.Hyper(lr=5e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0, max_grad_norm=1.0),
            O.Hyper(lr=2e-4, beta1=0.8, beta2=0.95, eps=1e-6, weight_decay=0.05, max_grad_norm=1.0)]
    offs = [0, 0, 2]
    host = _lib.DsxState()
    host.scale, host.hyst_left, host.t = 8.0, 1, 2
    st = torch.frombuffer(bytearray(bytes(host)), dtype=torch.uint8).to(gpu)
    tabs = [BiasCorrectionTable(gpu, h.beta1, h.beta2) for h in hyps]
    out = torch.zeros(ops.SCALARS_BYTES * 3, dtype=torch.uint8, device=gpu)
    parts = torch.tensor([4.0, 5.0, 7.0], dtype=torch.float64, device=gpu)  # sumsq 16 -> norm 4 -> clipped
    cfg = ScalerConfig(mode="static", init_scale=8.0).to_c()
    hc = [_lib.DsxAdamwHyper(h.lr, h.beta1, h.beta2, h.eps, h.weight_decay, h.max_grad_norm, h.clip_eps)
          for h in hyps]
    for t in range(3, 7):
        ops.finalize_groups(parts, 3, st, cfg, hc, [x.table for x in tabs], offs, tabs[0].length, out)
        s = ops.read_state(st)
        assert s.error == 0 and s.t == t and s.scale == 8.0
        for k, h in enumerate(hyps):
            got = ops.read_scalars(out[k * ops.SCALARS_BYTES:(k + 1) * ops.SCALARS_BYTES])
            ref = O.step_scalars(h, t - offs[k], O.inv_scale_of(8.0), O.clip_coef(4.0, 1.0))
            assert got.skip == 0 and got.t == t - offs[k]
            assert got.norm == 4.0
            for name in ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2", "eps", "bc2s", "nss"):
                assert np.float32(getattr(got, name)) == np.float32(getattr(ref, name)), (t, k, name)
    # an offset beyond the current step is an error: the step is skipped and flagged
    ops.finalize_groups(parts, 3, st, cfg, hc, [x.table for x in tabs], [0, 0, 7], tabs[0].length, out)
    s = ops.read_state(st)
    assert s.error & _lib.DSX_STATE_ERR_BC_TABLE and s.t == 6
    assert ops.read_scalars(out[:ops.SCALARS_BYTES]).skip == 1


def test_multi_tensor_groups(gpu, oracle):
    """K3 with two parameter groups: each tensor uses its group's scalars."""
    import torch
    from distributedspeed_amd import _lib, ops
    O = oracle
    sizes = [1000, 4096, 7, 20000]
    groups = [0, 1, 0, 1]
    hyps = [O.Hyper(lr=1e-3, weight_decay=0.1), O.Hyper(lr=3e-3, beta1=0.5, beta2=0.9, weight_decay=0.0)]
    t = 2
    arrs = [make_state(s, 40 + i, BF16, 1e-3, edges=False) for i, s in enumerate(sizes)]
    tens = [[f32_to_torch(a[j], gpu) for j in range(3)] for a in arrs]
    tg = [np16_to_torch(a[3], BF16, gpu) for a in arrs]
    tp16 = [torch.empty(s, dtype=torch.bfloat16, device=gpu) for s in sizes]
    table = ops.ChunkTable([x[0] for x in tens], [x[1] for x in tens], [x[2] for x in tens], tp16, tg,
                           groups=groups, chunk_elems=1024)
    scal = torch.zeros(2 * ops.SCALARS_BYTES, dtype=torch.uint8, device=gpu)
    for k, h in enumerate(hyps):
        sc = O.step_scalars(h, t, 1.0, 1.0)
        c = _lib.DsxStepScalars()
        for f in ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2", "eps", "bc2s", "nss"):
            setattr(c, f, getattr(sc, f))
        scal[k * ops.SCALARS_BYTES:(k + 1) * ops.SCALARS_BYTES] = ops.scalars_from_host(c, gpu)
    ops.adamw_multi(table, scal)
    torch.cuda.synchronize()
    for i, (p, m, v, g16) in enumerate(arrs):
        p16 = np.empty(p.size, np.uint16)
        O.adamw(p, m, v, p16, BF16, g16, BF16, O.step_scalars(hyps[groups[i]], t, 1.0, 1.0))
        assert np.array_equal(tens[i][0].cpu().numpy().view(np.uint32), p.view(np.uint32)), i
        assert np.array_equal(tens[i][1].cpu().numpy().view(np.uint32), m.view(np.uint32)), i
        assert np.array_equal(tens[i][2].cpu().numpy().view(np.uint32), v.view(np.uint32)), i
        assert np.array_equal(torch16_to_np(tp16[i]), p16), i


def test_traffic_probe_changes_nothing(gpu):
    """dsx_traffic_probe_flat (K2's traffic without its math, for bench.py)
    writes back what it reads: on a partition whose param16 is the cast of
    its master every buffer keeps its bits, in both 16-bit types, through the
    vector slots and the tail, in the small and the large launch shapes."""
    import torch
    from distributedspeed_amd import ops
    for n, dt in ((1_000_003, torch.bfloat16), (3_000_011, torch.float16), (402_653_187, torch.bfloat16)):
        _say(f"traffic probe n={n} {dt}")
        gen = torch.Generator(device=gpu).manual_seed(n)
        master = torch.randn(n, device=gpu, generator=gen)
        m = torch.randn(n, device=gpu, generator=gen)
        v = torch.rand(n, device=gpu, generator=gen)
        p16 = master.to(dt)
        g = torch.randn(n, device=gpu, generator=gen).to(dt)
        bits = [t.view(torch.int32 if t.dtype == torch.float32 else torch.int16) for t in (master, m, v, p16, g)]
        before = [b.clone() for b in bits]
        ops.traffic_probe_flat(master, m, v, p16, g)
        torch.cuda.synchronize()
        for name, a, b in zip(("master", "exp_avg", "exp_avg_sq", "param16", "grad"), bits, before):
            assert torch.equal(a, b), (n, name)
        del master, m, v, p16, g, bits, before
        torch.cuda.empty_cache()


def test_k2_in_parts_gives_identical_bits(gpu, oracle):
    """K2 issued as consecutive launches over parts of the partition
    (dsx_set_tuning_k2_chunk; the default splits above 2^26 elements)
    computes the oracle's bits: parts of ~2^20 elements, the last one
    shorter and holding the ragged tail, in both 16-bit types; one launch
    (chunk 0) agrees too; the default is restored afterwards."""
    from distributedspeed_amd import _lib
    O = oracle
    try:
        for n, dt, chunk in ((3_000_011, BF16, 1 << 20), (2_621_443, F16, 1 << 20), (3_000_011, BF16, 0)):
            p, m, v, g16 = make_state(n, 23, dt, 1e-3)
            sc = O.step_scalars(O.Hyper(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1), 3, 1.0, 0.7)
            rp, rm, rv, rp16 = p.copy(), m.copy(), v.copy(), np.empty(n, np.uint16)
            O.adamw(rp, rm, rv, rp16, dt, g16, dt, sc)
            assert _lib.call("dsx_set_tuning_k2_chunk", chunk) == 0
            _say(f"k2 in parts n={n} dtype={dt} chunk={chunk}")
            gp, gm, gv, gp16 = _run_k2(gpu, p, m, v, g16, dt, dt, sc)
            for name, a, b in (("master", gp, rp), ("exp_avg", gm, rm), ("exp_avg_sq", gv, rv)):
                assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (name, n, chunk)
            assert np.array_equal(gp16, rp16), (n, chunk)
    finally:
        _lib.call("dsx_set_tuning_k2_chunk", 1 << 26)


def test_k2_launch_shapes_give_identical_bits(gpu, oracle):
    """Every K2 launch shape the tuning calls can select (one block per CU
    or the automatic grid -- here one trip per block --, slots per thread
    2/4/8, drain on/off, grids on 1, 7 or 8 eighths of the CUs) computes the
    same bits as the oracle; the automatic shape is restored afterwards."""
    from distributedspeed_amd import _lib
    O = oracle
    n = 3_000_011
    p, m, v, g16 = make_state(n, 21, BF16, 1e-3)
    sc = O.step_scalars(O.Hyper(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1), 4, 1.0, 0.6)
    rp, rm, rv, rp16 = p.copy(), m.copy(), v.copy(), np.empty(n, np.uint16)
    O.adamw(rp, rm, rv, rp16, BF16, g16, BF16, sc)
    try:
        for bpc in (0, 1):
            for unroll in (2, 4, 8):
                for drain in (0, 1):
                    for eighths in (1, 7, 8):
                        assert _lib.call("dsx_set_tuning", 2, bpc, unroll, 1) == 0
                        assert _lib.call("dsx_set_tuning_k2", eighths, drain) == 0
                        case = (bpc, unroll, drain, eighths)
                        _say(f"k2 shape bpc={bpc} unroll={unroll} drain={drain} eighths={eighths}")
                        gp, gm, gv, gp16 = _run_k2(gpu, p, m, v, g16, BF16, BF16, sc)
                        for name, a, b in (("master", gp, rp), ("exp_avg", gm, rm), ("exp_avg_sq", gv, rv)):
                            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (name,) + case
                        assert np.array_equal(gp16, rp16), case
    finally:
        _lib.call("dsx_set_tuning", 2, 0, 0, 1)
        _lib.call("dsx_set_tuning_k2", 0, -1)


def test_k3_launch_shapes_give_identical_bits(gpu, oracle):
    """Every K3 shape the tuning can select (one block per CU up to many
    blocks per CU, 1/2/4 slots, drain on/off, and the automatic choice) is
    bit-identical to K2 over the same elements of a ragged list that has
    aligned and unaligned tensors; the automatic shape is restored afterwards."""
    import torch
    from distributedspeed_amd import _lib, ops
    O = oracle
    sizes = [65536 * 3 + 8, 3, 4096 * 5, 17, 65536 + 1, 4096 * 2]
    offs, pos = [], 0
    for i, s in enumerate(sizes):
        pos += (i % 2)
        offs.append(pos)
        pos += s
    total = pos
    p, m, v, g16 = make_state(total, 12, BF16, 1e-3)
    sc = O.step_scalars(O.Hyper(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1), 2, 1.0, 0.8)
    gp, gm, gv, gp16 = _run_k2(gpu, p, m, v, g16, BF16, BF16, sc)
    hs = _lib.DsxStepScalars()
    for k in ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2", "eps", "bc2s", "nss"):
        setattr(hs, k, getattr(sc, k))
    covered = np.zeros(total, bool)
    for o, s in zip(offs, sizes):
        covered[o:o + s] = True
    try:
        for shape in ((0, 1, 1, -1), (1, 1, 1, 0), (1, 2, 1, 1), (1, 4, 1, 0), (8, 1, 1, 1), (64, 2, 1, 1),
                      (64, 4, 0, 1), (512, 2, 1, 0)):
            _lib.call("dsx_set_tuning_multi", *shape)
            _say(f"k3 shape {shape}")
            tp, tm, tv = (f32_to_torch(a, gpu) for a in (p, m, v))
            tg = np16_to_torch(g16, BF16, gpu)
            tp16 = torch.zeros(total, dtype=torch.bfloat16, device=gpu)
            views = lambda t: [t[o:o + s] for o, s in zip(offs, sizes)]  # noqa: E731
            table = ops.ChunkTable(views(tp), views(tm), views(tv), views(tp16), views(tg), chunk_elems=4096)
            ops.adamw_multi(table, ops.scalars_from_host(hs, gpu))
            torch.cuda.synchronize()
            for name, a, b in (("master", tp.cpu().numpy(), gp), ("exp_avg", tm.cpu().numpy(), gm),
                               ("exp_avg_sq", tv.cpu().numpy(), gv)):
                assert np.array_equal(a[covered].view(np.uint32), b[covered].view(np.uint32)), (name, shape)
            assert np.array_equal(torch16_to_np(tp16)[covered], gp16[covered]), shape
    finally:
        _lib.call("dsx_set_tuning_multi", 0, 1, 1, -1)


def test_k3_several_chunks_per_block_give_identical_bits(gpu, oracle):
    """K3 with more chunks than blocks, so that every block steps several in
    turn (each chunk's records read while the previous one streams): 700
    tensors of 1 to 20000 elements, every third one off the 16-byte grid
    (element-wise path) and the others with ragged tails, in 4096-element
    chunks; one block per CU with 1, 2 and 4 slots, drain on and off.
    Bit-identical to K2 over the same elements."""
    import torch
    from distributedspeed_amd import _lib, ops
    O = oracle
    rng = np.random.default_rng(31)
    sizes = [int(x) for x in rng.integers(1, 20001, size=700)]
    offs, pos = [], 0
    for i, s in enumerate(sizes):
        pos = (pos + 3) // 4 * 4 + (1 if i % 3 == 2 else 0)
        offs.append(pos)
        pos += s
    total = pos
    p, m, v, g16 = make_state(total, 13, F16, 1e-3 * 1024)
    sc = O.step_scalars(O.Hyper(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01), 3, 1.0 / 1024, 0.6)
    gp, gm, gv, gp16 = _run_k2(gpu, p, m, v, g16, F16, F16, sc)
    hs = _lib.DsxStepScalars()
    for k in ("inv_scale", "clip_coef", "decay", "w1", "w1c", "b2", "val2", "eps", "bc2s", "nss"):
        setattr(hs, k, getattr(sc, k))
    covered = np.zeros(total, bool)
    for o, s in zip(offs, sizes):
        covered[o:o + s] = True
    try:
        for shape in ((1, 1, 1, 0), (1, 2, 1, 0), (1, 2, 1, 1), (1, 4, 1, 1), (1, 2, 0, 0)):
            _lib.call("dsx_set_tuning_multi", *shape)
            tp, tm, tv = (f32_to_torch(a, gpu) for a in (p, m, v))
            tg = np16_to_torch(g16, F16, gpu)
            tp16 = torch.zeros(total, dtype=torch.float16, device=gpu)
            views = lambda t: [t[o:o + s] for o, s in zip(offs, sizes)]  # noqa: E731
            table = ops.ChunkTable(views(tp), views(tm), views(tv), views(tp16), views(tg), chunk_elems=4096)
            _say(f"k3 shape {shape}, {table.nchunks} chunks")
            assert table.nchunks > 2 * 256  # more chunks than any one-block-per-CU grid holds
            ops.adamw_multi(table, ops.scalars_from_host(hs, gpu))
            torch.cuda.synchronize()
            for name, a, b in (("master", tp.cpu().numpy(), gp), ("exp_avg", tm.cpu().numpy(), gm),
                               ("exp_avg_sq", tv.cpu().numpy(), gv)):
                assert np.array_equal(a[covered].view(np.uint32), b[covered].view(np.uint32)), (name, shape)
            assert np.array_equal(torch16_to_np(tp16)[covered], gp16[covered]), shape
            assert not torch16_to_np(tp16)[~covered].any()  # nothing written between the tensors
    finally:
        _lib.call("dsx_set_tuning_multi", 0, 1, 1, -1)


@pytest.mark.parametrize("gdt", [F16, BF16, 0], ids=["fp16", "bf16", "fp32"])
def test_k1_multi_both_shapes_match_oracle(gpu, oracle, gdt):
    """K1 over a chunk table in both of its shapes -- one wave per chunk (at
    most 16 chunks per partial block) and one block per chunk (more) -- over
    the same ragged list (tensors off the 16-byte grid, ragged tails, tiny
    tensors): each within 1e-12 of the oracle's fp64 sum. The shape follows
    from the chunk and partial counts alone, which the one-call step shares."""
    import torch
    from distributedspeed_amd import ops
    O = oracle
    rng = np.random.default_rng(41)
    sizes = [int(x) for x in rng.integers(1, 9000, size=60)] + [2048, 4096, 3, 20000]
    offs, pos = [], 0
    for i, s in enumerate(sizes):
        pos += i % 3
        offs.append(pos)
        pos += s
    total = pos
    scale = 2.0 ** 10 if gdt == F16 else 1.0
    g32 = (rng.standard_normal(total) * 1e-3 * scale).astype(np.float32)
    g = g32 if gdt == 0 else O.cast16(g32, gdt)
    tdt = {F16: torch.float16, BF16: torch.bfloat16, 0: torch.float32}[gdt]
    tg = (torch.from_numpy(g.view(np.int16)).view(tdt) if gdt else torch.from_numpy(g)).to(gpu)
    f32 = torch.zeros(total, device=gpu)
    views = lambda t: [t[o:o + s] for o, s in zip(offs, sizes)]  # noqa: E731
    table = ops.ChunkTable(views(f32), views(f32), views(f32), None, views(tg), chunk_elems=2048)
    ref = sum(O.sumsq(np.ascontiguousarray(g[o:o + s]), gdt if gdt else 0, O.inv_scale_of(scale))
              for o, s in zip(offs, sizes))
    st = ops.new_state(gpu, scale, 1)
    for nparts in (4, (table.nchunks + 15) // 16, 256):  # block, wave (the bound), wave
        parts = torch.zeros(nparts, dtype=torch.float64, device=gpu)
        ops.unscale_norm_multi(table, st, parts, nparts)
        torch.cuda.synchronize()
        got = float(parts.sum().item())
        assert got == pytest.approx(ref, rel=1e-12), (nparts, table.nchunks, got, ref)
