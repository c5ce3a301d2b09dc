"""BASELINE configs at their real shapes (parity-test cases).

GPT-2-small fp16 partition, 148 tensors / 124,439,808 elements,
            dynamic scale 2^16, hysteresis 1, clip 1.0, 20 steps, one +inf at
            a seeded index in step 3 -> skip and halve. Every step is compared
            bit-for-bit with the oracle.
the ragged Llama layout, 289 tensors / 8,310,226,944 elements,
            through K3 (one launch per pass over the chunk table). Checked by
            a size-independent property: K3 over the ragged list and K2 over
            the same values laid out flat give identical results, compared by
            exact per-tensor integer checksums of the fp32/16-bit bit patterns.
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

from helpers import F16, torch16_to_np

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def gpt2_small_shapes():
    """wte, wpe, 12 x {ln_1 w,b; c_attn w,b; attn c_proj w,b; ln_2 w,b;
    c_fc w,b; mlp c_proj w,b}, ln_f w,b (head tied to wte): 148 tensors."""
    d, ff, vocab, ctx = 768, 3072, 50257, 1024
    shapes = [(vocab, d), (ctx, d)]
    for _ in range(12):
        shapes += [(d,), (d,), (d, 3 * d), (3 * d,), (d, d), (d,), (d,), (d,), (d, ff), (ff,), (ff, d), (d,)]
    shapes += [(d,), (d,)]
    return shapes


def llama_ragged_shapes():
    """32 x (4096^2 x4, 4096x14336 x2, 14336x4096, 4096 x2) + 128256x4096."""
    shapes = []
    for _ in range(32):
        shapes += [(4096, 4096)] * 4 + [(4096, 14336)] * 2 + [(14336, 4096)] + [(4096,)] * 2
    shapes.append((128256, 4096))
    return shapes


def test_shape_counts():
    g = gpt2_small_shapes()
    assert len(g) == 148 and sum(math.prod(s) for s in g) == 124_439_808
    r = llama_ragged_shapes()
    assert len(r) == 289 and sum(math.prod(s) for s in r) == 8_310_226_944


def test_config2_gpt2_full_size_twenty_steps(gpu, oracle):
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer
    O = oracle
    params = [torch.nn.Parameter(torch.empty(s, device=gpu).normal_(0, 0.02)) for s in gpt2_small_shapes()]
    opt = AdamWOptimizer(params, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, max_grad_norm=1.0,
                         param_dtype=torch.float16,
                         loss_scaler=ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, window=1000, hysteresis=1,
                                                  min_scale=1.0))
    flat = opt.flat
    n = flat.numel
    assert n == 124_439_808  # every GPT-2 tensor size is a multiple of 8: no padding
    p = flat.master.cpu().numpy().copy()
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    p16 = torch16_to_np(flat.param16).copy()
    spec = O.LossScalerSpec(scale=2.0 ** 16, window=1000, hysteresis=1, min_scale=1.0)
    orc = O.ZeroStepOracle(p, m, v, p16, F16, F16, O.Hyper(lr=1e-4, weight_decay=0.01, max_grad_norm=1.0), spec)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(1)
    inj = int(np.random.default_rng(1001).integers(0, n))
    skips = []
    for step in range(1, 21):
        _say(f"config2 step {step}")
        g = torch.empty(n, device=gpu).normal_(0.0, 1e-3, generator=gen).mul_(spec.scale).to(torch.float16)
        if step == 3:
            g[inj] = float("inf")
        flat.grad.copy_(g)
        g16 = torch16_to_np(g)
        opt.step()
        r = orc.step(g16)
        st = opt.read_state()
        skips.append(bool(st.last_skip))
        assert bool(st.last_skip) == r.skipped and st.scale == r.scale_next and st.t == r.t, step
        assert np.array_equal(flat.master.cpu().numpy().view(np.uint32), p.view(np.uint32)), step
        assert np.array_equal(flat.exp_avg.cpu().numpy().view(np.uint32), m.view(np.uint32)), step
        assert np.array_equal(flat.exp_avg_sq.cpu().numpy().view(np.uint32), v.view(np.uint32)), step
        assert np.array_equal(torch16_to_np(flat.param16), p16), step
    assert skips == [False, False, True] + [False] * 17
    st = opt.read_state()
    assert st.scale == 2.0 ** 15 and st.t == 19 and st.overflow_count == 1


def _checksums(tensors):
    """Exact integer checksums of bit patterns: (sum, index-weighted sum) as int64."""
    import torch
    out = []
    for t in tensors:
        iv = t.view(torch.int32) if t.dtype == torch.float32 else t.view(torch.int16).to(torch.int32)
        w = torch.arange(1, iv.numel() + 1, device=iv.device, dtype=torch.int64) % 65521
        out.append((int(iv.sum(dtype=torch.int64)), int((iv.to(torch.int64) * w).sum())))
    return out


def test_config4_ragged_k3_equals_flat_k2_full_size(gpu, oracle):
    """configs[3] at full size, three steps (the second with an inf grad,
    tolerated under hysteresis 2): K3 over the 289 tensors and K2 over the
    same values laid out flat give bit-identical master / exp_avg / exp_avg_sq
    / fp16 params and the same skip, clip and scaler decisions. Both forms are
    resident at once (249 GB): the ragged tensors' grads are views of the
    flat grad buffer, which both steps read."""
    import torch
    from distributedspeed_amd import ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    shapes = llama_ragged_shapes()
    sizes = [math.prod(s) for s in shapes]
    n = sum(sizes)
    hyper = AdamWHyper(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, max_grad_norm=1.0)
    scfg = ScalerConfig(mode="dynamic", init_scale=2.0 ** 16, window=1000, hysteresis=2, min_scale=1.0)
    bc = BiasCorrectionTable(gpu, hyper.beta1, hyper.beta2)
    _say("config4 full size: flat buffers")
    flat = [torch.empty(n, device=gpu) for _ in range(3)]
    p16f = torch.empty(n, dtype=torch.float16, device=gpu)
    g = torch.empty(n, dtype=torch.float16, device=gpu)
    off = 0
    bounds = []
    for i, k in enumerate(sizes):
        gen = torch.Generator(device=gpu)
        gen.manual_seed(10_000 + i)
        flat[0][off:off + k].normal_(0.0, 0.02, generator=gen)
        flat[1][off:off + k].normal_(0.0, 1e-4, generator=gen)
        flat[2][off:off + k].normal_(0.0, 1e-6, generator=gen).abs_()
        g[off:off + k].copy_(torch.empty(k, device=gpu).normal_(0.0, 1e-3, generator=gen).mul_(2.0 ** 16))
        bounds.append((off, off + k))
        off += k
    _say("config4 full size: ragged tensors")
    rag = [[flat[j][a:b].clone() for (a, b) in bounds] for j in range(3)]
    rp16 = [torch.empty(b - a, dtype=torch.float16, device=gpu) for (a, b) in bounds]
    rg = [g[a:b] for (a, b) in bounds]
    table = ops.ChunkTable(rag[0], rag[1], rag[2], rp16, rg)
    st_r, st_f = ops.new_state(gpu, scfg.init_scale, scfg.hysteresis), ops.new_state(gpu, scfg.init_scale,
                                                                                     scfg.hysteresis)
    nparts = ops.suggest_partials(n)
    parts_r = torch.zeros(nparts, dtype=torch.float64, device=gpu)
    parts_f = torch.zeros(nparts, dtype=torch.float64, device=gpu)
    out_r, out_f = ops.new_scalars(gpu), ops.new_scalars(gpu)
    bad = bounds[150][0] + 12_345
    for step in range(3):
        _say(f"config4 full size: step {step}")
        if step == 1:
            keep = g[bad].clone()
            g[bad] = float("inf")
        ops.unscale_norm_multi(table, st_r, parts_r, nparts)
        ops.finalize(parts_r, nparts, st_r, scfg.to_c(), hyper.to_c(), bc.table, bc.length, out_r)
        ops.adamw_multi(table, out_r)
        ops.zero_step_flat(flat[0], flat[1], flat[2], p16f, g, st_f, scfg.to_c(), hyper.to_c(), bc.table,
                           bc.length, parts_f, nparts, out_f)
        if step == 1:
            g[bad] = keep
        sr, sf = ops.read_scalars(out_r), ops.read_scalars(out_f)
        assert sr.skip == sf.skip == (1 if step == 1 else 0), step
        if not sr.skip:
            assert sr.norm == pytest.approx(sf.norm, rel=1e-12)
            assert sr.clip_coef == sf.clip_coef and sr.clip_coef < 1.0
        ar, af = ops.read_state(st_r), ops.read_state(st_f)
        for k in ("scale", "good_steps", "hyst_left", "t", "overflow_count", "error"):
            assert getattr(ar, k) == getattr(af, k), (step, k)
    assert (ar.t, ar.overflow_count, ar.hyst_left, ar.scale) == (2, 1, 1, 2.0 ** 16)
    _say("config4 full size: compare")
    for i, (a, b) in enumerate(bounds):
        for j, name in enumerate(("master", "exp_avg", "exp_avg_sq")):
            assert torch.equal(rag[j][i].view(torch.int32), flat[j][a:b].view(torch.int32)), f"tensor {i}: {name}"
        assert torch.equal(rp16[i].view(torch.int16), p16f[a:b].view(torch.int16)), f"tensor {i}: param16"


@pytest.mark.parametrize("name", ["scaler_config4_llama_ragged.json", "scaler_config4_llama_ragged_backoff.json"])
def test_config4_golden_scaler_sequence_through_k3(gpu, name):
    """configs[3]'s committed 2000-step loss-scale sequences (torch's
    _amp_update_scale_ with the hysteresis of the ds_config key; the second
    seed reaches a tolerated overflow, a growth that re-arms the hysteresis
    and two back-offs) replayed through the ragged path (K1 over a chunk
    table, K0, K3): the device scale after every step equals the golden one,
    and the step count and overflow count match."""
    import json
    import os
    import torch
    from distributedspeed_amd import ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    with open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)) as f:
        gold = json.load(f)
    sizes = [4096, 1000, 77]
    gen = torch.Generator(device=gpu).manual_seed(6)
    ts = [(torch.empty(k, device=gpu).normal_(0.0, 0.02, generator=gen), torch.zeros(k, device=gpu),
           torch.zeros(k, device=gpu), torch.empty(k, dtype=torch.float16, device=gpu),
           (torch.empty(k, device=gpu).normal_(0.0, 1e-3, generator=gen) * 64).half()) for k in sizes]
    table = ops.ChunkTable(*[[t[j] for t in ts] for j in range(5)], chunk_elems=1024)
    scfg = ScalerConfig(mode="dynamic", init_scale=gold["init_scale"], window=gold["window"],
                        hysteresis=gold["hysteresis"], min_scale=gold["min_scale"])
    hyper = AdamWHyper(lr=1e-5, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0)
    bc = BiasCorrectionTable(gpu, hyper.beta1, hyper.beta2, capacity=len(gold["overflow"]) + 8)
    st = ops.new_state(gpu, scfg.init_scale, scfg.hysteresis)
    nparts = ops.suggest_partials(table.numel)
    parts = torch.zeros(nparts, dtype=torch.float64, device=gpu)
    out = ops.new_scalars(gpu)
    scale_view = ops.scale_view(st)
    got = torch.empty(len(gold["overflow"]), dtype=torch.float32, device=gpu)
    g1 = ts[1][4]
    _say(f"golden scaler sequence {name} through K3")
    for i, f in enumerate(gold["overflow"]):
        if f:
            g1[500] = float("inf")
        ops.unscale_norm_multi(table, st, parts, nparts)
        ops.finalize(parts, nparts, st, scfg.to_c(), hyper.to_c(), bc.table, bc.length, out)
        ops.adamw_multi(table, out)
        got[i] = scale_view[0]
        if f:
            g1[500] = 0.0
    seq = got.cpu().tolist()
    bad = [i + 1 for i, (a, b) in enumerate(zip(seq, gold["scale_after"])) if a != b]
    assert not bad, f"scale differs from the golden sequence at steps {bad[:10]}"
    s = ops.read_state(st)
    assert s.t == gold["final_t"] and s.overflow_count == sum(gold["overflow"]) and s.error == 0
