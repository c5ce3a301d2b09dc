"""clip_grad_norm_ on the GPU: the norm kernels of every norm type
(dsx_norm_partials / _multi + dsx_clip_prepare) against the oracle's norm_p,
and the one-shot contract of Src/zero/optimizer.py:324-341 ->
Src/zero/utils.py:187-216 through both storage forms: the call returns the
pre-clip norm, the next fused step clips once by max_norm / (norm + 1e-6)
instead of the configured max_grad_norm, and the step after that is back to
the configured clip. Norms within 1e-12 relative of the oracle's (inf: exact,
a maximum has no rounding); coefficients and every step's state bit-exact."""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

from helpers import BF16, F16, make_state, np16_to_torch, torch16_to_np

pytestmark = pytest.mark.gpu

F32 = 0
NORM_TYPES = [1.0, 2.0, 3.0, 0.5, math.inf]


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _grads(O, n, dt, seed, scale):
    if dt == F32:
        rng = np.random.default_rng(seed)
        g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
        g[: min(n, 3)] = np.array([0.0, -0.0, 65504.0], np.float32)[: min(n, 3)]
        return g
    return make_state(n, seed, dt, 1e-3, scale=scale)[3]


def _to_dev(g, dt, gpu):
    import torch
    return torch.from_numpy(g.copy()).to(gpu) if dt == F32 else np16_to_torch(g, dt, gpu)


def _close(got, ref, p, tag):
    if math.isinf(p) or math.isnan(ref) or math.isinf(ref):
        assert (math.isnan(got) and math.isnan(ref)) or got == ref, f"{tag}: {got!r} vs {ref!r}"
    else:
        assert got == pytest.approx(ref, rel=1e-12, abs=0.0), f"{tag}: {got!r} vs {ref!r}"


def _norm_and_arm(gpu, tg, state, p, max_norm, table=None):
    import torch
    from distributedspeed_amd import ops
    n = table.numel if table is not None else tg.numel()
    nparts = ops.suggest_partials(n)
    partials = torch.full((nparts,), float("nan"), dtype=torch.float64, device=gpu)
    s = ops.stream_of(gpu)
    if table is None:
        ops.plan_norm_partials(tg, state, p, partials, nparts)(s)
    else:
        ops.plan_norm_partials_multi(table, state, p, partials, nparts)(s)
    out = torch.zeros(1, dtype=torch.float64, device=gpu)
    ops.clip_prepare(partials, nparts, p, max_norm, 1e-6, state, out)
    torch.cuda.synchronize()
    return float(out.item()), ops.read_state(state)


@pytest.mark.parametrize("n", [1, 7, 1000, 262147])
@pytest.mark.parametrize("dt", [F32, F16, BF16])
@pytest.mark.parametrize("p", NORM_TYPES)
def test_norm_kernels_match_oracle(gpu, oracle, p, dt, n):
    from distributedspeed_amd import ops
    O = oracle
    scale = 2.0 ** 10 if dt == F16 else 1.0
    g = _grads(O, n, dt, 900 + n + dt, scale)
    tg = _to_dev(g, dt, gpu)
    ref = O.norm_p(g, dt, O.inv_scale_of(scale), p)
    for max_norm in (0.5 * ref, 2.0 * ref + 1.0):
        state = ops.new_state(gpu, scale, 1)
        _say(f"norm p={p} dt={dt} n={n} max={max_norm:.4g}")
        got, st = _norm_and_arm(gpu, tg, state, p, max_norm)
        _close(got, ref, p, "norm")
        assert st.clip_once == 1
        assert st.clip_once_coef == np.float32(O.clip_once_coef(ref, max_norm)), (st.clip_once_coef, ref, max_norm)


@pytest.mark.parametrize("p", NORM_TYPES)
def test_norm_over_a_chunk_table_matches_flat(gpu, oracle, p):
    """The ragged form's norm (dsx_norm_partials_multi) over tensors at
    aligned and misaligned addresses equals the oracle's over their
    concatenation."""
    import torch
    from distributedspeed_amd import ops
    O = oracle
    dt, scale = F16, 2.0 ** 8
    sizes = [70_001, 1, 4096, 123_457]
    g = _grads(O, sum(sizes), dt, 77, scale)
    buf = torch.zeros(sum(sizes) + 16, dtype=torch.float16, device=gpu)
    grads, off, a = [], 0, 0
    for k, sz in enumerate(sizes):
        off += 1 if k == 1 else 0  # tensors from the second on sit one element off
        v = buf[off:off + sz]
        v.copy_(np16_to_torch(g[a:a + sz], dt, gpu))
        grads.append(v)
        off += sz
        a += sz
    f32 = [torch.zeros(sz, dtype=torch.float32, device=gpu) for sz in sizes]
    table = ops.ChunkTable(f32, f32, f32, None, grads, chunk_elems=4096)
    ref = O.norm_p(g, dt, O.inv_scale_of(scale), p)
    got, st = _norm_and_arm(gpu, None, ops.new_state(gpu, scale, 1), p, 0.25 * ref, table=table)
    _close(got, ref, p, "ragged norm")
    assert st.clip_once_coef == np.float32(O.clip_once_coef(ref, 0.25 * ref))


@pytest.mark.parametrize("bad", [math.inf, math.nan])
@pytest.mark.parametrize("p", NORM_TYPES)
def test_nonfinite_grads(gpu, oracle, p, bad):
    """An inf grad makes every norm inf (coefficient max / inf = 0, as the
    reference computes it); a NaN makes it NaN (NaN > max is false: no clip)."""
    O = oracle
    from distributedspeed_amd import ops
    n = 50_000
    g = _grads(O, n, F32, 5, 1.0)
    g[31_337] = bad
    ref = O.norm_p(g, F32, 1.0, p)
    got, st = _norm_and_arm(gpu, _to_dev(g, F32, gpu), ops.new_state(gpu, 1.0, 1), p, 1.0)
    _close(got, ref, p, "non-finite norm")
    assert st.clip_once_coef == (0.0 if bad == math.inf else 1.0)


def _params(gpu, seed, dtype):
    import torch
    gen = torch.Generator().manual_seed(seed)
    shapes = [(300, 77), (77,), (1000, 31), (5,)]
    return [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.05).to(gpu, dtype)) for s in shapes]


def _host(opt, grads):
    """master, exp_avg, exp_avg_sq, param16 (numpy, step order) and the
    given grads as one uint16 array (the flat form includes its padding)."""
    import torch
    if hasattr(opt, "flat"):
        f = opt.flat
        return (f.master.cpu().numpy().copy(), f.exp_avg.cpu().numpy().copy(), f.exp_avg_sq.cpu().numpy().copy(),
                torch16_to_np(f.param16).copy(), torch16_to_np(f.grad).copy())
    st = opt.store
    cat = lambda ts: torch.cat([t.detach().reshape(-1) for t in ts])  # noqa: E731
    return (cat(st.master).cpu().numpy(), cat(st.exp_avg).cpu().numpy(), cat(st.exp_avg_sq).cpu().numpy(),
            torch16_to_np(cat([p.data for p in st.params])), torch16_to_np(cat(grads)))


# flat: the one-call eager step; graph: K1 + K0 (device-memory form) + K2
# replayed from one HIP graph; capturable: the launches a caller may capture,
# here issued eagerly; offload: state in pinned host memory, K2 streamed.
FORMS = {"flat": {}, "graph": {"graph": True}, "capturable": {"capturable": True},
         "offload": {"offload": True, "offload_chunk_elems": 8192}, "ragged": None}


@pytest.mark.parametrize("form", list(FORMS))
def test_clip_grad_norm_is_one_shot(gpu, oracle, form):
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    from distributedspeed_amd.zero import ZeROOptimizer
    O = oracle
    cls = MultiTensorAdamWOptimizer if form == "ragged" else AdamWOptimizer
    kw = FORMS[form] or {}
    ps = _params(gpu, 3, torch.float32)
    sc = ScalerConfig(mode="dynamic", init_scale=2.0 ** 10, window=1000, hysteresis=1)
    opt = cls(ps, lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, max_grad_norm=1.0,
              param_dtype=torch.float16, loss_scaler=sc, device=gpu, **kw)
    zero = ZeROOptimizer(opt, {"stage": 2})
    gen = torch.Generator(device=gpu).manual_seed(8)
    # (explicit clip before the step: (max_norm, norm_type) or None, inject an inf)
    plan = [((0.05, 3.0), False), (None, False), ((0.05, math.inf), True), (None, False), ((100.0, 1.0), False)]
    orc = None
    for step, (clip, inf) in enumerate(plan):
        scale = float(opt.read_state().scale)
        grads = []
        for i, p in enumerate(opt.dsx_params):
            g = (torch.randn(p.shape, generator=gen, device=gpu) * 0.02 * scale).half()
            if inf and i == 2:
                g.view(-1)[17] = float("inf")
            if form != "ragged":
                p.grad.copy_(g)
                grads.append(p.grad)
            else:
                p.grad = g
                grads.append(g)
        master, m, v, p16, g16 = _host(opt, grads)
        if orc is None:
            orc = O.ZeroStepOracle(master, m, v, p16, F16, F16,
                                   O.Hyper(lr=1e-3, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1,
                                           max_grad_norm=1.0),
                                   O.LossScalerSpec(scale=2.0 ** 10, window=1000, hysteresis=1))
        coef = None
        _say(f"one-shot clip {form} step={step} clip={clip} inf={inf}")
        if clip is not None:
            norm_t = zero.clip_grad_norm_(*clip)
            ref = O.norm_p(g16, F16, O.inv_scale_of(scale), clip[1])
            got_norm = float(norm_t.item())  # fp32, as the reference returns it
            assert got_norm == pytest.approx(ref, rel=1.2e-7) or got_norm == ref, (step, got_norm, ref)
            assert norm_t.dtype == torch.float32 and norm_t.device.type == "cuda" and norm_t.dim() == 0
            coef = O.clip_once_coef(ref, clip[0])
        zero.step()
        torch.cuda.synchronize(gpu)  # the offloaded form writes host memory from its own streams
        r = orc.step(g16, clip_once=coef)
        st = opt.read_state()
        assert st.clip_once == 0, f"step {step}: the one-shot clip was not consumed"
        assert bool(st.last_skip) == r.skipped == inf
        assert st.scale == r.scale_next
        sc_host = opt.last_scalars()
        if not r.skipped:
            assert sc_host.clip_coef == np.float32(r.clip_coef), (step, sc_host.clip_coef, r.clip_coef)
        got = _host(opt, grads)
        for name, a, b in (("master", got[0], orc.p), ("exp_avg", got[1], orc.m), ("exp_avg_sq", got[2], orc.v)):
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {step}: {name} differs"
        assert np.array_equal(got[3], orc.p16), f"step {step}: param16 differs"
        assert opt.max_grad_norm == 1.0
    assert opt.read_state().t == 4


def test_clip_grad_norm_argument_checks(gpu):
    import torch
    from distributedspeed_amd.optimizers import AdamWOptimizer
    opt = AdamWOptimizer(_params(gpu, 1, torch.float32), param_dtype=torch.bfloat16, device=gpu)
    for bad in (0.0, -1.0, float("nan"), "two"):
        with pytest.raises(ValueError, match="norm_type"):
            opt.clip_grad_norm_(1.0, bad)
    with pytest.raises(ValueError, match="max_norm"):
        opt.clip_grad_norm_(-1.0)
    assert float(opt.clip_grad_norm_(1.0, "inf")) >= 0.0
