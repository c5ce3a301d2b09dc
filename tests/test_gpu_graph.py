"""GPU tests of the captured step (AdamWOptimizer(graph=True)): every replay
is compared bit for bit with an eager optimizer fed the same grads, with
eager work and host synchronisations between replays, across lr changes,
fp16 overflow (skip + scale back-off), bias-table growth and a checkpoint
load; plus the device-side checks of dsx_finalize_dev."""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _pair(gpu, dtype, scaler, shapes=((257, 33), (1000,), (64, 64), (5,)), lr=(1e-3, 3e-4), wd=(0.01, 0.0)):
    """Two optimizers over identical parameters in two parameter groups:
    one eager, one graphed."""
    import torch
    from distributedspeed_amd.optimizers import AdamWOptimizer
    out = []
    for graph in (False, True):
        g = torch.Generator().manual_seed(7)
        ps = [torch.nn.Parameter((torch.randn(s, generator=g) * 0.05).to(gpu)) for s in shapes]
        groups = [{"params": ps[:2], "lr": lr[0], "weight_decay": wd[0]},
                  {"params": ps[2:], "lr": lr[1], "weight_decay": wd[1], "betas": (0.8, 0.95)}]
        out.append(AdamWOptimizer(groups, lr=lr[0], max_grad_norm=1.0, param_dtype=dtype, loss_scaler=scaler,
                                  device=gpu, graph=graph))
    return out


def _same(a, b, tag):
    import torch
    for name in ("master", "exp_avg", "exp_avg_sq", "grad"):
        x, y = getattr(a.flat, name), getattr(b.flat, name)
        assert torch.equal(x.view(torch.int32) if x.dtype == torch.float32 else x.view(torch.int16),
                           y.view(torch.int32) if y.dtype == torch.float32 else y.view(torch.int16)), f"{tag}: {name}"
    if a.flat.param16 is not None:
        assert torch.equal(a.flat.param16.view(torch.int16), b.flat.param16.view(torch.int16)), f"{tag}: param16"
    assert torch.equal(a.dstate, b.dstate), f"{tag}: DsxState"
    assert torch.equal(a.scalars, b.scalars), f"{tag}: scalars"


def _feed(opts, gen, scale, inject_inf=False):
    import torch
    n = opts[0].flat.numel
    g = torch.randn(n, generator=gen, device=opts[0].device) * 0.02 * scale
    if inject_inf:
        g[n // 3] = float("inf")
    for o in opts:
        o.flat.grad.copy_(g.to(o.flat.grad.dtype))


@pytest.mark.parametrize("dtype_name", ["float16", "bfloat16"])
def test_graph_replays_match_eager_step_by_step(gpu, dtype_name):
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    dtype = getattr(torch, dtype_name)
    _say(f"graph vs eager {dtype_name}")
    sc = (ScalerConfig(mode="dynamic", init_scale=2.0 ** 10, window=3, hysteresis=2)
          if dtype == torch.float16 else ScalerConfig(mode="none"))
    eager, graphed = _pair(gpu, dtype, sc)
    gen = torch.Generator(device=gpu).manual_seed(11)
    side = torch.randn(1 << 16, device=gpu)
    for step in range(14):
        scale = float(eager.read_state().scale)
        # an lr schedule on both (the graph reads it from device memory)
        for o in (eager, graphed):
            o.param_groups[0]["lr"] = 1e-3 * (0.9 ** step)
            o.param_groups[1]["weight_decay"] = 0.001 * step
        _feed((eager, graphed), gen, scale, inject_inf=(step in (4, 5, 9) and dtype == torch.float16))
        eager.step()
        graphed.step()
        # unrelated eager work between replays, then a host synchronisation
        side.mul_(1.0001).add_(0.5).sqrt_()
        torch.cuda.synchronize()
        _same(eager, graphed, f"step {step}")
    assert graphed._graph is not None and graphed._graph.replays == 14
    assert graphed._graph.uploads == 14  # lr changed every step
    st = graphed.read_state()
    if dtype == torch.float16:
        assert st.overflow_count == 3 and st.t == 11 and st.iter == 14
    else:
        assert st.t == 14


def test_graph_survives_bias_table_growth_and_checkpoint_load(gpu):
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    _say("graph: bias table growth + load_state_dict")
    eager, graphed = _pair(gpu, torch.bfloat16, ScalerConfig(mode="none"), shapes=((40,), (24,), (16,)))
    gen = torch.Generator(device=gpu).manual_seed(3)
    for step in range(1030):  # the table starts with 1024 steps, so it is regrown once
        _feed((eager, graphed), gen, 1.0)
        eager.step()
        graphed.step()
        if step % 257 == 0 or step >= 1020:
            torch.cuda.synchronize()
            _same(eager, graphed, f"step {step}")
    assert min(t.length for t in graphed._bc.values()) >= 1030
    assert graphed._graph.uploads == 2  # constant lr: the first step and the table regrowth
    # load an earlier checkpoint into the graphed optimizer: same addresses, so
    # the captured graph keeps working from the loaded state
    sd = eager.state_dict()
    for _ in range(3):
        _feed((eager, graphed), gen, 1.0)
        graphed.step()
    graphed.load_state_dict(sd)
    for step in range(4):
        _feed((eager, graphed), gen, 1.0)
        eager.step()
        graphed.step()
        torch.cuda.synchronize()
        _same(eager, graphed, f"after load, step {step}")


def test_graph_rejects_bad_hyper_like_eager(gpu):
    import torch
    from distributedspeed_amd._lib import DsxError
    from distributedspeed_amd.flat_step import ScalerConfig
    eager, graphed = _pair(gpu, torch.bfloat16, ScalerConfig(mode="none"), shapes=((16,), (8,), (8,)))
    for o in (eager, graphed):
        o.step()
        o.param_groups[1]["lr"] = -1.0
        with pytest.raises(DsxError, match="Invalid learning rate"):
            o.step()


def test_finalize_dev_device_checks(gpu):
    """A group block that is bad on the device (ngroups out of range, a
    negative lr) skips the step in every output slot and flags the state."""
    import ctypes
    import torch
    from distributedspeed_amd import _lib, ops
    from distributedspeed_amd.flat_step import AdamWHyper, BiasCorrectionTable, ScalerConfig
    _say("finalize_dev device checks")
    tab = BiasCorrectionTable(gpu, 0.9, 0.999)
    parts = torch.full((4,), 0.25, dtype=torch.float64, device=gpu)
    scfg = ScalerConfig(mode="none").to_c()
    h = AdamWHyper(lr=1e-3).to_c()
    good = _lib.DsxGroupsDev.from_buffer_copy(ops.pack_groups([h, h], [tab.table, tab.table], [0, 0], tab.length))
    for case in ("ngroups", "lr", "ok_fewer"):
        g = _lib.DsxGroupsDev.from_buffer_copy(bytes(good))
        if case == "ngroups":
            g.ngroups = 5
        elif case == "lr":
            g.hyper[1].lr = -1.0
        else:
            g.ngroups = 1
        dev_g = torch.frombuffer(bytearray(bytes(g)), dtype=torch.uint8).to(gpu)
        st = ops.new_state(gpu)
        out = torch.zeros(ops.SCALARS_BYTES * 3, dtype=torch.uint8, device=gpu)
        out.fill_(0x7F)
        ops.finalize_dev(parts, 4, st, scfg, dev_g, 3, out)
        s = ops.read_state(st)
        sc = [ops.read_scalars(out[k * ops.SCALARS_BYTES:(k + 1) * ops.SCALARS_BYTES]) for k in range(3)]
        assert s.iter == 1 and s.last_norm == 1.0
        if case == "ok_fewer":
            assert s.error == 0 and s.t == 1 and s.last_skip == 0
            assert sc[0].skip == 0 and sc[0].t == 1 and sc[0].nss < 0
            assert sc[1].skip == 1 and sc[2].skip == 1  # slots past ngroups are written as skipped
        else:
            assert s.error & _lib.DSX_STATE_ERR_GROUPS and s.t == 0 and s.last_skip == 1, case
            assert all(x.skip == 1 for x in sc), case
    assert ctypes.sizeof(_lib.DsxGroupsDev) == ops.GROUPS_BYTES == 1112


def test_engine_hip_graph_config_matches_eager(gpu):
    import torch
    import distributedspeed_amd as ds
    _say("engine hip_graph")
    base = {"train_batch_size": 8, "optimizer": {"type": "AdamW", "params": {"lr": 1e-3}},
            "fp16": {"enabled": True, "initial_scale_power": 12}, "max_grad_norm": 1.0}
    runs = []
    for graph in (False, True):
        torch.manual_seed(0)
        model = torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.GELU(), torch.nn.Linear(128, 8))
        engine, opt, _, _ = ds.initialize(model, dict(base, hip_graph=graph))
        gen = torch.Generator(device=gpu).manual_seed(1)
        for _ in range(5):
            x = torch.randn(8, 64, device=gpu, generator=gen)
            loss = engine(x).float().pow(2).mean()
            engine.backward(loss)
            engine.step()
        torch.cuda.synchronize()
        runs.append(opt.base_optimizer)
    assert runs[1]._graph is not None and runs[0]._graph is None
    _same(runs[0], runs[1], "engine")


def test_graphed_optimizer_is_freed_by_refcount(gpu):
    """The optimizer -> GraphedStep link is one-way, so dropping a graphed
    optimizer frees it (and its graph) at once, not at some later cyclic
    collection that might land inside another graph's capture."""
    import gc
    import weakref
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    _, graphed = _pair(gpu, torch.bfloat16, ScalerConfig(mode="none"), shapes=((16,), (8,), (8,)))
    graphed.step()
    torch.cuda.synchronize()
    refs = [weakref.ref(graphed), weakref.ref(graphed._graph)]
    was = gc.isenabled()
    gc.disable()
    try:
        del graphed
        assert all(r() is None for r in refs)
    finally:
        if was:
            gc.enable()


def test_capturable_whole_iteration_in_one_graph(gpu):
    """AdamWOptimizer(capturable=True): a small fp16 model's whole iteration
    -- zero_grad, forward, loss * loss scale, backward, fused step -- is
    captured into one HIP graph by the caller and replayed, with
    prepare_step() before each replay; every replay is checked bit for bit
    against the same iteration run eagerly on a twin model (an lr change and
    an overflow-skipped step included), with unrelated eager work and a
    host synchronisation between replays."""
    import torch
    import torch.nn.functional as F
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer
    _say("capturable: whole iteration in one graph")

    def make():
        torch.manual_seed(0)
        model = torch.nn.Sequential(torch.nn.Linear(64, 128), torch.nn.GELU(), torch.nn.Linear(128, 16)).to(gpu)
        opt = AdamWOptimizer(model.parameters(), lr=1e-3, max_grad_norm=1.0, param_dtype=torch.float16,
                             loss_scaler=ScalerConfig(mode="dynamic", init_scale=2.0 ** 12, window=4, hysteresis=1),
                             device=gpu, capturable=True)
        return model, opt

    def iteration(model, opt, x, y):
        opt.zero_grad()
        loss = F.mse_loss(model(x).float(), y)
        (loss * opt.loss_scale_tensor()).backward()
        opt.step()

    gen = torch.Generator(device=gpu).manual_seed(5)
    data = [(torch.randn(32, 64, device=gpu, generator=gen).half(), torch.randn(32, 16, device=gpu, generator=gen))
            for _ in range(14)]
    data[8][1][0, 0] = float("inf")  # an overflow: the step is skipped, the scale halves
    m1, o1 = make()
    m2, o2 = make()
    sx, sy = data[0][0].clone(), data[0][1].clone()
    side = torch.cuda.Stream(gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):  # warm-up (eager) on a side stream, as torch's graph capture asks
        for x, y in data[:3]:
            sx.copy_(x)
            sy.copy_(y)
            iteration(m2, o2, sx, sy)
    torch.cuda.current_stream(gpu).wait_stream(side)
    for x, y in data[:3]:
        iteration(m1, o1, x, y)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        iteration(m2, o2, sx, sy)
    noise = torch.randn(1 << 16, device=gpu)
    for i, (x, y) in enumerate(data[3:], start=3):
        if i == 6:
            for o in (o1, o2):
                o.param_groups[0]["lr"] = 4e-4
        iteration(m1, o1, x, y)
        sx.copy_(x)
        sy.copy_(y)
        o2.prepare_step()
        graph.replay()
        noise.mul_(0.5).add_(1.0)  # unrelated eager work between replays
        torch.cuda.synchronize()
        for name in ("master", "exp_avg", "exp_avg_sq", "param16"):
            a, b = getattr(o1.flat, name), getattr(o2.flat, name)
            assert torch.equal(a.view(torch.int16 if a.dtype == torch.float16 else torch.int32),
                               b.view(torch.int16 if b.dtype == torch.float16 else torch.int32)), f"iter {i}: {name}"
        assert torch.equal(o1.dstate, o2.dstate), f"iter {i}: state"
    s = o2.read_state()
    assert s.iter == 14 and s.overflow_count == 1 and s.t == 13
