"""GPU tests of the drop-in API: initialize() -> engine(batch) ->
engine.backward(loss) -> engine.step(), checked step by step against the CPU
oracle fed the grads autograd produced (captured from the flat grad buffer
before each step)."""
from __future__ import annotations

import math
import os
import sys
import warnings

import numpy as np
import pytest

from helpers import BF16, F16, torch16_to_np

pytestmark = pytest.mark.gpu

F32 = 0


def _say(msg):
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _mlp(seed=0):
    import torch
    torch.manual_seed(seed)
    return torch.nn.Sequential(torch.nn.Linear(784, 1024), torch.nn.ReLU(), torch.nn.Linear(1024, 1024),
                               torch.nn.ReLU(), torch.nn.Linear(1024, 10))


def _grads_np(opt):
    g = opt.flat.grad
    if g.dtype == __import__("torch").float32:
        return g.detach().cpu().numpy().copy(), F32
    return torch16_to_np(g).copy(), (F16 if g.dtype == __import__("torch").float16 else BF16)


class GroupOracle:
    """The oracle over a flat partition with per-group hyper-parameters and
    one global norm / skip / scaler."""

    def __init__(self, O, opt, hypers, scaler):
        self.O = O
        self.p = opt.flat.master.detach().cpu().numpy().copy()
        self.m = np.zeros_like(self.p)
        self.v = np.zeros_like(self.p)
        self.p16 = torch16_to_np(opt.flat.param16).copy() if opt.flat.param16 is not None else None
        self.pdt = None if opt.flat.param16 is None else (F16 if opt.flat.param16.dtype == __import__("torch").float16
                                                           else BF16)
        self.ranges = opt.flat.group_ranges
        self.hypers = hypers
        self.scaler = scaler
        self.t = 0

    def step(self, g, gdt, max_norm):
        O = self.O
        scale = self.scaler.scale
        inv = O.inv_scale_of(scale)
        ss = O.sumsq(g, gdt, inv)
        skipped = not math.isfinite(ss)
        if not skipped:
            self.t += 1
            coef = O.clip_coef(math.sqrt(ss), max_norm)
            for (a, b), h in zip(self.ranges, self.hypers):
                sl = slice(a, b)
                p16 = self.p16[sl] if self.p16 is not None else None
                pv, mv, vv = self.p[sl], self.m[sl], self.v[sl]
                # the oracle works on contiguous arrays: run on copies, write back
                pc, mc, vc = pv.copy(), mv.copy(), vv.copy()
                p16c = p16.copy() if p16 is not None else None
                O.adamw(pc, mc, vc, p16c, self.pdt or F16, np.ascontiguousarray(g[sl]), gdt,
                        O.step_scalars(h, self.t, inv, coef))
                pv[:], mv[:], vv[:] = pc, mc, vc
                if p16 is not None:
                    p16[:] = p16c
        self.scaler.update(skipped)
        return skipped, ss

    def compare(self, opt, tag):
        for name, ref, got in (("master", self.p, opt.flat.master), ("exp_avg", self.m, opt.flat.exp_avg),
                               ("exp_avg_sq", self.v, opt.flat.exp_avg_sq)):
            g = got.detach().cpu().numpy()
            assert np.array_equal(g.view(np.uint32), ref.view(np.uint32)), f"{tag}: {name} differs"
        if self.p16 is not None:
            assert np.array_equal(torch16_to_np(opt.flat.param16), self.p16), f"{tag}: param16 differs"


def _run_training(gpu, oracle, ds_config, steps, seed=0, groups=None, scheduler=None, batch=32, check=True):
    import torch
    import distributedspeed_amd as ds
    model = _mlp(seed)
    params = groups(model) if groups else None
    engine, opt, _, sched = ds.initialize(model, ds_config, model_parameters=params)
    base = opt.base_optimizer
    hyp = [oracle.Hyper(lr=g["lr"], beta1=g["betas"][0], beta2=g["betas"][1], eps=g["eps"],
                        weight_decay=g["weight_decay"], max_grad_norm=base.max_grad_norm) for g in base.param_groups]
    sc = base.scaler
    spec = oracle.LossScalerSpec(scale=sc.init_scale if sc.mode != "none" else 1.0, window=sc.window,
                                 hysteresis=sc.hysteresis if sc.mode == "dynamic" else 1, min_scale=sc.min_scale,
                                 dynamic=sc.mode == "dynamic")
    orc = GroupOracle(oracle, base, hyp, spec)
    gen = torch.Generator(device=gpu)
    gen.manual_seed(seed + 100)
    log = []
    for step in range(steps):
        x = torch.randn(batch, 784, device=gpu, generator=gen)
        y = torch.randint(0, 10, (batch,), device=gpu, generator=gen)
        out = engine(x)
        loss = torch.nn.functional.cross_entropy(out.float(), y)
        engine.backward(loss)
        if check:
            g, gdt = _grads_np(base)
            skipped, ss = orc.step(g, gdt, base.max_grad_norm)
        engine.step()
        if check:
            st = base.read_state()
            assert bool(st.last_skip) == skipped, f"step {step}: skip {st.last_skip} vs {skipped}"
            assert st.scale == spec.scale, f"step {step}: scale {st.scale} vs {spec.scale}"
            orc.compare(base, f"step {step}")
            log.append((skipped, st.scale, float(loss.detach())))
    return engine, log


def test_engine_fp16_mlp_matches_oracle(gpu, oracle):
    _say("engine fp16 mlp")
    cfg = {"train_batch_size": 32, "optimizer": {"type": "AdamW", "params": {"lr": 1e-4, "betas": [0.9, 0.999],
                                                                             "eps": 1e-8, "weight_decay": 0.01}},
           "fp16": {"enabled": True, "loss_scale": 0, "initial_scale_power": 16, "loss_scale_window": 1000,
                    "hysteresis": 2, "min_loss_scale": 1},
           "zero_optimization": {"stage": 2}, "max_grad_norm": 1.0}
    engine, log = _run_training(gpu, oracle, cfg, steps=6)
    assert engine.global_steps == 6
    assert all(math.isfinite(l) for _, _, l in log)


def test_engine_bf16_two_groups_with_scheduler(gpu, oracle):
    import torch
    _say("engine bf16 groups")

    def groups(model):
        decay = [p for n, p in model.named_parameters() if n.endswith("weight")]
        no_decay = [p for n, p in model.named_parameters() if n.endswith("bias")]
        return [{"params": decay, "weight_decay": 0.1}, {"params": no_decay, "weight_decay": 0.0, "lr": 5e-4}]

    cfg = {"optimizer": {"type": "AdamW", "params": {"lr": 3e-4, "betas": [0.9, 0.95], "eps": 1e-8,
                                                     "weight_decay": 0.1}},
           "bf16": {"enabled": True}, "max_grad_norm": 0.5}
    engine, log = _run_training(gpu, oracle, cfg, steps=5, groups=groups)
    base = engine.optimizer.base_optimizer
    assert len(base.param_groups) == 2 and base.param_groups[1]["lr"] == 5e-4
    assert base.flat.param16.dtype == torch.bfloat16


def test_engine_fp32_no_mixed_precision(gpu, oracle):
    import torch
    _say("engine fp32")
    cfg = {"optimizer": {"type": "AdamW", "params": {"lr": 1e-3}}, "max_grad_norm": 0.0}
    engine, _ = _run_training(gpu, oracle, cfg, steps=4)
    base = engine.optimizer.base_optimizer
    assert base.flat.param16 is None and base.flat.grad.dtype == torch.float32
    # the model's parameters are the fp32 master itself
    p0 = next(engine.module.parameters())
    assert base.flat.master.data_ptr() <= p0.data_ptr() < base.flat.master.data_ptr() + 4 * base.flat.numel


def test_autograd_accumulates_into_flat_grad_buffer(gpu):
    import torch
    import distributedspeed_amd as ds
    model = _mlp(1)
    engine, opt, _, _ = ds.initialize(model, {"fp16": {"enabled": True}})
    flat = opt.base_optimizer.flat
    x = torch.randn(8, 784, device=gpu)
    engine.backward(engine(x).float().pow(2).mean())
    lo, hi = flat.grad.data_ptr(), flat.grad.data_ptr() + 2 * flat.numel
    for p in engine.module.parameters():
        assert p.grad is not None and lo <= p.grad.data_ptr() < hi
    assert float(flat.grad.float().abs().sum()) > 0


def test_gradient_accumulation(gpu, oracle):
    """Two micro-batches accumulate into the 16-bit grads; one step."""
    import torch
    import distributedspeed_amd as ds
    cfg = {"bf16": {"enabled": True}, "gradient_accumulation_steps": 2, "max_grad_norm": 0.0,
           "optimizer": {"params": {"lr": 1e-3}}}
    engine, opt, _, _ = ds.initialize(_mlp(2), cfg)
    base = opt.base_optimizer
    p_before = base.flat.master.clone()
    x1, x2 = torch.randn(16, 784, device=gpu), torch.randn(16, 784, device=gpu)
    engine.backward(engine(x1).float().pow(2).mean())
    engine.step()  # not a boundary: no update
    assert torch.equal(base.flat.master, p_before) and engine.global_steps == 0
    engine.backward(engine(x2).float().pow(2).mean())
    g = torch16_to_np(base.flat.grad).copy()
    engine.step()
    assert engine.global_steps == 1
    # after the boundary step the grads are None (zero_grad(set_to_none=True));
    # before anything reads the flat buffer, views without a grad are zeroed
    assert all(p.grad is None for p in base.flat.params)
    base.flat.check_grads_bound()
    assert float(base.flat.grad.float().abs().sum()) == 0.0
    p, m, v = p_before.cpu().numpy(), np.zeros(base.flat.numel, np.float32), np.zeros(base.flat.numel, np.float32)
    h = oracle.Hyper(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01)
    oracle.adamw(p, m, v, None, BF16, g, BF16, oracle.step_scalars(h, 1, 1.0, 1.0))
    assert np.array_equal(base.flat.master.cpu().numpy().view(np.uint32), p.view(np.uint32))


def test_torch_adamw_is_adopted(gpu):
    import torch
    import distributedspeed_amd as ds
    model = _mlp(3)
    topt = torch.optim.AdamW(model.parameters(), lr=2e-4, betas=(0.8, 0.9), weight_decay=0.05)
    engine, opt, _, _ = ds.initialize(model.cuda(), {"bf16": {"enabled": True}}, optimizer=topt)
    g = opt.param_groups[0]
    assert (g["lr"], tuple(g["betas"]), g["weight_decay"]) == (2e-4, (0.8, 0.9), 0.05)
    with pytest.raises(NotImplementedError):
        ds.initialize(_mlp(4), {}, optimizer=torch.optim.SGD(_mlp(4).parameters(), lr=0.1))


@pytest.mark.parametrize("cls_name", ["AdamWOptimizer", "MultiTensorAdamWOptimizer"])
def test_rebuilt_from_param_groups_and_defaults(gpu, cls_name):
    """The ZeRO stages rebuild their optimizer as
    type(opt)(groups, **opt.defaults) (Src/zero/stage1.py:358). A fused
    optimizer rebuilt that way takes the parameters over (their storage and
    grads move to it) and steps bit for bit as one built fresh over the same
    weights; attributes of the base optimizer reach through ZeROOptimizer."""
    import torch
    from distributedspeed_amd import optimizers as O
    from distributedspeed_amd.zero import ZeROOptimizer
    _say(f"rebuilt from param_groups and defaults: {cls_name}")
    cls = getattr(O, cls_name)
    m1, m2 = _mlp(11).to(gpu), _mlp(11).to(gpu)
    o1 = cls(m1.parameters(), lr=1e-3, betas=(0.8, 0.95), weight_decay=0.01)
    rebuilt = type(o1)(o1.param_groups, **o1.defaults)
    fresh = cls(m2.parameters(), lr=1e-3, betas=(0.8, 0.95), weight_decay=0.01)
    assert rebuilt.defaults == fresh.defaults == o1.defaults
    x = torch.randn(8, 784, device=gpu)
    for model, opt in ((m1, rebuilt), (m2, fresh)):
        for _ in range(3):
            opt.zero_grad()
            model(x).pow(2).mean().backward()
            opt.step()
    for a, b in zip(m1.parameters(), m2.parameters()):
        assert torch.equal(a.detach(), b.detach())
    z = ZeROOptimizer(rebuilt, {"stage": 1})
    assert z.numel == rebuilt.numel and z.layout() == rebuilt.layout() and z.defaults == rebuilt.defaults


@pytest.mark.parametrize("contiguous", [True, False])
def test_checkpoint_round_trip_is_bit_exact(gpu, tmp_path, contiguous):
    import torch
    import distributedspeed_amd as ds
    _say(f"checkpoint round trip, contiguous_gradients={contiguous}")
    cfg = {"fp16": {"enabled": True, "hysteresis": 1}, "max_grad_norm": 1.0,
           "zero_optimization": {"stage": 2, "contiguous_gradients": contiguous}}
    gen = torch.Generator(device=gpu)
    gen.manual_seed(9)
    data = [(torch.randn(16, 784, device=gpu, generator=gen), torch.randint(0, 10, (16,), device=gpu, generator=gen))
            for _ in range(5)]

    def train(engine, batches):
        for x, y in batches:
            engine.backward(torch.nn.functional.cross_entropy(engine(x).float(), y))
            engine.step()

    e1, _, _, _ = ds.initialize(_mlp(5), cfg)
    train(e1, data[:3])
    e1.save_checkpoint(str(tmp_path), client_state={"epoch": 1})
    train(e1, data[3:])
    e2, _, _, _ = ds.initialize(_mlp(6), cfg)  # different init: everything must come from the checkpoint
    _, client = e2.load_checkpoint(str(tmp_path))
    assert client == {"epoch": 1} and e2.global_steps == 3
    train(e2, data[3:])
    b1, b2 = e1.optimizer.base_optimizer, e2.optimizer.base_optimizer
    for i in range(len(b1.dsx_params)):
        v1, v2 = b1.store.views_of(i), b2.store.views_of(i)
        for name in ("master", "exp_avg", "exp_avg_sq"):
            assert torch.equal(v1[name], v2[name]), (i, name)
        assert torch.equal(b1.dsx_params[i].detach(), b2.dsx_params[i].detach()), (i, "param16")
    s1, s2 = b1.read_state(), b2.read_state()
    assert (s1.scale, s1.t, s1.good_steps, s1.overflow_count) == (s2.scale, s2.t, s2.good_steps, s2.overflow_count)


_FORM_CFG = {"flat": {}, "ragged": {"contiguous_gradients": False}, "offload": {"cpu_offload": True},
             "graph": None}


@pytest.mark.parametrize("src,dst", [("flat", "ragged"), ("flat", "offload"), ("flat", "graph"),
                                     ("ragged", "flat"), ("offload", "ragged")])
def test_checkpoint_moves_between_storage_forms(gpu, tmp_path, src, dst):
    """The checkpoint is keyed by parameter name and offset, not by the
    storage it came from: one saved by one step form (flat HBM partition,
    ragged list, state offloaded to pinned host memory, graph-replayed step)
    loads into another, and training continues bit for bit as it would have
    in the saving engine. No clipping here: the flat form's norm comes from
    the hooks' copies, the ragged form's from K1 over the list, equal to
    1e-12 but not bit for bit, and the clip coefficient is rounded from it."""
    import torch
    import distributedspeed_amd as ds
    _say(f"checkpoint from {src} into {dst}")

    def cfg(form):
        zo = {"stage": 2, "contiguous_gradients": True}
        zo.update(_FORM_CFG[form] or {})
        c = {"fp16": {"enabled": True, "hysteresis": 1, "initial_scale_power": 12}, "max_grad_norm": 0.0,
             "zero_optimization": zo}
        if form == "graph":
            c["hip_graph"] = True
        return c

    gen = torch.Generator(device=gpu)
    gen.manual_seed(21)
    data = [(torch.randn(16, 784, device=gpu, generator=gen), torch.randint(0, 10, (16,), device=gpu, generator=gen))
            for _ in range(6)]

    def train(engine, batches):
        for x, y in batches:
            engine.backward(torch.nn.functional.cross_entropy(engine(x).float(), y))
            engine.step()

    e1, _, _, _ = ds.initialize(_mlp(5), cfg(src))
    train(e1, data[:3])
    e1.save_checkpoint(str(tmp_path))
    train(e1, data[3:])
    e2, _, _, _ = ds.initialize(_mlp(6), cfg(dst))
    e2.load_checkpoint(str(tmp_path))
    assert e2.global_steps == 3
    train(e2, data[3:])
    torch.cuda.synchronize(gpu)
    b1, b2 = e1.optimizer.base_optimizer, e2.optimizer.base_optimizer
    for i in range(len(b1.dsx_params)):
        v1, v2 = b1.store.views_of(i), b2.store.views_of(i)
        for name in ("master", "exp_avg", "exp_avg_sq"):
            assert torch.equal(v1[name].cpu(), v2[name].cpu()), (i, name)
        assert torch.equal(b1.dsx_params[i].detach(), b2.dsx_params[i].detach()), (i, "param16")
    s1, s2 = b1.read_state(), b2.read_state()
    assert (s1.scale, s1.t, s1.good_steps, s1.overflow_count) == (s2.scale, s2.t, s2.good_steps, s2.overflow_count)
    assert s1.t == 6


@pytest.mark.parametrize("contiguous", [True, False])
def test_model_state_loaded_after_initialize_is_kept(gpu, contiguous):
    """A model state dict loaded into the module after initialize() writes
    the 16-bit params; the fp32 master follows them, so the next step starts
    from the loaded weights (the reference steps the params themselves).
    With lr 0 and no weight decay that step leaves them exactly as loaded;
    a stale master would write the initial weights back."""
    import torch
    import distributedspeed_amd as ds
    _say(f"model state loaded after initialize, contiguous_gradients={contiguous}")
    cfg = {"fp16": {"enabled": True, "hysteresis": 1},
           "optimizer": {"type": "AdamW", "params": {"lr": 0.0, "weight_decay": 0.0}},
           "zero_optimization": {"stage": 2, "contiguous_gradients": contiguous}}
    engine, _, _, _ = ds.initialize(_mlp(5), cfg)
    target = {k: v.clone() for k, v in _mlp(6).half().state_dict().items()}
    engine.module.load_state_dict(target)
    x = torch.randn(16, 784, device=gpu)
    engine.backward(engine(x).float().pow(2).mean())
    engine.step()
    after = engine.module.state_dict()
    for k, v in target.items():
        assert torch.equal(after[k].cpu(), v), k


def test_reference_format_state_dict_loads(gpu):
    """The reference's ZeROOptimizer.state_dict() over torch.optim.AdamW
    (Src/zero/optimizer.py:356-381: torch's AdamW state dict plus
    zero_stage, current_step, overflow_count, gradient_accumulation_count
    and a torch GradScaler's state dict) loads into the fused optimizer: the
    moments by parameter index, the master from the params, the step count,
    the overflow count and the dynamic loss scale. The state dict written
    back carries torch's GradScaler keys, which torch's GradScaler loads."""
    import torch
    import distributedspeed_amd as ds
    _say("reference-format state dict")
    ref_model = _mlp(7).to(gpu)
    topt = torch.optim.AdamW(ref_model.parameters(), lr=1e-3, weight_decay=0.01)
    gen = torch.Generator(device=gpu).manual_seed(4)
    for _ in range(3):
        ref_model(torch.randn(8, 784, device=gpu, generator=gen)).pow(2).mean().backward()
        topt.step()
        topt.zero_grad()
    gs = torch.amp.GradScaler("cuda", init_scale=4096.0)
    gs_sd = gs.state_dict()
    gs_sd["_growth_tracker"] = 7
    ref_sd = topt.state_dict()
    ref_sd.update(zero_stage=2, current_step=3, overflow_count=1, gradient_accumulation_count=0, grad_scaler=gs_sd)

    model = _mlp(8)
    model.load_state_dict({k: v.detach().cpu() for k, v in ref_model.state_dict().items()})
    cfg = {"fp16": {"enabled": True, "initial_scale_power": 16, "hysteresis": 1},
           "optimizer": {"type": "AdamW", "params": {"lr": 1e-3, "weight_decay": 0.01}}}
    engine, opt, _, _ = ds.initialize(model, cfg)
    opt.load_state_dict(ref_sd)
    assert opt.current_step == 3 and opt.overflow_count == 1
    assert opt.loss_scale == 4096.0 and opt.base_optimizer.read_state().good_steps == 7
    base = opt.base_optimizer
    for i, p in enumerate(ref_model.parameters()):
        v = base.store.views_of(i)
        assert torch.equal(v["exp_avg"].cpu(), topt.state[p]["exp_avg"].cpu()), i
        assert torch.equal(v["exp_avg_sq"].cpu(), topt.state[p]["exp_avg_sq"].cpu()), i
        assert torch.equal(v["master"].cpu(), p.detach().half().float().cpu()), i

    back = opt.state_dict()["grad_scaler"]
    gs2 = torch.amp.GradScaler("cuda", init_scale=1.0)
    gs2.load_state_dict(back)
    assert gs2.get_scale() == 4096.0 and gs2.state_dict()["_growth_tracker"] == 7


def test_initialize_refuses_multi_rank(gpu, monkeypatch):
    import distributedspeed_amd as ds
    monkeypatch.setenv("WORLD_SIZE", "2")
    with pytest.raises(NotImplementedError):
        ds.initialize(_mlp(7), {})


def test_offloaded_state_matches_in_hbm_step(gpu):
    """configs[4]'s path at reduced size: master/m/v in pinned host memory,
    streamed through HBM in small chunks (so that every stage of the copy-in /
    K2 / copy-out pipeline wraps around its buffers several times), two
    parameter groups, fp16 dynamic scaling with an overflow step. Results are
    bit-identical to the same steps with the state in HBM."""
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer
    shapes = [(1000, 1003), (4096,), (3, 777), (2048, 1024), (17,)]
    torch.manual_seed(0)
    init = [torch.randn(s) * 0.02 for s in shapes]

    def build(offload):
        ps = [torch.nn.Parameter(t.clone().to(gpu)) for t in init]
        groups = [{"params": ps[:3], "weight_decay": 0.1}, {"params": ps[3:], "weight_decay": 0.0, "lr": 3e-3}]
        return AdamWOptimizer(groups, lr=1e-3, betas=(0.9, 0.95), max_grad_norm=1.0, param_dtype=torch.float16,
                              loss_scaler=ScalerConfig(mode="dynamic", init_scale=2.0 ** 12, hysteresis=1),
                              offload=offload, offload_chunk_elems=131072)

    a, b = build(False), build(True)
    assert b.flat.master.device.type == "cpu" and b.flat.master.is_pinned()
    gen = torch.Generator(device=gpu)
    gen.manual_seed(5)
    for step in range(6):
        g = (torch.randn(a.flat.numel, device=gpu, generator=gen) * 1e-3 * 2.0 ** 12).to(torch.float16)
        if step == 2:
            g[12345] = float("inf")
        a.flat.grad.copy_(g)
        b.flat.grad.copy_(g)
        a.step()
        b.step()
    torch.cuda.synchronize()
    for name in ("master", "exp_avg", "exp_avg_sq"):
        assert torch.equal(getattr(a.flat, name).cpu(), getattr(b.flat, name)), name
    assert torch.equal(a.flat.param16, b.flat.param16)
    sa, sb = a.read_state(), b.read_state()
    assert (sa.t, sa.scale, sa.overflow_count) == (sb.t, sb.scale, sb.overflow_count) == (5, 2.0 ** 11, 1)


def test_engine_cpu_offload_config(gpu):
    import torch
    import distributedspeed_amd as ds
    cfg = {"bf16": {"enabled": True}, "zero_optimization": {"stage": 2, "cpu_offload": True}}
    engine, opt, _, _ = ds.initialize(_mlp(8), cfg)
    assert opt.base_optimizer.flat.master.device.type == "cpu"
    x = torch.randn(8, 784, device=gpu)
    for _ in range(2):
        engine.backward(engine(x).float().pow(2).mean())
        engine.step()
    assert opt.base_optimizer.read_state().t == 2
    with pytest.raises(ValueError):
        ds.initialize(_mlp(9), {"zero_optimization": {"cpu_offload": True}})  # fp32 params cannot offload


def test_scheduler_on_adopted_optimizer_and_overflow_skip(gpu):
    """A scheduler built on the user's torch.optim.AdamW drives the fused
    step after initialize() adopts it, and (as in DeepSpeed's engine) is not
    stepped on a step skipped for overflow; the skip flag is read on the host
    from the pinned mirror written after K0."""
    import torch
    import distributedspeed_amd as ds
    _say("scheduler + overflow skip")
    torch.manual_seed(0)
    model = torch.nn.Sequential(torch.nn.Linear(32, 64), torch.nn.ReLU(), torch.nn.Linear(64, 4)).to(gpu)
    topt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=0.0)
    sched = torch.optim.lr_scheduler.LambdaLR(topt, lambda e: 0.5 ** e)
    cfg = {"fp16": {"enabled": True, "initial_scale_power": 8, "hysteresis": 1}}
    engine, opt, _, sch = ds.initialize(model, cfg, optimizer=topt, lr_scheduler=sched)
    base = opt.base_optimizer
    assert sch is sched and base.param_groups[0] is topt.param_groups[0]
    gen = torch.Generator(device=gpu).manual_seed(4)
    skips = []
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        for step in range(6):
            x = torch.randn(8, 32, device=gpu, generator=gen)
            loss = engine(x).float().pow(2).mean()
            if step == 2:
                loss = loss * float("inf")  # every grad becomes non-finite: the step is skipped
            engine.backward(loss)
            engine.step()
            skips.append(base.last_step_skipped())
            assert skips[-1] == bool(base.read_state().last_skip)
    # the scheduler sees that the optimizer stepped before it (no order warning)
    assert not [w for w in caught if "lr_scheduler.step()" in str(w.message)]
    assert skips == [False, False, True, False, False, False]
    assert sched.last_epoch == 5  # six boundaries, one skipped
    assert base.param_groups[0]["lr"] == 1e-3 * 0.5 ** 5
    st = base.read_state()
    assert st.t == 5 and st.overflow_count == 1 and st.scale == 2.0 ** 7


def test_zero_optimizer_counters_and_accessors(gpu):
    """The reference's ZeROOptimizer counters and accessors
    (Src/zero/optimizer.py:212-274, 407-559): current_step counts clean
    optimizer steps only (an overflow-skipped step and accumulation-only calls
    do not), overflow_count the skipped ones; both survive state_dict /
    load_state_dict and reset_stats clears overflow_count; the memory figures
    are this layout's bytes (2-byte params and grads, 12 bytes of fp32 state per
    padded element)."""
    import torch
    import distributedspeed_amd as ds
    _say("ZeROOptimizer counters and accessors")
    torch.manual_seed(1)
    model = torch.nn.Sequential(torch.nn.Linear(32, 64), torch.nn.ReLU(), torch.nn.Linear(64, 4))
    cfg = {"fp16": {"enabled": True, "initial_scale_power": 8, "hysteresis": 1},
           "gradient_accumulation_steps": 2, "zero_optimization": {"stage": 1}}
    engine, opt, _, _ = ds.initialize(model, cfg)
    gen = torch.Generator(device=gpu).manual_seed(2)
    for it in range(5):
        for micro in range(2):
            with opt.no_sync():
                loss = engine(torch.randn(8, 32, device=gpu, generator=gen)).float().pow(2).mean()
                if it == 1 and micro == 1:
                    loss = loss * float("inf")
                engine.backward(loss)
            engine.step()
    assert opt.current_step == 4 and opt.overflow_count == 1
    thr = opt.get_throughput_stats()
    assert set(thr) == {"steps_per_second", "avg_step_time", "overflow_rate"}
    assert thr["overflow_rate"] == 0.25
    assert opt.get_communication_stats()["total_comm_bytes"] == 0

    numel = opt.base_optimizer.numel
    assert numel % 8 == 0 and numel >= sum(p.numel() for p in model.parameters())
    est = opt.estimate_memory_usage()
    assert est["parameters_gb"] == est["gradients_gb"] == 2 * numel / 1e9
    assert est["optimizer_states_gb"] == 12 * numel / 1e9
    assert est["memory_per_gpu_gb"] == est["total_gb"] == pytest.approx(16 * numel / 1e9, rel=1e-12)
    info = opt.get_memory_info()
    assert info["allocated_gb"] > 0 and info["optimizer_states_on_host"] is False
    gp = opt.gather_params()
    assert list(gp) == [f"param_{i}" for i in range(4)] and gp["param_0"] is opt.model_parameters[0]
    assert opt.partition_params(gp) is None

    sd = opt.state_dict()
    assert sd["current_step"] == 4 and sd["overflow_count"] == 1
    opt.reset_stats()
    assert opt.overflow_count == 0 and opt.current_step == 4
    opt.load_state_dict(sd)
    assert opt.current_step == 4 and opt.overflow_count == 1
    sd["current_step"], sd["overflow_count"] = 10, 3
    opt.load_state_dict(sd)
    assert opt.current_step == 10 and opt.overflow_count == 3
    opt.current_step = 7
    assert opt.current_step == 7 and opt.base_optimizer.read_state().t == 4


def test_grad_hand_over_matches_in_place_zeroing(gpu):
    """zero_grad(set_to_none=True) (autograd's grads copied into the flat
    buffer by the post-accumulate hook) and zero_grad(set_to_none=False)
    (flat buffer zeroed, autograd accumulates into it) train bit-identically:
    fp16 with a dynamic loss scale, two micro-batches per step, one parameter
    that never receives a grad."""
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer
    _say("grad hand-over vs in-place zeroing")

    def build():
        torch.manual_seed(11)
        model = torch.nn.Sequential(torch.nn.Linear(64, 96), torch.nn.GELU(), torch.nn.Linear(96, 8)).to(gpu)
        spare = torch.nn.Parameter(torch.randn(37, device=gpu) * 0.1)  # never used in forward
        opt = AdamWOptimizer(list(model.parameters()) + [spare], lr=1e-3, weight_decay=0.05, max_grad_norm=1.0,
                             param_dtype=torch.float16, device=gpu,
                             loss_scaler=ScalerConfig(mode="dynamic", init_scale=2.0 ** 12, window=1000,
                                                      hysteresis=1))
        return model, opt

    runs = []
    for set_to_none in (True, False):
        model, opt = build()
        gen = torch.Generator(device=gpu).manual_seed(3)
        for _ in range(4):
            opt.zero_grad(set_to_none=set_to_none)
            for _ in range(2):
                x = torch.randn(16, 64, device=gpu, generator=gen).half()
                loss = model(x).float().pow(2).mean() / 2
                (loss * opt.loss_scale_tensor()).backward()
            opt.step()
        torch.cuda.synchronize()
        assert opt.read_state().t == 4
        runs.append({k: getattr(opt.flat, k).clone() for k in ("master", "exp_avg", "exp_avg_sq", "param16")})
    for k in runs[0]:
        assert torch.equal(runs[0][k].view(torch.int16 if k == "param16" else torch.int32),
                           runs[1][k].view(torch.int16 if k == "param16" else torch.int32)), k


def test_norm_taken_by_the_hand_over_copy(gpu):
    """K1 folded into the hooks' copies: after zero_grad(set_to_none=True) and
    one backward the step finalizes from the copies' partials (no K1 pass)
    and trains bit-identically to the K1 path (in-place zeroing), with the
    norm equal to 1e-12; the step falls back to K1 when the partials may be
    stale -- a torch in-place edit of a grad after backward, a parameter with
    no grad, two micro-batches -- and still matches the K1 path."""
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer
    _say("norm folded into the hand-over copy")

    def build(spare_used):
        torch.manual_seed(21)
        model = torch.nn.Sequential(torch.nn.Linear(96, 160), torch.nn.GELU(), torch.nn.Linear(160, 24)).to(gpu)
        spare = torch.nn.Parameter(torch.randn(29, device=gpu) * 0.1)
        opt = AdamWOptimizer(list(model.parameters()) + [spare], lr=1e-3, weight_decay=0.05, max_grad_norm=0.5,
                             param_dtype=torch.float16, device=gpu,
                             loss_scaler=ScalerConfig(mode="dynamic", init_scale=2.0 ** 10, window=1000,
                                                      hysteresis=1))
        return model, spare, opt

    def run(set_to_none, case):
        model, spare, opt = build(case != "unused")
        gen = torch.Generator(device=gpu).manual_seed(5)
        ready, norms = [], []
        for _ in range(3):
            opt.zero_grad(set_to_none=set_to_none)
            for _ in range(2 if case == "accumulate" else 1):
                x = torch.randn(24, 96, device=gpu, generator=gen).half()
                out = model(x).float().pow(2).mean()
                if case != "unused":
                    out = out + spare.float().pow(2).sum() * 1e-3
                (out * opt.loss_scale_tensor()).backward()
            if case == "edit":
                for p in model.parameters():
                    p.grad.mul_(0.5)
            opt.flat.check_grads_bound()
            ready.append(opt.flat.hook_norm_ready())
            opt.step()
            norms.append(float(opt.grad_norm_tensor().item()))
        torch.cuda.synchronize()
        state = {k: getattr(opt.flat, k).clone() for k in ("master", "exp_avg", "exp_avg_sq", "param16")}
        return ready, norms, state

    for case in ("plain", "edit", "unused", "accumulate"):
        r_fold, n_fold, s_fold = run(True, case)
        r_k1, n_k1, s_k1 = run(False, case)
        assert r_k1 == [False] * 3
        assert r_fold == ([True] * 3 if case == "plain" else [False] * 3), (case, r_fold)
        for a, b in zip(n_fold, n_k1):
            assert a == pytest.approx(b, rel=1e-12), case
        for k in s_fold:
            dt = torch.int16 if k == "param16" else torch.int32
            assert torch.equal(s_fold[k].view(dt), s_k1[k].view(dt)), (case, k)


def test_one_call_step_matches_three_launches(gpu):
    """The eager flat step issues K1 -> K0 -> K2 through one C call
    (dsx_zero_step_plan) unless the skip flag is tracked, which keeps the
    launches separate: both give the same bits over 1030 steps with two
    groups, learning rates changed every 100 steps, betas changed once, an
    overflow skip and the bias-correction tables growing past 1024 steps."""
    import torch
    from distributedspeed_amd.flat_step import ScalerConfig
    from distributedspeed_amd.optimizers import AdamWOptimizer
    shapes = [(130, 7), (9,), (64, 33)]
    torch.manual_seed(3)
    init = [torch.randn(s) * 0.05 for s in shapes]

    def build(track):
        ps = [torch.nn.Parameter(t.clone().to(gpu)) for t in init]
        opt = AdamWOptimizer([{"params": ps[:2]}, {"params": ps[2:], "lr": 2e-3, "weight_decay": 0.0}],
                             lr=1e-3, betas=(0.9, 0.95), weight_decay=0.1, max_grad_norm=0.5,
                             param_dtype=torch.float16, device=gpu,
                             loss_scaler=ScalerConfig(mode="dynamic", init_scale=2.0 ** 8, window=50, hysteresis=1))
        opt.track_skips(track)
        return opt

    a, b = build(False), build(True)
    assert a._plan is not None
    gen = torch.Generator(device=gpu).manual_seed(4)
    _say("one-call step vs three launches, 1030 steps")
    for step in range(1030):
        g = (torch.randn(a.flat.numel, device=gpu, generator=gen) * 1e-2 * 256).half()
        if step == 5:
            g[100] = float("inf")
        a.flat.grad.copy_(g)
        b.flat.grad.copy_(g)
        if step % 100 == 99:
            for o in (a, b):
                o.param_groups[0]["lr"] *= 0.9
        if step == 500:
            for o in (a, b):
                o.param_groups[1]["betas"] = (0.8, 0.99)
        a.step()
        b.step()
    torch.cuda.synchronize()
    for name in ("master", "exp_avg", "exp_avg_sq", "param16"):
        x, y = getattr(a.flat, name), getattr(b.flat, name)
        assert torch.equal(x.view(torch.int16 if x.element_size() == 2 else torch.int32),
                           y.view(torch.int16 if y.element_size() == 2 else torch.int32)), name
    sa, sb = a.read_state(), b.read_state()
    assert bytes(sa) == bytes(sb)
    assert sa.t > 1024 and sa.overflow_count >= 1 and sa.error == 0


@pytest.mark.parametrize("contiguous", [True, False], ids=["flat", "ragged"])
def test_frozen_parameters_are_not_stepped(gpu, contiguous):
    """torch's AdamW steps a parameter only when it has a grad, so a frozen
    one (requires_grad=False) given with the others -- model.parameters() in
    a fine-tune -- keeps its values bit for bit, and the others step exactly
    as when it is left out. The state dict keeps torch's indexing over every
    parameter of the groups (no state for the frozen one) and loads back; a
    grad that later appears on the frozen parameter is refused."""
    import torch
    from distributedspeed_amd.optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer
    cls = AdamWOptimizer if contiguous else MultiTensorAdamWOptimizer

    def model():
        torch.manual_seed(0)
        m = torch.nn.Sequential(torch.nn.Linear(16, 32), torch.nn.ReLU(), torch.nn.Linear(32, 4)).to(gpu)
        m[0].weight.requires_grad_(False)
        return m

    a, b, c = model(), model(), model()
    frozen = a[0].weight.detach().clone()
    oa = cls(list(a.parameters()), lr=1e-2, weight_decay=0.1, device=gpu)
    ob = cls([p for p in b.parameters() if p.requires_grad], lr=1e-2, weight_decay=0.1, device=gpu)
    x = torch.randn(8, 16, device=gpu, generator=torch.Generator(device=gpu).manual_seed(1))
    print(f"[gpu-test] frozen parameters, {'flat' if contiguous else 'ragged'}", file=sys.stderr, flush=True)
    for _ in range(3):
        for m, o in ((a, oa), (b, ob)):
            o.zero_grad()
            m(x).square().sum().backward()
            o.step()
    torch.cuda.synchronize()
    assert torch.equal(a[0].weight, frozen)
    for pa, pb in zip(a.parameters(), b.parameters()):
        assert torch.equal(pa, pb)
    sd = oa.state_dict()
    assert sorted(sd["state"]) == [1, 2, 3] and sd["param_groups"][0]["params"] == [0, 1, 2, 3]
    oc = cls(list(c.parameters()), lr=1e-2, weight_decay=0.1, device=gpu)
    oc.load_state_dict(sd)
    sc = oc.state_dict()
    assert sorted(sc["state"]) == [1, 2, 3]
    for k in (1, 2, 3):
        for name in ("exp_avg", "exp_avg_sq", "master"):
            assert torch.equal(sc["state"][k][name], sd["state"][k][name]), (k, name)
    a[0].weight.requires_grad_(True)
    oa.zero_grad()
    a(x).square().sum().backward()
    with pytest.raises(RuntimeError, match="did not require grad when the optimizer was built"):
        oa.step()


@pytest.mark.parametrize("contiguous", [True, False], ids=["flat", "ragged"])
def test_engine_fine_tune_with_a_frozen_layer(gpu, contiguous):
    """The fine-tune pattern: a frozen first layer and torch's AdamW over
    model.parameters() handed to initialize() under bf16. The frozen layer
    takes the 16-bit dtype with the rest, so the module runs in one; it
    keeps its values through the steps while the trained layers move."""
    import torch
    import distributedspeed_amd as ds
    model = _mlp(7).cuda()
    model[0].weight.requires_grad_(False)
    model[0].bias.requires_grad_(False)
    topt = torch.optim.AdamW(model.parameters(), lr=1e-3, weight_decay=0.1)
    cfg = {"bf16": {"enabled": True}, "max_grad_norm": 1.0,
           "zero_optimization": {"stage": 2, "contiguous_gradients": contiguous}}
    engine, opt, _, _ = ds.initialize(model, cfg, optimizer=topt)
    assert all(p.dtype == torch.bfloat16 for p in model.parameters())
    frozen = [model[0].weight.detach().clone(), model[0].bias.detach().clone()]
    trained = model[2].weight.detach().clone()
    x = torch.randn(16, 784, device=gpu, generator=torch.Generator(device=gpu).manual_seed(3))
    y = torch.randint(0, 10, (16,), device=gpu, generator=torch.Generator(device=gpu).manual_seed(4))
    _say(f"fine-tune with a frozen layer, contiguous={contiguous}")
    for _ in range(3):
        loss = torch.nn.functional.cross_entropy(engine(x).float(), y)
        engine.backward(loss)
        engine.step()
    torch.cuda.synchronize()
    assert torch.equal(model[0].weight, frozen[0]) and torch.equal(model[0].bias, frozen[1])
    assert not torch.equal(model[2].weight, trained)
    assert opt.current_step == 3


@pytest.mark.parametrize("contiguous", [True, False])
def test_refused_checkpoints_and_state_dicts_change_nothing(gpu, tmp_path, contiguous):
    """What does not fit is refused before anything changes. load_checkpoint
    refuses a checkpoint of another model: layers of another width, or a
    parameter of the same name and size but another shape, which a check of
    names and sizes alone would have let through. load_state_dict (the
    ZeROOptimizer's, and so the base optimizer's, Src/zero/optimizer.py:
    356-404) refuses a state dict with another group count, a group of
    another size, or a state tensor of another shape. Each refusal is a
    ValueError. Afterwards master, exp_avg, exp_avg_sq, params, the device
    state, lr and the accumulation count are what they were, and the good
    state dict still loads."""
    import copy

    import torch
    import distributedspeed_amd as ds
    from distributedspeed_amd import _lib
    _say(f"refused loads, contiguous_gradients={contiguous}")

    class Reshaped(torch.nn.Module):
        """One 784x1024 weight stored in a given shape (the same size either
        way), then a 10-way head."""

        def __init__(self, shape, seed):
            super().__init__()
            g = torch.Generator().manual_seed(seed)
            self.w = torch.nn.Parameter(torch.randn(*shape, generator=g) * 0.02)
            self.head = torch.nn.Linear(1024, 10)

        def forward(self, x):
            return self.head(x @ self.w.reshape(784, 1024))

    cfg = {"fp16": {"enabled": True, "hysteresis": 1}, "max_grad_norm": 1.0,
           "zero_optimization": {"stage": 2, "contiguous_gradients": contiguous}}
    gen = torch.Generator(device=gpu)
    gen.manual_seed(31)
    data = [(torch.randn(16, 784, device=gpu, generator=gen), torch.randint(0, 10, (16,), device=gpu, generator=gen))
            for _ in range(2)]

    def train(engine):
        for x, y in data:
            engine.backward(torch.nn.functional.cross_entropy(engine(x).float(), y))
            engine.step()

    def snapshot(engine):
        b = engine.optimizer.base_optimizer
        torch.cuda.synchronize(gpu)
        views = [{k: v.detach().cpu().clone() for k, v in b.store.views_of(i).items()} for i in range(len(b.dsx_params))]
        params = [p.detach().cpu().clone() for p in b.dsx_params]
        st = bytes(b.read_state())
        return views, params, st, [g["lr"] for g in b.param_groups], engine.optimizer.gradient_accumulation_count

    def same(a, b):
        assert a[2] == b[2] and a[3] == b[3] and a[4] == b[4]
        for va, vb in zip(a[0], b[0]):
            for k in va:
                assert torch.equal(va[k].view(torch.int32), vb[k].view(torch.int32)), k
        for pa, pb in zip(a[1], b[1]):
            assert torch.equal(pa.view(torch.int16), pb.view(torch.int16))

    wide, _, _, _ = ds.initialize(_mlp(5), cfg)
    train(wide)
    wide.save_checkpoint(str(tmp_path / "wide"))
    narrow_model = torch.nn.Sequential(torch.nn.Linear(784, 512), torch.nn.ReLU(), torch.nn.Linear(512, 1024),
                                       torch.nn.ReLU(), torch.nn.Linear(1024, 10))
    narrow, _, _, _ = ds.initialize(narrow_model, cfg)
    train(narrow)
    before = snapshot(narrow)
    with pytest.raises(ValueError, match="layout does not match"):
        narrow.load_checkpoint(str(tmp_path / "wide"))
    same(before, snapshot(narrow))

    a, _, _, _ = ds.initialize(Reshaped((784, 1024), 1), cfg)
    train(a)
    a.save_checkpoint(str(tmp_path / "a"))
    b, _, _, _ = ds.initialize(Reshaped((1024, 784), 2), cfg)
    train(b)
    before = snapshot(b)
    with pytest.raises(ValueError, match="layout does not match"):
        b.load_checkpoint(str(tmp_path / "a"))
    same(before, snapshot(b))

    zo = wide.optimizer
    good = zo.state_dict()
    before = snapshot(wide)
    bad_count = copy.deepcopy(good)
    bad_count["param_groups"].append(dict(bad_count["param_groups"][0], params=[]))
    bad_size = copy.deepcopy(good)
    bad_size["param_groups"][0]["params"] = bad_size["param_groups"][0]["params"][:-1]
    bad_shape = copy.deepcopy(good)
    k0 = bad_shape["param_groups"][0]["params"][0]
    bad_shape["state"][k0]["exp_avg"] = bad_shape["state"][k0]["exp_avg"].reshape(-1)
    for bad, what in ((bad_count, "number of parameter groups"), (bad_size, "doesn't match the size"),
                      (bad_shape, "has shape")):
        for g in bad["param_groups"]:
            g["lr"] = 123.0  # would show if the hyper-parameters were taken before the refusal
        bad["gradient_accumulation_count"] = 3
        with pytest.raises(ValueError, match=what):
            zo.load_state_dict(bad)
        same(before, snapshot(wide))
    zo.load_state_dict(good)
    after = snapshot(wide)
    # a load carries the state, not the last step's record (last_norm, last_skip)
    fields = ("scale", "good_steps", "hyst_left", "t", "iter", "overflow_count", "error")
    sa, sb = (_lib.DsxState.from_buffer_copy(x[2]) for x in (before, after))
    assert [getattr(sa, f) for f in fields] == [getattr(sb, f) for f in fields]
    same(before[:2] + (b"",) + before[3:], after[:2] + (b"",) + after[3:])
