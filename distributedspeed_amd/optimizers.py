"""AdamWOptimizer: the fused ZeRO optimizer step behind torch's Optimizer API.

The reference's stages call `optimizer.step_fused()` when the optimizer has
one and `optimizer.step()` otherwise (Src/zero/stage1.py:522-525,
Src/zero/stage2.py:609-612); its public name for a fused AdamW is
`optimizers.AdamWOptimizer` (Src/__init__.py:109-114). This class is that
optimizer: torch.optim.AdamW's constructor arguments, param_groups,
state[p] (exp_avg / exp_avg_sq / master / step as live views), zero_grad,
state_dict / load_state_dict, and a step that runs entirely on the GPU:

    K1 unscale + inf/NaN + norm partials   over the whole flat grad buffer
    K0 finalize                            skip, norm, clip, t, per-group
                                           scalars, loss-scaler update
    K2 AdamW + 16-bit cast                 one launch per parameter group

with no host synchronisation. Parameters are re-homed into one
FlatPartition at construction (param.data / param.grad become views).
MultiTensorAdamWOptimizer is the same optimizer over parameters left in
their own storage (K1 and K3 over a chunk table instead of K1 and K2 over
one buffer), for zero_optimization.contiguous_gradients = false.
With graph=True the three stages are captured into one HIP graph at the
first step and replayed afterwards (K0 then reads the per-group values from
device memory; see graph.py).
"""
from __future__ import annotations

import ctypes
import math
from itertools import chain
from typing import Iterable

import torch
from torch.optim import optimizer as _topt

from . import _lib, ops
from ._lib import DSX_MAX_GROUPS, DsxAdamwHyper
from .flat import FlatPartition
from .flat_step import BiasCorrectionTable, ScalerConfig
from .offload import HostStateStreamer
from .ragged import RaggedParams


def _check_hyper(lr, betas, eps, weight_decay, max_grad_norm) -> None:
    if not 0.0 <= lr:
        raise ValueError(f"Invalid learning rate: {lr}")
    if not 0.0 <= eps:
        raise ValueError(f"Invalid epsilon value: {eps}")
    if not 0.0 <= betas[0] < 1.0:
        raise ValueError(f"Invalid beta parameter at index 0: {betas[0]}")
    if not 0.0 <= betas[1] < 1.0:
        raise ValueError(f"Invalid beta parameter at index 1: {betas[1]}")
    if not 0.0 <= weight_decay:
        raise ValueError(f"Invalid weight_decay value: {weight_decay}")
    if math.isnan(max_grad_norm) or max_grad_norm < 0:
        raise ValueError(f"Invalid max_grad_norm: {max_grad_norm}")


class _FusedAdamWBase(torch.optim.Optimizer):
    """What both storage forms share: torch.optim.AdamW's constructor
    checks and param_groups, the device-resident DsxState / partials /
    per-group scalars, the bias-correction tables, the readers and the
    checkpoint format. A subclass provides `store` (the parameter storage:
    params, numel, views_of, refresh_params16, layout, zero_grad) and
    step_fused()."""

    def _init_common(self, params, lr, betas, eps, weight_decay, max_grad_norm, loss_scaler, device):
        _check_hyper(lr, betas, eps, weight_decay, max_grad_norm)
        defaults = dict(lr=lr, betas=tuple(betas), eps=eps, weight_decay=weight_decay)
        super().__init__(params, defaults)
        if len(self.param_groups) > DSX_MAX_GROUPS:
            raise ValueError(f"at most {DSX_MAX_GROUPS} parameter groups are supported")
        everything = [p for g in self.param_groups for p in g["params"]]
        if not everything:
            raise ValueError("optimizer got an empty parameter list")
        # torch's AdamW steps a parameter only when it has a grad, so a frozen
        # one (requires_grad=False) is never touched. Such parameters stay out
        # of the stepped storage here; the state dict keeps torch's indexing
        # over every parameter of the groups (_state_index maps a stepped
        # parameter to its index there).
        self._stepped = [[p for p in g["params"] if p.requires_grad] for g in self.param_groups]
        self._frozen = [p for p in everything if not p.requires_grad]
        self._state_index = [i for i, p in enumerate(everything) if p.requires_grad]
        plist = [p for ps in self._stepped for p in ps]
        if not plist:
            raise ValueError("optimizer got no parameter that requires grad")
        if device is None:
            device = plist[0].device if plist[0].is_cuda else torch.device("cuda", torch.cuda.current_device())
        self.device = torch.device(device)
        self.max_grad_norm = float(max_grad_norm)
        self.clip_eps = 1e-6
        self.scaler = loss_scaler or ScalerConfig(mode="none")
        self.scaler.validate()
        return plist

    def _init_device(self, numel: int) -> None:
        self.nparts = ops.suggest_partials(numel)
        self.partials = torch.zeros(self.nparts, dtype=torch.float64, device=self.device)
        self.dstate = ops.new_state(self.device, self.scaler.init_scale if self.scaler.mode != "none" else 1.0,
                                    self.scaler.hysteresis if self.scaler.mode == "dynamic" else 1)
        self.scalars = torch.zeros(ops.SCALARS_BYTES * len(self.param_groups), dtype=torch.uint8, device=self.device)
        self._bc: dict[tuple[float, float], BiasCorrectionTable] = {}
        self._t_offsets = [0] * len(self.param_groups)
        self.steps_issued = 0
        self._skip_host = None  # pinned mirror of DsxState.last_skip (see track_skips)
        self._skip_event = None
        self._adopted_from = None  # the torch optimizer whose param groups were adopted, if any

    def _note_stepped(self) -> None:
        """What torch's LR schedulers look for to know that the optimizer
        stepped before them (the flag their step() wrapper sets): the step
        usually runs through step_fused(), which that wrapper does not see,
        and a scheduler may be attached to an adopted torch optimizer."""
        self._opt_called = True
        if self._adopted_from is not None:
            self._adopted_from._opt_called = True
        for p in self._frozen:
            if p.grad is not None:
                raise RuntimeError("a parameter that did not require grad when the optimizer was built has a grad: "
                                   "torch would step it, this optimizer holds no state for it; build the "
                                   "optimizer again after changing requires_grad")

    # ---- skip flag on the host, without waiting for K2 ---------------------------------

    def track_skips(self, on: bool = True) -> None:
        """After every step's skip decision, copy DsxState.last_skip into
        pinned host memory and record an event, so that last_step_skipped()
        need not synchronise the whole device. In the eager forms the step
        then runs as separate launches and the copy sits right after K0, so
        the wait covers K1 and K0 only. In the capturable and graph forms the
        step is one recorded sequence (with K0 folded into K2 where the fold
        applies), so the copy follows the whole step and the wait covers K2
        too. Costs one small device-to-host copy per step in stream order;
        off by default."""
        if on and self._skip_host is None:
            self._skip_host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
            self._skip_event = torch.cuda.Event()
        elif not on:
            self._skip_host = self._skip_event = None

    def _after_finalize(self) -> None:
        if self._skip_host is not None:
            self._skip_host.copy_(self.dstate[36:40].view(torch.int32), non_blocking=True)  # DsxState.last_skip
            self._skip_event.record(torch.cuda.current_stream(self.device))

    def last_step_skipped(self) -> bool:
        """Whether the last step was skipped (overflow). With track_skips on
        this waits for the event track_skips records (after K0 in the eager
        forms, after the whole step in the capturable and graph forms);
        otherwise it synchronises."""
        if self._skip_host is not None and self._skip_event is not None and self.steps_issued:
            self._skip_event.synchronize()
            return bool(int(self._skip_host[0]))
        return bool(self.read_state().last_skip)

    # ---- torch.optim.Optimizer protocol ---------------------------------------------

    @property
    def dsx_params(self) -> list:
        """The parameters in step order."""
        return self.store.params

    @property
    def numel(self) -> int:
        return self.store.numel

    def layout(self) -> list[dict]:
        return self.store.layout()

    def _bind_state(self) -> None:
        t_view = self.dstate[12:16].view(torch.int32)  # DsxState.t
        for i, p in enumerate(self.store.params):
            st = dict(self.store.views_of(i))
            st["step"] = t_view
            self.state[p] = st

    def zero_grad(self, set_to_none: bool = True) -> None:
        """set_to_none (torch's default): p.grad becomes None. In the flat
        form the next backward's grads are then copied into the flat buffer by
        a post-accumulate-grad hook (4 B/elt instead of zeroing plus
        accumulating, 8 B/elt); in the ragged form they are read where
        autograd puts them (the tensor table's grad pointers are refreshed at
        the next step). The grads are zeroed in place instead for
        capturable=True (a captured iteration must not depend on Python-side
        state)."""
        self.store.zero_grad(set_to_none=set_to_none and self._grads_may_move())
        for p in self._frozen:  # as torch's zero_grad does for every parameter of the groups
            if p.grad is not None:
                if set_to_none:
                    p.grad = None
                else:
                    p.grad.zero_()

    def _grads_may_move(self) -> bool:
        return True

    def add_param_group(self, param_group: dict) -> None:
        if getattr(self, "store", None) is not None:
            raise NotImplementedError("add_param_group after construction would move the parameter storage; "
                                      "build the optimizer with all groups")
        super().add_param_group(param_group)

    def step(self, closure=None):
        """torch's Optimizer.step protocol: the closure, the step pre / post
        hooks (global and per optimizer) and the profiler range. torch wraps
        step() to run that machinery at every call, which costs ~10 us of host
        time -- as much as the three launches of a small partition's step.
        Here it runs only when a hook is registered or the profiler records;
        otherwise step() is the closure plus step_fused()."""
        if (self._optimizer_step_pre_hooks or self._optimizer_step_post_hooks
                or _topt._global_optimizer_pre_hooks or _topt._global_optimizer_post_hooks
                or torch.autograd._profiler_enabled()):
            return self._step_with_hooks(closure)
        return self._step_plain(closure)

    step.hooked = True  # torch's _patch_step_function leaves a step marked hooked unwrapped

    def _step_plain(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self.step_fused()
        return loss

    def _step_with_hooks(self, closure=None):
        args, kwargs = (self,), ({"closure": closure} if closure is not None else {})
        with torch.autograd.profiler.record_function(f"Optimizer.step#{type(self).__name__}.step"):
            for pre in chain(_topt._global_optimizer_pre_hooks.values(), self._optimizer_step_pre_hooks.values()):
                result = pre(self, args, kwargs)
                if result is not None:
                    if not (isinstance(result, tuple) and len(result) == 2):
                        raise RuntimeError(f"step pre-hook must return None or a tuple of (new_args, new_kwargs), "
                                           f"but got {result}.")
                    args, kwargs = result
            out = self._step_plain(*args[1:], **kwargs)
            self._optimizer_step_code()
            for post in chain(self._optimizer_step_post_hooks.values(), _topt._global_optimizer_post_hooks.values()):
                post(self, args, kwargs)
        return out

    def _refresh_group_block(self) -> None:
        """The host group block (self._gblock: per-group hyper-parameters,
        bias tables, t offsets) of the one-call steps, refilled only when a
        value in param_groups or max_grad_norm changed or the bias tables
        must grow."""
        key = (tuple((float(g["lr"]), g["betas"], g["eps"], g["weight_decay"]) for g in self.param_groups),
               self.max_grad_norm, self.clip_eps)
        if key != self._gkey or self.steps_issued > self._gblock.bc_len:
            hs, tables, bc_len = self._hypers()
            blk = self._gblock
            for k, h in enumerate(hs):
                blk.hyper[k] = h
                blk.bc_table[k] = tables[k].data_ptr()
                blk.t_offset[k] = self._t_offsets[k]
            blk.ngroups, blk.bc_len = len(hs), bc_len
            self._gtables = tables  # the block holds their addresses
            self._gkey = key

    def _hypers(self):
        hs, tabs = [], []
        for g in self.param_groups:
            b1, b2 = float(g["betas"][0]), float(g["betas"][1])
            hs.append(DsxAdamwHyper(float(g["lr"]), b1, b2, float(g["eps"]), float(g["weight_decay"]),
                                    self.max_grad_norm, self.clip_eps))
            key = (b1, b2)
            if key not in self._bc:
                self._bc[key] = BiasCorrectionTable(self.device, b1, b2)
            self._bc[key].ensure(self.steps_issued)
            tabs.append(self._bc[key])
        bc_len = min(t.length for t in tabs)
        return hs, [t.table for t in tabs], bc_len

    # ---- clip_grad_norm_ ---------------------------------------------------------------------

    def clip_grad_norm_(self, max_norm: float, norm_type: float = 2.0) -> torch.Tensor:
        """The reference's contract (Src/zero/optimizer.py:324-341, which the
        stages implement at Src/zero/stage1.py:549-582 and
        Src/zero/stage2.py:683-725, and Src/zero/utils.py:187-216): the norm of
        type norm_type (any p > 0, or inf) of the current unscaled grads is
        taken now, and the grads are clipped once by max_norm / (norm + 1e-6)
        if norm > max_norm. The grads are not rewritten here: the coefficient
        is armed in the device state and the next fused step applies it (in
        fp32, inside K2) instead of the configured max_grad_norm; the step
        after that clips by the configured max_grad_norm again. A skipped
        (overflow) step consumes it too. Returns the pre-clip norm as a 0-dim
        fp32 device tensor, with no host synchronisation."""
        p = ops.norm_type_of(norm_type)
        max_norm = float(max_norm)
        if not max_norm >= 0:
            raise ValueError(f"max_norm must be >= 0, got {max_norm}")
        s = ops.stream_of(self.device)
        self._norm_launch(p)(s)
        if getattr(self, "_clip_norm", None) is None:
            self._clip_norm = torch.zeros(1, dtype=torch.float64, device=self.device)
        ops.clip_prepare(self.partials, self.nparts, p, max_norm, self.clip_eps, self.dstate, self._clip_norm)
        return self._clip_norm[0].to(torch.float32)

    def _norm_launch(self, p: float) -> ops.Launch:
        raise NotImplementedError

    # ---- device-side values, read on demand --------------------------------------------------

    def refresh_master(self) -> None:
        """Take the fp32 master from the current params. Needed after the
        16-bit params were written from outside the step, e.g. a model state
        dict loaded after this optimizer was built (the engine does this by
        itself for its module); the step reads only the master and would
        otherwise write the old values back."""
        self.store.refresh_master()

    def set_scaler_state(self, scale: float, good_steps: int = 0) -> None:
        """Loss scale and clean-step count of a dynamic scaler (as from a
        torch GradScaler's state dict); other modes keep their own scale."""
        if self.scaler.mode != "dynamic":
            return
        if not (scale > 0 and math.isfinite(scale)):
            raise ValueError(f"loss scale must be finite and > 0, got {scale}")
        hs = self.read_state()
        hs.scale = float(scale)
        hs.good_steps = int(good_steps)
        self.dstate.copy_(torch.frombuffer(bytearray(bytes(hs)), dtype=torch.uint8).to(self.device))

    def loss_scale_tensor(self) -> torch.Tensor:
        """The loss scale as a one-element fp32 device tensor (no sync)."""
        return ops.scale_view(self.dstate)

    def read_state(self):
        """DsxState on the host (synchronises)."""
        return ops.read_state(self.dstate)

    def init_warm_step(self) -> None:
        """The reference's construction-time warm step, on request
        (Src/zero/stage1.py:330-374, Src/zero/stage2.py:386-430: its ZeRO
        stages 1 and 2 give every owned parameter a zero grad and call step()
        on a throwaway copy of the optimizer, then keep that copy's state).
        One AdamW step over zero grads: each parameter decays once by
        (1 - lr * weight_decay), exp_avg and exp_avg_sq stay zero, and the
        AdamW step count becomes 1, so later steps take the bias corrections
        of t = 2, 3, ... The loss scaler takes no part (the reference calls
        the torch optimizer's step directly). Only before the first step;
        the grads are set to None afterwards, as the reference leaves them."""
        if self.steps_issued:
            raise RuntimeError("init_warm_step() is the construction-time step: call it before any other step")
        self._zero_grads_in_place()
        saved = self.scaler
        self.scaler = ScalerConfig(mode="none")
        try:
            self._warm_launch()
        finally:
            self.scaler = saved
        self.zero_grad(set_to_none=True)

    def _zero_grads_in_place(self) -> None:
        raise NotImplementedError

    def _warm_launch(self) -> None:
        self.step_fused()

    def last_scalars(self, group: int = 0):
        return ops.read_scalars(self.scalars[group * ops.SCALARS_BYTES:(group + 1) * ops.SCALARS_BYTES])

    def grad_norm_tensor(self) -> torch.Tensor:
        """Norm seen by the last step, as an fp64 device tensor (no sync)."""
        return self.dstate[40:48].view(torch.float64)

    # ---- checkpoints ----------------------------------------------------------------------------

    def state_dict(self) -> dict:
        """torch-compatible layout (state keyed by parameter index with
        exp_avg / exp_avg_sq / step) plus the fp32 master and the device
        scaler state; tensors are host copies."""
        if getattr(self, "streamer", None) is not None:
            # offloaded state: pinned host memory written by asynchronous
            # copies, whichever stream the caller is on now
            torch.cuda.synchronize(self.device)
        s = self.read_state()
        groups = []
        idx = 0
        for g in self.param_groups:
            gd = {k: v for k, v in g.items() if k != "params"}
            gd["params"] = list(range(idx, idx + len(g["params"])))
            idx += len(g["params"])
            groups.append(gd)
        state = {}
        for i in range(len(self.store.params)):
            v = self.store.views_of(i)
            state[self._state_index[i]] = {"step": torch.tensor(float(s.t)), "exp_avg": v["exp_avg"].detach().cpu().clone(),
                        "exp_avg_sq": v["exp_avg_sq"].detach().cpu().clone(),
                        "master": v["master"].detach().cpu().clone()}
        return {"state": state, "param_groups": groups,
                "dsx": {"scale": s.scale, "good_steps": s.good_steps, "hyst_left": s.hyst_left, "t": s.t,
                        "iter": s.iter, "overflow_count": s.overflow_count, "steps_issued": self.steps_issued,
                        "layout": self.store.layout(), "scaler": dict(vars(self.scaler))}}

    def load_state_dict(self, state_dict: dict) -> None:
        """Loads this optimizer's state dict or torch AdamW's (the
        reference's, Src/zero/optimizer.py:356-404). Every check runs before
        anything changes: a refused state dict (ValueError: another group
        count or group size, a state tensor of another shape) leaves the
        optimizer as it was."""
        if getattr(self, "streamer", None) is not None:
            torch.cuda.synchronize(self.device)  # no copy of an earlier step may still write the host state
        groups = state_dict["param_groups"]
        if len(groups) != len(self.param_groups):
            raise ValueError("loaded state dict has a different number of parameter groups")
        for g, sg in zip(self.param_groups, groups):
            if len(g["params"]) != len(sg["params"]):
                raise ValueError("loaded state dict contains a parameter group that doesn't match the size "
                                 "of optimizer's group")
        st = state_dict["state"]
        ix = self._state_index
        for i in range(len(self.store.params)):
            if ix[i] not in st:
                continue
            views = self.store.views_of(i)
            for key in ("exp_avg", "exp_avg_sq", "master"):
                if key in st[ix[i]] and tuple(st[ix[i]][key].shape) != tuple(views[key].shape):
                    raise ValueError(f"state for parameter {ix[i]} has shape {tuple(st[ix[i]][key].shape)}, "
                                     f"expected {tuple(views[key].shape)}")
        dsx = state_dict.get("dsx")
        t = int(dsx["t"]) if dsx else int(max((float(v["step"]) for v in st.values()), default=0))
        from ._lib import DsxState
        hs = DsxState()
        hs.scale = float(dsx["scale"]) if dsx else (self.scaler.init_scale if self.scaler.mode != "none" else 1.0)
        hs.good_steps = int(dsx["good_steps"]) if dsx else 0
        hs.hyst_left = int(dsx["hyst_left"]) if dsx else max(1, self.scaler.hysteresis)
        hs.t = t
        hs.iter = int(dsx["iter"]) if dsx else t
        hs.overflow_count = int(dsx["overflow_count"]) if dsx else 0
        steps_issued = int(dsx["steps_issued"]) if dsx else t
        # checked: now change
        for g, sg in zip(self.param_groups, groups):
            for k, v in sg.items():
                if k != "params":
                    g[k] = tuple(v) if k == "betas" else v
        # A torch (or the reference's) state dict holds no master: those
        # parameters take theirs from the current params, which the caller
        # loads from the same checkpoint.
        self.store.refresh_master([i for i in range(len(self.store.params)) if "master" not in st.get(ix[i], {})])
        with torch.no_grad():
            for i in range(len(self.store.params)):
                if ix[i] not in st:
                    continue
                views = self.store.views_of(i)
                for key in ("exp_avg", "exp_avg_sq", "master"):
                    if key in st[ix[i]]:
                        views[key].copy_(st[ix[i]][key].to(views[key].device, torch.float32))
            self.store.refresh_params16()
        self.dstate.copy_(torch.frombuffer(bytearray(bytes(hs)), dtype=torch.uint8).to(self.device))
        self.steps_issued = steps_issued
        self._bind_state()


class AdamWOptimizer(_FusedAdamWBase):
    """The flat form: every parameter re-homed into one FlatPartition (the
    reference's contiguous_gradients layout, Src/zero/stage2.py:108-193)."""

    def __init__(self, params: Iterable, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2, *, max_grad_norm: float = 0.0, param_dtype: torch.dtype | None = None,
                 loss_scaler: ScalerConfig | None = None, device: torch.device | None = None,
                 param_names: dict | None = None, offload: bool = False, offload_chunk_elems: int = 64 << 20,
                 graph: bool = False, capturable: bool = False):
        plist = self._init_common(params, lr, betas, eps, weight_decay, max_grad_norm, loss_scaler, device)
        if param_dtype is None and plist[0].dtype in (torch.float16, torch.bfloat16):
            param_dtype = plist[0].dtype
        if (graph or capturable) and offload:
            raise ValueError("graph=True / capturable=True need HBM-resident state (offload=False)")
        if graph and capturable:
            raise ValueError("graph=True captures the step itself; capturable=True is for callers that capture it")
        self.flat = FlatPartition(self._stepped, self.device, param_dtype, param_names,
                                  offload=offload)
        self.store = self.flat
        self.streamer = HostStateStreamer(self.device, offload_chunk_elems) if offload else None
        self._init_device(self.flat.numel)
        self.use_graph = bool(graph)
        self._graph = None
        self._bind_state()
        # The flat buffers never move, so every launch of the step is checked
        # and bound once here; a step then costs one ctypes call per launch.
        self._k1 = ops.plan_unscale_norm(self.flat.grad, self.dstate, self.partials, self.nparts)
        self._k0 = ops.FinalizeGroups(self.partials, self.nparts, self.dstate, self.scalars, len(self.param_groups))
        self._k2 = []
        if self.streamer is None:
            for gi in range(len(self.param_groups)):
                master, m, v, p16, g = self.flat.group_views(gi)
                if master.numel():
                    sc = self.scalars[gi * ops.SCALARS_BYTES:(gi + 1) * ops.SCALARS_BYTES]
                    self._k2.append(ops.plan_adamw_flat(master, m, v, p16, g, sc))
        self.capturable = bool(capturable)
        # The eager step as one C call (dsx_zero_step_plan: K1, K0 and each
        # group's K2), with its fixed arguments packed here once.
        self._plan = None
        if self.streamer is None and not self.use_graph and not self.capturable:
            self._build_plan()
        # K1 folded into the hooks' copies (eager form only: a captured or
        # graph-replayed step keeps its K1).
        self._k0_hook = None
        if not self.capturable and not self.use_graph and self.flat.enable_hook_norm(self.dstate):
            self._k0_hook = ops.FinalizeGroups(self.flat.hook_norm_partials, len(self.flat.params), self.dstate,
                                               self.scalars, len(self.param_groups))
        if self.capturable:
            # The kernels read the per-group values from device memory, so the
            # launches can be recorded into a caller's graph and replayed.
            self.groups_dev = torch.zeros(ops.GROUPS_BYTES, dtype=torch.uint8, device=self.device)
            self._dev_step = ops.plan_zero_step_dev(self.pack_plan(), self.groups_dev,
                                                    keep=(self.flat, self.partials, self.dstate, self.scalars))
            self._uploaded = None
            self._prepared = False

    def _grads_may_move(self) -> bool:
        return not self.capturable

    def _zero_grads_in_place(self) -> None:
        self.flat.zero_grad(set_to_none=False)

    def _warm_launch(self) -> None:
        if not (self.use_graph or self.capturable):
            self.step_fused()
            return
        # Not through the graph or the device group block: a one-off eager
        # dsx_zero_step_plan call with this step's (scaler-free) plan.
        self.steps_issued += 1
        hs, tables, bc_len = self._hypers()
        G = _lib.DsxGroupsDev.from_buffer_copy(ops.pack_groups(hs, tables, self._t_offsets, bc_len))
        P = self.pack_plan()
        _lib.call("dsx_zero_step_plan", ctypes.byref(P), ctypes.byref(G), ops.stream_of(self.device))

    # ---- the eager step in one call ------------------------------------------------------

    def pack_plan(self) -> _lib.DsxFlatPlan:
        """The flat step's fixed arguments as a DsxFlatPlan (host struct):
        buffers, dtypes, partials, step records, group boundaries, scaler."""
        f = self.flat
        P = _lib.DsxFlatPlan()
        P.master, P.exp_avg, P.exp_avg_sq = f.master.data_ptr(), f.exp_avg.data_ptr(), f.exp_avg_sq.data_ptr()
        P.param16 = f.param16.data_ptr() if f.param16 is not None else None
        P.grad = f.grad.data_ptr()
        P.n = f.numel
        P.param_dtype = ops.dtype_code(f.param16.dtype) if f.param16 is not None else _lib.DSX_F16
        P.grad_dtype = ops.grad_code(f.grad.dtype)
        P.state, P.partials, P.out = self.dstate.data_ptr(), self.partials.data_ptr(), self.scalars.data_ptr()
        P.nparts, P.ngroups = self.nparts, len(self.param_groups)
        P.scaler = self.scaler.to_c()
        for k, (_, b) in enumerate(f.group_ranges):
            P.group_end[k] = b
        return P

    def _build_plan(self) -> None:
        P = self.pack_plan()
        self._plan = P
        self._gblock = _lib.DsxGroupsDev()
        self._gkey = None  # what the group block was last filled from
        self._skey = None  # the scaler settings packed into the plan
        self._plan_fn = _lib.load().dsx_zero_step_plan
        self._plan_args = (ctypes.byref(P), ctypes.byref(self._gblock))

    def _step_plan(self) -> None:
        """K1 -> K0 -> K2 (or K1 and K2 with K0 folded in) through
        dsx_zero_step_plan. The group block is refilled only when it must be
        (_refresh_group_block); the scaler settings only when they changed."""
        self._refresh_group_block()
        sc = self.scaler
        skey = (sc.mode, sc.window, sc.hysteresis, sc.min_scale, sc.growth_factor, sc.backoff_factor)
        if skey != self._skey:
            self._plan.scaler = sc.to_c()
            self._skey = skey
        rc = self._plan_fn(*self._plan_args, ops.stream_of(self.device))
        if rc:
            raise _lib.DsxError("dsx_zero_step_plan", rc, _lib.last_error())

    # ---- capturable form ----------------------------------------------------------------

    def prepare_step(self) -> None:
        """capturable=True: the host half of a step, outside any capture --
        count the step, grow the bias-correction tables if needed, and upload
        the per-group block (lr, betas, eps, weight decay, tables) when it
        changed (a kernel launch in stream order; no host wait). Eager step()
        calls it; a caller replaying a captured step calls it before each
        replay."""
        if not self.capturable:
            raise RuntimeError("prepare_step() belongs to capturable=True")
        self.steps_issued += 1
        hs, tables, bc_len = self._hypers()
        key = (tuple((h.lr, h.beta1, h.beta2, h.eps, h.weight_decay, h.max_grad_norm, h.clip_eps) for h in hs),
               tuple(t.data_ptr() for t in tables), tuple(self._t_offsets), int(bc_len))
        if key != self._uploaded:
            ops.groups_upload(ops.pack_groups(hs, tables, self._t_offsets, bc_len), self.groups_dev)
            self._uploaded = key
        self._prepared = True

    def _step_capturable(self) -> None:
        capturing = torch.cuda.is_current_stream_capturing()
        if not capturing and not self._prepared:
            self.prepare_step()
        self._prepared = False
        self.flat.check_grads_bound()
        self._dev_step(ops.stream_of(self.device))
        if not capturing:
            self._after_finalize()

    def launch_norm(self) -> None:
        """K1 alone over the current grads (partials <- squared norms)."""
        self.flat.check_grads_bound()
        self._k1(ops.stream_of(self.device))

    def _norm_launch(self, p: float) -> ops.Launch:
        self.flat.check_grads_bound()
        return ops.plan_norm_partials(self.flat.grad, self.dstate, p, self.partials, self.nparts)

    def step_fused(self) -> None:
        """K1 -> K0 -> K2 on the current stream; no host synchronisation."""
        self._note_stepped()
        if self.capturable:
            self._step_capturable()
            return
        self.flat.check_grads_bound()
        self.steps_issued += 1
        if (self._plan is not None and self._skip_host is None
                and not (self._k0_hook is not None and self.flat.hook_norm_ready())):
            # one C call; with track_skips on, the three launches are issued
            # one by one so that the skip flag's copy sits between K0 and K2
            self._step_plan()
            self.flat.disarm_hook_norm()
            return
        hs, tables, bc_len = self._hypers()
        if self.use_graph:
            # Captured once (first step), replayed after uploading this step's
            # per-group block; the same kernels, buffers and order as below.
            if self._graph is None:
                from .graph import GraphedStep
                self._graph = GraphedStep(self)
            self._graph.replay(hs, tables, self._t_offsets, bc_len)
            self._after_finalize()  # after the replay: waits for the graph's K2 too
            return
        s = ops.stream_of(self.device)
        if self._k0_hook is not None and self.flat.hook_norm_ready():
            # the hooks' copies already took the norm's partials: no K1 pass
            self.flat.reduce_hook_norm(s)
            self._k0_hook(self.scaler.to_c(), hs, tables, self._t_offsets, bc_len, s)
        else:
            self._k1(s)
            self._k0(self.scaler.to_c(), hs, tables, self._t_offsets, bc_len, s)
        self.flat.disarm_hook_norm()
        self._after_finalize()
        if self.streamer is not None:
            # State in pinned host memory: stream it through HBM chunk by chunk.
            # A skipped step streams too (K2 leaves the chunks unchanged), which
            # keeps the host free of any wait on the device.
            pieces = [(a, b, self.scalars[gi * ops.SCALARS_BYTES:(gi + 1) * ops.SCALARS_BYTES])
                      for gi, (a, b) in enumerate(self.flat.group_ranges) if b > a]
            self.streamer.run((self.flat.master, self.flat.exp_avg, self.flat.exp_avg_sq), self.flat.param16,
                              self.flat.grad, pieces)
            return
        for k2 in self._k2:
            k2(s)



class MultiTensorAdamWOptimizer(_FusedAdamWBase):
    """The ragged form: parameters keep their own storage and autograd's
    grads; the step runs over the tensor list through a chunk table (K1 over
    the list, K0, K3), two streaming launches whatever the number of tensors;
    a mid-size list takes its large tensors through K2 one by one (see
    ragged.K2_TENSOR_ELEMS). Chosen by zero_optimization.contiguous_gradients
    = false."""

    def __init__(self, params: Iterable, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8,
                 weight_decay: float = 1e-2, *, max_grad_norm: float = 0.0, param_dtype: torch.dtype | None = None,
                 loss_scaler: ScalerConfig | None = None, device: torch.device | None = None,
                 param_names: dict | None = None, chunk_elems: int | None = None, offload: bool = False,
                 graph: bool = False):
        if offload or graph:
            raise ValueError("offload and graph capture need the flat form (contiguous_gradients = true)")
        plist = self._init_common(params, lr, betas, eps, weight_decay, max_grad_norm, loss_scaler, device)
        if param_dtype is None and plist[0].dtype in (torch.float16, torch.bfloat16):
            param_dtype = plist[0].dtype
        self.store = RaggedParams(self._stepped, self.device, param_dtype, param_names,
                                  chunk_elems)
        self.streamer = None
        self.use_graph = False
        self._graph = None
        self._init_device(self.store.numel)
        self._bind_state()
        self._k0 = ops.FinalizeGroups(self.partials, self.nparts, self.dstate, self.scalars, len(self.param_groups))
        self._plans_for = None  # the chunk table the bound K1 / K3 launches point at
        self._gblock = _lib.DsxGroupsDev()  # the one-call step's host group block
        self._gkey = None
        self._one_call = None

    def _zero_grads_in_place(self) -> None:
        with torch.no_grad():
            for p in self.store.params:
                if p.grad is None:
                    p.grad = torch.zeros_like(p)
                else:
                    p.grad.zero_()

    def _plans(self):
        table = self.store.table()
        if table is not self._plans_for:  # rebuilt after storage moved: bind again
            st = self.store
            self._k1 = ops.plan_unscale_norm_multi(table, self.dstate, self.partials, self.nparts)
            k3_table = st.small_table if st.k2_tensors else table
            self._k3 = ops.plan_adamw_multi(k3_table, self.scalars) if k3_table is not None else None
            # K2 per large tensor: everything but the grad is bound here; the
            # grad's address is read at each step (autograd's grads move).
            pdt = ops.dtype_code(st.param_dtype) if st.param_dtype is not None else ops.DSX_F16
            gdt = ops.grad_code(st.grad_dtype)
            base = self.scalars.data_ptr()
            self._k2_each = [(st.params[i], st.master[i].data_ptr(), st.exp_avg[i].data_ptr(),
                              st.exp_avg_sq[i].data_ptr(),
                              st.params[i].data.data_ptr() if st.param_dtype is not None else None,
                              st.master[i].numel(), base + ops.SCALARS_BYTES * st.group_of[i])
                             for i in st.k2_tensors]
            self._k2_meta = (pdt, gdt)
            # The whole step in one call (dsx_zero_step_multi) when no tensor
            # goes through K2: its fixed arguments, bound once per table.
            self._one_call = None
            if not st.k2_tensors:
                self._one_call = (_lib.load().dsx_zero_step_multi,
                                  (ops._ptr(table.tensors), ops._ptr(table.chunks), ctypes.c_int64(table.nchunks),
                                   ctypes.c_int64(table.numel), table.pdt, table.gdt, ops._ptr(self.dstate)),
                                  (ctypes.byref(self._gblock), ops._ptr(self.partials), int(self.nparts),
                                   ops._ptr(self.scalars)))
            self._plans_for = table
        return self._k1, self._k3

    def _k2_tensors(self, s) -> None:
        """K2 (dsx_adamw_flat) over each large tensor of the list."""
        if not self._k2_each:
            return
        fn = _lib.load().dsx_adamw_flat
        pdt, gdt = self._k2_meta
        for p, mp, ep, vp, pp, n, sp in self._k2_each:
            rc = fn(mp, ep, vp, pp, pdt, p.grad.data_ptr(), gdt, n, sp, s)
            if rc:
                raise _lib.DsxError("dsx_adamw_flat", rc, _lib.last_error())

    def launch_norm(self) -> None:
        k1, _ = self._plans()
        k1(ops.stream_of(self.device))

    def _norm_launch(self, p: float) -> ops.Launch:
        self._plans()
        return ops.plan_norm_partials_multi(self.store.table(), self.dstate, p, self.partials, self.nparts)

    def step_fused(self) -> None:
        """K1 (list) -> K0 -> K3 on the current stream (with K2 for each large
        tensor when the list is in K3's one-block-per-CU range); no host
        synchronisation (a chunk-table rebuild, after storage moved, uploads
        the new table)."""
        self._note_stepped()
        k1, k3 = self._plans()
        self.steps_issued += 1
        s = ops.stream_of(self.device)
        if self._one_call is not None and self._skip_host is None:
            # one C call (K1, K0, K3, or K1 and K3 with K0 folded in); with
            # track_skips on, the launches stay separate so that the skip
            # flag's copy sits between K0 and K3
            self._refresh_group_block()
            fn, head, tail = self._one_call
            rc = fn(*head, self.scaler.to_c(), *tail, s)
            if rc:
                raise _lib.DsxError("dsx_zero_step_multi", rc, _lib.last_error())
            return
        hs, tables, bc_len = self._hypers()
        k1(s)
        self._k0(self.scaler.to_c(), hs, tables, self._t_offsets, bc_len, s)
        self._after_finalize()
        self._k2_tensors(s)
        if k3 is not None:
            k3(s)


def adopt_torch_optimizer(opt: torch.optim.Optimizer, contiguous: bool = True, **kwargs) -> _FusedAdamWBase:
    """torch.optim.AdamW (or Adam without weight decay, where Adam and AdamW
    coincide) -> AdamWOptimizer over the same param groups (the same dict
    objects: a scheduler attached to `opt` keeps working) and
    hyper-parameters. Anything else is refused rather than silently changed
    into a different update rule."""
    if not isinstance(opt, torch.optim.Optimizer):
        raise TypeError(f"expected a torch.optim.Optimizer, got {type(opt).__name__}")
    if isinstance(opt, _FusedAdamWBase):
        return opt
    is_adamw = isinstance(opt, torch.optim.AdamW) or (isinstance(opt, torch.optim.Adam)
                                                      and opt.defaults.get("decoupled_weight_decay", False))
    plain_adam_no_wd = isinstance(opt, torch.optim.Adam) and all(g.get("weight_decay", 0) == 0
                                                                 for g in opt.param_groups)
    if not (is_adamw or plain_adam_no_wd):
        raise NotImplementedError(f"{type(opt).__name__} is not supported by the fused step; use AdamW")
    if any(g.get("amsgrad") or g.get("maximize") for g in opt.param_groups):
        raise NotImplementedError("amsgrad / maximize are not supported by the fused step")
    # The group dicts themselves are handed over (torch's add_param_group keeps
    # the dict it is given), so an LR scheduler built on `opt` -- which writes
    # into these dicts -- drives the fused step too.
    groups = list(opt.param_groups)
    d = opt.defaults
    cls = AdamWOptimizer if contiguous else MultiTensorAdamWOptimizer
    new = cls(groups, lr=float(d["lr"]), betas=d["betas"], eps=d["eps"], weight_decay=d["weight_decay"], **kwargs)
    new._adopted_from = opt
    return new
