"""ZeROOptimizer: the reference's ZeRO front-end over the fused step.

Same constructor, methods and counters as Src/zero/optimizer.py:52-569 --
step(closure) with the gradient-accumulation gate (:212-233), backward(loss)
scaling the loss by 1/accumulation and the loss scale (:300-322),
clip_grad_norm_ (:324-341), zero_grad, get_lr / set_lr, state_dict /
load_state_dict with zero_stage / current_step / overflow_count /
gradient_accumulation_count / grad_scaler (:356-404), no_sync,
gather_params / partition_params, the memory, communication and throughput
statistics and reset_stats (:407-559), and attribute delegation to the base
optimizer (:563-569).

What differs, by design: the overflow check, unscale, norm, clip, AdamW,
cast and loss-scale update all run on the device inside one fused step
(AdamWOptimizer.step_fused), so the host never waits for the GPU; the skip
decision lives on the device, and `overflow_count` and `current_step`
(clean steps only, as the reference counts them: :238-242, :269) read it back
on demand, which synchronises with the device.
The reference's own overflow check is inert as wired (_check_overflow
always returns False, :276-291); this one is real. At world size 1 every ZeRO
stage runs the same single-partition step.
"""
from __future__ import annotations

import logging
import time
from collections import defaultdict
from contextlib import contextmanager
from typing import Any, Dict, List, Optional

import torch

from .flat_step import ScalerConfig
from .optimizers import _FusedAdamWBase, adopt_torch_optimizer

logger = logging.getLogger(__name__)


def _config_get(cfg, key, default):
    if cfg is None:
        return default
    if isinstance(cfg, dict):
        return cfg.get(key, default)
    return getattr(cfg, key, default)


class ZeROOptimizer:
    """Wraps a base optimizer (an AdamWOptimizer, or a torch.optim.AdamW /
    Adam whose param_groups and hyper-parameters are moved onto one)."""

    def __init__(self, optimizer, config=None, model_parameters: Optional[List[torch.nn.Parameter]] = None,
                 comm_manager: Any = None):
        self.config = config
        self.comm_manager = comm_manager
        self.stage = int(_config_get(config, "stage", 0))
        if self.stage not in (0, 1, 2, 3):
            raise ValueError(f"ZeRO stage must be 0, 1, 2, or 3, got {self.stage}")
        self.gradient_accumulation_steps = int(_config_get(config, "gradient_accumulation_steps", 1))
        if self.gradient_accumulation_steps <= 0:
            raise ValueError("gradient_accumulation_steps must be positive")
        if not isinstance(optimizer, _FusedAdamWBase):
            optimizer = self._adopt(optimizer, config)
        self.base_optimizer = optimizer
        self.model_parameters = list(model_parameters) if model_parameters is not None else list(optimizer.dsx_params)
        self.param_groups = optimizer.param_groups
        self.gradient_accumulation_count = 0
        self.timers = defaultdict(float)
        self.communication_data_bytes = 0
        self.parameter_gathering_time = 0.0
        # current_step and overflow_count are read from the device counters
        # (DsxState.t, DsxState.overflow_count) plus these host offsets, which
        # load_state_dict and reset_stats move.
        self._step_base = 0
        self._overflow_base = 0

    @staticmethod
    def _adopt(opt, config) -> _FusedAdamWBase:
        scaler = _config_get(config, "loss_scaler", None)
        return adopt_torch_optimizer(opt, contiguous=bool(_config_get(config, "contiguous_gradients", True)),
                                     max_grad_norm=float(_config_get(config, "max_grad_norm", 0.0) or 0.0),
                                     loss_scaler=ScalerConfig(**scaler) if isinstance(scaler, dict) else scaler)

    # ---- the step --------------------------------------------------------------------------

    def zero_grad(self, set_to_none: bool = True) -> None:
        self.base_optimizer.zero_grad(set_to_none=set_to_none)
        self.gradient_accumulation_count = 0

    def step(self, closure=None):
        start = time.time()
        self.gradient_accumulation_count += 1
        if self.gradient_accumulation_count < self.gradient_accumulation_steps:
            return None
        self.gradient_accumulation_count = 0
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self.base_optimizer.step_fused()
        self.timers["step_time"] += time.time() - start
        return loss

    def backward(self, loss: torch.Tensor, retain_graph: bool = False) -> None:
        """loss / gradient_accumulation_steps * loss_scale, then backward. The
        scale is a device tensor: no host sync."""
        scaled = loss / self.gradient_accumulation_steps
        if self.base_optimizer.scaler.mode != "none":
            scaled = scaled.float() * self.base_optimizer.loss_scale_tensor()
        scaled.backward(retain_graph=retain_graph)

    def clip_grad_norm_(self, max_norm: float, norm_type: float = 2.0) -> torch.Tensor:
        """Clips the current grads once, as the reference does
        (Src/zero/optimizer.py:324-341 -> Src/zero/utils.py:187-216): the
        norm of type norm_type (p > 0 or inf) is taken now and returned as a
        0-dim device tensor (the pre-clip norm); if it exceeds max_norm, the
        next fused step multiplies the grads by max_norm / (norm + 1e-6) in
        place of the configured clip, which applies again from the step
        after. See AdamWOptimizer.clip_grad_norm_."""
        return self.base_optimizer.clip_grad_norm_(max_norm, norm_type)

    def init_warm_step(self) -> None:
        """The reference stages' construction-time warm step (one AdamW step
        over zero grads: Src/zero/stage1.py:330-374, stage2.py:386-430), on
        request, for runs that must follow the reference's trajectory; see
        AdamWOptimizer.init_warm_step. current_step stays 0, as the
        reference's counter does not see that step."""
        self.base_optimizer.init_warm_step()
        self._step_base -= 1

    def grad_norm(self) -> torch.Tensor:
        """sqrt(sum of squared unscaled grads) of the current grads, computed
        by K1 into a device tensor (no host sync)."""
        opt = self.base_optimizer
        opt.launch_norm()
        return opt.partials[:opt.nparts].sum().sqrt()

    # ---- counters and properties --------------------------------------------------------------

    @property
    def overflow_count(self) -> int:
        """Steps skipped for a non-finite grad (since the last reset_stats)."""
        return int(self.base_optimizer.read_state().overflow_count) - self._overflow_base

    @property
    def current_step(self) -> int:
        """Optimizer steps taken: skipped (overflow) steps and
        accumulation-only calls do not count, as in the reference."""
        return int(self.base_optimizer.read_state().t) + self._step_base

    @current_step.setter
    def current_step(self, value: int) -> None:
        self._step_base = int(value) - int(self.base_optimizer.read_state().t)

    @property
    def loss_scale(self) -> float:
        return float(self.base_optimizer.read_state().scale)

    @property
    def skipped_last_step(self) -> bool:
        return bool(self.base_optimizer.read_state().last_skip)

    def get_lr(self) -> float:
        return self.param_groups[0]["lr"] if self.param_groups else 0.0

    def set_lr(self, lr: float) -> None:
        for g in self.param_groups:
            g["lr"] = lr

    def state_dict(self) -> Dict[str, Any]:
        sd = self.base_optimizer.state_dict()
        sd["zero_stage"] = self.stage
        sd["current_step"] = int(sd["dsx"]["t"]) + self._step_base
        sd["overflow_count"] = int(sd["dsx"]["overflow_count"]) - self._overflow_base
        sd["gradient_accumulation_count"] = self.gradient_accumulation_count
        # torch's GradScaler.state_dict keys (what the reference stores and
        # loads), plus the hysteresis count torch's scaler does not have
        sc = self.base_optimizer.scaler
        if sc.mode == "dynamic":
            sd["grad_scaler"] = {"scale": sd["dsx"]["scale"], "growth_factor": sc.growth_factor,
                                 "backoff_factor": sc.backoff_factor, "growth_interval": sc.window,
                                 "_growth_tracker": sd["dsx"]["good_steps"], "hysteresis_left": sd["dsx"]["hyst_left"]}
        return sd

    def load_state_dict(self, state_dict: Dict[str, Any]) -> None:
        """The reference's keys (Src/zero/optimizer.py:356-404) around the
        base optimizer's state dict. A state dict the base optimizer refuses
        (ValueError) leaves this object unchanged as well."""
        state_dict = dict(state_dict)
        current_step = state_dict.pop("current_step", None)
        overflow_count = state_dict.pop("overflow_count", None)
        accumulation = int(state_dict.pop("gradient_accumulation_count", 0))
        scaler = state_dict.pop("grad_scaler", None)
        state_dict.pop("zero_stage", None)
        self.base_optimizer.load_state_dict(state_dict)
        self.gradient_accumulation_count = accumulation
        if "dsx" not in state_dict and scaler and "scale" in scaler:
            # the reference's state dict: its GradScaler's state
            # (Src/zero/optimizer.py:375-376, 397-398; torch's GradScaler.state_dict keys)
            self.base_optimizer.set_scaler_state(float(scaler["scale"]), int(scaler.get("_growth_tracker", 0)))
        st = self.base_optimizer.read_state()
        self._step_base = 0 if current_step is None else int(current_step) - int(st.t)
        self._overflow_base = 0 if overflow_count is None else int(st.overflow_count) - int(overflow_count)

    # ---- the reference's remaining accessors (Src/zero/optimizer.py:407-559) -------------------
    # At world size 1 every ZeRO stage holds the whole partition: nothing is
    # synchronised, gathered or partitioned, and no bytes are communicated.

    @contextmanager
    def no_sync(self):
        """Accumulate without gradient synchronisation: nothing to skip at
        world size 1."""
        yield

    def gather_params(self) -> Dict[str, torch.Tensor]:
        """The parameters by position, as the reference returns them for
        stages that keep parameters whole."""
        return {f"param_{i}": p for i, p in enumerate(self.model_parameters)}

    def partition_params(self, params_dict: Dict[str, torch.Tensor]) -> None:
        """Nothing to partition at world size 1 (the reference acts only for
        a stage-3 partitioner)."""
        return None

    def _storage_gb(self) -> Dict[str, float]:
        b = self.base_optimizer.store.storage_bytes()
        return {"parameters_gb": b["params"] / 1e9, "gradients_gb": b["grads"] / 1e9,
                "optimizer_states_gb": b["optimizer_states"] / 1e9,
                "optimizer_states_on_host": bool(b["optimizer_states_on_host"])}

    def get_memory_info(self) -> Dict[str, float]:
        """torch's allocator figures for the optimizer's device, in GB, plus
        what the partition holds (optimizer_states_gb counts the fp32 master
        with exp_avg and exp_avg_sq)."""
        dev = self.base_optimizer.device
        info = {"allocated_gb": torch.cuda.memory_allocated(dev) / 1e9,
                "cached_gb": torch.cuda.memory_reserved(dev) / 1e9,
                "max_allocated_gb": torch.cuda.max_memory_allocated(dev) / 1e9}
        info.update(self._storage_gb())
        return info

    def get_communication_stats(self) -> Dict[str, Any]:
        return {"total_comm_bytes": self.communication_data_bytes,
                "avg_comm_time": self.timers.get("comm_time", 0.0) / max(1, self.current_step),
                "parameter_gathering_time": self.parameter_gathering_time}

    def get_throughput_stats(self) -> Dict[str, float]:
        """The reference's formulas. step_time sums the host time of step()
        calls, which here only enqueue work (the step runs asynchronously)."""
        total = self.timers.get("step_time", 1.0)
        steps = self.current_step
        return {"steps_per_second": steps / total if total > 0 else 0.0,
                "avg_step_time": total / max(1, steps),
                "overflow_rate": self.overflow_count / max(1, steps)}

    def reset_stats(self) -> None:
        self.timers.clear()
        self.communication_data_bytes = 0
        self.parameter_gathering_time = 0.0
        self._overflow_base = int(self.base_optimizer.read_state().overflow_count)

    def estimate_memory_usage(self) -> Dict[str, float]:
        """Memory this layout holds, in GB, under the reference's keys:
        16-bit params, grads of the grad dtype and 12 bytes of fp32 state per
        element (the reference's estimate assumes 4-byte params and grads and
        8 bytes of state). memory_per_gpu_gb leaves out state kept in host
        memory (cpu_offload)."""
        g = self._storage_gb()
        total = g["parameters_gb"] + g["gradients_gb"] + g["optimizer_states_gb"]
        on_gpu = total - (g["optimizer_states_gb"] if g["optimizer_states_on_host"] else 0.0)
        return {"parameters_gb": g["parameters_gb"], "gradients_gb": g["gradients_gb"],
                "optimizer_states_gb": g["optimizer_states_gb"], "total_gb": total, "memory_per_gpu_gb": on_gpu}

    def __repr__(self) -> str:
        return (f"ZeROOptimizer(stage={self.stage}, world_size=1, parameters={len(self.model_parameters)}, "
                f"numel={self.base_optimizer.numel})")

    def __getattr__(self, name: str):
        if name == "base_optimizer":
            raise AttributeError(name)
        base = self.__dict__.get("base_optimizer")
        if base is not None and hasattr(base, name):
            return getattr(base, name)
        raise AttributeError(f"'{type(self).__name__}' object has no attribute '{name}'")
