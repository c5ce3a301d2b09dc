"""ZeROOptimizer: the reference's ZeRO front-end over the fused step.

Same constructor, methods and counters as Src/zero/optimizer.py:52-569 --
step(closure) with the gradient-accumulation gate (:212-233), backward(loss)
scaling the loss by 1/accumulation and the loss scale (:300-322),
clip_grad_norm_ (:324-341), zero_grad, get_lr / set_lr, state_dict /
load_state_dict with zero_stage / current_step / overflow_count /
gradient_accumulation_count / grad_scaler (:356-404), and attribute
delegation to the base optimizer (:563-569).

What differs, by design: the overflow check, unscale, norm, clip, AdamW,
cast and loss-scale update all run on the device inside one fused step
(AdamWOptimizer.step_fused), so the host never waits for the GPU; the skip
decision lives on the device and `overflow_count` reads it back on demand.
The reference's own overflow check is inert as wired (_check_overflow
always returns False, :276-291); this one is real. At world size 1 every ZeRO
stage runs the same single-partition step.
"""
from __future__ import annotations

import logging
import time
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
        self.current_step = 0
        self.gradient_accumulation_count = 0
        self.timers = {"step_time": 0.0}

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
        self.current_step += 1
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
        """Sets the clipping threshold of the fused step and returns the
        current (unscaled) grad norm as a device tensor. The reference
        multiplies the grads in place here; the fused step applies the same
        coefficient max_norm / (norm + 1e-6) in fp32 inside K2 instead."""
        if norm_type != 2.0:
            raise NotImplementedError("the fused step computes the L2 norm only")
        self.base_optimizer.max_grad_norm = float(max_norm)
        return self.grad_norm()

    def grad_norm(self) -> torch.Tensor:
        """sqrt(sum of squared unscaled grads) of the current grads, computed
        by K1 into a device tensor (no host sync)."""
        opt = self.base_optimizer
        opt.launch_norm()
        return opt.partials[:opt.nparts].sum().sqrt()

    # ---- counters and properties --------------------------------------------------------------

    @property
    def overflow_count(self) -> int:
        return int(self.base_optimizer.read_state().overflow_count)

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
        sd["current_step"] = self.current_step
        sd["overflow_count"] = int(sd["dsx"]["overflow_count"])
        sd["gradient_accumulation_count"] = self.gradient_accumulation_count
        sd["grad_scaler"] = {"scale": sd["dsx"]["scale"], "growth_tracker": sd["dsx"]["good_steps"],
                             "hysteresis_left": sd["dsx"]["hyst_left"]}
        return sd

    def load_state_dict(self, state_dict: Dict[str, Any]) -> None:
        state_dict = dict(state_dict)
        self.current_step = state_dict.pop("current_step", 0)
        state_dict.pop("overflow_count", None)
        self.gradient_accumulation_count = state_dict.pop("gradient_accumulation_count", 0)
        state_dict.pop("grad_scaler", None)
        state_dict.pop("zero_stage", None)
        self.base_optimizer.load_state_dict(state_dict)

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
