"""Device-resident driver of the ZeRO optimizer step over one flat partition.

FlatStep owns the small device buffers the kernels need -- the DsxState
(loss scale, scaler counters, AdamW step t), this step's DsxStepScalars, the
fp64 norm partials and the bias-correction table -- and issues
K1 -> K0 -> K2 on the current stream with no host synchronisation.

It is the device half of ZeROOptimizer.step (Src/zero/optimizer.py:212-274)
for ZeRO stage 1/2 at one rank: overflow check / skip, unscale, norm, clip
(Src/zero/utils.py:187-216), AdamW (the torch.optim.AdamW call at
Src/zero/stage2.py:609-612), 16-bit cast and GradScaler.update
(Src/zero/optimizer.py:265-266).
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from . import ops
from ._lib import (DSX_MAX_PARTIALS, DSX_SCALE_DYNAMIC, DSX_SCALE_NONE, DSX_SCALE_STATIC, DsxAdamwHyper,
                   DsxScalerConfig)


@dataclass
class AdamWHyper:
    """optimizer.params of ds_config (Src/config.py:33-42) plus clipping
    (max_grad_norm, Src/config.py:249; coefficient max/(norm + 1e-6),
    Src/zero/utils.py:211-214)."""
    lr: float = 1e-4
    beta1: float = 0.9
    beta2: float = 0.999
    eps: float = 1e-8
    weight_decay: float = 0.01
    max_grad_norm: float = 0.0
    clip_eps: float = 1e-6

    def validate(self) -> None:
        # The messages torch.optim.Adam's constructor raises (torch/optim/adam.py).
        if not 0.0 <= self.lr:
            raise ValueError(f"Invalid learning rate: {self.lr}")
        if not 0.0 <= self.eps:
            raise ValueError(f"Invalid epsilon value: {self.eps}")
        if not 0.0 <= self.beta1 < 1.0:
            raise ValueError(f"Invalid beta parameter at index 0: {self.beta1}")
        if not 0.0 <= self.beta2 < 1.0:
            raise ValueError(f"Invalid beta parameter at index 1: {self.beta2}")
        if not 0.0 <= self.weight_decay:
            raise ValueError(f"Invalid weight_decay value: {self.weight_decay}")
        if math.isnan(self.max_grad_norm):
            raise ValueError("max_grad_norm must not be NaN")

    def to_c(self) -> DsxAdamwHyper:
        return DsxAdamwHyper(float(self.lr), float(self.beta1), float(self.beta2), float(self.eps),
                             float(self.weight_decay), float(self.max_grad_norm), float(self.clip_eps))


@dataclass
class ScalerConfig:
    """fp16 section of ds_config (Src/config.py:93-102): mode "dynamic" when
    fp16.loss_scale == 0, "static" when > 0; "none" for bf16/fp32."""
    mode: str = "none"
    init_scale: float = 1.0
    window: int = 1000
    hysteresis: int = 2
    min_scale: float = 1.0
    growth_factor: float = 2.0
    backoff_factor: float = 0.5

    def to_c(self) -> DsxScalerConfig:
        mode = {"none": DSX_SCALE_NONE, "static": DSX_SCALE_STATIC, "dynamic": DSX_SCALE_DYNAMIC}[self.mode]
        return DsxScalerConfig(mode, int(self.window), int(self.hysteresis), 0, float(self.min_scale),
                               float(self.growth_factor), float(self.backoff_factor), 0.0)

    def validate(self) -> None:
        if self.mode not in ("none", "static", "dynamic"):
            raise ValueError(f"unknown loss-scale mode {self.mode!r}")
        if not (self.init_scale > 0 and math.isfinite(self.init_scale)):
            raise ValueError(f"loss scale must be finite and > 0, got {self.init_scale}")
        if self.mode == "dynamic":
            if self.window < 1:
                raise ValueError(f"loss_scale_window must be >= 1, got {self.window}")
            if self.hysteresis < 1:
                raise ValueError(f"hysteresis must be >= 1, got {self.hysteresis}")
            if not self.min_scale > 0:
                raise ValueError(f"min_loss_scale must be > 0, got {self.min_scale}")


class BiasCorrectionTable:
    """Device table of {1 - beta1**t, (1 - beta2**t)**0.5} for t = 1..len,
    evaluated on the host in Python double exactly as torch/optim/adam.py:529-535
    does, so the device never evaluates pow(). It grows by doubling; the
    host keeps it at least as long as the number of steps issued."""

    def __init__(self, device: torch.device, beta1: float, beta2: float, capacity: int = 1024):
        self.device = device
        self.betas = (float(beta1), float(beta2))
        self.length = 0
        self.table = torch.empty(0, dtype=torch.float64, device=device)
        self._host = None
        self.ensure(capacity)

    @staticmethod
    def entries(beta1: float, beta2: float, t_max: int) -> list[float]:
        out = []
        for t in range(1, t_max + 1):
            step = float(t)
            out.append(1 - beta1 ** step)
            out.append((1 - beta2 ** step) ** 0.5)
        return out

    def ensure(self, t_max: int, betas: tuple[float, float] | None = None) -> None:
        betas = (float(betas[0]), float(betas[1])) if betas is not None else self.betas
        if t_max <= self.length and betas == self.betas:
            return
        cap = max(1024, self.length)
        while cap < t_max:
            cap *= 2
        self.betas = betas
        host = torch.tensor(self.entries(*betas, cap), dtype=torch.float64)
        if torch.cuda.is_available():
            host = host.pin_memory()
        self._host = host  # keep the pinned source alive until the copy has run
        self.table = host.to(self.device, non_blocking=True)
        self.length = cap


class FlatStep:
    """Steps one flat partition: fp32 master/exp_avg/exp_avg_sq, 16-bit grads
    and (optionally) 16-bit params, all contiguous and 16-byte aligned."""

    def __init__(self, numel: int, device: torch.device, hyper: AdamWHyper, scaler: ScalerConfig):
        hyper.validate()
        scaler.validate()
        self.numel = int(numel)
        self.device = torch.device(device)
        self.hyper = hyper
        self.scaler = scaler
        self.nparts = min(ops.suggest_partials(self.numel), DSX_MAX_PARTIALS)
        self.partials = torch.zeros(self.nparts, dtype=torch.float64, device=self.device)
        self.state = ops.new_state(self.device, scaler.init_scale if scaler.mode != "none" else 1.0,
                                   scaler.hysteresis if scaler.mode == "dynamic" else 1)
        self.scalars = ops.new_scalars(self.device)
        self.bc = BiasCorrectionTable(self.device, hyper.beta1, hyper.beta2)
        self.steps_issued = 0

    def loss_scale_tensor(self) -> torch.Tensor:
        """Device view of the current loss scale (no host sync)."""
        return ops.scale_view(self.state)

    def step(self, master: torch.Tensor, exp_avg: torch.Tensor, exp_avg_sq: torch.Tensor,
             param16: torch.Tensor | None, grad: torch.Tensor, lr: float | None = None) -> None:
        if master.numel() != self.numel:
            raise ValueError(f"partition has {master.numel()} elements, FlatStep was built for {self.numel}")
        if lr is not None:
            self.hyper.lr = float(lr)
        self.steps_issued += 1
        self.bc.ensure(self.steps_issued, (self.hyper.beta1, self.hyper.beta2))
        ops.zero_step_flat(master, exp_avg, exp_avg_sq, param16, grad, self.state, self.scaler.to_c(),
                           self.hyper.to_c(), self.bc.table, self.bc.length, self.partials, self.nparts,
                           self.scalars)

    def read_state(self):
        return ops.read_state(self.state)

    def read_scalars(self):
        return ops.read_scalars(self.scalars)
