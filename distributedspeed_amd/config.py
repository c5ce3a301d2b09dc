"""ds_config for the optimizer-step path.

Mirrors the parts of the reference's DistributedSpeedConfig
(Src/config.py:213-530) that the ZeRO optimizer step consumes, with the same
defaults, deep-merge loading (config.py:302-354), unknown-key behaviour (a
TypeError from the section's dataclass constructor), validation messages
(config.py:356-396) and DISTRIBUTEDSPEED_* environment overrides
(config.py:398-421):

  optimizer.{type, params.{lr, betas, eps, weight_decay}}     config.py:33-42
  fp16.{enabled, loss_scale, initial_scale_power, loss_scale_window,
        hysteresis, min_loss_scale, auto_cast}                 config.py:93-102
  bf16.{enabled, auto_cast}                                    config.py:105-109
  zero_optimization.{stage, cpu_offload, contiguous_gradients, ...}
                                                               config.py:56-90
  gradient_accumulation_steps, max_grad_norm (default 1.0)     config.py:245-249

DeepSpeed's top-level `gradient_clipping` is accepted as an alias of
max_grad_norm. Sections that do not feed the optimizer step (scheduler,
pipeline, communication, logging, ...) are kept verbatim in `extra`.
"""
from __future__ import annotations

import copy
import json
import logging
import os
from dataclasses import asdict, dataclass, field
from typing import Any, Dict, Optional, Union

logger = logging.getLogger(__name__)


@dataclass
class OptimizerConfig:
    type: str = "AdamW"
    params: Dict[str, Any] = field(default_factory=lambda: {
        "lr": 1e-4, "betas": [0.9, 0.999], "eps": 1e-8, "weight_decay": 0.01})


@dataclass
class FP16Config:
    enabled: bool = False
    loss_scale: float = 0.0  # 0 means dynamic scaling
    initial_scale_power: int = 16
    loss_scale_window: int = 1000
    hysteresis: int = 2
    min_loss_scale: float = 1.0
    auto_cast: bool = True


@dataclass
class BF16Config:
    enabled: bool = False
    auto_cast: bool = True


@dataclass
class ZeROConfig:
    stage: int = 0
    cpu_offload: bool = False
    cpu_offload_params: bool = False
    cpu_offload_use_pin_memory: bool = True
    allgather_partitions: bool = True
    allgather_bucket_size: float = 2e8
    overlap_comm: bool = True
    reduce_scatter: bool = True
    reduce_bucket_size: float = 2e8
    contiguous_gradients: bool = True
    param_persistence_threshold: float = 1e6
    model_persistence_threshold: float = 1e6
    max_live_parameters: float = 1e9
    max_reuse_distance: float = 1e9
    prefetch_bucket_size: float = 5e8
    param_round_robin: bool = False
    offload_optimizer_config: Optional[Dict[str, Any]] = None
    offload_param_config: Optional[Dict[str, Any]] = None
    sub_group_size: float = 1e9
    elastic_checkpoint: bool = True
    ignore_unused_parameters: bool = True
    partition_grads: bool = True
    round_robin_gradients: bool = False
    zero_hpz_partition_size: int = 1
    zero_quantized_weights: bool = False
    zero_quantized_gradients: bool = False


_SECTIONS = {"optimizer": OptimizerConfig, "fp16": FP16Config, "bf16": BF16Config, "zero_optimization": ZeROConfig}

_ENV = {
    "DISTRIBUTEDSPEED_TRAIN_BATCH_SIZE": ("train_batch_size", int),
    "DISTRIBUTEDSPEED_MICRO_BATCH_SIZE": ("train_micro_batch_size_per_gpu", int),
    "DISTRIBUTEDSPEED_GRAD_ACCUM_STEPS": ("gradient_accumulation_steps", int),
    "DISTRIBUTEDSPEED_LEARNING_RATE": ("optimizer.params.lr", float),
    "DISTRIBUTEDSPEED_ZERO_STAGE": ("zero_optimization.stage", int),
    "DISTRIBUTEDSPEED_FP16_ENABLED": ("fp16.enabled", lambda x: x.lower() == "true"),
    "DISTRIBUTEDSPEED_BF16_ENABLED": ("bf16.enabled", lambda x: x.lower() == "true"),
}


def _deep_update(base: dict, upd: dict) -> None:
    for k, v in upd.items():
        if k in base and isinstance(base[k], dict) and isinstance(v, dict):
            _deep_update(base[k], v)
        else:
            base[k] = v


class DistributedSpeedConfig:
    """The step-relevant subset of the reference's configuration object."""

    def __init__(self, config_dict: Optional[Dict[str, Any]] = None):
        self.train_batch_size = 32
        self.train_micro_batch_size_per_gpu = None
        self.gradient_accumulation_steps = 1
        self.max_grad_norm = 1.0
        self.optimizer = OptimizerConfig()
        self.fp16 = FP16Config()
        self.bf16 = BF16Config()
        self.zero_optimization = ZeROConfig()
        self.extra: Dict[str, Any] = {}
        if config_dict:
            self._load(copy.deepcopy(config_dict))
        self._validate()
        self._apply_env_overrides()

    def _load(self, d: Dict[str, Any]) -> None:
        merged = {name: asdict(getattr(self, name)) for name in _SECTIONS}
        sect = {k: v for k, v in d.items() if k in _SECTIONS}
        _deep_update(merged, sect)
        for name, cls in _SECTIONS.items():
            setattr(self, name, cls(**merged[name]))  # unknown keys raise TypeError, as the reference does
        for k, v in d.items():
            if k in _SECTIONS:
                continue
            if k == "gradient_clipping":
                self.max_grad_norm = float(v)
            elif k in ("train_batch_size", "train_micro_batch_size_per_gpu", "gradient_accumulation_steps",
                       "max_grad_norm"):
                setattr(self, k, v)
            else:
                self.extra[k] = v

    def _validate(self) -> None:
        errors = []
        if self.train_batch_size is not None and self.train_batch_size <= 0:
            errors.append("train_batch_size must be positive")
        if self.gradient_accumulation_steps <= 0:
            errors.append("gradient_accumulation_steps must be positive")
        if self.zero_optimization.stage not in [0, 1, 2, 3]:
            errors.append("ZeRO stage must be 0, 1, 2, or 3")
        if self.fp16.enabled and self.bf16.enabled:
            errors.append("Cannot enable both FP16 and BF16 simultaneously")
        if not self.optimizer.type:
            errors.append("Optimizer type must be specified")
        if self.max_grad_norm is not None and self.max_grad_norm < 0:
            errors.append("max_grad_norm must be non-negative")
        if self.fp16.enabled and self.fp16.loss_scale == 0:
            if self.fp16.loss_scale_window < 1:
                errors.append("fp16.loss_scale_window must be >= 1")
            if self.fp16.hysteresis < 1:
                errors.append("fp16.hysteresis must be >= 1")
            if self.fp16.min_loss_scale <= 0:
                errors.append("fp16.min_loss_scale must be positive")
        if errors:
            raise ValueError("Configuration validation failed:\n" + "\n".join(f"  - {e}" for e in errors))

    def _apply_env_overrides(self) -> None:
        for var, (path, conv) in _ENV.items():
            raw = os.environ.get(var)
            if raw is None:
                continue
            try:
                self._set_nested(path, conv(raw))
                logger.info("Applied environment override: %s=%s", var, raw)
            except (ValueError, TypeError) as e:
                logger.warning("Failed to apply environment override %s=%s: %s", var, raw, e)

    def _set_nested(self, path: str, value: Any) -> None:
        parts = path.split(".")
        obj = self
        for p in parts[:-1]:
            obj = obj[p] if isinstance(obj, dict) else getattr(obj, p)
        if isinstance(obj, dict):
            obj[parts[-1]] = value
        else:
            setattr(obj, parts[-1], value)

    # ---- derived settings the step uses -----------------------------------------

    @property
    def precision(self) -> str:
        return "fp16" if self.fp16.enabled else "bf16" if self.bf16.enabled else "fp32"

    def adamw_params(self) -> Dict[str, Any]:
        p = dict(self.optimizer.params)
        betas = p.get("betas", [0.9, 0.999])
        return {"lr": float(p.get("lr", 1e-4)), "betas": (float(betas[0]), float(betas[1])),
                "eps": float(p.get("eps", 1e-8)), "weight_decay": float(p.get("weight_decay", 0.01))}

    def loss_scaler(self) -> Dict[str, Any]:
        """fp16.loss_scale == 0 -> dynamic (init 2**initial_scale_power,
        window, hysteresis, min); > 0 -> static; bf16/fp32 -> none."""
        f = self.fp16
        if not f.enabled:
            return {"mode": "none", "init_scale": 1.0}
        if f.loss_scale and f.loss_scale > 0:
            return {"mode": "static", "init_scale": float(f.loss_scale)}
        return {"mode": "dynamic", "init_scale": float(2.0 ** f.initial_scale_power),
                "window": int(f.loss_scale_window), "hysteresis": int(f.hysteresis),
                "min_scale": float(f.min_loss_scale)}

    def to_dict(self) -> Dict[str, Any]:
        d = {name: asdict(getattr(self, name)) for name in _SECTIONS}
        d.update(train_batch_size=self.train_batch_size,
                 train_micro_batch_size_per_gpu=self.train_micro_batch_size_per_gpu,
                 gradient_accumulation_steps=self.gradient_accumulation_steps, max_grad_norm=self.max_grad_norm)
        d.update(copy.deepcopy(self.extra))
        return d

    def __getitem__(self, key: str) -> Any:
        return getattr(self, key) if hasattr(self, key) else self.extra[key]

    def get(self, key: str, default: Any = None) -> Any:
        try:
            return self[key]
        except KeyError:
            return default


def load_config(config: Union[str, Dict[str, Any], DistributedSpeedConfig, None]) -> DistributedSpeedConfig:
    """dict, JSON/YAML path or config object -> DistributedSpeedConfig
    (Src/config.py:533-573)."""
    if config is None:
        return DistributedSpeedConfig()
    if isinstance(config, DistributedSpeedConfig):
        return config
    if isinstance(config, str):
        if not os.path.exists(config):
            raise FileNotFoundError(f"Configuration file not found: {config}")
        with open(config) as f:
            if config.endswith((".yaml", ".yml")):
                import yaml
                data = yaml.safe_load(f)
            else:
                data = json.load(f)
        return DistributedSpeedConfig(data)
    if isinstance(config, dict):
        return DistributedSpeedConfig(config)
    raise TypeError(f"Unsupported config type: {type(config)}")


def fp16_config() -> Dict[str, Any]:
    """The reference's fp16 preset (Src/__init__.py:473-484)."""
    return {"fp16": {"enabled": True, "loss_scale": 0, "loss_scale_window": 1000, "initial_scale_power": 16,
                     "hysteresis": 2, "min_loss_scale": 1}}


def bf16_config() -> Dict[str, Any]:
    """The reference's bf16 preset (Src/__init__.py:486-492)."""
    return {"bf16": {"enabled": True}}


def zero_config(stage: int) -> Dict[str, Any]:
    return {"zero_optimization": {"stage": stage, "contiguous_gradients": True}}


__all__ = ["DistributedSpeedConfig", "OptimizerConfig", "FP16Config", "BF16Config", "ZeROConfig", "load_config",
           "fp16_config", "bf16_config", "zero_config"]
