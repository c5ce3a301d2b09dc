"""distributedspeed_amd -- MI355X-native ZeRO optimizer step.

The hot path of DistributedSpeed's ZeROOptimizer.step
(Src/zero/optimizer.py:212-274) -- unscale, inf/NaN detection, grad norm,
clipping, AdamW, the 16-bit cast and the dynamic loss scaler -- as gfx950
HIP kernels behind a C ABI (include/dsx.h, libdsx.so), with the reference's
`initialize() / engine.backward() / engine.step()` API and ds_config keys.

    engine, optimizer, _, scheduler = distributedspeed_amd.initialize(model, ds_config)
    loss = engine(batch); engine.backward(loss); engine.step()
"""
from __future__ import annotations

import logging
import os
from typing import Any, Optional, Tuple, Union

__version__ = "0.1.0"

logger = logging.getLogger("DistributedSpeed")

_GLOBAL = {"config": None, "initialized": False}


def initialize(model, config: Union[dict, str, Any], optimizer=None, lr_scheduler=None, training_data=None,
               mpu=None, collate_fn=None, dist_init_required: bool = True, model_parameters=None
               ) -> Tuple[Any, Any, Any, Any]:
    """Build the engine; returns (engine, optimizer, dataloader, lr_scheduler)
    like the reference's initialize (Src/__init__.py:209-300).

    One process drives one GPU. A WORLD_SIZE above 1 is refused: the
    multi-rank sharding around this step (reduce-scatter of grads, the scalar
    norm / overflow all-reduces, all-gather of params) is not built here."""
    import torch

    from .config import load_config
    from .engine import DistributedSpeedEngine

    cfg = load_config(config)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if world > 1:
        raise NotImplementedError(f"WORLD_SIZE={world}: this build runs the ZeRO step of one rank on one GPU")
    if mpu is not None:
        raise NotImplementedError("model-parallel units are not supported")
    if not torch.cuda.is_available():
        raise RuntimeError("distributedspeed_amd needs a ROCm GPU (the optimizer step has no CPU path)")
    local_rank = int(os.environ.get("LOCAL_RANK", "0"))
    torch.cuda.set_device(local_rank)
    engine = DistributedSpeedEngine(model, cfg, optimizer=optimizer, lr_scheduler=lr_scheduler,
                                    model_parameters=model_parameters, device=torch.device("cuda", local_rank))
    dataloader = None
    if training_data is not None:
        bs = cfg.train_micro_batch_size_per_gpu or max(1, cfg.train_batch_size // cfg.gradient_accumulation_steps)
        dataloader = torch.utils.data.DataLoader(training_data, batch_size=bs, shuffle=True, collate_fn=collate_fn)
    _GLOBAL.update(config=cfg, initialized=True)
    return engine, engine.optimizer, dataloader, lr_scheduler


def is_initialized() -> bool:
    return bool(_GLOBAL["initialized"])


def get_config():
    return _GLOBAL["config"]


def get_rank() -> int:
    return 0


def get_world_size() -> int:
    return 1


def get_local_rank() -> int:
    return int(os.environ.get("LOCAL_RANK", "0"))


def destroy() -> None:
    _GLOBAL.update(config=None, initialized=False)


def __getattr__(name: str):
    # lazy exports so that importing the package does not load torch / libdsx
    if name in ("DistributedSpeedEngine",):
        from .engine import DistributedSpeedEngine
        return DistributedSpeedEngine
    if name in ("ZeROOptimizer",):
        from .zero import ZeROOptimizer
        return ZeROOptimizer
    if name in ("AdamWOptimizer", "MultiTensorAdamWOptimizer"):
        from . import optimizers as _o
        return getattr(_o, name)
    if name in ("DistributedSpeedConfig", "load_config", "fp16_config", "bf16_config", "zero_config"):
        from . import config as _c
        return getattr(_c, name)
    raise AttributeError(name)


__all__ = ["initialize", "is_initialized", "get_config", "get_rank", "get_world_size", "get_local_rank", "destroy",
           "DistributedSpeedEngine", "ZeROOptimizer", "AdamWOptimizer", "MultiTensorAdamWOptimizer", "DistributedSpeedConfig", "load_config",
           "fp16_config", "bf16_config", "zero_config"]
