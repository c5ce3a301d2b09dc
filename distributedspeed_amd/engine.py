"""DistributedSpeedEngine: the training loop's entry points.

The reference's user loop is `loss = engine(batch); engine.backward(loss);
engine.step()` (README.md:96-106). Its engine (Src/engine.py:665-785) never
builds or steps an optimizer for ZeRO stages 0-2 (step :714-732 only calls a
`self.optimizer` nothing sets), has no backward and no __call__, and
`initialize` looks it up under a name that does not exist
(Src/__init__.py:90, 270-275). This engine supplies those semantics over the
fused step:

  __call__ / forward   the wrapped module (floating-point inputs are cast to
                       the 16-bit parameter dtype under fp16/bf16)
  backward(loss)       ZeROOptimizer.backward: / accumulation, * loss scale
  step()               ZeROOptimizer.step (accumulation gate, fused step),
                       then the LR scheduler (not on a step skipped for
                       overflow) and zero_grad, as DeepSpeed's engine does
                       after a boundary step
  save_checkpoint / load_checkpoint   flat state keyed by parameter name
  module.load_state_dict  after initialize: the fp32 master is taken from
                       the loaded params (a post-load hook on the module)
"""
from __future__ import annotations

import json
import os
import weakref
from typing import Any, Optional

import torch

from .config import DistributedSpeedConfig
from .flat_step import ScalerConfig
from .optimizers import AdamWOptimizer, MultiTensorAdamWOptimizer, _FusedAdamWBase, adopt_torch_optimizer
from .zero import ZeROOptimizer


def _cast_inputs(obj, dtype):
    if isinstance(obj, torch.Tensor):
        return obj.to(dtype) if obj.is_floating_point() else obj
    if isinstance(obj, (list, tuple)):
        return type(obj)(_cast_inputs(o, dtype) for o in obj)
    if isinstance(obj, dict):
        return {k: _cast_inputs(v, dtype) for k, v in obj.items()}
    return obj


class DistributedSpeedEngine(torch.nn.Module):
    def __init__(self, model: torch.nn.Module, config: DistributedSpeedConfig,
                 optimizer: Optional[torch.optim.Optimizer] = None, lr_scheduler=None,
                 model_parameters=None, device: Optional[torch.device] = None):
        super().__init__()
        self.config = config
        self.device = device or torch.device("cuda", torch.cuda.current_device())
        self.module = model.to(self.device)
        prec = config.precision
        self.param_dtype = {"fp16": torch.float16, "bf16": torch.bfloat16}.get(prec)
        scaler = ScalerConfig(**config.loss_scaler())
        names = {id(p): n for n, p in self.module.named_parameters()}
        common = dict(max_grad_norm=float(config.max_grad_norm or 0), param_dtype=self.param_dtype,
                      loss_scaler=scaler, device=self.device, param_names=names,
                      offload=bool(config.zero_optimization.cpu_offload),
                      graph=bool(config.get("hip_graph", False)))
        contiguous = bool(config.zero_optimization.contiguous_gradients)
        if optimizer is not None:
            if not isinstance(optimizer, _FusedAdamWBase):
                optimizer = adopt_torch_optimizer(optimizer, contiguous=contiguous, **common)
        else:
            if config.optimizer.type.lower() not in ("adamw", "adam"):
                raise NotImplementedError(f"optimizer.type {config.optimizer.type!r}: the fused step is AdamW")
            params = list(model_parameters) if model_parameters is not None else list(self.module.parameters())
            if params and isinstance(params[0], dict):
                groups = [dict(g, params=[p for p in g["params"] if p.requires_grad]) for g in params]
            else:
                groups = [p for p in params if p.requires_grad]
            hp = config.adamw_params()
            cls = AdamWOptimizer if contiguous else MultiTensorAdamWOptimizer
            optimizer = cls(groups, lr=hp["lr"], betas=hp["betas"], eps=hp["eps"], weight_decay=hp["weight_decay"],
                            **common)
        zcfg = {"stage": config.zero_optimization.stage,
                "gradient_accumulation_steps": config.gradient_accumulation_steps}
        self.optimizer = ZeROOptimizer(optimizer, zcfg, list(optimizer.dsx_params))
        if self.param_dtype is not None:
            # The stepped parameters now live in the 16-bit buffer and forward
            # takes 16-bit inputs; the parameters the optimizer does not step
            # (frozen ones) take the same dtype, so the module runs in one.
            stepped = {id(p) for p in optimizer.dsx_params}
            with torch.no_grad():
                for p in self.module.parameters():
                    if id(p) not in stepped and p.is_floating_point() and p.dtype != self.param_dtype:
                        p.data = p.data.to(self.param_dtype)
        # With 16-bit params the step reads and writes the fp32 master; a state
        # dict loaded into the module later writes only the params, so the
        # master follows them (the reference steps the params themselves).
        opt_ref = weakref.ref(optimizer)

        def _master_follows_params(module, incompatible_keys):
            opt = opt_ref()
            if opt is not None:
                opt.refresh_master()

        self.module.register_load_state_dict_post_hook(_master_follows_params)
        self.lr_scheduler = lr_scheduler
        # DeepSpeed's engine leaves the LR scheduler alone on a step skipped for
        # overflow. Under dynamic loss scaling the engine therefore needs the
        # skip flag on the host; it is mirrored right after K0, so reading it
        # waits for the norm pass only, not for the AdamW pass.
        self._skip_aware = lr_scheduler is not None and optimizer.scaler.mode == "dynamic"
        if self._skip_aware:
            optimizer.track_skips(True)
        self.global_steps = 0
        self.micro_steps = 0

    # ---- training loop -------------------------------------------------------------------

    def forward(self, *args, **kwargs):
        if self.param_dtype is not None:
            args = _cast_inputs(args, self.param_dtype)
            kwargs = _cast_inputs(kwargs, self.param_dtype)
        return self.module(*args, **kwargs)

    def backward(self, loss: torch.Tensor, retain_graph: bool = False) -> None:
        self.optimizer.backward(loss, retain_graph=retain_graph)

    def is_gradient_accumulation_boundary(self) -> bool:
        return (self.optimizer.gradient_accumulation_count + 1) % self.optimizer.gradient_accumulation_steps == 0

    def step(self) -> None:
        self.micro_steps += 1
        boundary = self.is_gradient_accumulation_boundary()
        self.optimizer.step()
        if boundary:
            self.global_steps += 1
            if self.lr_scheduler is not None:
                if not (self._skip_aware and self.optimizer.base_optimizer.last_step_skipped()):
                    self.lr_scheduler.step()
            self.optimizer.base_optimizer.zero_grad()

    def zero_grad(self) -> None:
        self.optimizer.zero_grad()

    # ---- observability (each reads the device: one sync) ------------------------------------

    @property
    def loss_scale(self) -> float:
        return self.optimizer.loss_scale

    @property
    def skipped_steps(self) -> int:
        return self.optimizer.overflow_count

    def get_global_grad_norm(self) -> float:
        return float(self.optimizer.base_optimizer.grad_norm_tensor().item())

    def get_lr(self):
        return [g["lr"] for g in self.optimizer.param_groups]

    # ---- checkpoints ---------------------------------------------------------------------------

    def save_checkpoint(self, save_dir: str, tag: Optional[str] = None, client_state: Optional[dict] = None) -> str:
        """<save_dir>/<tag>/{model_states.pt, optim_states.pt, layout.json}; the
        optimizer state is keyed by parameter name and flat offset."""
        tag = tag or f"global_step{self.global_steps}"
        path = os.path.join(save_dir, tag)
        os.makedirs(path, exist_ok=True)
        opt = self.optimizer.base_optimizer
        torch.save({"module": {k: v.detach().cpu() for k, v in self.module.state_dict().items()},
                    "global_steps": self.global_steps, "micro_steps": self.micro_steps,
                    "client_state": client_state or {}}, os.path.join(path, "model_states.pt"))
        torch.save(self.optimizer.state_dict(), os.path.join(path, "optim_states.pt"))
        with open(os.path.join(path, "layout.json"), "w") as f:
            json.dump({"numel": opt.numel, "precision": self.config.precision, "params": opt.layout()}, f)
        with open(os.path.join(save_dir, "latest"), "w") as f:
            f.write(tag)
        return path

    def load_checkpoint(self, load_dir: str, tag: Optional[str] = None) -> tuple[str, dict]:
        if tag is None:
            with open(os.path.join(load_dir, "latest")) as f:
                tag = f.read().strip()
        path = os.path.join(load_dir, tag)
        with open(os.path.join(path, "layout.json")) as f:
            layout = json.load(f)
        mine = self.optimizer.base_optimizer.layout()
        # Names, shapes and group indices (not offsets: a checkpoint moves
        # between storage forms) are checked before anything is loaded, so
        # that a refused checkpoint leaves the engine as it was.
        def key(p, shape=True):
            return (p["name"], int(p["numel"]), tuple(p["shape"]) if shape else None, int(p.get("group", 0)))

        shaped = all("shape" in p for p in layout["params"])  # every layout this library writes has shapes
        if [key(p, shaped) for p in layout["params"]] != [key(p, shaped) for p in mine]:
            raise ValueError("checkpoint parameter layout does not match this model")
        ms = torch.load(os.path.join(path, "model_states.pt"), weights_only=True)
        osd = torch.load(os.path.join(path, "optim_states.pt"), weights_only=True)
        with torch.no_grad():
            self.module.load_state_dict(ms["module"], strict=False)  # buffers; params follow from the master
        self.optimizer.load_state_dict(osd)
        self.global_steps = int(ms["global_steps"])
        self.micro_steps = int(ms["micro_steps"])
        return path, ms.get("client_state", {})
