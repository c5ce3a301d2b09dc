"""Writes the committed golden fixtures of this directory.

    python tests/golden/make_golden.py

The reference ships no golden vectors for its optimizer step (it has no
tests); its arithmetic is torch's. These fixtures are therefore produced by
the library routines the reference calls, run on the CPU:

  adamw_torch_cpu.npz
      torch.optim.AdamW(foreach=False) -- the call at Src/zero/stage1.py:525 /
      Src/zero/stage2.py:612 -- over 1024 elements for 5 steps, for four
      hyper-parameter sets (configs[0], configs[2], and two that reach the
      other lerp branch and weight_decay = 0 / beta = 0), from zero state.
      Grads are exactly representable in bf16. Records torch's CPU capability:
      exp_avg / exp_avg_sq are bit-reproducible on AVX2/AVX512 hosts.

  scaler_config2_gpt2.json
      configs[1]'s loss-scale sequence: init 2^16, window 1000, hysteresis 1,
      min 1, 20 steps, overflow at step 3. Produced by torch._amp_update_scale_
      (GradScaler.update, Src/zero/optimizer.py:265-266), which is the whole
      scaler when hysteresis is 1.

  scaler_config4_llama_ragged.json
      configs[3]'s sequence: init 2^16, window 1000, hysteresis 2, min 1, 2000
      steps, Bernoulli(1e-3) overflows from numpy's default_rng(1004). The scale
      arithmetic and the growth window are torch._amp_update_scale_'s; the
      hysteresis decision on top of it follows the ds_config key's meaning:
      an overflow while more than one is still tolerated resets the growth
      tracker without backing off (the op with backoff factor 1.0).

  scaler_config4_llama_ragged_backoff.json
      the same configuration from default_rng(1022), a seed whose sequence
      reaches every branch: tolerated overflow, growth re-arming the
      hysteresis, and back-offs.
"""
from __future__ import annotations

import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))

HYPERS = [
    dict(lr=1e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01),
    dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1),
    dict(lr=1e-2, beta1=0.3, beta2=0.5, eps=1e-6, weight_decay=0.0),
    dict(lr=1.5e-4, beta1=0.0, beta2=0.0, eps=1e-3, weight_decay=0.5),
]


def bf16_exact(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(x).to(torch.bfloat16).float().numpy()


def adamw_fixture(n: int = 1024, steps: int = 5, device: str = "cpu", foreach=False) -> dict:
    """torch.optim.AdamW on `device` (foreach=None: torch's default dispatch)."""
    out = {"capability": np.array(torch.backends.cpu.get_cpu_capability()),
           "torch_version": np.array(torch.__version__)}
    if device != "cpu":
        out["device"] = np.array(torch.cuda.get_device_name(0))
        out["foreach"] = np.array(str(foreach))
    for k, h in enumerate(HYPERS):
        rng = np.random.default_rng(500 + k)
        p0 = (rng.standard_normal(n) * 0.02).astype(np.float32)
        p0[:4] = [0.0, -0.0, 1e-30, -3.0]
        grads = np.stack([bf16_exact((rng.standard_normal(n) * 1e-3).astype(np.float32)) for _ in range(steps)])
        grads[:, 4:8] = bf16_exact(np.array([0.0, -0.0, 1e-20, 65504.0], np.float32))
        param = torch.nn.Parameter(torch.from_numpy(p0.copy()).to(device))
        opt = torch.optim.AdamW([param], lr=h["lr"], betas=(h["beta1"], h["beta2"]), eps=h["eps"],
                                weight_decay=h["weight_decay"], foreach=foreach)
        ps, ms, vs = [], [], []
        for t in range(steps):
            param.grad = torch.from_numpy(grads[t].copy()).to(device)
            opt.step()
            st = opt.state[param]
            ps.append(param.detach().cpu().numpy().copy())
            ms.append(st["exp_avg"].cpu().numpy().copy())
            vs.append(st["exp_avg_sq"].cpu().numpy().copy())
        out[f"h{k}_hyper"] = np.array([h["lr"], h["beta1"], h["beta2"], h["eps"], h["weight_decay"]])
        out[f"h{k}_p0"] = p0
        out[f"h{k}_grads"] = grads
        out[f"h{k}_p"] = np.stack(ps)
        out[f"h{k}_m"] = np.stack(ms)
        out[f"h{k}_v"] = np.stack(vs)
    return out


def scaler_sequence(flags, init, window, hysteresis, min_scale):
    s = torch.tensor([float(init)])
    tracker = torch.zeros(1, dtype=torch.int32)
    hyst_left = hysteresis
    scales = []
    for f in flags:
        if f and hysteresis > 1 and hyst_left > 1:
            hyst_left -= 1
            torch._amp_update_scale_(s, tracker, torch.tensor([1.0]), 2.0, 1.0, window)  # reset only
        else:
            before = float(s.item())
            torch._amp_update_scale_(s, tracker, torch.tensor([1.0 if f else 0.0]), 2.0, 0.5, window)
            if f and float(s.item()) < min_scale:
                s.fill_(min_scale)
            if not f and float(s.item()) != before:  # grew: hysteresis re-armed
                hyst_left = hysteresis
            if not f and int(tracker.item()) == 0 and float(s.item()) == before:
                hyst_left = hysteresis  # window reached but growth was not finite
        scales.append(float(s.item()))
    return scales


def main() -> None:
    np.savez_compressed(os.path.join(HERE, "adamw_torch_cpu.npz"), **adamw_fixture())

    flags2 = [s == 3 for s in range(1, 21)]
    seq2 = scaler_sequence(flags2, 2.0 ** 16, 1000, 1, 1.0)
    with open(os.path.join(HERE, "scaler_config2_gpt2.json"), "w") as f:
        json.dump({"init_scale": 2.0 ** 16, "window": 1000, "hysteresis": 1, "min_scale": 1.0,
                   "overflow": [int(x) for x in flags2], "scale_after": seq2,
                   "final_t": sum(1 for x in flags2 if not x)}, f)

    rng = np.random.default_rng(1004)
    flags4 = (rng.random(2000) < 1e-3).tolist()
    seq4 = scaler_sequence(flags4, 2.0 ** 16, 1000, 2, 1.0)
    with open(os.path.join(HERE, "scaler_config4_llama_ragged.json"), "w") as f:
        json.dump({"init_scale": 2.0 ** 16, "window": 1000, "hysteresis": 2, "min_scale": 1.0,
                   "rng": "numpy default_rng(1004).random(2000) < 1e-3",
                   "overflow": [int(x) for x in flags4], "scale_after": seq4,
                   "final_t": sum(1 for x in flags4 if not x)}, f)
    print("overflows in config4 sequence:", sum(flags4), "final scale", seq4[-1])

    # a second seed for the same configuration, chosen so that the sequence
    # holds every hysteresis-2 branch: a tolerated overflow (step 1), a growth
    # that re-arms the hysteresis (1001), another tolerated overflow (1010),
    # then two back-offs (1300, 1919)
    rng = np.random.default_rng(1022)
    flags4b = (rng.random(2000) < 1e-3).tolist()
    seq4b = scaler_sequence(flags4b, 2.0 ** 16, 1000, 2, 1.0)
    with open(os.path.join(HERE, "scaler_config4_llama_ragged_backoff.json"), "w") as f:
        json.dump({"init_scale": 2.0 ** 16, "window": 1000, "hysteresis": 2, "min_scale": 1.0,
                   "rng": "numpy default_rng(1022).random(2000) < 1e-3",
                   "overflow": [int(x) for x in flags4b], "scale_after": seq4b,
                   "final_t": sum(1 for x in flags4b if not x)}, f)
    print("overflows in the second config4 sequence:", sum(flags4b), "final scale", seq4b[-1])


if __name__ == "__main__":
    main()
