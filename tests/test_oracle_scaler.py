"""Pins the oracle's loss-scaler state machine (LossScalerSpec).

* hysteresis = 1 with a reachable minimum: identical, step for step, to
  torch._amp_update_scale_ -- the op the GradScaler the reference builds
  (Src/zero/optimizer.py:102-110) runs in update() (optimizer.py:265-266).
* hysteresis > 1 and min_loss_scale (ds_config keys the reference parses,
  Src/config.py:100-101, but never consumes): sequences derived by hand from
  the keys' meaning -- `hysteresis` overflows in a row are tolerated before
  the scale backs off, the scale never drops below min_loss_scale, and a
  growth re-arms the hysteresis.
* the committed golden sequences of configs[1] and configs[3].
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest
import torch
from hypothesis import given, settings
from hypothesis import strategies as st

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _torch_sequence(flags, init, window):
    s = torch.tensor([float(init)])
    gt = torch.zeros(1, dtype=torch.int32)
    out = []
    for f in flags:
        torch._amp_update_scale_(s, gt, torch.tensor([1.0 if f else 0.0]), 2.0, 0.5, window)
        out.append((float(s.item()), int(gt.item())))
    return out


@settings(max_examples=200, deadline=None)
@given(flags=st.lists(st.booleans(), min_size=1, max_size=300), window=st.integers(1, 12),
       power=st.integers(0, 24))
def test_hysteresis1_equals_torch_amp_update_scale(oracle, flags, window, power):
    spec = oracle.LossScalerSpec(scale=2.0 ** power, window=window, hysteresis=1, min_scale=2.0 ** -126)
    ref = _torch_sequence(flags, 2.0 ** power, window)
    for f, (scale, tracker) in zip(flags, ref):
        spec.update(f)
        assert spec.scale == scale
        assert spec.good == tracker


def test_growth_stops_at_fp32_max(oracle):
    spec = oracle.LossScalerSpec(scale=2.0 ** 126, window=1, hysteresis=1)
    ref = _torch_sequence([False] * 4, 2.0 ** 126, 1)
    got = []
    for _ in range(4):
        spec.update(False)
        got.append(spec.scale)
    assert got == [s for s, _ in ref] == [2.0 ** 127] * 4


def test_hysteresis_two_hand_sequence(oracle):
    # window 3, hysteresis 2, min 1, start 16.
    #   step: 1 ovf  -> tolerated (hyst 2 -> 1), scale 16
    #         2 ovf  -> back off to 8, hyst stays 1
    #         3 ok   -> good 1
    #         4 ovf  -> hyst is 1 -> back off to 4; good 0
    #         5,6,7 ok -> good 3 == window -> grow to 8, hyst re-armed to 2
    #         8 ovf  -> tolerated (hyst 2 -> 1), scale 8
    #         9 ok, 10 ovf -> back off to 4 (hyst still 1: no growth since)
    flags = [1, 1, 0, 1, 0, 0, 0, 1, 0, 1]
    expect_scale = [16, 8, 8, 4, 4, 4, 8, 8, 8, 4]
    expect_hyst = [1, 1, 1, 1, 1, 1, 2, 1, 1, 1]
    spec = oracle.LossScalerSpec(scale=16.0, window=3, hysteresis=2, min_scale=1.0)
    for f, s, h in zip(flags, expect_scale, expect_hyst):
        spec.update(bool(f))
        assert (spec.scale, spec.hyst_left) == (s, h)


def test_min_loss_scale_clamps(oracle):
    spec = oracle.LossScalerSpec(scale=8.0, window=1000, hysteresis=1, min_scale=2.0)
    seq = []
    for _ in range(4):
        spec.update(True)
        seq.append(spec.scale)
    assert seq == [4.0, 2.0, 2.0, 2.0]
    # a non-power-of-two minimum is honoured exactly
    spec = oracle.LossScalerSpec(scale=8.0, window=1000, hysteresis=1, min_scale=3.0)
    spec.update(True)
    spec.update(True)
    assert spec.scale == 3.0


def test_static_scale_never_changes(oracle):
    spec = oracle.LossScalerSpec(scale=2.0 ** 16, dynamic=False)
    for f in [True, False] * 10:
        spec.update(f)
    assert spec.scale == 2.0 ** 16


def test_skip_does_not_advance_step_counter(oracle):
    n = 64
    p = np.ones(n, np.float32)
    m = np.zeros(n, np.float32)
    v = np.zeros(n, np.float32)
    orc = oracle.ZeroStepOracle(p, m, v, None, 1, 1, oracle.Hyper(), oracle.LossScalerSpec(scale=4.0, hysteresis=1))
    g = oracle.cast16(np.full(n, 0.5, np.float32), 1)
    bad = g.copy()
    bad[3] = 0x7C00
    r1 = orc.step(g)
    p_after1 = p.copy()
    r2 = orc.step(bad)
    assert (r1.t, r2.t, r2.skipped) == (1, 1, True)
    assert np.array_equal(p, p_after1)
    assert r2.scale_used == 4.0 and r2.scale_next == 2.0


@pytest.mark.parametrize("name", ["scaler_config2_gpt2.json", "scaler_config4_llama_ragged.json",
                                  "scaler_config4_llama_ragged_backoff.json"])
def test_golden_scaler_sequences(oracle, name):
    with open(os.path.join(GOLDEN, name)) as f:
        g = json.load(f)
    spec = oracle.LossScalerSpec(scale=g["init_scale"], window=g["window"], hysteresis=g["hysteresis"],
                                 min_scale=g["min_scale"])
    skipped = [False] * len(g["overflow"])
    for i, f in enumerate(g["overflow"]):
        skipped[i] = bool(f)
        spec.update(bool(f))
        assert spec.scale == g["scale_after"][i], f"step {i + 1}"
    t = sum(1 for s in skipped if not s)
    assert t == g["final_t"]
