"""Writes tests/golden/*.json: known-answer vectors computed independently of
the C oracle (plain Python / numpy float64 from the published formulas), used
to pin it.

  flow_schedule.json      flow-match Euler schedule for (steps, shift) pairs
                          (src/models/common/scheduler.cpp:26-55 restated)
  timestep_embedding.json 256-d sinusoidal embedding, cos first
                          (src/models/gwp05/engine/text_encoder.cpp:1-12)
  gelu.json               GELU tanh / erf at fixed points
  rope.json               NORMAL RoPE of a small tensor via complex rotation
  normal_sample.json      first values of the seeded splitmix64 / Box-Muller
                          sample, from exact integer arithmetic in Python

Run: python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

OUT = Path(__file__).resolve().parent


def f32(x):
    return float(np.float32(x))


def flow_schedule(steps: int, shift: float):
    s = np.float32(shift)
    train = np.float32(1.0) / np.float32(1000.0)
    shifted_min = s * train / (np.float32(1.0) + (s - np.float32(1.0)) * train)
    t_min = float(shifted_min) * 1000.0
    sig, ts = [], []
    for i in range(steps):
        t = 1000.0 if steps == 1 else 1000.0 + (t_min - 1000.0) * i / (steps - 1)
        g = t / 1000.0
        v = float(s) * g / (1.0 + (float(s) - 1.0) * g)
        sig.append(f32(v))
        ts.append(f32(np.float32(v) * np.float32(1000.0)))
    sig.append(0.0)
    return ts, sig


def timestep_embedding(t: float, dim: int):
    half = dim // 2
    out = [0.0] * dim
    for i in range(half):
        freq = math.exp(-math.log(10000.0) * i / half)
        out[i] = math.cos(t * freq)
        out[i + half] = math.sin(t * freq)
    return out


def gelu_tanh(x):
    return 0.5 * x * (1.0 + math.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def gelu_erf(x):
    return 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))


def rope(x: np.ndarray, pos: np.ndarray, n_dims: int, base: float):
    """x [tokens][heads][head_dim]: pair (2i, 2i+1) as the complex number
    x[2i] + j x[2i+1] multiplied by exp(j pos base^(-2i/n_dims))."""
    y = x.astype(np.float64).copy()
    T, H, D = x.shape
    for t in range(T):
        for i in range(n_dims // 2):
            theta = pos[t] * base ** (-2.0 * i / n_dims)
            z = (x[t, :, 2 * i] + 1j * x[t, :, 2 * i + 1]) * np.exp(1j * theta)
            y[t, :, 2 * i] = z.real
            y[t, :, 2 * i + 1] = z.imag
    return y


M64 = (1 << 64) - 1


def splitmix64(z: int) -> int:
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def normal_sample(n: int, seed: int, mean: float, std: float):
    out = []
    for i in range(n):
        z = splitmix64((seed + (i + 1) * 0x9E3779B97F4A7C15) & M64)
        u1 = ((z >> 40) + 0.5) / 16777216.0
        u2 = (((z >> 16) & 0xFFFFFF) + 0.5) / 16777216.0
        out.append(mean + std * math.sqrt(-2.0 * math.log(u1)) * math.cos(2.0 * math.pi * u2))
    return out


def main():
    sched = {f"{n}_{s}": dict(zip(("timesteps", "sigmas"), flow_schedule(n, s)))
             for n, s in [(10, 5.0), (1, 5.0), (4, 1.0), (20, 3.0)]}
    (OUT / "flow_schedule.json").write_text(json.dumps(sched, indent=1))

    emb = {str(t): timestep_embedding(t, 256) for t in (0.0, 1.0, 999.0, 500.5)}
    (OUT / "timestep_embedding.json").write_text(json.dumps(emb))

    xs = [-8.0, -3.0, -1.0, -0.5, -1e-3, 0.0, 1e-3, 0.5, 1.0, 2.0, 3.0, 8.0]
    (OUT / "gelu.json").write_text(json.dumps({"x": xs, "tanh": [gelu_tanh(x) for x in xs],
                                               "erf": [gelu_erf(x) for x in xs]}))

    rng = np.random.default_rng(1234)
    x = rng.standard_normal((3, 2, 16)).astype(np.float32)
    pos = np.array([0, 1, 47], np.int32)
    (OUT / "rope.json").write_text(json.dumps({
        "x": x.tolist(), "pos": pos.tolist(), "n_dims": 12, "base": 10000.0,
        "y": rope(x, pos, 12, 10000.0).tolist()}))

    (OUT / "normal_sample.json").write_text(json.dumps({
        "seed": 0x5EED0001, "mean": 0.0, "std": 1.0, "values": normal_sample(16, 0x5EED0001, 0.0, 1.0)}))


if __name__ == "__main__":
    main()
