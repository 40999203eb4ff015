"""Writes tests/golden/gwp_full_depth.json: the oracle's action chunk, and the
velocity (action decoder output) of every denoise step, for the
synthetic GWP-0.5 MoT at full depth and width (30 layers, d = 3072, 24 x 128
heads, FFN 14336 in both experts, 48 x 32 actions, 10 flow-matching steps,
512 prompt tokens of width 4096, 8 x 32 visual tokens from a 48-channel
latent), on weights and inputs drawn by oracle.fill_normal with the seeds
stored in the file.

tests/test_gpu_full_depth.py regenerates the same weights and inputs on the
host, uploads them to the HIP model and compares its chunk with this one.

    python tests/golden/make_full_depth.py      # ~5 minutes on 8 cores, ~21 GB of RAM
"""
from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "oracle"))
import oracle  # noqa: E402

CONFIG = dict(n_layers=30, hidden=3072, n_heads=24, head_dim=128, ffn_dim=14336, action_hidden=3072,
              action_ffn_dim=14336, action_chunk=48, action_dim=32, grid_h=8, grid_w=32, n_lang=512, t5_hidden=4096,
              z_dim=48, num_steps=10, enc_hidden=128, shift=5.0, eps=1e-6)
WEIGHT_SEED = 0x5EED0D00
WEIGHT_STD = 0.02
INPUT_SEED = 0x5EED0D10


def inputs(cfg, seed):
    """state [action_dim], latent [z][2gh][2gw], prompt [n_lang][t5], noise [chunk][action_dim]."""
    c = cfg
    return (oracle.fill_normal(c["action_dim"], seed + 1),
            oracle.fill_normal(c["z_dim"] * 4 * c["grid_h"] * c["grid_w"], seed + 2),
            oracle.fill_normal(c["n_lang"] * c["t5_hidden"], seed + 3),
            oracle.fill_normal(c["action_chunk"] * c["action_dim"], seed + 4))


def main(out: Path = HERE / "gwp_full_depth.json") -> None:
    oracle.load()
    t0 = time.time()
    w = oracle.gwp_synthetic_weights(CONFIG, WEIGHT_SEED, WEIGHT_STD)
    t1 = time.time()
    state, latent, prompt, noise = inputs(CONFIG, INPUT_SEED)
    g = oracle.Gwp(CONFIG, w)
    g.prompt(prompt)
    g.prefix(state, latent, prompt)
    action = g.denoise(noise)
    t2 = time.time()
    doc = {
        "what": "oracle action chunk (bf16 state widened to f32) of the synthetic GWP-0.5 MoT at full depth",
        "config": CONFIG, "weight_seed": WEIGHT_SEED, "weight_std": WEIGHT_STD, "input_seed": INPUT_SEED,
        "weights": "oracle.gwp_synthetic_weights(config, weight_seed, weight_std)",
        "inputs": "make_full_depth.inputs(config, input_seed)",
        "action": [float(v) for v in action.ravel()],
        "velocity": [[float(v) for v in g.velocity(s)] for s in range(CONFIG["num_steps"])],
        "noise_bf16_rel_change": float(np.linalg.norm(action - noise) / np.linalg.norm(noise)),
        "oracle_threads": oracle.num_threads(), "weights_s": round(t1 - t0, 1), "oracle_s": round(t2 - t1, 1),
    }
    out.write_text(json.dumps(doc, indent=1) + "\n")
    print(f"wrote {out}: weights {t1 - t0:.0f} s, oracle {t2 - t1:.0f} s, |action| {np.linalg.norm(action):.3f}")


if __name__ == "__main__":
    main()
