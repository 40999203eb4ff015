"""The action chunk of the synthetic GWP-0.5 MoT at full depth and width
(30 layers x 10 flow-matching steps, d = 3072, 24 x 128 heads, FFN 14336 in
both experts, 512 prompt tokens, 8 x 32 visual tokens) on the HIP backend
against the oracle's chunk for the same weights and inputs, committed as a
fixture (tests/golden/gwp_full_depth.json, written by
tests/golden/make_full_depth.py).

The weights are drawn on the host with the oracle's fill (every named weight
of the model) and uploaded through wamx_backend_tensor_set, so both sides see
the same bits.  Bar (the full-step bound): the reference's action gates of
its BF16 latency profile (apps/wam-bench.cpp:172-176: mean |delta| <= 1e-3,
max |delta| <= 1e-2), which the no-op bf16(noise) must fail, and every
step's velocity (the action decoder's output, the fixture's "velocity")
within the velocity bar: cosine >= 0.9999 as per op, max-rel <= 3e-2 (the
per-op 1e-2 widened for a whole step's composition).
"""
from __future__ import annotations

import ctypes as C
import json
import sys
from pathlib import Path

import numpy as np
import pytest

from test_gpu_gwp import action_gate, check_velocities

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))


def test_full_depth_action_chunk_matches_oracle(wx, be, orc):
    import make_full_depth
    doc = json.loads((GOLDEN / "gwp_full_depth.json").read_text())
    cfg = doc["config"]
    assert cfg == make_full_depth.CONFIG
    lib = be.lib
    print("gwp full depth: create", flush=True)
    c = wx.GwpConfig(**cfg)
    m = lib.wamx_gwp_create(be.ptr, C.byref(c))
    assert m, wx.last_error()
    try:
        specs = dict(orc.gwp_weight_specs(cfg))
        names = [lib.wamx_gwp_weight_name(m, i).decode() for i in range(lib.wamx_gwp_n_weights(m))]
        assert sorted(names) == sorted(specs)
        for i, name in enumerate(names):
            t = lib.wamx_gwp_weight(m, name.encode())
            n = lib.wamx_nelements(t)
            assert n == specs[name], name
            a = orc.gwp_synthetic_weight(name, n, doc["weight_seed"], doc["weight_std"])
            wx.check(lib.wamx_backend_tensor_set(t, a.ctypes.data, 0, a.nbytes), f"upload {name}")
            if i % 200 == 0:
                print(f"gwp full depth: uploaded {i + 1}/{len(names)} weights", flush=True)
        state, latent, prompt, noise = make_full_depth.inputs(cfg, doc["input_seed"])
        wx.check(lib.wamx_gwp_set_inputs(m, state.ctypes.data, latent.ctypes.data, prompt.ctypes.data,
                                          noise.ctypes.data), "set_inputs")
        print("gwp full depth: predict", flush=True)
        wx.check(lib.wamx_gwp_predict(m, None), "predict")
        got = np.empty(noise.size, np.float32)
        wx.check(lib.wamx_gwp_get_action(m, got.ctypes.data), "get_action")
        ref = np.asarray(doc["action"], np.float32)
        assert np.all(np.isfinite(got))
        action_gate(got, ref, "full-depth action chunk (30 layers x 10 steps)", noise)
        ref_v = [np.asarray(v, np.float32) for v in doc["velocity"]]
        # the neighbouring step's velocity (another action state and timestep)
        # must fail the bar
        check_velocities(wx, be, m, ref_v, ref_v[1:] + ref_v[:1], "full depth")
    finally:
        lib.wamx_gwp_free(m)
