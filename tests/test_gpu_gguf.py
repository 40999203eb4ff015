"""A GWP-0.5 model loaded from a GGUF artifact (wamx_gwp_create_from_gguf).

The artifact is written in the reference's layout (tests/gguf_io.py
gwp_artifact): compact tensor names, one adaLN table per layer and expert,
the state / action encoder in_proj and decoder out_proj as
[num_embodiments][in][out] with embodiment 1 selected and the other slices
random, self-attention q / k / v packed (mot-vae-bf16-qkv-v1) or split
(mot-vae-bf16-v1), plus T5 / VAE / statistic / unused tensors the loader must
skip.  The loaded model must hold exactly the weights of a model given the
same weights by name, produce the same action chunk bit for bit, and match
the oracle.  Artifacts the reference refuses (artifact.cpp:57-95, 232-268;
semantics.cpp:35-56), or this backend cannot run (an F32 MoT policy), are
refused with a message.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import gguf_io as gi
from test_gpu_gwp import action_gate, inputs, run_gpu

pytestmark = pytest.mark.gpu

CFG = dict(n_layers=2, hidden=256, n_heads=2, head_dim=128, ffn_dim=512, action_hidden=256, action_ffn_dim=384,
           action_chunk=48, action_dim=32, grid_h=4, grid_w=8, n_lang=16, t5_hidden=64, z_dim=16, num_steps=3,
           enc_hidden=128, shift=5.0, eps=1e-6)
SEED = 0x5EED0A00


def by_name_model(wx, be, weights):
    lib = be.lib
    m = lib.wamx_gwp_create(be.ptr, C.byref(wx.GwpConfig(**CFG)))
    assert m, wx.last_error()
    shapes = {}
    for name, a in weights.items():
        t = lib.wamx_gwp_weight(m, name.encode())
        assert t, name
        shapes[name] = list(t.contents.ne)
        wx.check(lib.wamx_backend_tensor_set(t, a.ctypes.data, 0, a.nbytes), f"upload {name}")
    return m, shapes


def load(wx, be, path, expect_ok=True):
    lib = be.lib
    g = lib.wamx_gguf_open(str(path).encode())
    assert g, wx.last_error()
    try:
        m = lib.wamx_gwp_create_from_gguf(be.ptr, g, CFG["n_lang"], 1)
        if expect_ok:
            assert m, wx.last_error()
        return m, wx.last_error()
    finally:
        lib.wamx_gguf_close(g)


@pytest.mark.parametrize("packed", [True, False])
def test_artifact_model_matches_direct_upload_and_oracle(wx, be, orc, tmp_path, packed):
    print(f"gguf artifact model packed_qkv={packed}", flush=True)
    lib = be.lib
    weights = orc.gwp_synthetic_weights(CFG, SEED, 0.02)
    ref, shapes = by_name_model(wx, be, weights)
    path = gi.gwp_artifact(CFG, weights, shapes, packed_qkv=packed).write(tmp_path / "gwp.gguf")
    m, _ = load(wx, be, path)
    try:
        # every weight as the model holds it
        for name, a in weights.items():
            t = lib.wamx_gwp_weight(m, name.encode())
            got = np.empty_like(a)
            wx.check(lib.wamx_backend_tensor_get(t, got.ctypes.data, 0, got.nbytes), name)
            assert np.array_equal(got, a), name
        ins = inputs(CFG)
        got = run_gpu(wx, be, m, ins)
        want = run_gpu(wx, be, ref, ins)
        assert np.array_equal(got, want)
        g = orc.Gwp(CFG, weights)
        g.prompt(ins[2])
        g.prefix(ins[0], ins[1], ins[2])
        action_gate(got, g.denoise(ins[3]).ravel(), "artifact model vs oracle", ins[3])
    finally:
        lib.wamx_gwp_free(m)
        lib.wamx_gwp_free(ref)


REFUSALS = {
    "source_f32_policy": (dict(policy="source-f32-v1"), "conversion policy"),
    "no_policy": (dict(policy=""), "conversion policy"),
    "two_views": (dict(num_views=2), "three camera views"),
    "image_not_multiple_of_32": (dict(image_height=100), "divisible by 32"),
    "embodiment_out_of_range": (dict(embodiment_id=5), "embodiment id"),
    "head_dim_64": (dict(head_dim=64, n_heads=4), "head_dim"),
    "hidden_mismatch": (dict(hidden=300), "heads x head_dim"),
    "zero_steps": (dict(inference_steps=0), "zero dimension"),
    "bad_shift": (dict(flow_shift=-1.0), "finite and positive"),
}


@pytest.mark.parametrize("case", sorted(REFUSALS))
def test_artifact_metadata_refused(wx, be, tmp_path, case):
    over, why = REFUSALS[case]
    over = dict(over)
    policy = over.pop("policy", "mot-vae-bf16-qkv-v1")
    emb = over.pop("embodiment_id", 1)
    w = gi.GgufWriter()
    gi.geometry_keys(w, CFG, policy, 3, emb, **over)
    m, err = load(wx, be, w.write(tmp_path / f"{case}.gguf"), expect_ok=False)
    assert not m
    assert why in err, (case, err)


@pytest.mark.parametrize("case", ["missing_tensor", "wrong_shape", "f32_tensor"])
def test_artifact_weights_refused(wx, be, orc, tmp_path, case):
    print(f"gguf artifact refused: {case}", flush=True)
    weights = orc.gwp_synthetic_weights(CFG, SEED, 0.02)
    ref, shapes = by_name_model(wx, be, weights)
    be.lib.wamx_gwp_free(ref)
    w = gi.gwp_artifact(CFG, weights, shapes, packed_qkv=True)
    target = "gwp.blk.1.a.ffn.out.weight"
    i = [t[0] for t in w.tensors].index(target)
    name, gtype, ne, payload = w.tensors[i]
    if case == "missing_tensor":
        del w.tensors[i]
    elif case == "wrong_shape":
        w.tensors[i] = (name, gtype, (ne[1], ne[0]), payload)
    else:
        f32 = np.frombuffer(payload, np.uint16).astype(np.uint32) << 16
        w.tensors[i] = (name, gi.GGML_F32, ne, f32.view(np.float32).tobytes())
    m, err = load(wx, be, w.write(tmp_path / f"{case}.gguf"), expect_ok=False)
    assert not m
    assert target in err, (case, err)
