"""End-to-end parity of the synthetic GWP-0.5 MoT action step (prompt
projection, prefix pass, unrolled denoise) on the HIP backend against the
oracle's independent CPU restatement, on identical seeded weights and inputs.

Full-step bar: the action chunk is a bf16 state rounded every step, so it is
compared through its relative L2 error and cosine (rel-L2 <= 2e-2, cosine >=
0.9998) plus the wam-compare style mean |delta| gate (<= 2e-2).  Prefix K/V
caches are compared per layer with the per-op bar (max-rel <= 1e-2 scaled to
the tensor, cosine >= 0.9999).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from conftest import assert_parity, cosine

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_heads=2, head_dim=128, ffn_dim=512, action_hidden=256, action_ffn_dim=384,
             action_chunk=48, action_dim=32, grid_h=4, grid_w=8, n_lang=16, t5_hidden=64, z_dim=16, num_steps=3,
             enc_hidden=32, shift=5.0, eps=1e-6)


def make_model(wx, be, cfg, seed=0x5EED0003):
    c = wx.GwpConfig(**cfg)
    m = be.lib.wamx_gwp_create(be.ptr, C.byref(c))
    assert m, wx.last_error()
    wx.check(be.lib.wamx_gwp_init_synthetic(m, seed, 0.02), "init_synthetic")
    return m


def read_weights(wx, be, m):
    lib = be.lib
    out = {}
    for i in range(lib.wamx_gwp_n_weights(m)):
        name = lib.wamx_gwp_weight_name(m, i).decode()
        t = lib.wamx_gwp_weight(m, name.encode())
        n = lib.wamx_nelements(t)
        a = np.empty(n, np.uint16)
        wx.check(lib.wamx_backend_tensor_get(t, a.ctypes.data, 0, n * 2), f"read {name}")
        out[name] = a
    return out


def inputs(cfg, seed=7):
    import oracle
    A, T, Z = cfg["action_dim"], cfg["action_chunk"], cfg["z_dim"]
    state = oracle.fill_normal(A, seed + 1)
    latent = oracle.fill_normal(Z * 4 * cfg["grid_h"] * cfg["grid_w"], seed + 2)
    prompt = oracle.fill_normal(cfg["n_lang"] * cfg["t5_hidden"], seed + 3)
    noise = oracle.fill_normal(T * A, seed + 4)
    return state, latent, prompt, noise


def run_gpu(wx, be, m, ins, timing=None):
    lib = be.lib
    state, latent, prompt, noise = ins
    wx.check(lib.wamx_gwp_set_inputs(m, state.ctypes.data, latent.ctypes.data, prompt.ctypes.data,
                                     noise.ctypes.data), "set_inputs")
    wx.check(lib.wamx_gwp_predict(m, C.byref(timing) if timing is not None else None), "predict")
    out = np.empty(noise.size, np.float32)
    wx.check(lib.wamx_gwp_get_action(m, out.ctypes.data), "get_action")
    return out


def tensor_bytes(wx, be, t, shape):
    """Read a tensor's memory span (a padded view reads fewer bytes than the
    full shape; the tail stays zero)."""
    n = int(np.prod(shape))
    a = np.zeros(n, np.uint16)
    nbytes = min(n * 2, be.lib.wamx_nbytes(t))
    wx.check(be.lib.wamx_backend_tensor_get(t, a.ctypes.data, 0, nbytes))
    return a.reshape(shape)


def action_gate(got, ref, what):
    rel_l2 = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    mean_abs = float(np.mean(np.abs(got - ref)))
    cos = cosine(got, ref)
    print(f"{what}: rel-L2 {rel_l2:.3e} mean|d| {mean_abs:.3e} max|d| {np.max(np.abs(got - ref)):.3e} cos {cos:.6f}")
    assert rel_l2 <= 2e-2 and cos >= 0.9998 and mean_abs <= 2e-2, what


def test_small_model_matches_oracle(wx, be, orc):
    print("gwp small model vs oracle", flush=True)
    m = make_model(wx, be, SMALL)
    try:
        w = read_weights(wx, be, m)
        ins = inputs(SMALL)
        got = run_gpu(wx, be, m, ins)
        ref_model = orc.Gwp(SMALL, w)
        state, latent, prompt, noise = ins
        ref_model.prompt(prompt)
        ref_model.prefix(state, latent, prompt)
        H, dh, P = SMALL["n_heads"], SMALL["head_dim"], 1 + SMALL["grid_h"] * SMALL["grid_w"]
        for layer in range(SMALL["n_layers"]):
            k = tensor_bytes(wx, be, be.lib.wamx_gwp_prefix_key(m, layer), (H, P, dh))
            vt = be.lib.wamx_gwp_prefix_value(m, layer)
            ld = vt.contents.nb[1] // 2
            v = tensor_bytes(wx, be, vt, (H, dh, ld))[:, :, :P]
            assert_parity(wx.bf16_to_f32(k), wx.bf16_to_f32(ref_model.prefix_key(layer)), what=f"prefix K {layer}")
            assert_parity(wx.bf16_to_f32(v), wx.bf16_to_f32(ref_model.prefix_value(layer)), what=f"prefix V {layer}")
        ref = ref_model.denoise(noise)
        action_gate(got, ref, "action chunk")
    finally:
        be.lib.wamx_gwp_free(m)


def test_graph_replay_is_deterministic(wx, be):
    """The second predict replays the captured HIP graphs; eager work and
    synchronisation in between; every replay must equal the first result."""
    print("gwp replay determinism", flush=True)
    m = make_model(wx, be, SMALL, seed=11)
    try:
        ins = inputs(SMALL, seed=3)
        first = run_gpu(wx, be, m, ins)
        for _ in range(3):
            be.sync()
            assert np.array_equal(run_gpu(wx, be, m, ins), first)
        other = run_gpu(wx, be, m, inputs(SMALL, seed=4))
        assert not np.array_equal(other, first)
        assert np.array_equal(run_gpu(wx, be, m, ins), first)
    finally:
        be.lib.wamx_gwp_free(m)


def test_projected_prompt_cache(wx, be):
    """Projected-prompt reuse across requests (cache.cpp:53-67, :131): with a
    nonzero capacity a request whose prompt has the same bytes as the last
    projected one skips the prompt graphs, and its action equals, bit for bit,
    that of a model that projects every prompt; a changed prompt, new weights
    and a zero capacity all project again."""
    print("gwp projected-prompt cache", flush=True)
    lib = be.lib
    ref = make_model(wx, be, SMALL, seed=21)
    m = make_model(wx, be, SMALL, seed=21)

    def stats():
        h, mi = C.c_uint64(), C.c_uint64()
        wx.check(lib.wamx_gwp_prompt_cache_stats(m, C.byref(h), C.byref(mi)), "stats")
        return h.value, mi.value

    try:
        wx.check(lib.wamx_gwp_set_prompt_cache(m, 4), "set_prompt_cache")
        a, b = inputs(SMALL, seed=5), inputs(SMALL, seed=9)
        a_other = (b[0], b[1], a[2], b[3])  # prompt a, everything else from b
        expect = [(0, 1), (1, 1), (1, 2), (2, 2)]
        for req, st in zip((a, a_other, b, b), expect):
            got = run_gpu(wx, be, m, req)
            assert np.array_equal(got, run_gpu(wx, be, ref, req))
            assert stats() == st
        # New weights: the caches no longer hold the prompt's projection.
        for x in (m, ref):
            wx.check(lib.wamx_gwp_init_synthetic(x, 0x77, 0.02), "init_synthetic")
        assert np.array_equal(run_gpu(wx, be, m, b), run_gpu(wx, be, ref, b))
        assert stats() == (2, 3)
        # Capacity 0: every prompt is projected again and nothing is counted.
        wx.check(lib.wamx_gwp_set_prompt_cache(m, 0), "set_prompt_cache")
        assert np.array_equal(run_gpu(wx, be, m, a), run_gpu(wx, be, ref, a))
        assert np.array_equal(run_gpu(wx, be, m, a_other), run_gpu(wx, be, ref, a_other))
        assert stats() == (2, 3)
    finally:
        lib.wamx_gwp_free(m)
        lib.wamx_gwp_free(ref)


def test_full_width_one_layer_matches_oracle(wx, be, orc):
    """Full GWP-0.5 widths (d = 3072, 24 heads, FFN 14336, 48 action tokens,
    512 prompt tokens) on two layers and 2 denoise steps with 256 visual tokens."""
    cfg = dict(n_layers=2, hidden=3072, n_heads=24, head_dim=128, ffn_dim=14336, action_hidden=3072,
               action_ffn_dim=14336, action_chunk=48, action_dim=32, grid_h=8, grid_w=32, n_lang=512,
               t5_hidden=4096, z_dim=48, num_steps=2, enc_hidden=128, shift=5.0, eps=1e-6)
    print("gwp full-width one-layer vs oracle", flush=True)
    m = make_model(wx, be, cfg, seed=0x5EED0004)
    try:
        w = read_weights(wx, be, m)
        ins = inputs(cfg, seed=21)
        got = run_gpu(wx, be, m, ins)
        ref_model = orc.Gwp(cfg, w)
        state, latent, prompt, noise = ins
        ref_model.prompt(prompt)
        ref_model.prefix(state, latent, prompt)
        ref = ref_model.denoise(noise)
        action_gate(got, ref, "full-width action chunk")
    finally:
        be.lib.wamx_gwp_free(m)


def test_baseline_size_runs_and_is_deterministic(wx, be):
    """The 30-layer, 3x1024-visual-token, 512-prompt-token configuration: the
    chunk is finite, deterministic across graph replays, and its prefix cache
    layout is [H][P][dh] / [H][dh][P]."""
    print("gwp full size", flush=True)
    c = be.lib.wamx_gwp_default_config()
    cfg = {k: getattr(c, k) for k, _ in wx.GwpConfig._fields_}
    m = make_model(wx, be, cfg, seed=0x5EED0003)
    try:
        params = be.lib.wamx_gwp_param_count(m)
        assert 9.5e9 < params < 1.1e10, params
        ins = inputs(cfg, seed=5)
        t = wx.GwpTiming()
        a1 = run_gpu(wx, be, m, ins, t)
        a2 = run_gpu(wx, be, m, ins, t)
        print(f"timing prompt {t.prompt_ms:.2f} prefix {t.prefix_ms:.2f} denoise {t.denoise_ms:.2f} "
              f"total {t.total_ms:.2f} ms")
        assert np.all(np.isfinite(a1)) and np.array_equal(a1, a2)
        assert np.std(a1) > 0.1
        k = be.lib.wamx_gwp_prefix_key(m, 29)
        assert tuple(k.contents.ne)[:3] == (128, 3073, 24)
    finally:
        be.lib.wamx_gwp_free(m)


def inputs_batch(cfg, B, seed):
    """Chunk-major inputs of B independent chunks."""
    per = [inputs(cfg, seed + 17 * b) for b in range(B)]
    return tuple(np.concatenate([p[i] for p in per]) for i in range(4)), per


def test_batched_chunks_match_oracle(wx, be, orc):
    """Three independent chunks in one request (each with its own state,
    latent, prompt and noise) against three oracle runs on the same weights."""
    B = 3
    cfg = dict(SMALL, batch=B)
    print(f"gwp batch {B} vs oracle", flush=True)
    m = make_model(wx, be, cfg, seed=0x5EED0008)
    try:
        w = read_weights(wx, be, m)
        ins, per = inputs_batch(SMALL, B, 40)
        got = run_gpu(wx, be, m, ins).reshape(B, -1)
        k = tensor_bytes(wx, be, be.lib.wamx_gwp_prefix_key(m, 1), (B, SMALL["n_heads"], 1 + 32, 128))
        for b in range(B):
            ref_model = orc.Gwp(SMALL, w)
            state, latent, prompt, noise = per[b]
            ref_model.prompt(prompt)
            ref_model.prefix(state, latent, prompt)
            assert_parity(wx.bf16_to_f32(k[b]), wx.bf16_to_f32(ref_model.prefix_key(1)), what=f"chunk {b} prefix K 1")
            action_gate(got[b], ref_model.denoise(noise), f"chunk {b} of {B}")
        assert not np.array_equal(got[0], got[1])
    finally:
        be.lib.wamx_gwp_free(m)


def test_batch8_full_width_properties(wx, be):
    """Batch 8 at full width (d = 3072, 24 heads, FFN 14336, 512 prompt
    tokens; 2 layers, 2 steps, 256 visual tokens): the denoise projections
    run on 384 rows.  Reordering the chunks reorders the results bit for bit
    (rows never mix), and each chunk matches a batch-1 model on its own."""
    cfg = dict(n_layers=2, hidden=3072, n_heads=24, head_dim=128, ffn_dim=14336, action_hidden=3072,
               action_ffn_dim=14336, action_chunk=48, action_dim=32, grid_h=8, grid_w=32, n_lang=512,
               t5_hidden=4096, z_dim=48, num_steps=2, enc_hidden=128, shift=5.0, eps=1e-6)
    B = 8
    print("gwp batch 8 full width", flush=True)
    m8 = make_model(wx, be, dict(cfg, batch=B), seed=0x5EED0009)
    m1 = make_model(wx, be, cfg, seed=0x5EED0009)
    try:
        ins, per = inputs_batch(cfg, B, 70)
        got = run_gpu(wx, be, m8, ins).reshape(B, -1)
        perm = np.array([3, 0, 7, 1, 6, 2, 5, 4])
        ins_p = tuple(np.concatenate([per[p][i] for p in perm]) for i in range(4))
        got_p = run_gpu(wx, be, m8, ins_p).reshape(B, -1)
        assert np.array_equal(got_p, got[perm])
        for b in (0, 5):
            one = run_gpu(wx, be, m1, per[b])
            action_gate(got[b], one, f"batch-8 chunk {b} vs batch 1")
    finally:
        be.lib.wamx_gwp_free(m8)
        be.lib.wamx_gwp_free(m1)
