"""End-to-end parity of the synthetic GWP-0.5 MoT action step (prompt
projection, prefix pass, unrolled denoise) on the HIP backend against the
oracle's independent CPU restatement, on identical seeded weights and inputs.

Full-step bar, two parts:
* the action chunk (a bf16 state rounded every step) passes the reference's
  own comparison gates of its BF16 latency profile (apps/wam-bench.cpp
  :172-176, apps/wam-compare.cpp:39): finite, mean |delta| <= 1e-3 and max
  |delta| <= 1e-2.  Models with inflated weights (std 0.05) and batch 8
  against batch 1 (two GPU paths) hold the max gate relative above |a| = 1
  (|delta| <= 1e-2 * max(1, |a|)), since a single rounding flip of a bf16
  state element at |a| >= 2 is 1.56e-2.  Every such check also asserts that
  the no-op result bf16(noise) FAILS the same gate against the same
  reference, so the gate can fail;
* the velocity of every denoise step (the action decoder's output, which the
  reference dumps as velocity_step0 / denoise_%02d_velocity,
  engine.cpp:416-421) passes the velocity bar: the per-op cosine >= 0.9999
  and max-rel <= 3e-2 (VEL_REL_TOL).  The bar must also reject the
  velocities of another input on the same weights (other noise, another
  prompt or another chunk's inputs).
Prefix K/V caches are compared per layer with the per-op bar.  rel-L2 and
cosine of the chunk are printed as extra reporting.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest
import wamx

from conftest import COS_TOL, assert_parity, cosine, rel_err

pytestmark = pytest.mark.gpu

SMALL = dict(n_layers=2, hidden=256, n_heads=2, head_dim=128, ffn_dim=512, action_hidden=256, action_ffn_dim=384,
             action_chunk=48, action_dim=32, grid_h=4, grid_w=8, n_lang=16, t5_hidden=64, z_dim=16, num_steps=3,
             enc_hidden=32, shift=5.0, eps=1e-6)


# Weight std of the small-geometry parity tests: at 0.02 the 32-wide encoder
# and decoder MLPs squash the inputs and the velocity hardly depends on them;
# at 0.05 each of state, latent, prompt and noise moves it past the per-op
# bar (tests/test_oracle_mot.py::test_small_parity_weights_are_input_sensitive).
SMALL_WSTD = 0.05


def make_model(wx, be, cfg, seed=0x5EED0003, wstd=0.02):
    c = wx.GwpConfig(**cfg)
    m = be.lib.wamx_gwp_create(be.ptr, C.byref(c))
    assert m, wx.last_error()
    wx.check(be.lib.wamx_gwp_init_synthetic(m, seed, wstd), "init_synthetic")
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


# The reference's action comparison gates in the BF16 latency profile
# (apps/wam-bench.cpp:172-176; apps/wam-compare.cpp:39 defaults).
MEAN_GATE, MAX_GATE = 1e-3, 1e-2


def gate_passes(got, ref, scaled=False) -> bool:
    """The reference's gates; scaled=True holds the max gate relative above
    |a| = 1 (|delta| <= 1e-2 * max(1, |a|)): one rounding flip of a bf16
    state element at |a| >= 2 is 1.56e-2."""
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    ok_max = np.all(d <= MAX_GATE * np.maximum(1.0, np.abs(ref))) if scaled else d.max() <= MAX_GATE
    return bool(np.all(np.isfinite(got)) and d.mean() <= MEAN_GATE and ok_max)


def action_gate(got, ref, what, noise, scaled=False):
    """The chunk passes the gates against `ref`, and the no-op chunk
    bf16(noise) does not."""
    got, ref = np.asarray(got, np.float32).ravel(), np.asarray(ref, np.float32).ravel()
    d = np.abs(got.astype(np.float64) - ref)
    rel_l2 = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    noop = wamx.round_bf16(np.asarray(noise, np.float32).ravel())
    dn = np.abs(noop.astype(np.float64) - ref)
    print(f"{what}: mean|d| {d.mean():.3e} max|d| {d.max():.3e} (gates {MEAN_GATE}, {MAX_GATE}"
          f"{' x max(1,|a|)' if scaled else ''}); rel-L2 {rel_l2:.3e} cos {cosine(got, ref):.6f}; "
          f"no-op bf16(noise) mean|d| {dn.mean():.3e} max|d| {dn.max():.3e}")
    assert not gate_passes(noop, ref, scaled), f"{what}: the gate cannot tell bf16(noise) from the reference"
    assert gate_passes(got, ref, scaled), what


# Velocity bar: the per-op cosine (>= 0.9999) and max-rel <= 3e-2, the
# per-op 1e-2 widened for a whole step's composition (prompt, prefix and
# denoise layers of bf16 rounding; from step 1 on the bf16 action states
# already differ by rounding flips).  Measured: <= 1.23e-2 on the 2-layer
# models, <= 2.25e-2 at 30 + 30 layers; cosine >= 0.99993 everywhere.
VEL_REL_TOL = 3e-2


def velocity_passes(got, ref, rel=VEL_REL_TOL) -> bool:
    return rel_err(got, ref) <= rel and cosine(got, ref) >= COS_TOL


def velocity_gate(got, ref, what, rel=VEL_REL_TOL):
    """The velocity bar on one step's velocity."""
    print(f"{what}: max-rel {rel_err(got, ref):.3e} cosine {cosine(got, ref):.7f} |v|max {np.max(np.abs(ref)):.3e}")
    assert np.max(np.abs(ref)) > 0
    assert_parity(got, ref, rel=rel, what=what)


def gpu_velocity(wx, be, m, step, n):
    out = np.empty(n, np.float32)
    wx.check(be.lib.wamx_gwp_get_velocity(m, step, out.ctypes.data), f"get_velocity {step}")
    return out


def check_velocities(wx, be, m, ref_v, other_v, what, chunks=1, chunk=None, rel=VEL_REL_TOL):
    """Every step's velocity of the GPU model (chunk `chunk` of `chunks`, or
    all) against the reference velocities `ref_v[s]`.  `other_v[s]` are
    reference velocities of another input (other noise or another chunk's
    inputs, same weights): the bar must reject them at every step, so a
    backend that lost its input would fail."""
    steps = len(ref_v)
    n = ref_v[0].size
    for s in range(steps):
        got = gpu_velocity(wx, be, m, s, n * chunks)
        if chunk is not None:
            got = got.reshape(chunks, n)[chunk]
        velocity_gate(got, ref_v[s], f"{what} velocity step {s}", rel)
        if other_v is not None:
            assert not velocity_passes(other_v[s], ref_v[s], rel), f"{what}: the bar accepts another input's step {s}"


@pytest.mark.parametrize("wstd", [0.02, SMALL_WSTD])
def test_small_model_matches_oracle(wx, be, orc, wstd):
    """Prefix K/V per layer (the per-op bar), the chunk and every step's
    velocity (the velocity bar) against the oracle, at the 0.02 weight std of
    the other tests (the chunk under the reference's gates) and at
    SMALL_WSTD, where the inputs move the velocity past the bar (the chunk
    under the magnitude-scaled max gate; the bar must reject the velocities
    of other noise)."""
    print(f"gwp small model vs oracle, weight std {wstd}", flush=True)
    m = make_model(wx, be, SMALL, wstd=wstd)
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
        action_gate(got, ref, "action chunk", noise, scaled=wstd != 0.02)
        ref_v = [ref_model.velocity(s) for s in range(SMALL["num_steps"])]
        if wstd == 0.02:
            check_velocities(wx, be, m, ref_v, None, "small model")
        else:
            ref_model.denoise(inputs(SMALL, seed=8)[3])
            other_v = [ref_model.velocity(s) for s in range(SMALL["num_steps"])]
            check_velocities(wx, be, m, ref_v, other_v, "small model")
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
    (also written through a weight handle) and a zero capacity all project
    again."""
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
        # A weight handle may be written through: the same prompt is
        # projected again, with the weights as they now are.
        for x in (m, ref):
            t = lib.wamx_gwp_weight(x, b"gwp.blocks.0.action_expert.attn2.to_k.weight")
            assert t, wx.last_error()
            n = lib.wamx_nelements(t)
            w = np.empty(n, np.uint16)
            wx.check(lib.wamx_backend_tensor_get(t, w.ctypes.data, 0, n * 2), "read")
            w = wamx.f32_to_bf16(wamx.bf16_to_f32(w) * 1.5)
            wx.check(lib.wamx_backend_tensor_set(t, w.ctypes.data, 0, n * 2), "write")
        assert np.array_equal(run_gpu(wx, be, m, b), run_gpu(wx, be, ref, b))
        assert stats() == (2, 4)
        # Capacity 0: every prompt is projected again and nothing is counted.
        wx.check(lib.wamx_gwp_set_prompt_cache(m, 0), "set_prompt_cache")
        assert np.array_equal(run_gpu(wx, be, m, a), run_gpu(wx, be, ref, a))
        assert np.array_equal(run_gpu(wx, be, m, a_other), run_gpu(wx, be, ref, a_other))
        assert stats() == (2, 4)
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
        action_gate(got, ref, "full-width action chunk", noise)
        ref_v = [ref_model.velocity(s) for s in range(cfg["num_steps"])]
        # another prompt (the input the velocity depends on most at this
        # weight scale: rel 1.3e-1 on the oracle)
        other_prompt = inputs(cfg, seed=22)[2]
        ref_model.prompt(other_prompt)
        ref_model.prefix(state, latent, other_prompt)
        ref_model.denoise(noise)
        other_v = [ref_model.velocity(s) for s in range(cfg["num_steps"])]
        check_velocities(wx, be, m, ref_v, other_v, "full width")
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


@pytest.mark.parametrize("B", [3, 8])
def test_batched_chunks_match_oracle(wx, be, orc, B):
    """B independent chunks in one request (each with its own state, latent,
    prompt and noise) against B oracle runs on the same weights (std
    SMALL_WSTD): the prefix K of layer 1, the chunk under the
    magnitude-scaled gates and every step's velocity under the velocity bar,
    which must reject the next chunk's.  B x 48 rows take the tile GEMMs in the denoise step (144
    rows at B = 3; 384 at B = 8, the batch of config 5)."""
    cfg = dict(SMALL, batch=B)
    print(f"gwp batch {B} vs oracle", flush=True)
    m = make_model(wx, be, cfg, seed=0x5EED0008, wstd=SMALL_WSTD)
    try:
        w = read_weights(wx, be, m)
        ins, per = inputs_batch(SMALL, B, 40)
        got = run_gpu(wx, be, m, ins).reshape(B, -1)
        k = tensor_bytes(wx, be, be.lib.wamx_gwp_prefix_key(m, 1), (B, SMALL["n_heads"], 1 + 32, 128))
        refs, ref_vs = [], []
        for b in range(B):
            ref_model = orc.Gwp(SMALL, w)
            state, latent, prompt, noise = per[b]
            ref_model.prompt(prompt)
            ref_model.prefix(state, latent, prompt)
            assert_parity(wx.bf16_to_f32(k[b]), wx.bf16_to_f32(ref_model.prefix_key(1)), what=f"chunk {b} prefix K 1")
            refs.append(ref_model.denoise(noise))
            ref_vs.append([ref_model.velocity(s) for s in range(SMALL["num_steps"])])
        for b in range(B):
            action_gate(got[b], refs[b], f"chunk {b} of {B}", per[b][3], scaled=True)
            # the next chunk's velocities come from other inputs on the same weights
            check_velocities(wx, be, m, ref_vs[b], ref_vs[(b + 1) % B], f"chunk {b} of {B}", chunks=B, chunk=b)
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
            action_gate(got[b], one, f"batch-8 chunk {b} vs batch 1", per[b][3], scaled=True)
    finally:
        be.lib.wamx_gwp_free(m8)
        be.lib.wamx_gwp_free(m1)


def test_batch8_full_size_matches_batch1(wx, be):
    """BASELINE config 5 at batch 8 with its full KV: 30 layers, 8 chunks each
    with its own 3073 prefix + 512 prompt keys, 10 steps; the 384-row denoise
    projections run on the K-sliced tile GEMMs and the attention on 192
    virtual heads.  Every chunk equals the same chunk run alone by a batch-1
    model with the same weights (the few-token path) under the reference's
    gates, and its step-0 velocity under the per-op bar."""
    c = be.lib.wamx_gwp_default_config()
    cfg = {k: getattr(c, k) for k, _ in wx.GwpConfig._fields_}
    B = 8
    print("gwp batch 8 full size: create", flush=True)
    m8 = make_model(wx, be, dict(cfg, batch=B), seed=0x5EED0005)
    m1 = make_model(wx, be, dict(cfg, batch=1), seed=0x5EED0005)
    try:
        ins, per = inputs_batch(cfg, B, 90)
        got = run_gpu(wx, be, m8, ins).reshape(B, -1)
        n = cfg["action_chunk"] * cfg["action_dim"]
        v8 = gpu_velocity(wx, be, m8, 0, B * n).reshape(B, n)
        print("gwp batch 8 full size: chunks alone", flush=True)
        v1 = []
        for b in range(B):
            one = run_gpu(wx, be, m1, per[b])
            action_gate(got[b], one, f"full-size batch-8 chunk {b} vs batch 1", per[b][3], scaled=True)
            v1.append(gpu_velocity(wx, be, m1, 0, n))
            velocity_gate(v8[b], v1[b], f"full-size batch-8 chunk {b} step-0 velocity")
        for b in range(B):
            assert not velocity_passes(v1[(b + 1) % B], v1[b]), "the bar accepts another chunk's"
    finally:
        be.lib.wamx_gwp_free(m8)
        be.lib.wamx_gwp_free(m1)


def test_non_finite_inputs_and_outputs_refused(wx, be):
    """A NaN or Inf in any input is refused before upload (engine.cpp:238-247,
    :274, :320, :350-357), leaving the model's inputs as they were; a
    non-finite action fails get_action (model.cpp:246-251)."""
    print("gwp non-finite inputs and outputs", flush=True)
    lib = be.lib
    m = make_model(wx, be, SMALL, seed=31)
    try:
        ins = inputs(SMALL, seed=12)
        first = run_gpu(wx, be, m, ins)
        names = ("state", "latent", "prompt", "noise")
        for i, bad in ((0, np.nan), (1, np.inf), (2, -np.inf), (3, np.nan)):
            arrs = [a.copy() for a in inputs(SMALL, seed=13)]
            arrs[i][len(arrs[i]) // 2] = bad
            st = lib.wamx_gwp_set_inputs(m, *[a.ctypes.data for a in arrs])
            assert st != 0 and f"{names[i]} contains NaN or Inf (element {len(arrs[i]) // 2})" in wx.last_error()
        # the refused requests uploaded nothing: the last good inputs remain
        wx.check(lib.wamx_gwp_predict(m, None), "predict")
        out = np.empty(first.size, np.float32)
        wx.check(lib.wamx_gwp_get_action(m, out.ctypes.data), "get_action")
        assert np.array_equal(out, first)
        # an infinite decoder bias makes every action non-finite
        t = lib.wamx_gwp_weight(m, b"gwp.action_decoder.out_proj.bias")
        inf = np.full(lib.wamx_nelements(t), 0x7F80, np.uint16)
        wx.check(lib.wamx_backend_tensor_set(t, inf.ctypes.data, 0, inf.nbytes), "set bias")
        wx.check(lib.wamx_gwp_predict(m, None), "predict")
        assert lib.wamx_gwp_get_action(m, out.ctypes.data) != 0
        assert "action contains NaN or Inf" in wx.last_error()
        assert not np.all(np.isfinite(out))
    finally:
        lib.wamx_gwp_free(m)
