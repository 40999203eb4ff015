"""Pins the CPU oracle (oracle/liboracle.so) before anything is compared to it.

The reference ships no tests or golden vectors for this path (its /tests is
git-ignored, .gitignore:58-60), and ggml b9866 is not available to build, so
each oracle function is pinned by what the mathematics fixes: known-answer
integer GEMMs that are exact in f32, closed forms computed independently in
float64 (tests/golden/make_golden.py), invariants, and brute force at tiny
sizes.  Every check is chosen so that a plausible slip (dropped term, wrong
sign or index, transposed operand) fails it.
"""
from __future__ import annotations

import json
import math

import numpy as np
import pytest

from conftest import GOLDEN, cosine, rel_err


def bf16(x):
    import wamx
    return wamx.f32_to_bf16(np.asarray(x, np.float32))


def f32(h):
    import wamx
    return wamx.bf16_to_f32(h)


# --- bf16 rounding -----------------------------------------------------------
def test_bf16_round_to_nearest_even(orc):
    # 1 + 2^-8 is the tie between 1 and 1 + 2^-7: even mantissa (1.0) wins;
    # 1 + 3*2^-8 ties to 1 + 2^-6 (even).  1 + 2^-8 + 2^-20 rounds up.
    cases = {1.0: 0x3F80, 1.0 + 2 ** -8: 0x3F80, 1.0 + 3 * 2 ** -8: 0x3F82, 1.0 + 2 ** -8 + 2 ** -20: 0x3F81,
             -2.0: 0xC000, float("inf"): 0x7F80, 65280.0: 0x477F, 3.0e38: 0x7F62}
    for v, bits in cases.items():
        assert int(orc.f32_to_bf16([v])[0]) == bits, v
    nan = orc.f32_to_bf16([float("nan")])[0]
    assert (nan & 0x7F80) == 0x7F80 and (nan & 0x7F) != 0
    # the Python helper used by the tests agrees with the oracle on random values
    x = np.random.default_rng(1).standard_normal(4096).astype(np.float32) * 100
    assert np.array_equal(orc.f32_to_bf16(x), bf16(x))


# --- MUL_MAT -----------------------------------------------------------------
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (7, 5, 3), (33, 17, 64), (64, 48, 3072), (130, 3, 4096)])
def test_mul_mat_integer_kat_is_exact(orc, M, N, K):
    """Entries in {-4..4}: products are exact in bf16/f32 and |sum| <= 16K
    < 2^24, so the GEMM result is an exact integer."""
    rng = np.random.default_rng(M * 1000 + N * 10 + K)
    w = rng.integers(-4, 5, (M, K))
    x = rng.integers(-4, 5, (N, K))
    ref = (x @ w.T).astype(np.float64)
    got = orc.mul_mat(bf16(w), x.astype(np.float32))
    assert np.array_equal(got.astype(np.float64), ref)
    got_bf = orc.mul_mat(bf16(w), bf16(x), y_type=orc.BF16)
    assert np.array_equal(got_bf, bf16(ref))


def test_mul_mat_orientation_one_hot(orc):
    """y[n][m] = sum_k w[m][k] x[n][k]: a one-hot weight row selects one input column."""
    M, N, K = 4, 3, 5
    w = np.zeros((M, K), np.float32)
    w[0, 2] = w[1, 0] = w[2, 4] = w[3, 1] = 1.0
    x = np.arange(N * K, dtype=np.float32).reshape(N, K)
    got = orc.mul_mat(bf16(w), x)
    assert np.array_equal(got, x[:, [2, 0, 4, 1]])


def test_mul_mat_rounds_activation_to_bf16(orc):
    # ggml converts the f32 activation to the weight's bf16 type before the dot.
    w = bf16(np.ones((1, 1)))
    x = np.array([[1.0 + 2 ** -9]], np.float32)  # not representable in bf16 -> 1.0
    assert orc.mul_mat(w, x)[0, 0] == 1.0


def test_mul_mat_matches_float64_reference(orc, rng):
    M, N, K = 96, 40, 777
    w = bf16(rng.standard_normal((M, K)) * 0.02)
    x = rng.standard_normal((N, K)).astype(np.float32)
    ref = f32(bf16(x)).astype(np.float64) @ f32(w).astype(np.float64).T
    got = orc.mul_mat(w, x)
    assert rel_err(got, ref) < 1e-6


# --- linear epilogues --------------------------------------------------------
def test_linear_epilogues_consistent(orc, rng):
    M, N, K = 24, 6, 64
    w = bf16(rng.standard_normal((M, K)) * 0.1)
    x = bf16(rng.standard_normal((N, K)))
    zero_b = bf16(np.zeros(M))
    base = orc.linear(w, x)
    assert np.array_equal(base, orc.mul_mat(w, x, y_type=orc.BF16))
    assert np.array_equal(orc.linear(w, x, zero_b, orc.EPI_BIAS), base)
    b = bf16(rng.standard_normal(M))
    withb = orc.linear(w, x, b, orc.EPI_BIAS)
    # bias enters after the bf16 store of the GEMM: bf16(bf16(acc) + b)
    assert np.array_equal(withb, bf16(f32(base) + f32(b)[None, :]))
    gelu = orc.linear(w, x, b, orc.EPI_BIAS_GELU)
    ref_gelu = np.array([[orc.gelu_tanh(v) for v in row] for row in (f32(base) + f32(b)[None, :])], np.float32)
    assert np.array_equal(gelu, bf16(ref_gelu))
    h = bf16(rng.standard_normal((N, M)))
    # gate 0 -> residual unchanged; gate 1 with zero residual -> biased branch
    assert np.array_equal(orc.linear(w, x, b, orc.EPI_BIAS_GATED, h, np.zeros(M, np.float32)), h)
    zero_h = bf16(np.zeros((N, M)))
    assert np.array_equal(orc.linear(w, x, b, orc.EPI_BIAS_GATED, zero_h, np.ones(M, np.float32)), withb)
    assert np.array_equal(orc.linear(w, x, b, orc.EPI_BIAS_RESIDUAL, zero_h), withb)
    g = rng.standard_normal(M).astype(np.float32)
    gated = orc.linear(w, x, b, orc.EPI_BIAS_GATED, h, g)
    assert np.array_equal(gated, orc.gated_residual_bf16(h, withb, g))


# --- GELU --------------------------------------------------------------------
def test_gelu_golden(orc):
    d = json.loads((GOLDEN / "gelu.json").read_text())
    for x, t, e in zip(d["x"], d["tanh"], d["erf"]):
        assert orc.gelu_tanh(x) == pytest.approx(t, rel=1e-6, abs=1e-12)
        assert orc.gelu_erf(x) == pytest.approx(e, rel=1e-6, abs=1e-12)


def test_gelu_identities(orc):
    for x in (0.1, 0.7, 1.9, 4.0):
        # gelu(x) - gelu(-x) = x for both forms (x*Phi(x) with Phi odd-symmetric about 1/2)
        assert orc.gelu_tanh(x) - orc.gelu_tanh(-x) == pytest.approx(x, rel=1e-6)
        assert orc.gelu_erf(x) - orc.gelu_erf(-x) == pytest.approx(x, rel=1e-6)
    assert orc.gelu_tanh(0.0) == 0.0
    assert orc.gelu_tanh(20.0) == pytest.approx(20.0)
    assert abs(orc.gelu_tanh(-20.0)) < 1e-30


def test_bias_gelu_bf16(orc, rng):
    width = 37
    x = bf16(rng.standard_normal((5, width)))
    b = bf16(rng.standard_normal(width))
    got = orc.bias_gelu_bf16(x, b)
    ref = np.vectorize(lambda v: orc.gelu_tanh(float(v)))(f32(x) + f32(b)[None, :])
    assert np.array_equal(got, bf16(ref))


# --- norms -------------------------------------------------------------------
def test_norm_mod_constant_row_gives_shift(orc):
    x = bf16(np.full((3, 64), 2.5))
    scale = np.linspace(-1, 1, 64).astype(np.float32)
    shift = np.linspace(0.5, -0.5, 64).astype(np.float32)
    assert np.array_equal(orc.norm_mod_bf16(x, scale, shift, 1e-6), bf16(np.tile(shift, (3, 1))))


def test_norm_mod_standardises(orc, rng):
    x = bf16(rng.standard_normal((4, 3072)) * 3 + 1)
    y = f32(orc.norm_mod_bf16(x, np.zeros(3072, np.float32), np.zeros(3072, np.float32), 1e-6)).astype(np.float64)
    assert np.allclose(y.mean(1), 0, atol=1e-3) and np.allclose(y.std(1), 1, atol=5e-3)
    xd = f32(x).astype(np.float64)
    ref = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6)
    sc = rng.standard_normal(3072).astype(np.float32) * 0.1
    sh = rng.standard_normal(3072).astype(np.float32) * 0.1
    got = f32(orc.norm_mod_bf16(x, sc, sh, 1e-6))
    assert rel_err(got, ref * (1 + sc) + sh) < 8e-3
    # per-row scale/shift (row stride = cols) equals broadcast when rows repeat
    got_rows = orc.norm_mod_bf16(x, np.tile(sc, (4, 1)), np.tile(sh, (4, 1)), 1e-6)
    assert np.array_equal(got_rows, orc.norm_mod_bf16(x, sc, sh, 1e-6))


def test_layer_norm_affine_identity_matches_modulation(orc, rng):
    x = bf16(rng.standard_normal((3, 128)))
    one, zero = bf16(np.ones(128)), bf16(np.zeros(128))
    z = np.zeros(128, np.float32)
    assert np.array_equal(orc.layer_norm_bf16(x, one, zero, 1e-6), orc.norm_mod_bf16(x, z, z, 1e-6))
    w = bf16(rng.standard_normal(128))
    b = bf16(rng.standard_normal(128))
    n = f32(orc.norm_mod_bf16(x, z, z, 1e-6)).astype(np.float64)
    assert rel_err(f32(orc.layer_norm_bf16(x, w, b, 1e-6)), n * f32(w) + f32(b)) < 1e-2


def test_rms_norm_scale_invariant_and_closed_form(orc, rng):
    x = bf16(rng.standard_normal((5, 3072)))
    w = bf16(1 + 0.02 * rng.standard_normal(3072))
    y = orc.rms_norm_bf16_f32(x, w, 1e-6)
    y4 = orc.rms_norm_bf16_f32(bf16(f32(x) * 4), w, 1e-6)  # power-of-two scale is exact in bf16
    assert np.allclose(y, y4, rtol=1e-6, atol=0)
    xd = f32(x).astype(np.float64)
    ref = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * f32(w)
    assert rel_err(y, ref) < 1e-6


def test_norm_mod_f32_closed_form(orc, rng):
    x = rng.standard_normal((6, 1024)).astype(np.float32) * 2 - 0.5
    sc = rng.standard_normal(1024).astype(np.float32) * 0.1
    sh = rng.standard_normal(1024).astype(np.float32) * 0.1
    xd = x.astype(np.float64)
    n = (xd - xd.mean(1, keepdims=True)) / np.sqrt(xd.var(1, keepdims=True) + 1e-6)
    got = orc.norm_mod_f32(x, sc, sh, 1e-6)
    assert rel_err(got, n + n * sc + sh) < 1e-5
    # constant row: variance 0 -> n = 0 -> y = shift
    c = orc.norm_mod_f32(np.full((1, 1024), 3.0, np.float32), sc, sh, 1e-6)
    assert np.allclose(c[0], sh, atol=1e-6)


def test_gated_residuals(orc, rng):
    h = bf16(rng.standard_normal((4, 50)))
    b = bf16(rng.standard_normal((4, 50)))
    g = rng.standard_normal(50).astype(np.float32)
    assert np.array_equal(orc.gated_residual_bf16(h, b, np.zeros(50, np.float32)), h)
    one = orc.gated_residual_bf16(h, b, np.ones(50, np.float32))
    assert np.array_equal(one, bf16(f32(h) + f32(b)))
    got = f32(orc.gated_residual_bf16(h, b, g)).astype(np.float64)
    assert rel_err(got, f32(h) + f32(b) * g) < 4e-3
    g_rows = np.tile(g, (4, 1))
    assert np.array_equal(orc.gated_residual_bf16(h, b, g_rows), orc.gated_residual_bf16(h, b, g))
    gb = bf16(g)
    assert np.array_equal(orc.gated_residual_bf16(h, b, gb), orc.gated_residual_bf16(h, b, f32(gb)))
    r = rng.standard_normal((3, 40)).astype(np.float32)
    bb = rng.standard_normal((3, 40)).astype(np.float32)
    gg = rng.standard_normal(40).astype(np.float32)
    exp = (r + (bb * gg).astype(np.float32)).astype(np.float32)
    assert np.array_equal(orc.gated_residual_f32(r, bb, gg), exp)


# --- RoPE ----------------------------------------------------------------------
def test_rope_golden(orc):
    d = json.loads((GOLDEN / "rope.json").read_text())
    x = np.array(d["x"], np.float32)
    got = orc.rope_f32(x, np.array(d["pos"]), d["n_dims"], d["base"])
    assert np.allclose(got, np.array(d["y"]), rtol=1e-6, atol=1e-6)


def test_rope_invariants(orc, rng):
    T, H, D = 6, 3, 128
    x = rng.standard_normal((T, H, D)).astype(np.float32)
    # position 0 is the identity
    assert np.array_equal(orc.rope_f32(x, np.zeros(T), D), x)
    pos = np.arange(T) * 7 + 3
    y = orc.rope_f32(x, pos, D)
    # each rotated pair keeps its norm
    nx = np.hypot(x[..., 0::2], x[..., 1::2])
    ny = np.hypot(y[..., 0::2], y[..., 1::2])
    assert np.allclose(nx, ny, rtol=1e-5)
    # <R(m)q, R(n)k> depends on m - n only
    q = rng.standard_normal((1, 1, D)).astype(np.float32)
    k = rng.standard_normal((1, 1, D)).astype(np.float32)
    dots = []
    for m, n in [(5, 2), (13, 10), (40, 37)]:
        rq = orc.rope_f32(q, [m], D)
        rk = orc.rope_f32(k, [n], D)
        dots.append(float((rq.astype(np.float64) * rk).sum()))
    assert np.allclose(dots, dots[0], rtol=1e-5)
    # dims past n_dims pass through
    part = orc.rope_f32(x, pos, 44)
    assert np.array_equal(part[..., 44:], x[..., 44:])


def test_qk_norm_rope_composition(orc, rng):
    """rms_norm_bf16_f32 -> rope -> bf16 -> [H][T][dh], for 1-D and 3-section rope."""
    H, dh, T = 3, 128, 5
    x = bf16(rng.standard_normal((T, H * dh)))
    w = bf16(1 + 0.02 * rng.standard_normal(H * dh))
    pos = np.array([1, 2, 3, 4, 48], np.int32)
    got = orc.qk_norm_rope(x, w, H, dh, 0, pos)
    normed = orc.rms_norm_bf16_f32(x, w, 1e-6).reshape(T, H, dh)
    ref = orc.rope_f32(normed, pos, dh)
    assert np.array_equal(got, bf16(ref).transpose(1, 0, 2))
    p0, p1, p2 = np.zeros(T, np.int32), np.array([0, 1, 2, 3, 15]), np.array([5, 6, 7, 31, 0])
    got3 = orc.qk_norm_rope(x, w, H, dh, 1, p0, p1, p2)
    parts = [orc.rope_f32(np.ascontiguousarray(normed[..., a:b]), p, b - a)
             for (a, b, p) in [(0, 44, p0), (44, 86, p1), (86, 128, p2)]]
    ref3 = np.concatenate(parts, axis=-1)
    assert np.array_equal(got3, bf16(ref3).transpose(1, 0, 2))
    # t == 0 for every token makes the first section the identity
    assert np.array_equal(got3[..., :44], bf16(normed[..., :44]).transpose(1, 0, 2))
    got_none = orc.qk_norm_rope(x, w, H, dh, 2)
    assert np.array_equal(got_none, bf16(normed).transpose(1, 0, 2))
    # token offset into a larger destination
    dst = np.zeros((H, T + 3, dh), np.uint16)
    orc.qk_norm_rope(x, w, H, dh, 0, pos, dst=dst, tok0=2)
    assert np.array_equal(dst[:, 2:2 + T], got) and not dst[:, :2].any() and not dst[:, 2 + T:].any()


# --- softmax / attention ----------------------------------------------------------
def test_softmax_rows(orc, rng):
    x = rng.standard_normal((7, 300)).astype(np.float32) * 5
    y = orc.softmax_f32(x, 0.3)
    assert np.allclose(y.sum(1), 1, atol=1e-6)
    assert np.allclose(orc.softmax_f32(x + 11, 0.3), y, atol=1e-6)  # shift invariance
    ref = np.exp(0.3 * x.astype(np.float64))
    assert rel_err(y, ref / ref.sum(1, keepdims=True)) < 1e-6


def _attn_inputs(rng, H, tq, na, nb, dh=128):
    q = bf16(rng.standard_normal((H, tq, dh)))
    ka = bf16(rng.standard_normal((H, na, dh)))
    va = bf16(rng.standard_normal((H, dh, na)))
    kb = bf16(rng.standard_normal((H, nb, dh)))
    vb = bf16(rng.standard_normal((H, dh, nb)))
    return q, ka, va, kb, vb


def test_attention_brute_force(orc, rng):
    H, tq, na, nb, dh = 2, 5, 9, 4, 128
    q, ka, va, kb, vb = _attn_inputs(rng, H, tq, na, nb)
    got = f32(orc.attention(q, ka, va, kb, vb, na_split=1)).reshape(tq, H, dh)
    for h in range(H):
        k = np.concatenate([f32(ka[h, :1]), f32(kb[h]), f32(ka[h, 1:])]).astype(np.float64)
        v = np.concatenate([f32(va[h, :, :1]), f32(vb[h]), f32(va[h, :, 1:])], axis=1).T.astype(np.float64)
        s = f32(q[h]).astype(np.float64) @ k.T / math.sqrt(dh)
        p = np.exp(s - s.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        ref = p @ v
        assert rel_err(got[:, h], ref) < 1e-2 and cosine(got[:, h], ref) > 0.9999


def test_attention_invariants(orc, rng):
    H, tq, dh = 1, 3, 128
    # identical keys -> uniform probabilities -> mean of V
    q = bf16(rng.standard_normal((H, tq, dh)))
    k = bf16(np.tile(rng.standard_normal((1, 1, dh)), (H, 8, 1)))
    v = bf16(rng.standard_normal((H, dh, 8)))
    got = f32(orc.attention(q, k, v))
    assert np.allclose(got, np.tile(f32(v)[0].mean(1), (tq, 1)), rtol=1e-2, atol=1e-2)
    # one dominant logit selects its value column
    k2 = bf16(np.zeros((H, 8, dh)))
    k2[0, 5] = bf16(np.full(dh, 8.0))
    q2 = bf16(np.full((H, tq, dh), 8.0))
    got2 = f32(orc.attention(q2, k2, v))
    assert np.allclose(got2, np.tile(f32(v)[0, :, 5], (tq, 1)), rtol=1e-2, atol=1e-2)
    # key order only changes rounding: split position and source assignment
    q3, ka, va, kb, vb = _attn_inputs(rng, 2, 4, 12, 8)
    a1 = f32(orc.attention(q3, ka, va, kb, vb, na_split=1))
    a2 = f32(orc.attention(q3, ka, va, kb, vb, na_split=7))
    kcat = np.concatenate([kb, ka], axis=1)
    vcat = np.concatenate([vb, va], axis=2)
    a3 = f32(orc.attention(q3, kcat, vcat))
    assert rel_err(a1, a2) < 1e-2 and rel_err(a1, a3) < 1e-2 and cosine(a1, a3) > 0.99999


def test_modulation_sum(orc, rng):
    mod = bf16(rng.standard_normal(6 * 16))
    tab = bf16(rng.standard_normal((3, 6 * 16)))
    out = orc.modulation(mod, tab)
    assert np.array_equal(out, (f32(mod)[None, :] + f32(tab)).astype(np.float32))


# --- schedule, timestep embedding, RNG ----------------------------------------------
def test_flow_schedule_golden(orc):
    d = json.loads((GOLDEN / "flow_schedule.json").read_text())
    for key, ref in d.items():
        n, s = key.split("_")
        t, sig = orc.flow_schedule(int(n), float(s))
        assert np.array_equal(t, np.array(ref["timesteps"], np.float32)), key
        assert np.array_equal(sig, np.array(ref["sigmas"], np.float32)), key
    t, sig = orc.flow_schedule(10, 5.0)
    assert sig[0] == 1.0 and sig[-1] == 0.0 and np.all(np.diff(sig) < 0)
    # shift 1 is the plain linspace from 1 down to the training sigma 1e-3
    t1, s1 = orc.flow_schedule(4, 1.0)
    assert np.allclose(s1[:4], np.linspace(1.0, 1e-3, 4), rtol=1e-6)


def test_timestep_embedding_golden(orc):
    d = json.loads((GOLDEN / "timestep_embedding.json").read_text())
    for t, ref in d.items():
        got = orc.timestep_embedding(float(t), 256)
        assert np.allclose(got, np.array(ref), atol=2e-4 * max(1.0, float(t) / 100)), t
    e0 = orc.timestep_embedding(0.0, 256)
    assert np.array_equal(e0[:128], np.ones(128, np.float32)) and not e0[128:].any()


def test_fill_normal_golden_and_moments(orc):
    d = json.loads((GOLDEN / "normal_sample.json").read_text())
    got = orc.fill_normal(len(d["values"]), d["seed"], d["mean"], d["std"])
    assert np.allclose(got, d["values"], rtol=1e-6, atol=1e-6)
    big = orc.fill_normal(1 << 20, 7).astype(np.float64)
    assert abs(big.mean()) < 5e-3 and abs(big.std() - 1) < 5e-3
    assert abs(((big - big.mean()) ** 3).mean()) < 2e-2  # symmetric
    assert not np.array_equal(orc.fill_normal(16, 1), orc.fill_normal(16, 2))


# --- the CPU port (cpu_port.c): the baseline bench.py times -------------------
def test_cpu_port_matches_the_exact_oracle(orc, rng):
    """The fp32 CPU port computes what the exact oracle computes, to fp32
    accumulation error: products (ragged M, N and K, f32 and bf16
    activations), two-source attention with a split, and the small MoT
    chunk under the reference's action gates.  Its outputs are timed by
    bench.py's cpu_baseline, so a port that computed something else would
    make that baseline meaningless."""
    import oracle as o
    try:
        for M, N, K, xt in ((37, 5, 300, o.F32), (64, 48, 3072, o.BF16), (130, 13, 513, o.BF16)):
            w = bf16(rng.standard_normal(M * K) * 0.05).reshape(M, K)
            x = rng.standard_normal((N, K)).astype(np.float32)
            if xt == o.BF16:
                x = bf16(x)
            o.set_port(False)
            ref = orc.mul_mat(w, x)
            o.set_port(True)
            got = orc.mul_mat(w, x)
            assert rel_err(got, ref) < 1e-5, (M, N, K)
        H, dh, tq, na, nb = 3, 64, 37, 150, 21
        q = bf16(rng.standard_normal((H, tq, dh)))
        ka, kb = bf16(rng.standard_normal((H, na, dh))), bf16(rng.standard_normal((H, nb, dh)))
        va, vb = bf16(rng.standard_normal((H, dh, na + 3))), bf16(rng.standard_normal((H, dh, nb)))
        o.set_port(False)
        ref = orc.attention(q, ka, va, kb, vb, na_split=1)
        o.set_port(True)
        got = orc.attention(q, ka, va, kb, vb, na_split=1)
        assert rel_err(f32(got), f32(ref)) < 1e-2 and cosine(f32(got), f32(ref)) > 0.9999
        # the small MoT chunk, exact against port
        import test_oracle_mot as tm
        w = orc.gwp_synthetic_weights(tm.CFG, tm.SEED, 0.05)
        ins = tm.inputs(orc)
        chunks = []
        for port in (False, True):
            o.set_port(port)
            g = tm.run(orc, w, ins)
            chunks.append(g.denoise(ins[3]))
            g.close()
        d = np.abs(chunks[1].astype(np.float64) - chunks[0])
        assert d.mean() <= 1e-3 and d.max() <= 1e-2 * max(1.0, float(np.abs(chunks[0]).max()))
    finally:
        o.set_port(False)
