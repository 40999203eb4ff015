"""The denoise step's glue ops on the GPU: the flow-matching update
(EULER_STEP, scheduler_step weights.cpp:885-902), the small two-layer MLP of
the action encoder and decoder (MLP_SMALL, mot.cpp:16-55) and the adaLN
modulation batched over timesteps (MODULATION with S columns,
mot.cpp:130-145).  The update and the modulation are exact f32 arithmetic and
must match bit for bit; the MLP is held to the oracle's linear layers and
GELU-erf at the per-op bar."""
from __future__ import annotations

import numpy as np
import pytest
from scipy.special import erf

from conftest import assert_parity
from test_gpu_fusion import Graph

pytestmark = pytest.mark.gpu


def bf16(x):
    import wamx
    return wamx.f32_to_bf16(np.asarray(x, np.float32))


def f32(h):
    import wamx
    return wamx.bf16_to_f32(h)


def test_euler_step_bit_exact(wx, be, rng):
    print("euler step", flush=True)
    g = Graph(wx, be)
    try:
        a = g.t(wx.TYPE_BF16, 32, 384)
        v = g.t(wx.TYPE_BF16, 32, 384)
        dt = g.t(wx.TYPE_F32, 1)
        out = be.lib.wamx_euler_step(g.ctx, a, v, dt)
        assert out, wx.last_error()
        g.alloc()
        ah = bf16(rng.standard_normal((384, 32)) * 2)
        vh = bf16(rng.standard_normal((384, 32)) * 0.05)
        dth = np.array([-0.0823], np.float32)
        g.set(a, ah)
        g.set(v, vh)
        g.set(dt, dth)
        g.compute(out)
        got = g.get(out, np.uint16, (384, 32))
        prod = (f32(vh) * dth[0]).astype(np.float32)  # MUL node, f32
        ref = bf16((f32(ah) + prod).astype(np.float32))  # ADD node, f32, then the bf16 cast
        assert np.array_equal(got, ref)
    finally:
        g.close()


def gelu_erf_bf16(h):
    x = f32(h).astype(np.float64)
    return bf16((0.5 * x * (1.0 + erf(x / np.sqrt(2.0)))).astype(np.float32))


@pytest.mark.parametrize("N", [48, 17, 384])
@pytest.mark.parametrize("which", ["encoder", "decoder", "ragged"])
def test_mlp_small_matches_oracle(wx, be, orc, rng, N, which):
    """Encoder form: x [32] -> 128 + GELU-erf -> 128 + GELU-erf; decoder form:
    GELU-erf(x [128]) -> 128 + GELU-erf -> 32 (both on the register-row
    kernel); ragged widths 20 -> 72 -> 30, which take the LDS-staged kernel."""
    print(f"mlp_small {which} N={N}", flush=True)
    K0, M1, M2, flags = {"encoder": (32, 128, 128, 2 | 4), "decoder": (128, 128, 32, 1 | 2),
                         "ragged": (20, 72, 30, 1 | 2 | 4)}[which]
    xh = bf16(rng.standard_normal((N, K0)))
    w1h = bf16(rng.standard_normal((M1, K0)) * 0.08)
    b1h = bf16(rng.standard_normal(M1) * 0.02)
    w2h = bf16(rng.standard_normal((M2, M1)) * 0.08)
    b2h = bf16(rng.standard_normal(M2) * 0.02)
    g = Graph(wx, be)
    try:
        x = g.t(wx.TYPE_BF16, K0, N)
        w1, b1 = g.t(wx.TYPE_BF16, K0, M1), g.t(wx.TYPE_BF16, M1)
        w2, b2 = g.t(wx.TYPE_BF16, M1, M2), g.t(wx.TYPE_BF16, M2)
        y = be.lib.wamx_mlp_small(g.ctx, x, w1, b1, w2, b2, flags)
        assert y, wx.last_error()
        g.alloc()
        for t, a in ((x, xh), (w1, w1h), (b1, b1h), (w2, w2h), (b2, b2h)):
            g.set(t, a)
        g.compute(y)
        got = g.get(y, np.uint16, (N, M2))
    finally:
        g.close()
    h = gelu_erf_bf16(xh) if flags & 1 else xh
    h = orc.linear(w1h, h, b1h, orc.EPI_BIAS)
    if flags & 2:
        h = gelu_erf_bf16(h)
    h = orc.linear(w2h, h, b2h, orc.EPI_BIAS)
    if flags & 4:
        h = gelu_erf_bf16(h)
    assert_parity(f32(got), f32(h), what=f"mlp_small {which}")
    assert np.mean(got != h) < 0.02


def test_modulation_over_steps_bit_exact(wx, be, rng):
    print("modulation over timesteps", flush=True)
    d, L, S = 64, 30, 10
    g = Graph(wx, be)
    try:
        mod = g.t(wx.TYPE_F32, 6 * d, S)
        tab = g.t(wx.TYPE_BF16, d, 6, L)
        out = be.lib.wamx_modulation(g.ctx, mod, tab)
        assert out, wx.last_error()
        g.alloc()
        mh = (rng.standard_normal((S, 6 * d)) * 0.1).astype(np.float32)
        th = bf16(rng.standard_normal((L, 6 * d)) * 0.1)
        g.set(mod, mh)
        g.set(tab, th)
        g.compute(out)
        got = g.get(out, np.float32, (S, L, 6 * d))
        ref = (mh[:, None, :] + f32(th)[None, :, :]).astype(np.float32)
        assert np.array_equal(got, ref)
    finally:
        g.close()
