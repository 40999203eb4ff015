"""The vision front-end on the GPU against the oracle (pinned in
test_vision.py).

* wamx_preprocess_views (preprocess_kernel, cuda_preprocess.cu:45-137):
  three camera views, u8 and f32, composed into the 384 x 320 canvas of the
  GWP-0.5 artifact and an odd 35 x 23 one; shrinking, enlarging and
  cropping views; a second call with larger views (the staging buffers
  grow).  Bar: within 1e-5 of the oracle (f32 filter arithmetic; the oracle
  sums in float64).  Refused: not three views, an invalid view.
* CONV_2D (ggml_conv_2d_direct, the VAE convolution vae.cpp:140-157)
  through the drop-in import, followed by the bias ADD as vae_conv does, at
  the Wan VAE encoder's shapes for a 384 x 320 image: conv_in 12 -> 160 at
  192 x 160, a 160-channel 3x3 (on a 48 x 40 crop: the kernel is spatially
  uniform), the 1x1 shortcut 160 -> 320, the stride-2 downsampler 320 ->
  320 on the padded 49 x 41 map, 640 -> 640 3x3 at 24 x 20, and an f32
  convolution with two images, stride 2, dilation 2.  Bar: the per-op bar
  (max-rel <= 1e-2, cosine >= 0.9999) on the rounded output.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import ggml_mirror as gm
from conftest import assert_parity
from test_gpu_dropin import Runner

pytestmark = pytest.mark.gpu


def preprocess(wx, be, p, views, W, H):
    arr = (wx.ImageView * len(views))()
    keep = []
    for i, v in enumerate(views):
        a = np.ascontiguousarray(v)
        keep.append(a)
        arr[i] = wx.ImageView(a.ctypes.data, a.shape[1], a.shape[0], 0 if a.dtype == np.uint8 else 1)
    out = be.empty(12 * (W // 2) * (H // 2) * 4)
    st = be.lib.wamx_preprocess_views(p, arr, len(views), W, H, C.c_void_p(out.ptr))
    return st, (out.download(np.float32, (12, H // 2, W // 2)) if st == 0 else None)


def test_preprocess_views_match_oracle(wx, be, orc):
    print("preprocess views", flush=True)
    rng = np.random.default_rng(11)
    p = be.lib.wamx_preprocessor_create(be.ptr)
    assert p, wx.last_error()
    try:
        cases = [
            # high camera 640x480 u8 (shrink + crop), wrists 320x240 f32 (enlarge) and 200x150 u8
            ([rng.integers(0, 256, (480, 640, 3), dtype=np.uint8), rng.random((240, 320, 3), np.float32),
              rng.integers(0, 256, (150, 200, 3), dtype=np.uint8)], 384, 320),
            # larger views on the next call: the staging buffers grow
            ([rng.random((720, 1280, 3), np.float32), rng.integers(0, 256, (480, 640, 3), dtype=np.uint8),
              rng.random((481, 641, 3), np.float32)], 384, 320),
            # an odd canvas: regions of 35 x 11, 17 x 12 and 18 x 12, the last row and column unused
            ([rng.random((9, 13, 3), np.float32), rng.integers(0, 256, (40, 30, 3), dtype=np.uint8),
              rng.random((11, 17, 3), np.float32)], 35, 23),
        ]
        for views, W, H in cases:
            st, got = preprocess(wx, be, p, views, W, H)
            wx.check(st, "preprocess_views")
            ref = orc.compose_and_patchify(views, W, H)
            assert got.shape == ref.shape
            err = np.max(np.abs(got - ref))
            assert err <= 1e-5, (W, H, err)
        # refusals
        views = cases[0][0]
        st, _ = preprocess(wx, be, p, views[:2], 384, 320)
        assert st != 0 and "three camera views" in wx.last_error()
        px = np.zeros(3, np.uint8)
        bad = (wx.ImageView * 3)(*[wx.ImageView(px.ctypes.data, 1, 1, 0)] * 3)
        bad[1] = wx.ImageView(None, 4, 4, 0)
        out = be.empty(12 * 4)
        st = be.lib.wamx_preprocess_views(p, bad, 3, 4, 4, C.c_void_p(out.ptr))
        assert st != 0 and "invalid image 1" in wx.last_error()
    finally:
        be.lib.wamx_preprocessor_free(p)


def _bf(wx, a):
    return wx.f32_to_bf16(np.asarray(a, np.float32))


# (name, IC, OC, k, stride, pad, IW, IH) at a 384 x 320 image
VAE = [("conv_in", 12, 160, 3, 1, 1, 192, 160),
       ("res0.conv1 (crop)", 160, 160, 3, 1, 1, 48, 40),
       ("shortcut 1x1", 160, 320, 1, 1, 0, 24, 20),
       ("downsample", 320, 320, 3, 2, 0, 49, 41),
       ("res3.conv1", 640, 640, 3, 1, 1, 24, 20)]


@pytest.mark.parametrize("name,IC,OC,k,s,p,IW,IH", VAE, ids=[v[0] for v in VAE])
def test_vae_conv_matches_oracle(wx, be, orc, name, IC, OC, k, s, p, IW, IH):
    print(f"vae conv {name}: {IC}->{OC} k{k} s{s} p{p} at {IW}x{IH}", flush=True)
    rng = np.random.default_rng(IC * OC + IW)
    wt = _bf(wx, rng.standard_normal((OC, IC, k, k)) / np.sqrt(IC * k * k))
    x = _bf(wx, rng.standard_normal((1, IC, IH, IW)))
    b = _bf(wx, rng.standard_normal(OC) * 0.1)
    r = Runner(wx, be, 1 << 28)
    tk = r.leaf("bf16", (k, k, IC, OC), wt, "weight")
    tx = r.leaf("bf16", (IW, IH, IC, 1), x, "input")
    tb = r.leaf("bf16", (OC,), b, "bias")
    y = gm.add(gm.conv_2d_direct(tk, tx, s, s, p, p, 1, 1), gm.reshape(tb, 1, 1, OC, 1))
    r.run([y])
    OW, OH = y.ne[0], y.ne[1]
    got = wx.bf16_to_f32(r.fetch(y, np.uint16, (1, OC, OH, OW)))
    ref = orc.conv_2d(wx.bf16_to_f32(wt), wx.bf16_to_f32(x), s, s, p, p) + wx.bf16_to_f32(b)[None, :, None, None]
    assert_parity(got, ref.astype(np.float32), what=f"conv {name}")


def test_f32_conv_batched_strided_dilated(wx, be, orc):
    print("f32 conv, 2 images, stride 2, dilation 2", flush=True)
    rng = np.random.default_rng(5)
    k = rng.standard_normal((24, 8, 3, 3)).astype(np.float32)
    x = rng.standard_normal((2, 8, 37, 29)).astype(np.float32)
    r = Runner(wx, be, 1 << 24)
    tk = r.leaf("f32", (3, 3, 8, 24), k, "weight")
    tx = r.leaf("f32", (29, 37, 8, 2), x, "input")
    y = gm.conv_2d_direct(tk, tx, 2, 2, 2, 2, 2, 2)
    r.run([y])
    got = r.fetch(y, np.float32, (2, 24, y.ne[1], y.ne[0]))
    ref = orc.conv_2d(k, x, 2, 2, 2, 2, 2, 2)
    assert np.allclose(got, ref, rtol=1e-4, atol=1e-4)
