"""The vision front-end's oracle and host side, on the CPU.

The oracle's canvas (oracle.compose_and_patchify, vae.cpp:1-133) is pinned
by checks a misreading would fail:
  * views sized exactly to their regions pass through unchanged: the output
    equals a brute-force 2x2 unshuffle of the hand-assembled canvas
    (channel 4c + 2dx + dy, high camera on top, wrist cameras bottom-left /
    bottom-right), u8 read as v / 255;
  * a constant view stays constant at every scale (normalised taps, to
    the rounding of float32 weights);
  * interior pixels equal torch's antialiased bilinear resize (PIL's
    triangle filter) to the rounded cover size followed by the centre crop;
  * the border rule: taps outside the image are clamped, not dropped (the
    first pixel of a 2x shrink is (p0 + 0.75 p1 + 0.25 p2) / 2, where
    dropping them would give (0.75 p0 + 0.75 p1 + 0.25 p2) / 1.75);
  * the cover-and-crop geometry: a view twice the region's aspect at scale 1
    is its centre columns, the crop rounding down.
The oracle convolution (oracle.conv_2d, ggml_conv_2d_direct) equals torch's
float64 conv2d over strides, paddings and dilations, and a brute-force loop
on a tiny case.  CONV_2D graphs import through wamx_graph_from_ggml and pass
supports_op; malformed ones are refused.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import ggml_mirror as gm


def unshuffle_brute(canvas):
    h, w, _ = canvas.shape
    out = np.zeros((12, h // 2, w // 2))
    for c in range(3):
        for dx in range(2):
            for dy in range(2):
                for y in range(h // 2):
                    for x in range(w // 2):
                        out[4 * c + 2 * dx + dy, y, x] = canvas[2 * y + dy, 2 * x + dx, c] * 2 - 1
    return out


def test_identity_views_give_the_layout(orc):
    rng = np.random.default_rng(1)
    W, H = 16, 12
    top = rng.random((6, 16, 3)).astype(np.float32)
    bl = rng.integers(0, 256, (6, 8, 3)).astype(np.uint8)
    br = rng.random((6, 8, 3)).astype(np.float32)
    got = orc.compose_and_patchify([top, bl, br], W, H)
    canvas = np.zeros((H, W, 3))
    canvas[:6] = top
    canvas[6:, :8] = bl.astype(np.float32) * np.float32(1 / 255)
    canvas[6:, 8:] = br
    assert np.array_equal(got, unshuffle_brute(canvas))


@pytest.mark.parametrize("size", [(7, 5), (64, 48), (33, 90), (640, 480)])
def test_constant_views_stay_constant(orc, size):
    w, h = size
    views = [np.full((h, w, 3), v, np.float32) for v in (0.25, 0.5, 0.875)]
    got = orc.compose_and_patchify(views, 32, 24)
    canvas = np.zeros((24, 32, 3))
    canvas[:12], canvas[12:, :16], canvas[12:, 16:] = 0.25, 0.5, 0.875
    # float32 weights normalise to 1 within their rounding
    assert np.allclose(got, unshuffle_brute(canvas), rtol=0, atol=2e-6)


def _torch_cover_crop(img, dst_w, dst_h, rw, rh):
    t = torch.from_numpy(np.ascontiguousarray(img.transpose(2, 0, 1)[None]).astype(np.float64))
    r = torch.nn.functional.interpolate(t, size=(rh, rw), mode="bilinear", align_corners=False, antialias=True)
    cx, cy = (rw - dst_w) // 2, (rh - dst_h) // 2
    return r[0, :, cy:cy + dst_h, cx:cx + dst_w].numpy().transpose(1, 2, 0)


@pytest.mark.parametrize("src,dst", [((64, 48), (32, 24)), ((100, 60), (40, 24)), ((30, 20), (45, 30)),
                                     ((640, 480), (384, 160)), ((13, 11), (40, 24))])
def test_interior_matches_torch_antialiased_bilinear(orc, src, dst):
    rng = np.random.default_rng(src[0] * dst[0])
    img = rng.random((src[1], src[0], 3)).astype(np.float32)
    got = orc.resize_center_crop(img, *dst)
    f = np.float32
    s = max(f(dst[0]) / f(src[0]), f(dst[1]) / f(src[1]))
    rw, rh = int(np.floor(f(src[0]) * s + 0.5)), int(np.floor(f(src[1]) * s + 0.5))
    want = _torch_cover_crop(img, dst[0], dst[1], rw, rh)
    # interior: more than the filter support away from the image edges
    sup_x, sup_y = max(1.0, src[0] / rw), max(1.0, src[1] / rh)
    mx, my = int(np.ceil((sup_x + 1) * rw / src[0])) + 1, int(np.ceil((sup_y + 1) * rh / src[1])) + 1
    cx, cy = (rw - dst[0]) // 2, (rh - dst[1]) // 2
    xs = [x for x in range(dst[0]) if mx <= x + cx < rw - mx]
    ys = [y for y in range(dst[1]) if my <= y + cy < rh - my]
    assert xs and ys
    # The filter centres are float32 (as the reference computes them), torch's
    # double: at source coordinates near 640 that moves a centre by ~4e-5 px.
    assert np.allclose(got[np.ix_(ys, xs)], want[np.ix_(ys, xs)], rtol=0, atol=5e-5)


def test_border_taps_are_clamped(orc):
    rng = np.random.default_rng(3)
    img = rng.random((8, 16, 3)).astype(np.float32)          # 16 x 8 -> 8 x 4: a 2x shrink
    got = orc.resize_center_crop(img, 8, 4)
    row = img[:, :3, :].astype(np.float64)                  # y handled below: compare after the x pass
    # x pass at output 0, then y pass at output 0: both use (p0 + 0.75 p1 + 0.25 p2) / 2
    wx = np.array([1.0, 0.75, 0.25]) / 2
    want = np.einsum("yxc,x->yc", img[:3, :3, :].astype(np.float64), wx)
    want = np.einsum("yc,y->c", want, wx)
    assert np.allclose(got[0, 0], want, rtol=0, atol=1e-7)
    dropped = np.array([0.75, 0.75, 0.25]) / 1.75
    assert not np.allclose(got[0, 0], np.einsum("yc,y->c", np.einsum("yxc,x->yc", row[:3], dropped), dropped),
                           atol=1e-4)
    # the interior of a 2x shrink is the [1, 3, 3, 1] / 8 filter
    k = np.array([1, 3, 3, 1]) / 8
    want_in = np.einsum("yxc,y,x->c", img[1:5, 3:7, :].astype(np.float64), k, k)
    assert np.allclose(got[1, 2], want_in, rtol=0, atol=1e-7)


@pytest.mark.parametrize("w", [16, 17, 19])
def test_cover_then_centre_crop(orc, w):
    rng = np.random.default_rng(w)
    img = rng.random((6, w, 3)).astype(np.float32)          # region 8 x 6: scale max(8/w, 1) = 1
    got = orc.resize_center_crop(img, 8, 6)
    c = (w - 8) // 2
    assert np.allclose(got, img[:, c:c + 8], rtol=0, atol=0)


@pytest.mark.parametrize("s,p,d", [(1, 0, 1), (1, 1, 1), (2, 0, 1), (2, 1, 1), (1, 2, 2), (3, 1, 2)])
def test_conv_oracle_matches_torch(orc, s, p, d):
    rng = np.random.default_rng(s * 100 + p * 10 + d)
    k = rng.standard_normal((5, 4, 3, 3))
    x = rng.standard_normal((2, 4, 13, 11))
    got = orc.conv_2d(k, x, s, s, p, p, d, d)
    want = torch.nn.functional.conv2d(torch.from_numpy(x), torch.from_numpy(k), stride=s, padding=p,
                                      dilation=d).numpy()
    assert got.shape == want.shape
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def test_conv_oracle_brute_force_asymmetric(orc):
    rng = np.random.default_rng(7)
    k = rng.standard_normal((2, 3, 2, 3))
    x = rng.standard_normal((1, 3, 5, 6))
    s0, s1, p0, p1, d0, d1 = 2, 1, 1, 0, 1, 2
    got = orc.conv_2d(k, x, s0, s1, p0, p1, d0, d1)
    OW = (6 + 2 * p0 - d0 * 2 - 1) // s0 + 1
    OH = (5 + 2 * p1 - d1 * 1 - 1) // s1 + 1
    want = np.zeros((1, 2, OH, OW))
    for oc in range(2):
        for oy in range(OH):
            for ox in range(OW):
                acc = 0.0
                for ic in range(3):
                    for ky in range(2):
                        for kx in range(3):
                            iy, ix = oy * s1 - p1 + ky * d1, ox * s0 - p0 + kx * d0
                            if 0 <= iy < 5 and 0 <= ix < 6:
                                acc += k[oc, ic, ky, kx] * x[0, ic, iy, ix]
                want[0, oc, oy, ox] = acc
    assert np.allclose(got, want, rtol=1e-12, atol=1e-12)


def _import(wx, out):
    lib = wx.load()
    graph = gm.Graph()
    graph.expand(out)
    gm.place(graph.tensors(), 1 << 30, 1 << 30)
    arr, nodes, keep = gm.describe(graph)
    ctx = lib.wamx_init(len(arr) + 16)
    g = lib.wamx_graph_from_ggml(ctx, arr, len(arr), nodes, len(nodes))
    return lib, ctx, g, graph, keep


def test_conv_graph_imports_and_is_supported(wx):
    k = gm.new_tensor("bf16", 3, 3, 12, 160, name="vae.enc.in.weight")
    x = gm.new_tensor("bf16", 192, 160, 12, 1, name="patches")
    b = gm.new_tensor("bf16", 160, name="vae.enc.in.bias")
    y = gm.add(gm.conv_2d_direct(k, x, 1, 1, 1, 1, 1, 1), gm.reshape(b, 1, 1, 160, 1))
    lib, ctx, g, graph, _keep = _import(wx, y)
    try:
        assert g, wx.last_error()
        ops = [graph.nodes[i].op for i in range(lib.wamx_graph_n_nodes(g))]
        assert "CONV_2D" in ops
        bad = [i for i in range(len(ops)) if not lib.wamx_backend_supports_op(None, lib.wamx_graph_node(g, i))]
        assert not bad, [ops[i] for i in bad]
        conv = lib.wamx_graph_node(g, ops.index("CONV_2D"))
        assert list(conv.contents.ne) == [192, 160, 160, 1]
    finally:
        lib.wamx_free(ctx)


def test_conv_constructor_and_refusals(wx):
    lib = wx.load()
    ctx = lib.wamx_init(64)
    try:
        k = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 3, 3, 8, 16)
        x = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 49, 41, 8, 2)
        y = lib.wamx_conv_2d_direct(ctx, k, x, 2, 2, 0, 0, 1, 1)
        assert y and list(y.contents.ne) == [24, 20, 16, 2] and y.contents.type == wx.TYPE_BF16
        assert lib.wamx_backend_supports_op(None, y)
        xf = lib.wamx_new_tensor_4d(ctx, wx.TYPE_F32, 49, 41, 8, 2)
        assert not lib.wamx_conv_2d_direct(ctx, k, xf, 1, 1, 1, 1, 1, 1)       # mixed types
        assert "types" in wx.last_error()
        x7 = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 49, 41, 7, 2)
        assert not lib.wamx_conv_2d_direct(ctx, k, x7, 1, 1, 1, 1, 1, 1)       # channel mismatch
        assert not lib.wamx_conv_2d_direct(ctx, k, x, 0, 1, 1, 1, 1, 1)        # stride 0
        small = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 2, 2, 8, 1)
        assert not lib.wamx_conv_2d_direct(ctx, k, small, 1, 1, 0, 0, 1, 1)   # no output pixel
    finally:
        lib.wamx_free(ctx)


def test_preprocess_views_refusals_without_a_device(wx):
    lib = wx.load()
    assert not lib.wamx_preprocessor_create(None)
    assert "null backend" in wx.last_error()
