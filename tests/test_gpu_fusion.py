"""Row fusion in the graph executor: a LINEAR on a few tokens followed by the
row ops that consume its output (LayerNorm / adaLN modulation of the residual
stream; RMSNorm + RoPE of the Q and K column ranges and the V^T copy) runs as
the skinny GEMM plus one reduce that applies the row ops; on eight 48-token
chunks (384 rows, the batched denoise step) as the K-sliced 128 x 128 GEMM
plus the same reduce, with chunk-major Q/K and V^T destinations.  The fused graph
must produce the same bits as the standalone ops launched one at a time
(wamx_op_linear, wamx_op_norm_modulation_bf16 / wamx_op_layer_norm_bf16,
wamx_op_qk_norm_rope and a host transpose for V^T), which the per-op tests
hold to the oracle.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

D, H, DH = 3072, 24, 128


class Graph:
    """A no-alloc context whose tensors are placed in one backend buffer."""

    def __init__(self, wx, be):
        self.wx, self.be, self.lib = wx, be, be.lib
        self.ctx = self.lib.wamx_init(256)
        self.buf = None

    def t(self, typ, *ne):
        return getattr(self.lib, f"wamx_new_tensor_{len(ne)}d")(self.ctx, typ, *ne)

    def alloc(self):
        self.buf = self.lib.wamx_backend_alloc_ctx_tensors(self.ctx, self.be.ptr)
        assert self.buf, self.wx.last_error()

    def set(self, t, a):
        a = np.ascontiguousarray(a)
        self.wx.check(self.lib.wamx_backend_tensor_set(t, a.ctypes.data, 0, a.nbytes), "tensor_set")

    def get(self, t, dtype, shape):
        a = np.empty(shape, dtype)
        self.wx.check(self.lib.wamx_backend_tensor_get(t, a.ctypes.data, 0, a.nbytes), "tensor_get")
        return a

    def compute(self, *outs):
        g = self.lib.wamx_new_graph(self.ctx, 256)
        for o in outs:
            self.lib.wamx_build_forward_expand(g, o)
        self.wx.check(self.lib.wamx_backend_graph_compute(self.be.ptr, g), "graph_compute")
        self.be.sync()

    def close(self):
        if self.buf:
            self.lib.wamx_buffer_free(self.buf)
        self.lib.wamx_free(self.ctx)


def data(t):
    return t.contents.data


@pytest.mark.parametrize("T", [48, 17, 1, 384])
@pytest.mark.parametrize("kind", ["modulation", "layer_norm"])
def test_linear_then_norm_is_bit_exact(wx, be, rng, T, kind):
    print(f"fusion linear->norm {kind} T={T}", flush=True)
    lib = be.lib
    g = Graph(wx, be)
    try:
        w = g.t(wx.TYPE_BF16, D, D)
        x = g.t(wx.TYPE_BF16, D, T)
        b = g.t(wx.TYPE_BF16, D)
        h = g.t(wx.TYPE_BF16, D, T)
        gate = g.t(wx.TYPE_F32, D)
        y = lib.wamx_linear(g.ctx, w, x, b, wx.EPI_BIAS_GATED, h, gate)
        if kind == "modulation":
            sc, sh = g.t(wx.TYPE_F32, D), g.t(wx.TYPE_F32, D)
            n = lib.wamx_norm_modulation_bf16(g.ctx, y, sc, sh, 1e-6)
        else:
            sc, sh = g.t(wx.TYPE_BF16, D), g.t(wx.TYPE_BF16, D)
            n = lib.wamx_layer_norm_bf16(g.ctx, y, sc, sh, 1e-6)
        g.alloc()
        hw = wx.f32_to_bf16(rng.standard_normal(D * D).astype(np.float32) * 0.02)
        hx = wx.f32_to_bf16(rng.standard_normal(D * T).astype(np.float32))
        hb = wx.f32_to_bf16(rng.standard_normal(D).astype(np.float32) * 0.02)
        hh = wx.f32_to_bf16(rng.standard_normal(D * T).astype(np.float32))
        hg = (rng.standard_normal(D) * 0.5).astype(np.float32)
        if kind == "modulation":
            hsc, hsh = (rng.standard_normal(D) * 0.1).astype(np.float32), (rng.standard_normal(D) * 0.1).astype(np.float32)
        else:
            hsc = wx.f32_to_bf16(1.0 + rng.standard_normal(D).astype(np.float32) * 0.1)
            hsh = wx.f32_to_bf16(rng.standard_normal(D).astype(np.float32) * 0.1)
        for t, a in ((w, hw), (x, hx), (b, hb), (h, hh), (gate, hg), (sc, hsc), (sh, hsh)):
            g.set(t, a)
        g.compute(n)
        got_y = g.get(y, np.uint16, (T, D))
        got_n = g.get(n, np.uint16, (T, D))

        ref_y, ref_n = be.empty(T * D * 2), be.empty(T * D * 2)
        wx.check(lib.wamx_op_linear(be.ptr, data(w), data(x), wx.TYPE_BF16, data(b), wx.EPI_BIAS_GATED, data(h),
                                    C.cast(data(gate), C.POINTER(C.c_float)), ref_y.ptr, D, T, D))
        if kind == "modulation":
            wx.check(lib.wamx_op_norm_modulation_bf16(be.ptr, ref_y.ptr, D, C.cast(data(sc), C.POINTER(C.c_float)),
                                                      C.cast(data(sh), C.POINTER(C.c_float)), 0, ref_n.ptr, T, D,
                                                      1e-6))
        else:
            wx.check(lib.wamx_op_layer_norm_bf16(be.ptr, ref_y.ptr, D, data(sc), data(sh), ref_n.ptr, T, D, 1e-6))
        be.sync()
        assert np.array_equal(got_y, ref_y.download(np.uint16, (T, D)))
        assert np.array_equal(got_n, ref_n.download(np.uint16, (T, D)))
    finally:
        g.close()


@pytest.mark.parametrize("T", [48, 5, 1])
def test_qkv_split_is_bit_exact(wx, be, rng, T):
    print(f"fusion qkv T={T}", flush=True)
    lib = be.lib
    g = Graph(wx, be)
    try:
        w = g.t(wx.TYPE_BF16, D, 3 * D)
        x = g.t(wx.TYPE_BF16, D, T)
        b = g.t(wx.TYPE_BF16, 3 * D)
        nq, nk = g.t(wx.TYPE_BF16, D), g.t(wx.TYPE_BF16, D)
        pos = g.t(wx.TYPE_I32, T)
        tpad = (T + 3) // 4 * 4
        vraw = g.t(wx.TYPE_BF16, tpad, DH, H)
        qkv = lib.wamx_linear(g.ctx, w, x, b, wx.EPI_BIAS, None, None)
        pitch = qkv.contents.nb[1]
        q = lib.wamx_qk_norm_rope(g.ctx, lib.wamx_view_2d(g.ctx, qkv, D, T, pitch, 0), nq,
                                  g.t(wx.TYPE_BF16, DH, T, H), 0, 0, pos, None, None, 1e-6, 10000.0)
        k = lib.wamx_qk_norm_rope(g.ctx, lib.wamx_view_2d(g.ctx, qkv, D, T, pitch, 2 * D), nk,
                                  g.t(wx.TYPE_BF16, DH, T, H), 0, 0, pos, None, None, 1e-6, 10000.0)
        vsrc = lib.wamx_permute(g.ctx, lib.wamx_view_3d(g.ctx, qkv, DH, H, T, DH * 2, pitch, 4 * D), 1, 2, 0, 3)
        vdst = lib.wamx_view_3d(g.ctx, vraw, T, DH, H, vraw.contents.nb[1], vraw.contents.nb[2], 0)
        v = lib.wamx_cpy(g.ctx, vsrc, vdst)
        g.alloc()
        hw = wx.f32_to_bf16(rng.standard_normal(3 * D * D).astype(np.float32) * 0.02)
        hx = wx.f32_to_bf16(rng.standard_normal(D * T).astype(np.float32))
        hb = wx.f32_to_bf16(rng.standard_normal(3 * D).astype(np.float32) * 0.02)
        hnq = wx.f32_to_bf16(1.0 + rng.standard_normal(D).astype(np.float32) * 0.1)
        hnk = wx.f32_to_bf16(1.0 + rng.standard_normal(D).astype(np.float32) * 0.1)
        hpos = np.arange(1, T + 1, dtype=np.int32)
        for t, a in ((w, hw), (x, hx), (b, hb), (nq, hnq), (nk, hnk), (pos, hpos),
                     (vraw, np.zeros(tpad * DH * H, np.uint16))):
            g.set(t, a)
        g.compute(q, k, v)
        got_qkv = g.get(qkv, np.uint16, (T, 3 * D))
        got_q = g.get(q, np.uint16, (H, T, DH))
        got_k = g.get(k, np.uint16, (H, T, DH))
        got_vt = g.get(vraw, np.uint16, (H, DH, tpad))[:, :, :T]

        ref_qkv, ref_q, ref_k = be.empty(T * 3 * D * 2), be.empty(T * D * 2), be.empty(T * D * 2)
        wx.check(lib.wamx_op_linear(be.ptr, data(w), data(x), wx.TYPE_BF16, data(b), wx.EPI_BIAS, None, None,
                                    ref_qkv.ptr, 3 * D, T, D))
        pp = C.cast(data(pos), C.POINTER(C.c_int32))
        wx.check(lib.wamx_op_qk_norm_rope(be.ptr, ref_qkv.ptr, 3 * D, data(nq), ref_q.ptr, H, DH, T, T, 0, 0, pp,
                                          None, None, 1e-6, 10000.0))
        wx.check(lib.wamx_op_qk_norm_rope(be.ptr, ref_qkv.ptr + 2 * D, 3 * D, data(nk), ref_k.ptr, H, DH, T, T, 0,
                                          0, pp, None, None, 1e-6, 10000.0))
        be.sync()
        rq = ref_qkv.download(np.uint16, (T, 3 * D))
        assert np.array_equal(got_qkv, rq)
        assert np.array_equal(got_q, ref_q.download(np.uint16, (H, T, DH)))
        assert np.array_equal(got_k, ref_k.download(np.uint16, (H, T, DH)))
        assert np.array_equal(got_vt, rq[:, 2 * D:].reshape(T, H, DH).transpose(1, 2, 0))
    finally:
        g.close()


def test_qkv_row_ops_apart_are_not_fused(wx, be, rng):
    """A 48-token QKV product whose K norm and V^T store follow it but whose
    Q norm comes after another launch: the fused reduce writes the product
    only in its segments' columns, so the K and V segments alone (two thirds
    of the columns) must not be fused, and the Q norm must read the product
    as written.  The product's output holds a NaN pattern before the run; all
    three results are compared bit for bit with the standalone ops."""
    T = 48
    print(f"fusion qkv row ops apart T={T}", flush=True)
    lib = be.lib
    g = Graph(wx, be)
    try:
        w = g.t(wx.TYPE_BF16, D, 3 * D)
        x = g.t(wx.TYPE_BF16, D, T)
        b = g.t(wx.TYPE_BF16, 3 * D)
        nq, nk = g.t(wx.TYPE_BF16, D), g.t(wx.TYPE_BF16, D)
        pos = g.t(wx.TYPE_I32, T)
        vraw = g.t(wx.TYPE_BF16, 64, DH, H)
        other_in = g.t(wx.TYPE_BF16, D, T)
        qkv = lib.wamx_linear(g.ctx, w, x, b, wx.EPI_BIAS, None, None)
        pitch = qkv.contents.nb[1]
        k = lib.wamx_qk_norm_rope(g.ctx, lib.wamx_view_2d(g.ctx, qkv, D, T, pitch, 2 * D), nk,
                                  g.t(wx.TYPE_BF16, DH, T, H), 0, 0, pos, None, None, 1e-6, 10000.0)
        vsrc = lib.wamx_permute(g.ctx, lib.wamx_view_3d(g.ctx, qkv, DH, H, T, DH * 2, pitch, 4 * D), 1, 2, 0, 3)
        vdst = lib.wamx_view_3d(g.ctx, vraw, T, DH, H, vraw.contents.nb[1], vraw.contents.nb[2], 0)
        v = lib.wamx_cpy(g.ctx, vsrc, vdst)
        other = lib.wamx_gelu(g.ctx, other_in)  # a launch between the V^T store and the Q norm
        q = lib.wamx_qk_norm_rope(g.ctx, lib.wamx_view_2d(g.ctx, qkv, D, T, pitch, 0), nq,
                                  g.t(wx.TYPE_BF16, DH, T, H), 0, 0, pos, None, None, 1e-6, 10000.0)
        g.alloc()
        hw = wx.f32_to_bf16(rng.standard_normal(3 * D * D).astype(np.float32) * 0.02)
        hx = wx.f32_to_bf16(rng.standard_normal(D * T).astype(np.float32))
        hb = wx.f32_to_bf16(rng.standard_normal(3 * D).astype(np.float32) * 0.02)
        hnq = wx.f32_to_bf16(1.0 + rng.standard_normal(D).astype(np.float32) * 0.1)
        hnk = wx.f32_to_bf16(1.0 + rng.standard_normal(D).astype(np.float32) * 0.1)
        hpos = np.arange(1, T + 1, dtype=np.int32)
        for t, a in ((w, hw), (x, hx), (b, hb), (nq, hnq), (nk, hnk), (pos, hpos), (other_in, hx),
                     (vraw, np.zeros(64 * DH * H, np.uint16)), (qkv, np.full(T * 3 * D, 0x7FC1, np.uint16))):
            g.set(t, a)
        g.compute(k, v, other, q)
        got_qkv = g.get(qkv, np.uint16, (T, 3 * D))
        got_q = g.get(q, np.uint16, (H, T, DH))
        got_k = g.get(k, np.uint16, (H, T, DH))
        got_vt = g.get(vraw, np.uint16, (H, DH, 64))[:, :, :T]

        ref_qkv, ref_q, ref_k = be.empty(T * 3 * D * 2), be.empty(T * D * 2), be.empty(T * D * 2)
        wx.check(lib.wamx_op_linear(be.ptr, data(w), data(x), wx.TYPE_BF16, data(b), wx.EPI_BIAS, None, None,
                                    ref_qkv.ptr, 3 * D, T, D))
        pp = C.cast(data(pos), C.POINTER(C.c_int32))
        wx.check(lib.wamx_op_qk_norm_rope(be.ptr, ref_qkv.ptr, 3 * D, data(nq), ref_q.ptr, H, DH, T, T, 0, 0, pp,
                                          None, None, 1e-6, 10000.0))
        wx.check(lib.wamx_op_qk_norm_rope(be.ptr, ref_qkv.ptr + 2 * D, 3 * D, data(nk), ref_k.ptr, H, DH, T, T, 0,
                                          0, pp, None, None, 1e-6, 10000.0))
        be.sync()
        rq = ref_qkv.download(np.uint16, (T, 3 * D))
        assert np.array_equal(got_qkv, rq), "the product's output"
        assert np.array_equal(got_q, ref_q.download(np.uint16, (H, T, DH))), "Q norm after another launch"
        assert np.array_equal(got_k, ref_k.download(np.uint16, (H, T, DH)))
        assert np.array_equal(got_vt, rq[:, 2 * D:].reshape(T, H, DH).transpose(1, 2, 0))
    finally:
        g.close()


@pytest.mark.parametrize("tpad", [52, 64])
def test_qkv_split_chunked_is_bit_exact(wx, be, rng, tpad):
    """Eight chunks of 48 tokens: Q and K into [dh, 48, H, 8], V^T into
    [pad, dh, H, 8], each chunk's RoPE positions 1..48.  With V^T rows of
    64 keys (16-byte aligned) the reduce's V^T segment runs in blocks of 8
    tokens stored as 16-byte runs; with 52 it stores one token row at a
    time."""
    B, Tc = 8, 48
    T = B * Tc
    print(f"fusion qkv chunked B={B} Tc={Tc} tpad={tpad}", flush=True)
    lib = be.lib
    g = Graph(wx, be)
    try:
        w = g.t(wx.TYPE_BF16, D, 3 * D)
        x = g.t(wx.TYPE_BF16, D, T)
        b = g.t(wx.TYPE_BF16, 3 * D)
        nq, nk = g.t(wx.TYPE_BF16, D), g.t(wx.TYPE_BF16, D)
        pos = g.t(wx.TYPE_I32, Tc)
        vraw = g.t(wx.TYPE_BF16, tpad, DH, H, B)
        qkv = lib.wamx_linear(g.ctx, w, x, b, wx.EPI_BIAS, None, None)
        pitch = qkv.contents.nb[1]
        q = lib.wamx_qk_norm_rope(g.ctx, lib.wamx_view_2d(g.ctx, qkv, D, T, pitch, 0), nq,
                                  g.t(wx.TYPE_BF16, DH, Tc, H, B), 0, 0, pos, None, None, 1e-6, 10000.0)
        k = lib.wamx_qk_norm_rope(g.ctx, lib.wamx_view_2d(g.ctx, qkv, D, T, pitch, 2 * D), nk,
                                  g.t(wx.TYPE_BF16, DH, Tc, H, B), 0, 0, pos, None, None, 1e-6, 10000.0)
        vsrc = lib.wamx_permute(g.ctx, lib.wamx_view_4d(g.ctx, qkv, DH, H, Tc, B, DH * 2, pitch, pitch * Tc, 4 * D),
                                1, 2, 0, 3)
        vr = vraw.contents
        vdst = lib.wamx_view_4d(g.ctx, vraw, Tc, DH, H, B, vr.nb[1], vr.nb[2], vr.nb[3], 0)
        v = lib.wamx_cpy(g.ctx, vsrc, vdst)
        g.alloc()
        hw = wx.f32_to_bf16(rng.standard_normal(3 * D * D).astype(np.float32) * 0.02)
        hx = wx.f32_to_bf16(rng.standard_normal(D * T).astype(np.float32))
        hb = wx.f32_to_bf16(rng.standard_normal(3 * D).astype(np.float32) * 0.02)
        hnq = wx.f32_to_bf16(1.0 + rng.standard_normal(D).astype(np.float32) * 0.1)
        hnk = wx.f32_to_bf16(1.0 + rng.standard_normal(D).astype(np.float32) * 0.1)
        hpos = np.arange(1, Tc + 1, dtype=np.int32)
        for t, a in ((w, hw), (x, hx), (b, hb), (nq, hnq), (nk, hnk), (pos, hpos),
                     (vraw, np.zeros(tpad * DH * H * B, np.uint16))):
            g.set(t, a)
        g.compute(q, k, v)
        got_qkv = g.get(qkv, np.uint16, (T, 3 * D))
        got_q = g.get(q, np.uint16, (B, H, Tc, DH))
        got_k = g.get(k, np.uint16, (B, H, Tc, DH))
        got_vt = g.get(vraw, np.uint16, (B, H, DH, tpad))[..., :Tc]

        ref_qkv, ref_q, ref_k = be.empty(T * 3 * D * 2), be.empty(Tc * D * 2), be.empty(Tc * D * 2)
        wx.check(lib.wamx_op_linear(be.ptr, data(w), data(x), wx.TYPE_BF16, data(b), wx.EPI_BIAS, None, None,
                                    ref_qkv.ptr, 3 * D, T, D))
        be.sync()
        rq = ref_qkv.download(np.uint16, (T, 3 * D))
        assert np.array_equal(got_qkv, rq)
        pp = C.cast(data(pos), C.POINTER(C.c_int32))
        for c in range(B):
            row0 = ref_qkv.ptr + c * Tc * 3 * D * 2
            wx.check(lib.wamx_op_qk_norm_rope(be.ptr, row0, 3 * D, data(nq), ref_q.ptr, H, DH, Tc, Tc, 0, 0, pp,
                                              None, None, 1e-6, 10000.0))
            wx.check(lib.wamx_op_qk_norm_rope(be.ptr, row0 + 2 * D, 3 * D, data(nk), ref_k.ptr, H, DH, Tc, Tc, 0,
                                              0, pp, None, None, 1e-6, 10000.0))
            be.sync()
            assert np.array_equal(got_q[c], ref_q.download(np.uint16, (H, Tc, DH))), f"Q chunk {c}"
            assert np.array_equal(got_k[c], ref_k.download(np.uint16, (H, Tc, DH))), f"K chunk {c}"
            vt = rq[c * Tc:(c + 1) * Tc, 2 * D:].reshape(Tc, H, DH).transpose(1, 2, 0)
            assert np.array_equal(got_vt[c], vt), f"V^T chunk {c}"
    finally:
        g.close()


@pytest.mark.parametrize("T,k0", [(3072, 1), (512, 0), (3073, 0), (130, 0), (130, 7), (100, 3), (40, 0)])
def test_v_transpose_store_is_exact(wx, be, rng, T, k0):
    """The V^T store of the attention caches (CPY of a permuted token-major
    view into [head][dim][token] at token offset k0): the tiled transposing
    copy (T >= 64; 16-byte accesses, the destination offset k0 taken as a
    shift of the 16-byte grid, ragged first and last tiles) and the generic
    strided copy give the transposed bits."""
    print(f"V^T store T={T} k0={k0}", flush=True)
    lib = be.lib
    g = Graph(wx, be)
    try:
        width = 3 * D
        src = g.t(wx.TYPE_BF16, width, T)
        ld = (k0 + T + 63) // 64 * 64
        vraw = g.t(wx.TYPE_BF16, ld, DH, H)
        pitch = src.contents.nb[1]
        vsrc = lib.wamx_permute(g.ctx, lib.wamx_view_3d(g.ctx, src, DH, H, T, DH * 2, pitch, 4 * D), 1, 2, 0, 3)
        vdst = lib.wamx_view_3d(g.ctx, vraw, T, DH, H, vraw.contents.nb[1], vraw.contents.nb[2], 2 * k0)
        v = lib.wamx_cpy(g.ctx, vsrc, vdst)
        g.alloc()
        hs = wx.f32_to_bf16(rng.standard_normal(width * T).astype(np.float32)).reshape(T, width)
        fill = np.full(ld * DH * H, 0x7777, np.uint16)
        g.set(src, hs)
        g.set(vraw, fill)
        g.compute(v)
        got = g.get(vraw, np.uint16, (H, DH, ld))
        want = fill.reshape(H, DH, ld).copy()
        want[:, :, k0:k0 + T] = hs[:, 2 * D:].reshape(T, H, DH).transpose(1, 2, 0)
        assert np.array_equal(got, want)
    finally:
        g.close()


def _f32_chains(wx, lib, g, rows, cols):
    """The F32 profile's modulated norm (mot.cpp:154-158: norm + norm * scale
    + shift, scale and shift views of the modulation rows) and gated residual
    (mot.cpp:161-164: residual + branch * gate view), unfused ggml ops."""
    x = g.t(wx.TYPE_F32, cols, rows)
    comb = g.t(wx.TYPE_F32, cols, 6, 1)
    res = g.t(wx.TYPE_F32, cols, rows)
    br = g.t(wx.TYPE_F32, cols, rows)
    part = [lib.wamx_view_2d(g.ctx, comb, cols, 1, comb.contents.nb[2], i * comb.contents.nb[1]) for i in range(6)]
    n = lib.wamx_norm(g.ctx, x, 1e-6)
    y = lib.wamx_add(g.ctx, lib.wamx_add(g.ctx, n, lib.wamx_mul(g.ctx, n, part[1])), part[0])
    out = lib.wamx_add(g.ctx, res, lib.wamx_mul(g.ctx, br, part[2]))
    return x, comb, res, br, y, out


def test_f32_profile_fusions(wx, be, orc, rng):
    """The F32 chains run as norm_modulation_f32 and gated_residual_f32
    (p7-fusions.patch:173-245): the graph's results equal the standalone
    fused kernels bit for bit and the oracle's restatement of them; with the
    fusions switched off the unfused ops agree with the oracle too."""
    import os
    rows, cols = 2048, 3072
    print("f32 profile fusions", flush=True)
    xv = (rng.standard_normal((rows, cols)) * 2 + 0.5).astype(np.float32)
    cv = (rng.standard_normal((1, 6, cols)) * 0.1).astype(np.float32)
    rv = rng.standard_normal((rows, cols)).astype(np.float32)
    bv = rng.standard_normal((rows, cols)).astype(np.float32)
    ref_y = orc.norm_mod_f32(xv, cv[0, 1], cv[0, 0], 1e-6)
    ref_out = orc.gated_residual_f32(rv, bv, cv[0, 2])
    results = {}
    backends = {"fused": be}
    os.environ["WAMX_DISABLE_NORM_MODULATION_FUSION"] = "1"
    os.environ["WAMX_DISABLE_GATED_RESIDUAL_FUSION"] = "1"
    try:
        backends["unfused"] = wx.Backend(0)
    finally:
        del os.environ["WAMX_DISABLE_NORM_MODULATION_FUSION"]
        del os.environ["WAMX_DISABLE_GATED_RESIDUAL_FUSION"]
    for key, b in backends.items():
        g = Graph(wx, b)
        try:
            x, comb, res, br, y, out = _f32_chains(wx, b.lib, g, rows, cols)
            g.alloc()
            for t, a in ((x, xv), (comb, cv), (res, rv), (br, bv)):
                g.set(t, a)
            g.compute(y, out)
            results[key] = (g.get(y, np.float32, (rows, cols)), g.get(out, np.float32, (rows, cols)))
        finally:
            g.close()
    backends["unfused"].close()
    # the standalone fused kernels on the same inputs
    lib = be.lib
    dx, ds, dsh, dy = be.array(xv), be.array(cv[0, 1].copy()), be.array(cv[0, 0].copy()), be.empty(xv.nbytes)
    wx.check(lib.wamx_op_norm_modulation_f32(be.ptr, dx.ptr, cols, ds.ptr, dsh.ptr, 0, dy.ptr, rows, cols, 1e-6))
    dr, db, dg, do = be.array(rv), be.array(bv), be.array(cv[0, 2].copy()), be.empty(rv.nbytes)
    wx.check(lib.wamx_op_gated_residual_f32(be.ptr, dr.ptr, db.ptr, dg.ptr, 0, do.ptr, rows, cols))
    k_y, k_out = dy.download(np.float32, (rows, cols)), do.download(np.float32, (rows, cols))
    f_y, f_out = results["fused"]
    u_y, u_out = results["unfused"]
    assert np.array_equal(f_y, k_y) and np.array_equal(f_out, k_out)
    assert np.array_equal(f_out, ref_out)            # exact: r + b*g rounded per op
    for got in (f_y, u_y):
        assert np.max(np.abs(got - ref_y)) <= 1e-4 * np.max(np.abs(ref_y))
    assert np.max(np.abs(u_out - ref_out)) <= 1e-6 * np.max(np.abs(ref_out))


@pytest.mark.parametrize("hilo", [False, True])
def test_qk_norm_rope_layer_chunks(wx, be, rng, hilo):
    """The Q/K norm over every layer's column block of a packed projection
    ([d, T, C] rows, layer c's at columns 2c·d), each layer with its own norm
    weight ([d, C]) and its own destination chunk (strided among a batch of
    two, or hi/lo planes 2c and 2c + 1), in one launch, equals C launches on
    the layer's columns with the layer's weight, bit for bit.  This is how
    the prompt graph fills every layer's prompt-key cache."""
    print(f"qk norm layer chunks hilo={hilo}", flush=True)
    lib = be.lib
    d, H, DH, T, C, B, cb = 512, 4, 128, 24, 3, 2, 1
    g = Graph(wx, be)
    try:
        kv = g.t(wx.TYPE_BF16, 2 * C * d, T)
        wts = g.t(wx.TYPE_BF16, d, C)
        x = lib.wamx_view_3d(g.ctx, kv, d, T, C, kv.contents.nb[1], 2 * d * 2, 0)
        if hilo:
            store = g.t(wx.TYPE_BF16, DH, T, H, 2 * C)
            node = lib.wamx_qk_norm_rope_hilo(g.ctx, x, wts, store, 0, 2, None, None, None, 1e-6, 10000.0)
        else:
            store = g.t(wx.TYPE_BF16, DH, T, H, C * B)
            nb = store.contents.nb
            dst = lib.wamx_view_4d(g.ctx, store, DH, T, H, C, nb[1], nb[2], nb[3] * B, nb[3] * cb)
            node = lib.wamx_qk_norm_rope(g.ctx, x, wts, dst, 0, 2, None, None, None, 1e-6, 10000.0)
        assert node, wx.last_error()
        g.alloc()
        g.set(kv, wx.f32_to_bf16(rng.standard_normal((T, 2 * C * d)).astype(np.float32)))
        g.set(wts, wx.f32_to_bf16((1.0 + 0.1 * rng.standard_normal((C, d))).astype(np.float32)))
        if not hilo:
            g.set(store, np.full(DH * T * H * C * B, 0x7FC0, np.uint16))  # NaN: untouched chunks stay NaN
        g.compute(node)
        plane = DH * T * H
        got = g.get(store, np.uint16, (plane * (2 * C if hilo else C * B),))
        for c in range(C):
            x_ptr, w_ptr = data(kv) + 2 * c * d * 2, data(wts) + c * d * 2
            if hilo:
                ref = be.empty(2 * plane * 2)
                wx.check(lib.wamx_op_qk_norm_rope_hilo(be.ptr, x_ptr, 2 * C * d, w_ptr, ref.ptr, ref.ptr + plane * 2, H,
                                                       DH, T, T, 0, 2, None, None, None, 1e-6, 10000.0))
                be.sync()
                assert np.array_equal(got[2 * c * plane:(2 * c + 2) * plane], ref.download(np.uint16, (2 * plane,))), c
            else:
                ref = be.empty(plane * 2)
                wx.check(lib.wamx_op_qk_norm_rope(be.ptr, x_ptr, 2 * C * d, w_ptr, ref.ptr, H, DH, T, T, 0, 2, None,
                                                  None, None, 1e-6, 10000.0))
                be.sync()
                k = c * B + cb
                assert np.array_equal(got[k * plane:(k + 1) * plane], ref.download(np.uint16, (plane,))), c
                other = c * B + (1 - cb)
                assert np.all(got[other * plane:(other + 1) * plane] == 0x7FC0), "wrote outside its chunk"
            ref.free()
    finally:
        g.close()
