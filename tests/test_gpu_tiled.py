"""The tiled weight buffer type: a 2-D bf16 weight placed there is stored in the
MFMA-tiled layout ([M/16][K/32] tiles of 1 KB, lane l of tile (g, q) holding
w[16g + l%16][32q + 8(l//16) .. +8]) and read by the few-token GEMM path.

Checks: the stored bytes are that permutation of the row-major weight;
set/get/copy convert both ways; ineligible shapes stay row-major; integer
products through tiled weights are exact (bf16 products and fp32 sums of small
integers are exact, so any tiling or split order must give the same bits); the
LINEAR epilogues and the fused split-K reduce agree with row-major weights; and
supports_op rejects tiled weights on more than 64 tokens.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_parity

pytestmark = pytest.mark.gpu


def tiled_bytes(w: np.ndarray) -> np.ndarray:
    """Row-major [M][K] -> the tiled order, as a flat uint16 array."""
    M, K = w.shape
    t = w.reshape(M // 16, 16, K // 32, 4, 8)           # [g][r][q][lg][e]
    return np.ascontiguousarray(t.transpose(0, 2, 3, 1, 4)).reshape(-1)  # [g][q][lg][r][e]


class Bufs:
    """Contexts placed in the tiled and the default buffer types of device 0."""

    def __init__(self, wx, be):
        self.wx, self.be, self.lib = wx, be, be.lib
        self.tctx = self.lib.wamx_init(64)
        self.pctx = self.lib.wamx_init(256)
        self.bufs = []

    def tiled(self, *ne):
        return getattr(self.lib, f"wamx_new_tensor_{len(ne)}d")(self.tctx, self.wx.TYPE_BF16, *ne)

    def plain(self, typ, *ne):
        return getattr(self.lib, f"wamx_new_tensor_{len(ne)}d")(self.pctx, typ, *ne)

    def alloc(self):
        lib = self.lib
        bt = lib.wamx_backend_alloc_ctx_tensors_from_buft(self.tctx, lib.wamx_backend_tiled_buffer_type(0))
        bp = lib.wamx_backend_alloc_ctx_tensors(self.pctx, self.be.ptr)
        assert bt and bp, self.wx.last_error()
        self.bufs += [bt, bp]

    def set(self, t, a):
        a = np.ascontiguousarray(a)
        self.wx.check(self.lib.wamx_backend_tensor_set(t, a.ctypes.data, 0, a.nbytes), "tensor_set")

    def get(self, t, dtype, shape):
        a = np.empty(shape, dtype)
        self.wx.check(self.lib.wamx_backend_tensor_get(t, a.ctypes.data, 0, a.nbytes), "tensor_get")
        return a

    def compute(self, *outs):
        g = self.lib.wamx_new_graph(self.pctx, 256)
        for o in outs:
            self.lib.wamx_build_forward_expand(g, o)
        self.wx.check(self.lib.wamx_backend_graph_compute(self.be.ptr, g), "graph_compute")
        self.be.sync()

    def close(self):
        for b in self.bufs:
            self.lib.wamx_buffer_free(b)
        self.lib.wamx_free(self.tctx)
        self.lib.wamx_free(self.pctx)


def test_layout_and_conversions(wx, be, rng):
    print("tiled buffer layout and conversions", flush=True)
    lib = be.lib
    B = Bufs(wx, be)
    try:
        M, K = 96, 160
        wt = B.tiled(K, M)
        odd = B.tiled(96, 40)            # M % 16 != 0: stays row-major
        wp = B.plain(wx.TYPE_BF16, K, M)
        back = B.plain(wx.TYPE_BF16, K, M)
        B.alloc()
        assert wt.contents.extra and not odd.contents.extra and not wp.contents.extra
        w = wx.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32)).reshape(M, K)
        B.set(wt, w)
        raw = np.empty(M * K, np.uint16)
        wx.check(lib.wamx_memcpy_d2h(be.ptr, raw.ctypes.data, wt.contents.data, raw.nbytes))
        assert np.array_equal(raw, tiled_bytes(w))
        assert np.array_equal(B.get(wt, np.uint16, (M, K)), w)
        part = np.empty(100, np.uint16)  # a range of the row-major view
        wx.check(lib.wamx_backend_tensor_get(wt, part.ctypes.data, 2 * 1000, part.nbytes))
        assert np.array_equal(part, w.reshape(-1)[1000:1100])
        wx.check(lib.wamx_backend_tensor_copy(wt, back))   # tiled -> row-major
        assert np.array_equal(B.get(back, np.uint16, (M, K)), w)
        w2 = wx.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32)).reshape(M, K)
        B.set(wp, w2)
        wx.check(lib.wamx_backend_tensor_copy(wp, wt))     # row-major -> tiled
        assert np.array_equal(B.get(wt, np.uint16, (M, K)), w2)
        # a tiled weight is written whole
        assert lib.wamx_backend_tensor_set(wt, w.ctypes.data, 0, 64) != wx.STATUS_SUCCESS
        o = wx.f32_to_bf16(rng.standard_normal(96 * 40).astype(np.float32)).reshape(40, 96)
        B.set(odd, o)
        raw = np.empty(o.size, np.uint16)
        wx.check(lib.wamx_memcpy_d2h(be.ptr, raw.ctypes.data, odd.contents.data, raw.nbytes))
        assert np.array_equal(raw, o.reshape(-1))
    finally:
        B.close()


# One-token shapes (the state token's projections) run the K-split plans of
# grids in rounds of 64 workgroups; the rest in rounds of 256.
@pytest.mark.parametrize("M,K,N", [(3072, 3072, 48), (9216, 3072, 48), (3072, 14336, 48), (14336, 3072, 1),
                                   (3072, 3072, 1), (9216, 3072, 1), (3072, 14336, 1),
                                   (3072, 3072, 17), (128, 96, 5)])
def test_integer_products_exact(wx, be, M, K, N):
    print(f"tiled integer product M={M} K={K} N={N}", flush=True)
    lib = be.lib
    rng = np.random.default_rng(M + 3 * K + 7 * N)
    w = rng.integers(-4, 5, (M, K))
    x = rng.integers(-4, 5, (N, K))
    B = Bufs(wx, be)
    try:
        wt = B.tiled(K, M)
        xt = B.plain(wx.TYPE_BF16, K, N)
        y = lib.wamx_mul_mat(B.pctx, wt, xt)
        B.alloc()
        assert wt.contents.extra
        B.set(wt, wx.f32_to_bf16(w.astype(np.float32)))
        B.set(xt, wx.f32_to_bf16(x.astype(np.float32)))
        B.compute(y)
        got = B.get(y, np.float32, (N, M))
        assert np.array_equal(got.astype(np.int64), x @ w.T)
    finally:
        B.close()


@pytest.mark.parametrize("M,K,N", [(3072, 3072, 48), (3072, 3072, 1), (9216, 3072, 1), (3072, 14336, 1),
                                   (3072, 3072, 17), (128, 96, 5)])
def test_integer_products_f32_activations_exact(wx, be, M, K, N):
    """Tiled weights times f32 activations (gemm_skinny_tiled's f32 form, which
    rounds each activation to bf16 as it stages it). Small integers survive
    that rounding, and their fp32 sums are exact, so the output must equal
    x @ w.T exactly."""
    print(f"tiled integer product, f32 activations, M={M} K={K} N={N}", flush=True)
    lib = be.lib
    rng = np.random.default_rng(M + 13 * K + 5 * N)
    w = rng.integers(-4, 5, (M, K))
    x = rng.integers(-4, 5, (N, K))
    B = Bufs(wx, be)
    try:
        wt = B.tiled(K, M)
        xt = B.plain(wx.TYPE_F32, K, N)
        y = lib.wamx_mul_mat(B.pctx, wt, xt)
        B.alloc()
        B.set(wt, wx.f32_to_bf16(w.astype(np.float32)))
        B.set(xt, x.astype(np.float32))
        for rep in range(2):
            B.compute(y)
            got = B.get(y, np.float32, (N, M))
            assert np.array_equal(got.astype(np.int64), x @ w.T), f"launch {rep}"
    finally:
        B.close()


@pytest.mark.parametrize("M,K,N", [(14336, 3072, 48), (14336, 3072, 1), (12288, 4096, 17), (14336, 2048, 33),
                                   (14336, 3072, 64)])
def test_integer_products_bf16_out_exact(wx, be, M, K, N):
    """bf16 outputs of tiled few-token products with at least 192 groups of 64
    features: the K split over the waves of one workgroup (gemm_skinny_wk).
    The fp32 sums of small-integer products are exact, so the bf16 output
    equals the RNE rounding of the exact product."""
    print(f"tiled integer product, bf16 out, M={M} K={K} N={N}", flush=True)
    lib = be.lib
    rng = np.random.default_rng(M + 5 * K + 11 * N)
    w = rng.integers(-4, 5, (M, K))
    x = rng.integers(-4, 5, (N, K))
    B = Bufs(wx, be)
    try:
        wt = B.tiled(K, M)
        xt = B.plain(wx.TYPE_BF16, K, N)
        y = lib.wamx_mul_mat_out_type(B.pctx, wt, xt, wx.TYPE_BF16)
        B.alloc()
        B.set(wt, wx.f32_to_bf16(w.astype(np.float32)))
        B.set(xt, wx.f32_to_bf16(x.astype(np.float32)))
        for rep in range(2):
            B.compute(y)
            got = B.get(y, np.uint16, (N, M))
            ref = wx.f32_to_bf16((x @ w.T).astype(np.float32))
            assert np.array_equal(got, ref), f"launch {rep}: {np.count_nonzero(got != ref)} outputs differ"
    finally:
        B.close()


@pytest.mark.parametrize("epi", ["gelu", "gated"])
def test_linear_and_fused_reduce_match_row_major(wx, be, rng, epi):
    """The same LINEAR (and LINEAR -> adaLN norm, which runs fused) with the
    weight tiled and row-major.  The K splits differ, so the fp32 sums are
    reassociated: the bf16 results agree to the per-op bar."""
    print(f"tiled linear vs row-major ({epi})", flush=True)
    lib = be.lib
    M, K, N = (14336, 3072, 48) if epi == "gelu" else (3072, 14336, 48)
    B = Bufs(wx, be)
    try:
        wt = B.tiled(K, M)
        wp = B.plain(wx.TYPE_BF16, K, M)
        x = B.plain(wx.TYPE_BF16, K, N)
        b = B.plain(wx.TYPE_BF16, M)
        outs = []
        if epi == "gelu":
            for w in (wt, wp):
                outs.append(lib.wamx_linear(B.pctx, w, x, b, wx.EPI_BIAS_GELU, None, None))
        else:
            h = B.plain(wx.TYPE_BF16, M, N)
            gate = B.plain(wx.TYPE_F32, M)
            sc, sh = B.plain(wx.TYPE_F32, M), B.plain(wx.TYPE_F32, M)
            for w in (wt, wp):
                y = lib.wamx_linear(B.pctx, w, x, b, wx.EPI_BIAS_GATED, h, gate)
                outs.append(lib.wamx_norm_modulation_bf16(B.pctx, y, sc, sh, 1e-6))
        B.alloc()
        wv = wx.f32_to_bf16(rng.standard_normal(M * K).astype(np.float32) * 0.02).reshape(M, K)
        B.set(wt, wv)
        B.set(wp, wv)
        B.set(x, wx.f32_to_bf16(rng.standard_normal(N * K).astype(np.float32)))
        B.set(b, wx.f32_to_bf16(rng.standard_normal(M).astype(np.float32) * 0.02))
        if epi == "gated":
            B.set(h, wx.f32_to_bf16(rng.standard_normal(N * M).astype(np.float32)))
            B.set(gate, (rng.standard_normal(M) * 0.5).astype(np.float32))
            B.set(sc, (rng.standard_normal(M) * 0.1).astype(np.float32))
            B.set(sh, (rng.standard_normal(M) * 0.1).astype(np.float32))
        B.compute(*outs)
        got = [wx.bf16_to_f32(B.get(o, np.uint16, (N, M))) for o in outs]
        assert_parity(got[0], got[1], what=f"tiled vs row-major {epi}")
        assert np.mean(got[0] != got[1]) < 0.02
    finally:
        B.close()


def test_supports_op(wx, be):
    lib = be.lib
    B = Bufs(wx, be)
    try:
        wt = B.tiled(3072, 3072)
        b = B.plain(wx.TYPE_BF16, 3072)
        few = lib.wamx_linear(B.pctx, wt, B.plain(wx.TYPE_BF16, 3072, 48), b, wx.EPI_BIAS, None, None)
        many = lib.wamx_linear(B.pctx, wt, B.plain(wx.TYPE_BF16, 3072, 128), b, wx.EPI_BIAS, None, None)
        # other readers of a tiled weight, or of a view of one, would see the tiled order
        cont = lib.wamx_cont(B.pctx, wt)
        half = lib.wamx_view_2d(B.pctx, wt, 3072, 1536, wt.contents.nb[1], 0)
        on_view = lib.wamx_mul_mat(B.pctx, half, B.plain(wx.TYPE_BF16, 3072, 48))
        B.alloc()
        assert wt.contents.extra
        assert lib.wamx_backend_supports_op(be.ptr, few)
        assert not lib.wamx_backend_supports_op(be.ptr, many)
        assert not lib.wamx_backend_supports_op(be.ptr, cont)
        assert not lib.wamx_backend_supports_op(be.ptr, on_view)
    finally:
        B.close()
