"""wamx_op_linear_noalloc against wamx_op_linear, through the C ABI: the
same product on the same device arrays gives the same bits, on calls in a row
(each smaller than the one before, so it runs on what that one left in the
shared scratch array), on both K-split paths (the few-token skinny products
and the 384-token K-sliced 128 x 128 products of a batch of eight chunks), and
a product whose split-K partials would not fit in the scratch array is refused
before anything runs."""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(wx, be, orc, M, N, K, epi, seed):
    w = orc.fill_normal(M * K, seed, 0.0, 0.02, orc.BF16)
    x = orc.fill_normal(N * K, seed + 1, 0.0, 1.0, orc.BF16)
    b = orc.fill_normal(M, seed + 2, 0.0, 0.02, orc.BF16)
    r = orc.fill_normal(N * M, seed + 3, 0.0, 1.0, orc.BF16)
    g = orc.fill_normal(M, seed + 4, 0.0, 0.5)
    dw, dx, db, dr, dg = (be.array(a) for a in (w, x, b, r, g))
    y_ref, y_na = be.empty(N * M * 2), be.empty(N * M * 2)
    res = dr.ptr if epi in (wx.EPI_BIAS_GATED, wx.EPI_BIAS_RESIDUAL) else None
    gate = dg.ptr if epi == wx.EPI_BIAS_GATED else None
    lib = be.lib
    wx.check(lib.wamx_op_linear(be.ptr, dw.ptr, dx.ptr, wx.TYPE_BF16, db.ptr, epi, res, gate, y_ref.ptr, M, N, K),
             "linear")
    be.sync()
    stream = lib.wamx_backend_stream(be.ptr)
    wx.check(lib.wamx_op_linear_noalloc(stream, dw.ptr, dx.ptr, wx.TYPE_BF16, db.ptr, epi, res, gate, y_na.ptr, M, N,
                                        K), "linear_noalloc")
    be.sync()
    a = y_ref.download(np.uint16, (N, M))
    c = y_na.download(np.uint16, (N, M))
    assert np.array_equal(a, c), f"{N}x{M}x{K}"
    return dw, dx, db, y_na


def test_linear_noalloc_matches_linear(wx, be, orc):
    print("linear_noalloc: 384 x 3072 x 14336, 384 x 3072 x 3072, 48 x 14336 x 3072, 16 x 3072 x 14336, "
          "8 x 256 x 512", flush=True)
    lib = be.lib
    # batch-8 denoise FFN-down and 3072^2 projection: K-sliced 128 x 128 tiles
    # (7 and 6 slices), partials in the scratch array
    for M, K, seed in ((3072, 14336, 400), (3072, 3072, 500)):
        _case(wx, be, orc, M, 384, K, wx.EPI_BIAS_GATED, seed)
    _case(wx, be, orc, 14336, 48, 3072, wx.EPI_BIAS_GELU, 100)       # FFN-up of the 48-token step
    _case(wx, be, orc, 3072, 16, 14336, wx.EPI_BIAS_GATED, 200)      # smaller: FFN-down shape on 16 tokens
    dw, dx, db, y = _case(wx, be, orc, 256, 8, 512, wx.EPI_BIAS_RESIDUAL, 300)
    # 64 tokens x 65536 x 14336 would need far more split-K partials than the
    # scratch array holds: refused, nothing launched
    st = lib.wamx_op_linear_noalloc(lib.wamx_backend_stream(be.ptr), dw.ptr, dx.ptr, wx.TYPE_BF16, db.ptr,
                                    wx.EPI_BIAS, None, None, y.ptr, 65536, 64, 14336)
    assert st != 0 and "split-K scratch" in wx.last_error()
    be.sync()
