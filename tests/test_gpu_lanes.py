"""Two-lane graphs: nodes built after wamx_set_lane(ctx, 1) run on a second
stream, ordered against lane 0 only through the memory both touch, and the
graph allocator keeps each lane's recycled blocks apart.

A graph with chains on both lanes that hand data to each other through a
persistent tensor C (read-after-write both ways and a write-after-read) must
give the bits of the same graph with every node on lane 0, on captured-graph
replays and eager runs alike.  The prefix pass of the model runs this way
(state token on lane 1), and the model tests hold it to the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

D, T = 512, 48


class LaneGraph:
    """Persistent weights / inputs / C in one buffer; the graph's
    intermediates placed by the graph allocator (which recycles them)."""

    def __init__(self, wx, be, rng, lanes: bool, capture: bool):
        self.wx, self.be, self.lib = wx, be, be.lib
        lib = self.lib
        self.pctx = lib.wamx_init(64)
        self.gctx = lib.wamx_init(256)
        bf = wx.TYPE_BF16
        self.w1 = lib.wamx_new_tensor_2d(self.pctx, bf, D, D)
        self.w2 = lib.wamx_new_tensor_2d(self.pctx, bf, D, D)
        self.b1 = lib.wamx_new_tensor_1d(self.pctx, bf, D)
        self.b2 = lib.wamx_new_tensor_1d(self.pctx, bf, D)
        self.x = lib.wamx_new_tensor_2d(self.pctx, bf, D, T)
        self.c = lib.wamx_new_tensor_2d(self.pctx, bf, D, 2 * T)
        self.pbuf = lib.wamx_backend_alloc_ctx_tensors(self.pctx, be.ptr)
        assert self.pbuf, wx.last_error()
        r = np.random.default_rng(1234)  # the same data for every variant
        for t, a in ((self.w1, r.standard_normal(D * D) * 0.05), (self.w2, r.standard_normal(D * D) * 0.05),
                     (self.b1, r.standard_normal(D) * 0.1), (self.b2, r.standard_normal(D) * 0.1),
                     (self.x, r.standard_normal(D * T)), (self.c, np.zeros(2 * D * T))):
            self.set(t, wx.f32_to_bf16(a.astype(np.float32)))
        g, c = self.gctx, self.c
        lin = lambda w, x, b, epi, res=None: lib.wamx_linear(g, w, x, b, epi, res, None)
        half = lambda i: lib.wamx_view_2d(g, c, D, T, c.contents.nb[1], i * T * c.contents.nb[1])
        lane = lambda k: lib.wamx_set_lane(g, k if lanes else 0)
        E = wx
        lane(1)
        a1 = lin(self.w1, self.x, self.b1, E.EPI_BIAS_GELU)
        a2 = lin(self.w2, a1, self.b2, E.EPI_BIAS)
        c1 = lib.wamx_cpy(g, a2, half(0))                                # lane 1 writes C[0:T]
        lane(0)
        p1 = lin(self.w2, self.x, self.b2, E.EPI_BIAS_GELU)
        p2 = lin(self.w1, p1, self.b1, E.EPI_BIAS_RESIDUAL, c1)          # lane 0 reads it
        c2 = lib.wamx_cpy(g, p2, half(1))                                # lane 0 writes C[T:2T]
        lane(1)
        s1 = lin(self.w1, c2, self.b1, E.EPI_BIAS)                       # lane 1 reads it
        s2 = lin(self.w2, s1, self.b2, E.EPI_BIAS_GELU)
        s3 = lin(self.w1, c1, self.b2, E.EPI_BIAS)                       # lane 1 reads C[0:T] again
        lane(0)
        o1 = lin(self.w2, p2, self.b2, E.EPI_BIAS)
        o2 = lin(self.w1, o1, self.b1, E.EPI_BIAS)
        c3 = lib.wamx_cpy(g, o2, half(0))                                # and lane 0 overwrites it
        lane(0)
        self.outs = [s2, s3, o2]
        for o in self.outs:
            lib.wamx_set_output(o)
        self.graph = lib.wamx_new_graph(g, 256)
        for o in (s2, s3, o2, c3):
            lib.wamx_build_forward_expand(self.graph, o)
        if capture:
            lib.wamx_graph_assign_uid(self.graph)
        self.galloc = lib.wamx_gallocr_new(be.ptr)
        assert lib.wamx_gallocr_alloc_graph(self.galloc, self.graph), wx.last_error()

    def set(self, t, a):
        a = np.ascontiguousarray(a)
        self.wx.check(self.lib.wamx_backend_tensor_set(t, a.ctypes.data, 0, a.nbytes), "tensor_set")

    def get(self, t, shape):
        a = np.empty(shape, np.uint16)
        self.wx.check(self.lib.wamx_backend_tensor_get(t, a.ctypes.data, 0, a.nbytes), "tensor_get")
        return a

    def run(self):
        self.set(self.c, np.zeros(2 * D * T, np.uint16))
        self.wx.check(self.lib.wamx_backend_graph_compute(self.be.ptr, self.graph), "graph_compute")
        self.be.sync()
        return [self.get(o, (T, D)) for o in self.outs] + [self.get(self.c, (2 * T, D))]

    def close(self):
        self.lib.wamx_gallocr_free(self.galloc)
        self.lib.wamx_buffer_free(self.pbuf)
        self.lib.wamx_free(self.gctx)
        self.lib.wamx_free(self.pctx)


@pytest.mark.parametrize("capture", [True, False])
def test_two_lanes_match_one_lane(wx, be, rng, capture):
    print(f"two-lane graph vs one lane (capture={capture})", flush=True)
    one = LaneGraph(wx, be, rng, lanes=False, capture=capture)
    two = LaneGraph(wx, be, rng, lanes=True, capture=capture)
    try:
        ref = one.run()
        assert ref[3][:T].any() and ref[3][T:].any()
        for rep in range(3):  # capture, then replays
            got = two.run()
            for k, (a, b) in enumerate(zip(got, ref)):
                assert np.array_equal(a, b), f"output {k} differs on run {rep}"
    finally:
        one.close()
        two.close()


def test_allocator_keeps_lanes_apart(wx, be):
    """A tensor that lane 1 writes first and lane 0 reads later must not take
    memory lane 0 has recycled: lane 0 may still be running the nodes that
    used it.  It goes to lane 1's arena, away from every lane-0 intermediate."""
    lib = be.lib
    ctx = lib.wamx_init(64)
    pctx = lib.wamx_init(16)
    bf = wx.TYPE_BF16
    try:
        w = lib.wamx_new_tensor_2d(pctx, bf, D, D)
        b = lib.wamx_new_tensor_1d(pctx, bf, D)
        x = lib.wamx_new_tensor_2d(pctx, bf, D, T)
        pbuf = lib.wamx_backend_alloc_ctx_tensors(pctx, be.ptr)
        assert pbuf, wx.last_error()
        lin = lambda a: lib.wamx_linear(ctx, w, a, b, wx.EPI_BIAS, None, None)
        lib.wamx_set_lane(ctx, 0)
        p1 = lin(x)
        p2 = lin(p1)          # p1 is recycled after this node
        lib.wamx_set_lane(ctx, 1)
        z = lin(x)            # first touched on lane 1, read by lane 0 below
        lib.wamx_set_lane(ctx, 0)
        out = lib.wamx_linear(ctx, w, z, b, wx.EPI_BIAS_RESIDUAL, p2, None)
        lib.wamx_set_output(out)
        g = lib.wamx_new_graph(ctx, 64)
        lib.wamx_build_forward_expand(g, p2)  # node order: p1, p2, z, out
        lib.wamx_build_forward_expand(g, out)
        ga = lib.wamx_gallocr_new(be.ptr)
        try:
            assert lib.wamx_gallocr_alloc_graph(ga, g), wx.last_error()
            nbytes = D * T * 2
            zs, ps = z.contents.data, p1.contents.data
            assert zs + nbytes <= ps or ps + nbytes <= zs, "lane-1 tensor placed in recycled lane-0 memory"
        finally:
            lib.wamx_gallocr_free(ga)
        lib.wamx_buffer_free(pbuf)
    finally:
        lib.wamx_free(ctx)
        lib.wamx_free(pctx)
