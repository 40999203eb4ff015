"""CPU side of the drop-in path: the reference's unfused action layer, built
with the restated ggml constructors (tests/ggml_mirror.py), imports through
wamx_graph_from_ggml and every node passes supports_op.  Nothing runs on a
device here (addresses are placeholders); tests/test_gpu_dropin.py computes
the same graph against the oracle."""
from __future__ import annotations

import numpy as np

import ggml_mirror as gm
from test_gpu_dropin import action_layer_graph


class _Leaves:
    def leaf(self, typ, ne, data=None, name=""):
        return gm.new_tensor(typ, *ne, name=name)


def test_unfused_action_layer_imports_and_is_supported(wx):
    lib = wx.load()
    d, H, F, P, NL, T = 256, 2, 384, 129, 16, 48
    dh = d // H
    r = _Leaves()
    names = {"attn1.to_qkv.weight": (d, 3 * d), "attn1.to_qkv.bias": (3 * d,),
             "attn1.norm_q.weight": (d,), "attn1.norm_k.weight": (d,),
             "attn1.to_out.0.weight": (d, d), "attn1.to_out.0.bias": (d,),
             "norm2.weight": (d,), "norm2.bias": (d,), "attn2.to_q.weight": (d, d), "attn2.to_q.bias": (d,),
             "attn2.norm_q.weight": (d,), "attn2.to_out.0.weight": (d, d), "attn2.to_out.0.bias": (d,),
             "ffn.net.0.proj.weight": (d, F), "ffn.net.0.proj.bias": (F,),
             "ffn.net.2.weight": (F, d), "ffn.net.2.bias": (d,)}
    W = {n: r.leaf("bf16", ne, name=n) for n, ne in names.items()}
    out = action_layer_graph(r, W, r.leaf("bf16", (d, T)), r.leaf("bf16", (d, 6, 1)), r.leaf("bf16", (d, 6)),
                             r.leaf("i32", (T,)), r.leaf("bf16", (dh, P, H)), r.leaf("bf16", (P, dh, H)),
                             r.leaf("bf16", (dh, NL, H)), r.leaf("bf16", (NL, dh, H)), d, H, T, P, NL)
    assert out.ne[:2] == [d, T] and out.type == "bf16"
    graph = gm.Graph()
    graph.expand(out)
    used = gm.place(graph.tensors(), 1 << 30, 1 << 30)
    assert used > 0
    arr, nodes, _keep = gm.describe(graph)
    ctx = lib.wamx_init(len(arr) + 64)
    try:
        g = lib.wamx_graph_from_ggml(ctx, arr, len(arr), nodes, len(nodes))
        assert g, wx.last_error()
        n = lib.wamx_graph_n_nodes(g)
        assert n == len(graph.nodes)
        bad = [(i, graph.nodes[i].op) for i in range(n) if not lib.wamx_backend_supports_op(None, lib.wamx_graph_node(g, i))]
        assert not bad, bad
        counts = {}
        for t in graph.nodes:
            counts[t.op] = counts.get(t.op, 0) + 1
        # two attentions (scores and outputs: 4 MUL_MAT) and six projections
        assert counts["MUL_MAT"] == 10 and counts["SOFT_MAX"] == 2 and counts["CONCAT"] == 4
    finally:
        lib.wamx_free(ctx)
