"""The drop-in path on the GPU: graphs built the way wam.cpp's engine builds
them for ggml (its unfused constructors, ggml's op_params layouts, ggml op and
unary names), handed to libwamx through wamx_graph_from_ggml exactly as a
ggml backend shim fills the descriptors, run by wamx_backend_graph_compute,
and checked against the oracle.

Covered ggml nodes: batched MUL_MAT(K, Q) at GGML_PREC_F32, SOFT_MAX_EXT
(with and without a mask), MUL_MAT(V, P) with f32 probabilities, CONCAT of
the cached and current K/V, CONT of permutes, bf16 MUL_MAT_out + bias ADD,
the patch's NORM / RMS_NORM / ADD(src[2]) / UNARY(src[1]) extensions, ROPE
(1-D and apply_visual_rope's strided section views + CONCAT), CPY casts,
IM2COL, GELU_ERF and SILU.

Bars: the per-op bar (max-rel <= 1e-2, cosine >= 0.9999) on a layer's bf16
output; masked softmax within 1e-6 absolute of float64 numpy.
"""
from __future__ import annotations

import numpy as np
import pytest

import ggml_mirror as gm
from conftest import assert_parity

pytestmark = pytest.mark.gpu

EPS = 1e-6


class Runner:
    """Places a mirrored graph in one device arena, uploads its leaves,
    imports it through wamx_graph_from_ggml and computes it."""

    def __init__(self, wx, be, capacity: int):
        self.wx, self.be = wx, be
        self.arena = be.empty(capacity)
        self.host = {}

    def leaf(self, typ, ne, data, name=""):
        t = gm.new_tensor(typ, *ne, name=name)
        self.host[id(t)] = (t, np.ascontiguousarray(data))
        return t

    def run(self, outputs):
        lib = self.be.lib
        graph = gm.Graph()
        for o in outputs:
            graph.expand(o)
        tensors = graph.tensors()
        gm.place(tensors, self.arena.ptr, self.arena.nbytes)
        for t, a in self.host.values():
            assert a.nbytes == t.nbytes(), t.name
            self.wx.check(lib.wamx_memcpy_h2d(self.be.ptr, t.data, a.ctypes.data, a.nbytes), f"upload {t.name}")
        arr, nodes, keep = gm.describe(graph)
        ctx = lib.wamx_init(len(arr) + 64)
        try:
            g = lib.wamx_graph_from_ggml(ctx, arr, len(arr), nodes, len(nodes))
            assert g, self.wx.last_error()
            lib.wamx_graph_assign_uid(g)
            self.wx.check(lib.wamx_backend_graph_compute(self.be.ptr, g), "graph_compute")
            self.be.sync()
        finally:
            lib.wamx_free(ctx)
        del keep
        return graph

    def fetch(self, t, dtype, shape):
        out = np.empty(shape, dtype)
        assert out.nbytes == t.nbytes()
        self.wx.check(self.be.lib.wamx_memcpy_d2h(self.be.ptr, out.ctypes.data, t.data, out.nbytes), "download")
        return out


def bf(wx, a):
    return wx.bf16_to_f32(a)


def weights(orc, seed, shapes):
    out = {}
    for i, (name, shape) in enumerate(shapes.items()):
        n = int(np.prod(shape))
        if name.endswith("bias"):
            out[name] = orc.fill_normal(n, seed + i, 0.0, 0.02, orc.BF16).reshape(shape)
        elif "norm" in name:
            out[name] = orc.fill_normal(n, seed + i, 1.0, 0.02, orc.BF16).reshape(shape)
        else:
            out[name] = orc.fill_normal(n, seed + i, 0.0, 0.02, orc.BF16).reshape(shape)
    return out


def action_layer_graph(r, W, h, mod, table, apos, pk, pv, lk, lv, d, H, T, P, NL):
    """One action-expert layer of build_cached_action_body (mot.cpp:377-467)
    in the BF16 latency profile, op for op: modulation_add / modulation_part
    (mot.cpp:130-145), expert_qkv (:204-267) with packed QKV, the joint
    [state, action, reference] K/V CONCAT (:397-431), the unfused attention
    (:432-445), gated_residual (:161-173), expert_cross_ffn with the cached
    prompt K/V (:284-347), linear_with_activation / linear_gelu_with_activation
    (weights.cpp:819-849), rms_norm / layer_norm (weights.cpp:904-930)."""
    dh = d // H
    scale = 1.0 / np.sqrt(dh)

    def linear(wn, x):
        if x.type != "bf16":
            x = gm.cast(x, "bf16")
        y = gm.mul_mat_out_type(W[wn + ".weight"], x, "bf16")
        return gm.add(y, W[wn + ".bias"])

    def rms(x, wn):
        return gm.rms_norm_bf16_f32(x, W[wn], EPS)

    # modulation_add: f32(mod) + f32(table) -> [d, 6, 1]; parts are [d, 1] views
    comb = gm.add(gm.cast(mod, "f32"), gm.cast(table, "f32"))
    part = [gm.view_2d(comb, d, 1, comb.nb[2], i * comb.nb[1]) for i in range(6)]
    shift, scl, gate, cshift, cscale, cgate = part
    # expert_qkv, packed QKV
    n = gm.norm_modulation_bf16(h, scl, shift, EPS)
    qkv = linear("attn1.to_qkv", n)
    q = gm.cont(gm.view_2d(qkv, d, T, qkv.nb[1], 0))
    k = gm.cont(gm.view_2d(qkv, d, T, qkv.nb[1], d * 2))
    v = gm.cont(gm.view_2d(qkv, d, T, qkv.nb[1], 2 * d * 2))
    q = gm.reshape(rms(q, "attn1.norm_q.weight"), dh, H, T)
    k = gm.reshape(rms(k, "attn1.norm_k.weight"), dh, H, T)
    v = gm.reshape(v, dh, H, T)
    rope = dict(n_dims=dh, mode=gm.GGML_ROPE_TYPE_NORMAL, n_ctx_orig=0, freq_base=10000.0, freq_scale=1.0,
                ext_factor=0.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0)
    q = gm.cast(gm.rope_ext(q, apos, **rope), "bf16")
    k = gm.cast(gm.rope_ext(k, apos, **rope), "bf16")
    Q = gm.cont(gm.permute(q, 0, 2, 1, 3))
    ak = gm.cont(gm.permute(k, 0, 2, 1, 3))
    av = gm.cont(gm.permute(v, 1, 2, 0, 3))
    nimg = P - 1
    state_k = gm.view_3d(pk, dh, 1, H, pk.nb[1], pk.nb[2], 0)
    ref_k = gm.view_3d(pk, dh, nimg, H, pk.nb[1], pk.nb[2], pk.nb[1])
    state_v = gm.view_3d(pv, 1, dh, H, pv.nb[1], pv.nb[2], 0)
    ref_v = gm.view_3d(pv, nimg, dh, H, pv.nb[1], pv.nb[2], pv.nb[0])
    jk = gm.concat(gm.concat(state_k, ak, 1), ref_k, 1)
    jv = gm.concat(gm.concat(state_v, av, 0), ref_v, 0)
    scores = gm.mul_mat(jk, Q)
    gm.mul_mat_set_prec(scores, gm.GGML_PREC_F32)
    probs = gm.soft_max_ext(scores, None, scale, 0.0)
    att = gm.reshape(gm.cont(gm.permute(gm.mul_mat(jv, probs), 0, 2, 1, 3)), d, T)
    att = linear("attn1.to_out.0", att)
    h = gm.gated_residual_bf16(h, att, gate)
    # expert_cross_ffn, cached prompt K/V
    n2 = gm.layer_norm_bf16(h, W["norm2.weight"], W["norm2.bias"], EPS)
    cq = linear("attn2.to_q", n2)
    cq = gm.cast(gm.reshape(rms(cq, "attn2.norm_q.weight"), dh, H, T), "bf16")
    CQ = gm.cont(gm.permute(cq, 0, 2, 1, 3))
    cs = gm.mul_mat(lk, CQ)
    gm.mul_mat_set_prec(cs, gm.GGML_PREC_F32)
    cp = gm.soft_max_ext(cs, None, scale, 0.0)
    catt = gm.reshape(gm.cont(gm.permute(gm.mul_mat(lv, cp), 0, 2, 1, 3)), d, T)
    catt = linear("attn2.to_out.0", catt)
    h = gm.add(h, catt)
    n3 = gm.norm_modulation_bf16(h, cscale, cshift, EPS)
    u = gm.bias_gelu_bf16(gm.mul_mat_out_type(W["ffn.net.0.proj.weight"], n3, "bf16"), W["ffn.net.0.proj.bias"])
    dn = linear("ffn.net.2", u)
    return gm.gated_residual_bf16(h, dn, cgate)


def oracle_action_layer(orc, W, h, mod, table, apos, pk, pvt, lk, lvt, d, H, T):
    """The same layer from the oracle's pinned per-op functions."""
    dh = d // H
    m = orc.modulation(mod.reshape(-1), table.reshape(-1))[0].reshape(6, d)
    n = orc.norm_mod_bf16(h, m[1], m[0], EPS)
    qkv = orc.linear(W["attn1.to_qkv.weight"], n, W["attn1.to_qkv.bias"], orc.EPI_BIAS)
    Q = orc.qk_norm_rope(qkv[:, :d], W["attn1.norm_q.weight"], H, dh, 0, pos0=apos, eps=EPS)
    Ka = orc.qk_norm_rope(qkv[:, d:2 * d], W["attn1.norm_k.weight"], H, dh, 0, pos0=apos, eps=EPS)
    Vat = np.ascontiguousarray(qkv[:, 2 * d:].reshape(T, H, dh).transpose(1, 2, 0))
    att = orc.attention(Q, pk, pvt, Ka, Vat, na_split=1)
    h = orc.linear(W["attn1.to_out.0.weight"], att, W["attn1.to_out.0.bias"], orc.EPI_BIAS_GATED, h, m[2])
    n2 = orc.layer_norm_bf16(h, W["norm2.weight"], W["norm2.bias"], EPS)
    cq = orc.linear(W["attn2.to_q.weight"], n2, W["attn2.to_q.bias"], orc.EPI_BIAS)
    CQ = orc.qk_norm_rope(cq, W["attn2.norm_q.weight"], H, dh, 2, eps=EPS)
    catt = orc.attention(CQ, lk, lvt)
    h = orc.linear(W["attn2.to_out.0.weight"], catt, W["attn2.to_out.0.bias"], orc.EPI_BIAS_RESIDUAL, h)
    n3 = orc.norm_mod_bf16(h, m[4], m[3], EPS)
    u = orc.linear(W["ffn.net.0.proj.weight"], n3, W["ffn.net.0.proj.bias"], orc.EPI_BIAS_GELU)
    return orc.linear(W["ffn.net.2.weight"], u, W["ffn.net.2.bias"], orc.EPI_BIAS_GATED, h, m[5])


@pytest.mark.parametrize("d,H,F,P,NL", [(256, 2, 384, 129, 16), (3072, 24, 14336, 3073, 512)],
                         ids=["small", "config5-layer"])
def test_unfused_action_layer_matches_oracle(wx, be, orc, d, H, F, P, NL):
    """The reference's unfused action layer (48 queries over 1 + 48 + n_img
    self-attention keys and NL prompt keys) through the ggml import path."""
    print(f"drop-in unfused action layer d={d} H={H} F={F} P={P} NL={NL}", flush=True)
    T, dh = 48, d // H
    shapes = {"attn1.to_qkv.weight": (3 * d, d), "attn1.to_qkv.bias": (3 * d,),
              "attn1.norm_q.weight": (d,), "attn1.norm_k.weight": (d,),
              "attn1.to_out.0.weight": (d, d), "attn1.to_out.0.bias": (d,),
              "norm2.weight": (d,), "norm2.bias": (d,),
              "attn2.to_q.weight": (d, d), "attn2.to_q.bias": (d,), "attn2.norm_q.weight": (d,),
              "attn2.to_out.0.weight": (d, d), "attn2.to_out.0.bias": (d,),
              "ffn.net.0.proj.weight": (F, d), "ffn.net.0.proj.bias": (F,),
              "ffn.net.2.weight": (d, F), "ffn.net.2.bias": (d,)}
    Wh = weights(orc, 0x5EED0500, shapes)
    h = orc.fill_normal(T * d, 1, 0.0, 1.0, orc.BF16).reshape(T, d)
    mod = orc.fill_normal(6 * d, 2, 0.0, 0.5, orc.BF16).reshape(6, d)
    table = orc.fill_normal(6 * d, 3, 0.0, 0.1, orc.BF16).reshape(6, d)
    apos = np.arange(1, T + 1, dtype=np.int32)
    pk = orc.fill_normal(H * P * dh, 4, 0.0, 1.0, orc.BF16).reshape(H, P, dh)
    pvt = orc.fill_normal(H * dh * P, 5, 0.0, 1.0, orc.BF16).reshape(H, dh, P)
    lk = orc.fill_normal(H * NL * dh, 6, 0.0, 1.0, orc.BF16).reshape(H, NL, dh)
    lvt = orc.fill_normal(H * dh * NL, 7, 0.0, 1.0, orc.BF16).reshape(H, dh, NL)

    r = Runner(wx, be, 1 << 30)
    W = {}
    for name, a in Wh.items():
        ne = tuple(reversed(a.shape))
        W[name] = r.leaf("bf16", ne, a, name)
    th = r.leaf("bf16", (d, T), h, "hidden")
    tmod = r.leaf("bf16", (d, 6, 1), mod, "time_proj")
    ttab = r.leaf("bf16", (d, 6), table, "scale_shift_table")
    tpos = r.leaf("i32", (T,), apos, "positions")
    tpk = r.leaf("bf16", (dh, P, H), pk, "prefix_keys")
    tpv = r.leaf("bf16", (P, dh, H), pvt, "prefix_values")
    tlk = r.leaf("bf16", (dh, NL, H), lk, "prompt_keys")
    tlv = r.leaf("bf16", (NL, dh, H), lvt, "prompt_values")
    out = action_layer_graph(r, W, th, tmod, ttab, tpos, tpk, tpv, tlk, tlv, d, H, T, P, NL)
    graph = r.run([out])
    ops = {t.op for t in graph.nodes}
    assert {"MUL_MAT", "SOFT_MAX", "CONCAT", "CONT", "ROPE", "NORM", "RMS_NORM", "UNARY", "ADD", "CPY"} <= ops
    got = r.fetch(out, np.uint16, (T, d))
    ref = oracle_action_layer(orc, Wh, h, mod, table, apos, pk, pvt, lk, lvt, d, H, T)
    assert_parity(bf(wx, got), bf(wx, ref), what=f"unfused action layer d={d}")


def test_masked_soft_max_matches_numpy(wx, be):
    """SOFT_MAX_EXT with the complete-MoT mask (mot.cpp:1025-1027,
    semantics.cpp:260-287: state and visual queries do not see action keys)
    as an f32 [n, n, H] tensor, and an f16 mask broadcast over heads with
    padded rows."""
    print("drop-in masked soft_max", flush=True)
    n, H, A = 70, 3, 16       # 1 state + 16 action + 53 visual tokens
    rng = np.random.default_rng(11)
    x = rng.normal(0, 3, (H, n, n)).astype(np.float32)           # [H][query][key]
    q_act = (np.arange(n) >= 1) & (np.arange(n) < 1 + A)
    allowed = q_act[:, None] | ~q_act[None, :]
    mask = np.where(allowed, 0.0, -np.inf).astype(np.float32)
    mask3 = np.ascontiguousarray(np.broadcast_to(mask, (H, n, n)))
    mask16 = np.zeros((n + 5, n), np.float16)
    mask16[:n] = rng.normal(0, 1, (n, n)).astype(np.float16)
    scale = 0.125

    r = Runner(wx, be, 16 << 20)
    tx = r.leaf("f32", (n, n, H), x, "scores")
    tm = r.leaf("f32", (n, n, H), mask3, "mask")
    tm16 = r.leaf("f16", (n, n + 5), mask16, "mask16")
    y1 = gm.soft_max_ext(tx, tm, scale, 0.0)
    y2 = gm.soft_max_ext(tx, tm16, scale, 0.0)
    y3 = gm.soft_max_ext(tx, None, scale, 0.0)
    r.run([y1, y2, y3])

    def ref(m):
        w = x.astype(np.float64) * scale + (0 if m is None else m.astype(np.float64))
        w = w - w.max(axis=-1, keepdims=True)
        e = np.exp(w)
        return e / e.sum(axis=-1, keepdims=True)

    for t, m in ((y1, mask3), (y2, mask16[:n][None]), (y3, None)):
        got = r.fetch(t, np.float32, (H, n, n))
        assert np.max(np.abs(got - ref(m))) <= 1e-6
    got = r.fetch(y1, np.float32, (H, n, n))
    assert np.all(got[:, ~q_act][:, :, q_act] == 0.0)   # masked keys get exactly zero weight


def test_unfused_prefix_entry_matches_oracle(wx, be, orc):
    """The prefix pass's entry, unfused: the patch embedding as ggml_conv_2d
    lowers it (IM2COL to bf16 + MUL_MAT_out + reshape/permute/CONT + bias ADD,
    native-bf16.patch:683-695, cache.cpp:203-218), the state encoder MLP with
    GELU_ERF (mot.cpp:16-33), the condition path with SILU (mot.cpp:63-82),
    and apply_visual_rope's {44, 42, 42} strided ROPE views + CONCAT
    (mot.cpp:182-202) on a (t, h, w) grid with t > 0."""
    print("drop-in unfused prefix entry", flush=True)
    Z, gh, gw, d, H, E, A = 8, 4, 6, 256, 2, 32, 32
    dh = d // H
    nimg = gh * gw
    seed = 0x5EED0600
    patch_w = orc.fill_normal(d * Z * 4, seed, 0.0, 0.02, orc.BF16).reshape(d, Z, 2, 2)
    patch_b = orc.fill_normal(d, seed + 1, 0.0, 0.02, orc.BF16)
    latent = orc.fill_normal(Z * 2 * gh * 2 * gw, seed + 2).reshape(Z, 2 * gh, 2 * gw)
    enc = {n: orc.fill_normal(int(np.prod(s)), seed + 10 + i, 0.0, 0.02 if "w" in n else 0.02, orc.BF16).reshape(s)
           for i, (n, s) in enumerate({"in_w": (E, A), "in_b": (E,), "mid_w": (E, E), "mid_b": (E,),
                                       "out_w": (d, E), "out_b": (d,), "t1_w": (d, 256), "t1_b": (d,),
                                       "t2_w": (d, d), "t2_b": (d,), "tp_w": (6 * d, d), "tp_b": (6 * d,)}.items())}
    state = orc.fill_normal(A, seed + 3)
    freq = orc.timestep_embedding(0.0)
    x = orc.fill_normal(nimg * d, seed + 4, 0.0, 1.0, orc.BF16).reshape(nimg, d)
    norm_w = orc.fill_normal(d, seed + 5, 1.0, 0.02, orc.BF16)
    tpos = (np.arange(nimg) % 4).astype(np.int32)          # t in 0..3
    hpos = (np.arange(nimg) // gw).astype(np.int32)
    wpos = (np.arange(nimg) % gw).astype(np.int32)

    r = Runner(wx, be, 64 << 20)
    tw = r.leaf("bf16", (2, 2, Z, d), patch_w, "patch_embedding.weight")
    tb = r.leaf("bf16", (d,), patch_b, "patch_embedding.bias")
    tl = r.leaf("f32", (2 * gw, 2 * gh, Z, 1), latent, "reference")
    # ggml_conv_2d as patched: im2col (bf16) x kernel -> bf16 [OW*OH, OC] ... [OW, OH, OC, N]
    col = gm.im2col(tw, tl, 2, 2, 0, 0, 1, 1, True, "bf16")
    mm = gm.mul_mat_out_type(gm.reshape(col, col.ne[0], col.ne[3] * col.ne[2] * col.ne[1]),
                             gm.reshape(tw, 2 * 2 * Z, d), "bf16")
    conv = gm.cont(gm.permute(gm.reshape(mm, col.ne[1], col.ne[2], col.ne[3], d), 0, 1, 3, 2))
    vis = gm.add(conv, gm.reshape(tb, 1, 1, d, 1))
    vis = gm.reshape(gm.cont(gm.permute(vis, 1, 2, 0, 3)), d, nimg)
    # state encoder and condition path
    E_ = {k: r.leaf("bf16", tuple(reversed(v.shape)), v, k) for k, v in enc.items()}
    ts = r.leaf("f32", (A, 1), state, "state")
    tf = r.leaf("f32", (256, 1), freq, "frequency")

    def lin(w, b, inp):
        if inp.type != "bf16":
            inp = gm.cast(inp, "bf16")
        return gm.add(gm.mul_mat_out_type(E_[w], inp, "bf16"), E_[b])

    sh = lin("out_w", "out_b", gm.gelu_erf(lin("mid_w", "mid_b", gm.gelu_erf(lin("in_w", "in_b", ts)))))
    temb = lin("t2_w", "t2_b", gm.silu(lin("t1_w", "t1_b", tf)))
    mod = lin("tp_w", "tp_b", gm.silu(temb))
    # apply_visual_rope on RMSNorm(x) reshaped [dh, H, T]
    tx = r.leaf("bf16", (d, nimg), x, "visual_k")
    tn = r.leaf("bf16", (d,), norm_w, "norm_k")
    pt, ph, pw = (r.leaf("i32", (nimg,), p, n) for p, n in ((tpos, "t"), (hpos, "h"), (wpos, "w")))
    k = gm.reshape(gm.rms_norm_bf16_f32(tx, tn, EPS), dh, H, nimg)
    res, off = None, 0
    for sec, pos in zip((44, 42, 42), (pt, ph, pw)):
        view = gm.view_3d(k, sec, H, nimg, k.nb[1], k.nb[2], off)
        rot = gm.rope_ext(view, pos, sec, 0, 0, 10000.0, 1.0, 0.0, 1.0, 32.0, 1.0)
        res = rot if res is None else gm.concat(res, rot, 0)
        off += sec * k.nb[0]
    kk = gm.cast(gm.cont(res), "bf16")
    r.run([vis, sh, mod, kk])

    # oracle: conv as im2col (ic, kh, kw) x weight [OC][IC*KH*KW] + bias
    cols = np.zeros((nimg, Z * 4), np.float32)
    for y in range(gh):
        for xx in range(gw):
            cols[y * gw + xx] = latent[:, 2 * y:2 * y + 2, 2 * xx:2 * xx + 2].reshape(-1)
    ref_vis = orc.linear(patch_w.reshape(d, Z * 4), orc.f32_to_bf16(cols), patch_b, orc.EPI_BIAS)
    assert_parity(bf(wx, r.fetch(vis, np.uint16, (nimg, d))), bf(wx, ref_vis), what="patch embedding")

    def gelu_erf_bf16(a):
        from math import erf
        v = bf(wx, a).astype(np.float64)
        g = np.array([0.5 * t * (1 + erf(t / np.sqrt(2))) for t in v.ravel()], np.float32).reshape(v.shape)
        return wx.f32_to_bf16(g)

    def silu_bf16(a):
        v = bf(wx, a).astype(np.float64)
        return wx.f32_to_bf16((v / (1 + np.exp(-v))).astype(np.float32))

    h1 = gelu_erf_bf16(orc.linear(enc["in_w"], state[None], enc["in_b"], orc.EPI_BIAS))
    h2 = gelu_erf_bf16(orc.linear(enc["mid_w"], h1, enc["mid_b"], orc.EPI_BIAS))
    ref_sh = orc.linear(enc["out_w"], h2, enc["out_b"], orc.EPI_BIAS)
    assert_parity(bf(wx, r.fetch(sh, np.uint16, (1, d))), bf(wx, ref_sh), what="state encoder")
    t1 = silu_bf16(orc.linear(enc["t1_w"], freq[None], enc["t1_b"], orc.EPI_BIAS))
    ref_temb = orc.linear(enc["t2_w"], t1, enc["t2_b"], orc.EPI_BIAS)
    ref_mod = orc.linear(enc["tp_w"], silu_bf16(ref_temb), enc["tp_b"], orc.EPI_BIAS)
    assert_parity(bf(wx, r.fetch(mod, np.uint16, (1, 6 * d))), bf(wx, ref_mod), what="time_proj")
    ref_k = orc.qk_norm_rope(x, norm_w, H, dh, 1, pos0=tpos, pos1=hpos, pos2=wpos, eps=EPS)   # [H][T][dh]
    got_k = r.fetch(kk, np.uint16, (nimg, H, dh)).transpose(1, 0, 2)
    assert_parity(bf(wx, got_k), bf(wx, ref_k), what="visual rope t>0")


# --- the F32 reference profile ------------------------------------------------
def action_layer_graph_f32(W, h, mod, table, apos, pk, pv, lk, lv, d, H, T, P, NL):
    """The same layer in the F32 reference profile (Precision::f32_reference,
    engine.cpp:45-51; `source-f32-v1` artifacts: F32 weights, hidden states
    and caches), op for op:
    * modulation_add of two F32 tensors (mot.cpp:137-145);
    * modulated_norm's F32 form (mot.cpp:154-158): NORM, MUL, ADD, ADD, the
      chain the backend matches into norm_modulation_f32;
    * expert_qkv with separate q/k/v projections (no packed QKV outside the
      qkv policy, mot.cpp:225-236): linear_with_activation -> linear
      (weights.cpp:786-793, :819-829), MUL_MAT f32 x f32 + bias ADD;
    * rms_norm (weights.cpp:904-917): RMS_NORM, a CPY of the weight to f32,
      MUL; 1-D RoPE on f32 (mot.cpp:175-180); no bf16 casts;
    * the unfused f32 attention (mot.cpp:432-445);
    * gated_residual's F32 form (mot.cpp:164-166): MUL, ADD, matched into
      gated_residual_f32;
    * layer_norm (weights.cpp:919-930): NORM, MUL(CPY w), ADD(CPY b); the
      cross-attention over cached f32 prompt K/V; linear_gelu_with_activation's
      F32 form (weights.cpp:831-849): GELU of the linear."""
    dh = d // H
    scale = 1.0 / np.sqrt(dh)

    def linear(wn, x):
        return gm.add(gm.mul_mat(W[wn + ".weight"], x), W[wn + ".bias"])

    def rms(x, wn):
        return gm.mul(gm.rms_norm(x, EPS), gm.cast(W[wn], "f32"))

    def modulated_norm(x, scl, sft):
        n = gm.norm(x, EPS)
        return gm.add(gm.add(n, gm.mul(n, scl)), sft)

    def layer_norm(x, wn, bn):
        return gm.add(gm.mul(gm.norm(x, EPS), gm.cast(W[wn], "f32")), gm.cast(W[bn], "f32"))

    comb = gm.add(mod, table)
    shift, scl, gate, cshift, cscale, cgate = [gm.view_2d(comb, d, 1, comb.nb[2], i * comb.nb[1]) for i in range(6)]
    n = modulated_norm(h, scl, shift)
    q = gm.reshape(rms(linear("attn1.to_q", n), "attn1.norm_q.weight"), dh, H, T)
    k = gm.reshape(rms(linear("attn1.to_k", n), "attn1.norm_k.weight"), dh, H, T)
    v = gm.reshape(linear("attn1.to_v", n), dh, H, T)
    rope = dict(n_dims=dh, mode=gm.GGML_ROPE_TYPE_NORMAL, n_ctx_orig=0, freq_base=10000.0, freq_scale=1.0,
                ext_factor=0.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0)
    q = gm.rope_ext(q, apos, **rope)
    k = gm.rope_ext(k, apos, **rope)
    Q = gm.cont(gm.permute(q, 0, 2, 1, 3))
    ak = gm.cont(gm.permute(k, 0, 2, 1, 3))
    av = gm.cont(gm.permute(v, 1, 2, 0, 3))
    nimg = P - 1
    state_k = gm.view_3d(pk, dh, 1, H, pk.nb[1], pk.nb[2], 0)
    ref_k = gm.view_3d(pk, dh, nimg, H, pk.nb[1], pk.nb[2], pk.nb[1])
    state_v = gm.view_3d(pv, 1, dh, H, pv.nb[1], pv.nb[2], 0)
    ref_v = gm.view_3d(pv, nimg, dh, H, pv.nb[1], pv.nb[2], pv.nb[0])
    jk = gm.concat(gm.concat(state_k, ak, 1), ref_k, 1)
    jv = gm.concat(gm.concat(state_v, av, 0), ref_v, 0)
    scores = gm.mul_mat(jk, Q)
    gm.mul_mat_set_prec(scores, gm.GGML_PREC_F32)
    probs = gm.soft_max_ext(scores, None, scale, 0.0)
    att = gm.reshape(gm.cont(gm.permute(gm.mul_mat(jv, probs), 0, 2, 1, 3)), d, T)
    att = linear("attn1.to_out.0", att)
    h = gm.add(h, gm.mul(att, gate))
    n2 = layer_norm(h, "norm2.weight", "norm2.bias")
    cq = gm.reshape(rms(linear("attn2.to_q", n2), "attn2.norm_q.weight"), dh, H, T)
    CQ = gm.cont(gm.permute(cq, 0, 2, 1, 3))
    cs = gm.mul_mat(lk, CQ)
    gm.mul_mat_set_prec(cs, gm.GGML_PREC_F32)
    cp = gm.soft_max_ext(cs, None, scale, 0.0)
    catt = gm.reshape(gm.cont(gm.permute(gm.mul_mat(lv, cp), 0, 2, 1, 3)), d, T)
    h = gm.add(h, linear("attn2.to_out.0", catt))
    n3 = modulated_norm(h, cscale, cshift)
    u = gm.gelu(linear("ffn.net.0.proj", n3))
    return gm.add(h, gm.mul(linear("ffn.net.2", u), cgate))


def f64_action_layer(W, h, mod, table, apos, pk, pvt, lk, lvt, d, H, T):
    """The F32-profile layer in float64 numpy from textbook operations:
    LayerNorm (biased variance), RMSNorm, the GELU tanh form, 1-D RoPE on
    (even, odd) pairs with theta = pos * 10000^(-2i/dh), softmax attention."""
    dh = d // H
    f = {k: v.astype(np.float64) for k, v in W.items()}
    h = h.astype(np.float64)

    def ln(x):
        mu = x.mean(axis=1, keepdims=True)
        return (x - mu) / np.sqrt(((x - mu) ** 2).mean(axis=1, keepdims=True) + EPS)

    def rms(x, w):
        return x / np.sqrt((x ** 2).mean(axis=1, keepdims=True) + EPS) * w

    def lin(n, x):
        return x @ f[n + ".weight"].T + f[n + ".bias"]

    def rope(x):  # [T, H, dh]
        i = np.arange(dh // 2)
        th = apos[:, None].astype(np.float64) * 10000.0 ** (-2.0 * i / dh)
        c, s = np.cos(th)[:, None, :], np.sin(th)[:, None, :]
        a, b = x[..., 0::2], x[..., 1::2]
        out = np.empty_like(x)
        out[..., 0::2], out[..., 1::2] = a * c - b * s, a * s + b * c
        return out

    def attend(Q, K, Vt):  # Q [H,T,dh], K [H,n,dh], Vt [H,dh,n]
        sc = np.einsum("htd,hnd->htn", Q, K) / np.sqrt(dh)
        p = np.exp(sc - sc.max(axis=2, keepdims=True))
        p /= p.sum(axis=2, keepdims=True)
        return np.einsum("htn,hdn->thd", p, Vt).reshape(T, d)

    m = (mod.astype(np.float64) + table.astype(np.float64)).reshape(6, d)
    n = ln(h) * (1 + m[1]) + m[0]
    q = rope(rms(lin("attn1.to_q", n), f["attn1.norm_q.weight"]).reshape(T, H, dh)).transpose(1, 0, 2)
    k = rope(rms(lin("attn1.to_k", n), f["attn1.norm_k.weight"]).reshape(T, H, dh)).transpose(1, 0, 2)
    v = lin("attn1.to_v", n).reshape(T, H, dh).transpose(1, 2, 0)
    pk64, pv64 = pk.astype(np.float64), pvt.astype(np.float64)
    K = np.concatenate([pk64[:, :1], k, pk64[:, 1:]], axis=1)
    Vt = np.concatenate([pv64[:, :, :1], v, pv64[:, :, 1:]], axis=2)
    h = h + lin("attn1.to_out.0", attend(q, K, Vt)) * m[2]
    n2 = ln(h) * f["norm2.weight"] + f["norm2.bias"]
    cq = rms(lin("attn2.to_q", n2), f["attn2.norm_q.weight"]).reshape(T, H, dh).transpose(1, 0, 2)
    h = h + lin("attn2.to_out.0", attend(cq, lk.astype(np.float64), lvt.astype(np.float64)))
    n3 = ln(h) * (1 + m[4]) + m[3]
    u = lin("ffn.net.0.proj", n3)
    u = 0.5 * u * (1 + np.tanh(np.sqrt(2 / np.pi) * (u + 0.044715 * u ** 3)))
    return h + lin("ffn.net.2", u) * m[5]


@pytest.mark.parametrize("d,H,F,P,NL", [(256, 2, 384, 129, 16), (3072, 24, 14336, 3073, 512)],
                         ids=["small", "config5-layer"])
def test_f32_profile_action_layer(wx, be, orc, d, H, F, P, NL, monkeypatch):
    """The reference's action layer as its F32 reference profile builds it
    (F32 weights, hidden states and caches), through the ggml import, against
    a float64 restatement: max-rel <= 1e-4, cosine >= 0.999999.  At the small
    size the same graph also runs on a backend with the F32 chain fusions off
    (the reference's own switches): both results pass the bar and differ in
    their last bits, so the matched norm_modulation_f32 and gated_residual_f32
    kernels are what ran."""
    print(f"drop-in F32-profile action layer d={d} H={H} F={F} P={P} NL={NL}", flush=True)
    T, dh = 48, d // H
    shapes = {"attn1.to_q.weight": (d, d), "attn1.to_q.bias": (d,), "attn1.to_k.weight": (d, d),
              "attn1.to_k.bias": (d,), "attn1.to_v.weight": (d, d), "attn1.to_v.bias": (d,),
              "attn1.norm_q.weight": (d,), "attn1.norm_k.weight": (d,),
              "attn1.to_out.0.weight": (d, d), "attn1.to_out.0.bias": (d,),
              "norm2.weight": (d,), "norm2.bias": (d,),
              "attn2.to_q.weight": (d, d), "attn2.to_q.bias": (d,), "attn2.norm_q.weight": (d,),
              "attn2.to_out.0.weight": (d, d), "attn2.to_out.0.bias": (d,),
              "ffn.net.0.proj.weight": (F, d), "ffn.net.0.proj.bias": (F,),
              "ffn.net.2.weight": (d, F), "ffn.net.2.bias": (d,)}
    Wh = {}
    for i, (name, shape) in enumerate(shapes.items()):
        n = int(np.prod(shape))
        mean, std = (1.0, 0.02) if "norm" in name else (0.0, 0.02)
        Wh[name] = orc.fill_normal(n, 0x5EED0700 + i, mean, std, orc.F32).reshape(shape)
    h = orc.fill_normal(T * d, 11, 0.0, 1.0, orc.F32).reshape(T, d)
    mod = orc.fill_normal(6 * d, 12, 0.0, 0.5, orc.F32).reshape(6, d)
    table = orc.fill_normal(6 * d, 13, 0.0, 0.1, orc.F32).reshape(6, d)
    apos = np.arange(1, T + 1, dtype=np.int32)
    pk = orc.fill_normal(H * P * dh, 14, 0.0, 1.0, orc.F32).reshape(H, P, dh)
    pvt = orc.fill_normal(H * dh * P, 15, 0.0, 1.0, orc.F32).reshape(H, dh, P)
    lk = orc.fill_normal(H * NL * dh, 16, 0.0, 1.0, orc.F32).reshape(H, NL, dh)
    lvt = orc.fill_normal(H * dh * NL, 17, 0.0, 1.0, orc.F32).reshape(H, dh, NL)
    ref = f64_action_layer(Wh, h, mod, table, apos, pk, pvt, lk, lvt, d, H, T)

    def run(backend):
        r = Runner(wx, backend, 2 << 30 if d > 1024 else 64 << 20)
        W = {name: r.leaf("f32", tuple(reversed(a.shape)), a, name) for name, a in Wh.items()}
        out = action_layer_graph_f32(W, r.leaf("f32", (d, T), h, "hidden"), r.leaf("f32", (d, 6, 1), mod, "time_proj"),
                                     r.leaf("f32", (d, 6), table, "scale_shift_table"),
                                     r.leaf("i32", (T,), apos, "positions"),
                                     r.leaf("f32", (dh, P, H), pk, "prefix_keys"),
                                     r.leaf("f32", (P, dh, H), pvt, "prefix_values"),
                                     r.leaf("f32", (dh, NL, H), lk, "prompt_keys"),
                                     r.leaf("f32", (NL, dh, H), lvt, "prompt_values"), d, H, T, P, NL)
        graph = r.run([out])
        assert {"MUL_MAT", "SOFT_MAX", "CONCAT", "CONT", "ROPE", "NORM", "RMS_NORM", "UNARY", "ADD", "MUL",
                "CPY"} <= {t.op for t in graph.nodes}
        got = r.fetch(out, np.float32, (T, d))
        r.arena.free()
        return got

    got = run(be)
    assert_parity(got, ref, rel=1e-4, cos=0.999999, what=f"F32-profile action layer d={d}")
    if d <= 1024:
        monkeypatch.setenv("WAMX_DISABLE_NORM_MODULATION_FUSION", "1")
        monkeypatch.setenv("WAMX_DISABLE_GATED_RESIDUAL_FUSION", "1")
        be2 = wx.Backend(0)
        try:
            unfused = run(be2)
        finally:
            be2.close()
        assert_parity(unfused, ref, rel=1e-4, cos=0.999999, what="F32-profile action layer, fusions off")
        assert not np.array_equal(got, unfused), "the F32 chains were not matched"
