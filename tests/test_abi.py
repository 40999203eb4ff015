"""CPU checks of the C ABI: the library loads, exports every symbol the public
header declares, and the host-side IR (constructors, views, graph ordering,
supports_op) behaves like the ggml calls it restates.  No kernel runs here."""
from __future__ import annotations

import ctypes as C

import pytest


def test_exports_every_declared_symbol(wx):
    lib = wx.load()
    names = wx.declared_symbols()
    assert len(names) > 100
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_no_device_needed_to_load(wx):
    assert wx.load().wamx_get_device_count() >= 0


def test_check_finite_f32(wx):
    """The finite-value check the model driver applies to its inputs and
    outputs (copy_f32_tensor, input_validation.cpp:37-42): host only."""
    import numpy as np
    lib = wx.load()
    a = np.linspace(-3, 3, 1000).astype(np.float32)
    assert lib.wamx_check_finite_f32(a.ctypes.data, a.size, b"state") == 0
    assert lib.wamx_check_finite_f32(None, 0, b"state") == 0
    for i, bad in ((0, np.nan), (517, np.inf), (999, -np.inf)):
        b = a.copy()
        b[i] = bad
        assert lib.wamx_check_finite_f32(b.ctypes.data, b.size, b"noise") != 0
        assert wx.last_error() == f"noise contains NaN or Inf (element {i})"
    # the largest finite value and subnormals are finite
    c = np.array([np.finfo(np.float32).max, -np.finfo(np.float32).max, 1e-45], np.float32)
    assert lib.wamx_check_finite_f32(c.ctypes.data, c.size, b"x") == 0
    assert lib.wamx_check_finite_f32(None, 4, b"prompt") != 0


@pytest.fixture
def ctx(wx):
    lib = wx.load()
    c = lib.wamx_init(4096)
    yield c
    lib.wamx_free(c)


def shape(t):
    return tuple(t.contents.ne)


def strides(t):
    return tuple(t.contents.nb)


def test_mul_mat_shape_and_types(wx, ctx):
    lib = wx.load()
    w = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 3072, 9216)   # ne={K, M}
    x = lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 3072, 48)      # ne={K, N}
    y = lib.wamx_mul_mat(ctx, w, x)
    assert shape(y) == (9216, 48, 1, 1) and y.contents.type == wx.TYPE_F32
    yb = lib.wamx_mul_mat_out_type(ctx, w, x, wx.TYPE_BF16)
    assert yb.contents.type == wx.TYPE_BF16 and yb.contents.op == wx.OP["MUL_MAT"]
    lib.wamx_mul_mat_set_prec(y, 10)
    assert y.contents.op_params[0] == 10
    bad = lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 100, 48)
    assert not lib.wamx_mul_mat(ctx, w, bad)
    assert "mul_mat" in wx.last_error()
    # batched broadcast over dim 2 (attention: K [128, n, H] x Q [128, T, H])
    k = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 3121, 24)
    q = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 48, 24)
    assert shape(lib.wamx_mul_mat(ctx, k, q)) == (3121, 48, 24, 1)


def test_permute_transpose_views(wx, ctx):
    lib = wx.load()
    t = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 24, 48)  # [dh, H, T]
    p = lib.wamx_permute(ctx, t, 0, 2, 1, 3)                    # -> [dh, T, H]
    assert shape(p) == (128, 48, 24, 1)
    assert strides(p)[:3] == (2, 2 * 128 * 24, 2 * 128)
    assert not lib.wamx_is_contiguous(p)
    c = lib.wamx_cont(ctx, p)
    assert lib.wamx_is_contiguous(c) and shape(c) == shape(p)
    v = lib.wamx_permute(ctx, t, 1, 2, 0, 3)                    # V layout [T, dh, H]
    assert shape(v) == (48, 128, 24, 1)
    tr = lib.wamx_transpose(ctx, lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 5, 7))
    assert shape(tr) == (7, 5, 1, 1) and strides(tr)[:2] == (20, 4)
    base = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 9216, 48)
    view = lib.wamx_view_2d(ctx, base, 3072, 48, base.contents.nb[1], 3072 * 2)
    assert shape(view) == (3072, 48, 1, 1) and view.contents.view_offs == 6144
    assert C.addressof(view.contents.view_src.contents) == C.addressof(base.contents)
    r = lib.wamx_reshape_3d(ctx, lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 3072, 48), 128, 24, 48)
    assert shape(r) == (128, 24, 48, 1)
    assert not lib.wamx_reshape_2d(ctx, p, 128 * 48, 24)  # non-contiguous source


def test_concat_and_fused_constructors(wx, ctx):
    lib = wx.load()
    a = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 1, 24)
    b = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 48, 24)
    assert shape(lib.wamx_concat(ctx, a, b, 1)) == (128, 49, 24, 1)
    h = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 3072, 48)
    g = lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 3072, 1)
    gr = lib.wamx_gated_residual_bf16(ctx, h, h, g)
    assert gr.contents.op == wx.OP["ADD"] and bool(gr.contents.src[2])
    bias = lib.wamx_new_tensor_1d(ctx, wx.TYPE_BF16, 3072)
    bg = lib.wamx_bias_gelu_bf16(ctx, h, bias)
    assert bg.contents.op == wx.OP["UNARY"] and bg.contents.op_params[0] == wx.UNARY_GELU
    sc = lib.wamx_new_tensor_1d(ctx, wx.TYPE_F32, 3072)
    nm = lib.wamx_norm_modulation_bf16(ctx, h, sc, sc, 1e-6)
    assert nm.contents.op == wx.OP["NORM"] and nm.contents.type == wx.TYPE_BF16
    rn = lib.wamx_rms_norm_bf16_f32(ctx, h, bias, 1e-6)
    assert rn.contents.op == wx.OP["RMS_NORM"] and rn.contents.type == wx.TYPE_F32
    w = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 3072, 14336)
    lin = lib.wamx_linear(ctx, w, h, lib.wamx_new_tensor_1d(ctx, wx.TYPE_BF16, 14336), wx.EPI_BIAS_GELU, None, None)
    assert shape(lin) == (14336, 48, 1, 1) and lin.contents.op == wx.OP["LINEAR"]
    assert not lib.wamx_linear(ctx, w, h, bias, wx.EPI_BIAS, None, None)  # bias length must be M


def test_hilo_constructors(wx, ctx):
    """The f32-score attention pair (build_attention, text_encoder.cpp:26-73):
    QK norm into two bf16 planes, joint attention over one hi/lo source."""
    lib = wx.load()
    x = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 3072, 300)
    w = lib.wamx_new_tensor_1d(ctx, wx.TYPE_BF16, 3072)
    q2 = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 128, 300, 24, 2)
    q = lib.wamx_qk_norm_rope_hilo(ctx, x, w, q2, 0, 2, None, None, None, 1e-6, 10000.0)
    assert q and q.contents.op == wx.OP["QK_NORM_ROPE"] and q.contents.op_params[4] == 1
    assert lib.wamx_backend_supports_op(None, q)
    # one plane is not a hi/lo destination
    assert not lib.wamx_qk_norm_rope_hilo(ctx, x, w, lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 300, 24), 0, 2,
                                          None, None, None, 1e-6, 10000.0)
    kx = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 3072, 64)
    k = lib.wamx_qk_norm_rope_hilo(ctx, kx, w, lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 128, 64, 24, 2), 0, 2,
                                   None, None, None, 1e-6, 10000.0)
    vt = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 64, 128, 24)
    att = lib.wamx_joint_attn_hilo(ctx, q, k, vt, 0.088)
    assert att and shape(att) == (3072, 300, 1, 1) and att.contents.op_params[2] == 1
    assert lib.wamx_backend_supports_op(None, att)
    # planes of the bf16 q alone, too few keys, and V^T rows off 8 keys are refused
    assert not lib.wamx_joint_attn_hilo(ctx, lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 300, 24), k, vt, 0.088)
    k4 = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 128, 4, 24, 2)
    assert not lib.wamx_joint_attn_hilo(ctx, q, k4, lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 4, 128, 24), 0.088)
    k12 = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 128, 12, 24, 2)
    assert not lib.wamx_joint_attn_hilo(ctx, q, k12, lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 12, 128, 24), 0.088)


def test_qk_norm_rope_layer_chunks_constructor(wx, ctx):
    """The Q/K norm over the layers of a packed projection: x [d, T, C] with
    its own chunk stride, per-chunk norm weights [d, C], chunk-strided
    destinations (plain) or 2C contiguous planes (hi/lo); mismatched chunk
    counts, weights and plane counts are refused."""
    lib = wx.load()
    d, T, C, L = 3072, 512, 30, 30
    kv = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 2 * L * d, T)
    x = lib.wamx_view_3d(ctx, kv, d, T, C, kv.contents.nb[1], 2 * d * 2, 0)
    w = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, d, C)
    store = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 128, T, 24, 2 * C)
    nb = store.contents.nb
    dst = lib.wamx_view_4d(ctx, store, 128, T, 24, C, nb[1], nb[2], 2 * nb[3], nb[3])
    k = lib.wamx_qk_norm_rope(ctx, x, w, dst, 0, 2, None, None, None, 1e-6, 10000.0)
    assert k and lib.wamx_backend_supports_op(None, k), wx.last_error()
    kh = lib.wamx_qk_norm_rope_hilo(ctx, x, w, store, 0, 2, None, None, None, 1e-6, 10000.0)
    assert kh and lib.wamx_backend_supports_op(None, kh), wx.last_error()
    w1 = lib.wamx_new_tensor_1d(ctx, wx.TYPE_BF16, d)
    assert lib.wamx_qk_norm_rope(ctx, x, w1, dst, 0, 2, None, None, None, 1e-6, 10000.0)  # one shared weight
    bad = (
        (lib.wamx_view_3d(ctx, kv, d, T, C - 1, kv.contents.nb[1], 2 * d * 2, 0), w, dst, False),  # chunk count
        (x, lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, d, C - 1), dst, False),                     # weights
        (x, w, lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 128, T, 24, 2 * C - 1), True),            # odd planes
        (x, w, dst, True),                                                                        # strided planes
    )
    for xx, ww, dd, hl in bad:
        fn = lib.wamx_qk_norm_rope_hilo if hl else lib.wamx_qk_norm_rope
        assert not fn(ctx, xx, ww, dd, 0, 2, None, None, None, 1e-6, 10000.0)


def test_denoise_glue_constructors(wx, ctx):
    """EULER_STEP, MLP_SMALL and the timestep-batched MODULATION."""
    lib = wx.load()
    a = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 32, 48)
    dt = lib.wamx_new_tensor_1d(ctx, wx.TYPE_F32, 1)
    e = lib.wamx_euler_step(ctx, a, a, dt)
    assert e and e.contents.op == wx.OP["EULER_STEP"] and shape(e) == (32, 48, 1, 1)
    assert lib.wamx_backend_supports_op(None, e)
    assert not lib.wamx_euler_step(ctx, a, lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 32, 47), dt)
    assert not lib.wamx_euler_step(ctx, a, a, lib.wamx_new_tensor_1d(ctx, wx.TYPE_F32, 2))
    w1 = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 32, 128)
    b1 = lib.wamx_new_tensor_1d(ctx, wx.TYPE_BF16, 128)
    w2 = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 128, 96)
    b2 = lib.wamx_new_tensor_1d(ctx, wx.TYPE_BF16, 96)
    m = lib.wamx_mlp_small(ctx, a, w1, b1, w2, b2, 2 | 4)
    assert m and m.contents.op == wx.OP["MLP_SMALL"] and shape(m) == (96, 48, 1, 1)
    assert lib.wamx_backend_supports_op(None, m)
    assert not lib.wamx_mlp_small(ctx, a, w1, b1, w2, b1, 0)  # b2 length must be M2
    wide = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 128, 3072)
    assert not lib.wamx_mlp_small(ctx, lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 128, 48), w2, b2, wide,
                                  lib.wamx_new_tensor_1d(ctx, wx.TYPE_BF16, 3072), 0)  # 3072 wide
    mod = lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 6 * 64, 10)
    tab = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 64, 6, 30)
    md = lib.wamx_modulation(ctx, mod, tab)
    assert md and shape(md) == (64, 6, 30, 10) and lib.wamx_backend_supports_op(None, md)
    assert not lib.wamx_modulation(ctx, lib.wamx_new_tensor_1d(ctx, wx.TYPE_F32, 6 * 64 + 1), tab)


def test_graph_order_and_uid(wx, ctx):
    lib = wx.load()
    x = lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 16, 4)
    y = lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 16, 4)
    a = lib.wamx_add(ctx, x, y)
    m = lib.wamx_mul(ctx, a, x)
    s = lib.wamx_scale(ctx, m, 2.0)
    g = lib.wamx_new_graph(ctx, 64)
    lib.wamx_build_forward_expand(g, s)
    assert lib.wamx_graph_n_nodes(g) == 3
    ops = [lib.wamx_graph_node(g, i).contents.op for i in range(3)]
    assert ops == [wx.OP["ADD"], wx.OP["MUL"], wx.OP["SCALE"]]
    assert C.addressof(lib.wamx_graph_node(g, -1).contents) == C.addressof(s.contents)
    lib.wamx_build_forward_expand(g, s)  # idempotent
    assert lib.wamx_graph_n_nodes(g) == 3
    assert lib.wamx_graph_uid(g) == 0
    lib.wamx_graph_assign_uid(g)
    uid = lib.wamx_graph_uid(g)
    lib.wamx_graph_assign_uid(g)
    assert uid != 0 and lib.wamx_graph_uid(g) == uid
    g2 = lib.wamx_new_graph(ctx, 64)
    lib.wamx_graph_assign_uid(g2)
    assert lib.wamx_graph_uid(g2) != uid


def test_supports_op(wx, ctx):
    lib = wx.load()
    x = lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 64, 8)
    assert lib.wamx_backend_supports_op(None, lib.wamx_soft_max_ext(ctx, x, None, 0.1, 0.0))
    assert lib.wamx_backend_supports_op(None, lib.wamx_norm(ctx, x, 1e-6))
    pos = lib.wamx_new_tensor_1d(ctx, wx.TYPE_I32, 8)
    r = lib.wamx_rope_ext(ctx, lib.wamx_reshape_3d(ctx, x, 16, 4, 8), pos, None, 16, 0, 0, 10000.0, 1.0, 0.0,
                          1.0, 32.0, 1.0)
    assert r and lib.wamx_backend_supports_op(None, r)
    # NEOX-mode rope is not built
    assert not lib.wamx_rope_ext(ctx, lib.wamx_reshape_3d(ctx, x, 16, 4, 8), pos, None, 16, 2, 0, 10000.0, 1.0,
                                 0.0, 1.0, 32.0, 1.0)


def test_ggml_op_map(wx):
    """Names are the ones ggml_op_name() returns (bare, no GGML_OP_ prefix);
    the fused ops of this backend have no ggml name, FLASH_ATTN_EXT is not
    mapped (its operand layout is not JOINT_ATTN's)."""
    lib = wx.load()
    n = lib.wamx_ggml_op_count()
    names = {lib.wamx_ggml_op_name(i).decode(): lib.wamx_ggml_op_to_wamx(i) for i in range(n)}
    for op in ("MUL_MAT", "NORM", "RMS_NORM", "ROPE", "SOFT_MAX", "ADD", "UNARY", "CONCAT", "CPY", "CONT", "IM2COL",
               "VIEW", "PERMUTE", "RESHAPE", "TRANSPOSE", "GET_ROWS", "SCALE", "MUL", "REPEAT", "DUP", "NONE"):
        assert names[op] == wx.OP[op]
    assert not any(k.startswith("GGML_OP_") for k in names)
    assert "FLASH_ATTN_EXT" not in names
    assert not {"LINEAR", "QK_NORM_ROPE", "JOINT_ATTN", "MODULATION"} & set(names)


def test_supports_rejects_malformed_nodes(wx, ctx):
    """supports_op checks what the launch path assumes, for nodes built
    without the constructors (as a mirrored graph is)."""
    lib = wx.load()
    x = lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 64, 8)
    u = lib.wamx_gelu(ctx, x)
    assert lib.wamx_backend_supports_op(None, u)
    for code in (0, 1, 2, 3):        # ggml ABS, SGN, NEG, STEP: never run as GELU / SILU
        u.contents.op_params[0] = code
        assert not lib.wamx_backend_supports_op(None, u)
    # IM2COL reads its kernel size from src[0]: a kernel whose shape does not
    # give the output's shape is refused
    k = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 2, 2, 16, 256)
    inp = lib.wamx_new_tensor_4d(ctx, wx.TYPE_F32, 16, 8, 16, 1)
    col = lib.wamx_im2col(ctx, k, inp, 2, 2, 0, 0, 1, 1, wx.TYPE_BF16)
    assert shape(col) == (64, 8, 4, 1) and list(col.contents.op_params)[:7] == [2, 2, 0, 0, 1, 1, 1]
    assert lib.wamx_backend_supports_op(None, col)
    col.contents.src[0] = lib.wamx_new_tensor_4d(ctx, wx.TYPE_BF16, 3, 3, 16, 256)
    assert not lib.wamx_backend_supports_op(None, col)
    # a JOINT_ATTN whose V^T does not cover the keys
    q = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 48, 4)
    kk = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 256, 4)
    vt = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 256, 128, 4)
    at = lib.wamx_joint_attn(ctx, q, kk, vt, None, None, 0, 0.088)
    assert at and lib.wamx_backend_supports_op(None, at)
    at.contents.src[2] = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 255, 128, 4)
    assert not lib.wamx_backend_supports_op(None, at)
    # no keys at all (softmax over an empty set): refused by the constructor,
    # and by supports_op when a mirrored graph arrives without it
    k0 = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 128, 0, 4)
    v0 = lib.wamx_new_tensor_3d(ctx, wx.TYPE_BF16, 0, 128, 4)
    assert not lib.wamx_joint_attn(ctx, q, k0, v0, None, None, 0, 0.088)
    assert b"no keys" in lib.wamx_last_error()
    at0 = lib.wamx_joint_attn(ctx, q, kk, vt, None, None, 0, 0.088)
    at0.contents.src[1], at0.contents.src[2] = k0, v0
    assert not lib.wamx_backend_supports_op(None, at0)
    # an empty first source beside a non-empty second one is a valid key set
    assert lib.wamx_joint_attn(ctx, q, k0, v0, kk, vt, 0, 0.088)
    # MUL_MAT whose result shape does not follow from its operands
    w = lib.wamx_new_tensor_2d(ctx, wx.TYPE_BF16, 64, 32)
    mm = lib.wamx_mul_mat(ctx, w, x)
    assert lib.wamx_backend_supports_op(None, mm)
    mm.contents.ne[0] = 31
    assert not lib.wamx_backend_supports_op(None, mm)
    # ROPE with YaRN / frequency scaling is not what the kernel computes
    pos = lib.wamx_new_tensor_1d(ctx, wx.TYPE_I32, 8)
    r = lib.wamx_rope_ext(ctx, lib.wamx_reshape_3d(ctx, x, 16, 4, 8), pos, None, 16, 0, 0, 10000.0, 1.0, 0.0,
                          1.0, 32.0, 1.0)
    assert lib.wamx_backend_supports_op(None, r)
    r.contents.op_params[6] = 0x3F000000   # freq_scale 0.5
    assert not lib.wamx_backend_supports_op(None, r)


def test_soft_max_mask_constructor(wx, ctx):
    lib = wx.load()
    s = lib.wamx_new_tensor_3d(ctx, wx.TYPE_F32, 100, 48, 24)
    m = lib.wamx_new_tensor_3d(ctx, wx.TYPE_F32, 100, 48, 24)
    sm = lib.wamx_soft_max_ext(ctx, s, m, 0.088, 0.0)
    assert sm and lib.wamx_backend_supports_op(None, sm)
    assert C.addressof(sm.contents.src[1].contents) == C.addressof(m.contents)
    m16 = lib.wamx_new_tensor_2d(ctx, wx.TYPE_F16, 100, 64)      # broadcast over heads, padded rows
    assert lib.wamx_soft_max_ext(ctx, s, m16, 0.088, 0.0)
    assert not lib.wamx_soft_max_ext(ctx, s, lib.wamx_new_tensor_2d(ctx, wx.TYPE_F32, 99, 48), 0.088, 0.0)
    assert not lib.wamx_soft_max_ext(ctx, s, m, 0.088, 8.0)     # ALiBi


def test_graph_from_ggml_translation(wx, ctx):
    """A graph described the way a ggml shim describes it (names, ggml
    op_params) mirrors into wamx tensors with the same shapes, strides, data
    addresses and sources; unary ops are matched by name; unknown names fail
    with the tensor named."""
    import ggml_mirror as gm
    lib = wx.load()
    x = gm.new_tensor("bf16", 64, 8, name="x")
    w = gm.new_tensor("bf16", 64, 32, name="w")
    b = gm.new_tensor("bf16", 32, name="b")
    y = gm.add(gm.mul_mat_out_type(w, x, "bf16"), b)
    g = gm.gelu_erf(gm.cast(y, "f32"))
    v = gm.view_2d(g, 16, 8, g.nb[1], 16 * 4)
    out = gm.cont(gm.permute(gm.reshape(gm.cont(v), 4, 4, 8), 0, 2, 1, 3))
    graph = gm.Graph()
    graph.expand(out)
    gm.place(graph.tensors(), 1 << 20, 1 << 20)
    arr, nodes, _keep = gm.describe(graph)
    wg = lib.wamx_graph_from_ggml(ctx, arr, len(arr), nodes, len(nodes))
    assert wg, wx.last_error()
    n = lib.wamx_graph_n_nodes(wg)
    assert n == len(graph.nodes)
    for i, t in enumerate(graph.nodes):
        m = lib.wamx_graph_node(wg, i).contents
        assert wx.OP_NAMES[m.op] == t.op
        assert list(m.ne) == t.ne and list(m.nb) == t.nb and m.data == t.data
        if t.op == "UNARY":
            assert m.op_params[0] == wx.UNARY_GELU_ERF
        assert lib.wamx_backend_supports_op(None, lib.wamx_graph_node(wg, i)), t.op
    # a view keeps its root and offset
    mv = [lib.wamx_graph_node(wg, i).contents for i in range(n) if graph.nodes[i] is v][0]
    assert mv.view_offs == 64 and mv.view_src.contents.data == g.data
    # unknown names are refused, naming the tensor
    bad = gm.new_tensor("f32", 4, name="odd")
    z = gm.T("f32", [4], op="FLASH_ATTN_EXT", src=[bad])
    z.name = "fa"
    gr2 = gm.Graph()
    gr2.expand(z)
    gm.place(gr2.tensors(), 1 << 20, 1 << 16)
    arr2, nodes2, _k2 = gm.describe(gr2)
    assert not lib.wamx_graph_from_ggml(ctx, arr2, len(arr2), nodes2, len(nodes2))
    assert "FLASH_ATTN_EXT" in wx.last_error() and "fa" in wx.last_error()
    ab = gm._unary(gm.new_tensor("f32", 4), "ABS")
    gr3 = gm.Graph()
    gr3.expand(ab)
    gm.place(gr3.tensors(), 1 << 20, 1 << 16)
    arr3, nodes3, _k3 = gm.describe(gr3)
    assert not lib.wamx_graph_from_ggml(ctx, arr3, len(arr3), nodes3, len(nodes3))
    assert "ABS" in wx.last_error()
