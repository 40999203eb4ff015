"""A restatement of the ggml graph constructors the GWP-0.5 engine calls, for
the drop-in tests: tensors carry ggml's own shapes, byte strides, op names and
op_params layouts (ggml b9866, not vendored; restated from its upstream
semantics), and a graph is handed to libwamx through wamx_graph_from_ggml the
way a ggml backend shim fills the descriptors from ggml_tensor fields
(ggml_op_name, ggml_unary_op_name, ggml_type_name, ne, nb, op_params, src,
view_src, data).

Test infrastructure only: nothing here computes; the backend does.
"""
from __future__ import annotations

import ctypes as C
import struct

import numpy as np

TYPE_SIZE = {"f32": 4, "f16": 2, "bf16": 2, "i32": 4}
GGML_PREC_F32 = 10          # enum ggml_prec
GGML_ROPE_TYPE_NORMAL = 0


class Desc(C.Structure):
    """struct wamx_ggml_tensor (include/wamx/wamx.h)."""
    _fields_ = [
        ("op", C.c_char_p), ("unary_op", C.c_char_p), ("type", C.c_char_p),
        ("ne", C.c_int64 * 4), ("nb", C.c_size_t * 4), ("op_params", C.c_int32 * 16),
        ("flags", C.c_int32), ("src", C.c_int32 * 10), ("view_src", C.c_int32),
        ("view_offs", C.c_size_t), ("data", C.c_void_p), ("name", C.c_char_p),
    ]


def _f(v: float) -> int:
    return struct.unpack("<i", struct.pack("<f", v))[0]


class T:
    """A ggml_tensor: type name, ne/nb, op name (+ unary name), op_params,
    src[], view_src/view_offs, data (a device address once placed)."""

    def __init__(self, typ, ne, op="NONE", src=(), nb=None, view_of=None, view_offs=0, name=""):
        self.type = typ
        self.ne = list(ne) + [1] * (4 - len(ne))
        if nb is None:
            nb = [TYPE_SIZE[typ]]
            for i in range(1, 4):
                nb.append(nb[-1] * self.ne[i - 1])
        self.nb = list(nb)
        self.op = op
        self.unary = None
        self.params = [0] * 16
        self.src = list(src) + [None] * (10 - len(src))
        self.view_src = None
        self.view_offs = 0
        if view_of is not None:
            self.view_src = view_of.view_src or view_of
            self.view_offs = view_of.view_offs + view_offs
        self.data = None
        self.flags = 0
        self.name = name

    def nelements(self) -> int:
        return int(np.prod(self.ne))

    def nbytes(self) -> int:
        return TYPE_SIZE[self.type] + sum((n - 1) * b for n, b in zip(self.ne, self.nb))

    def is_contiguous(self) -> bool:
        exp = TYPE_SIZE[self.type]
        for n, b in zip(self.ne, self.nb):
            if n != 1 and b != exp:
                return False
            exp *= n
        return True


# --- constructors (ggml.c semantics) ----------------------------------------
def new_tensor(typ, *ne, name=""):
    return T(typ, ne, name=name)


def _view(a, ne, offset, op="VIEW"):
    t = T(a.type, ne, op=op, src=[a], view_of=a, view_offs=offset)
    t.params[0:2] = list(struct.unpack("<ii", struct.pack("<Q", offset)))  # ggml_view_impl stores the offset
    return t


def view_1d(a, ne0, offset):
    return _view(a, [ne0], offset)


def view_2d(a, ne0, ne1, nb1, offset):
    t = _view(a, [ne0, ne1], offset)
    t.nb[1] = nb1
    t.nb[2] = nb1 * ne1
    t.nb[3] = t.nb[2]
    return t


def view_3d(a, ne0, ne1, ne2, nb1, nb2, offset):
    t = _view(a, [ne0, ne1, ne2], offset)
    t.nb[1], t.nb[2] = nb1, nb2
    t.nb[3] = nb2 * ne2
    return t


def reshape(a, *ne):
    assert a.is_contiguous() and int(np.prod(ne)) == a.nelements()
    t = T(a.type, ne, op="RESHAPE", src=[a], view_of=a, view_offs=0)
    return t


def permute(a, ax0, ax1, ax2, ax3):
    axes = (ax0, ax1, ax2, ax3)
    t = T(a.type, a.ne, op="PERMUTE", src=[a], nb=a.nb, view_of=a, view_offs=0)
    ne, nb = [0] * 4, [0] * 4
    for i, ax in enumerate(axes):
        ne[ax], nb[ax] = a.ne[i], a.nb[i]
    t.ne, t.nb = ne, nb
    t.params[0:4] = list(axes)
    return t


def cont(a):
    return T(a.type, a.ne, op="CONT", src=[a])


def cast(a, typ):
    t = T(typ, a.ne, op="CPY", src=[a])
    t.src[1] = t                    # ggml_cast: src[1] is the result itself
    return t


def concat(a, b, dim):
    ne = list(a.ne)
    ne[dim] += b.ne[dim]
    t = T(a.type, ne, op="CONCAT", src=[a, b])
    t.params[0] = dim
    return t


def add(a, b):
    return T(a.type, a.ne, op="ADD", src=[a, b])


def mul(a, b):
    return T(a.type, a.ne, op="MUL", src=[a, b])


def mul_mat_out_type(a, b, typ="f32"):          # native-bf16.patch:566-592
    assert a.ne[0] == b.ne[0]
    return T(typ, [a.ne[1], b.ne[1], b.ne[2], b.ne[3]], op="MUL_MAT", src=[a, b])


def mul_mat(a, b):
    return mul_mat_out_type(a, b, "f32")


def mul_mat_set_prec(t, prec):
    t.params[0] = prec


def soft_max_ext(a, mask, scale, max_bias=0.0):
    t = T(a.type, a.ne, op="SOFT_MAX", src=[a, mask])
    t.params[0], t.params[1] = _f(scale), _f(max_bias)
    return t


def rope_ext(a, pos, n_dims, mode, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor, beta_fast,
             beta_slow):
    t = T(a.type, a.ne, op="ROPE", src=[a, pos, None])
    t.params[0:5] = [0, n_dims, mode, 0, n_ctx_orig]
    for i, v in enumerate((freq_base, freq_scale, ext_factor, attn_factor, beta_fast, beta_slow)):
        t.params[5 + i] = _f(v)
    return t


def _unary(a, name):
    t = T(a.type, a.ne, op="UNARY", src=[a])
    t.unary = name
    return t


def gelu(a):
    return _unary(a, "GELU")


def gelu_erf(a):
    return _unary(a, "GELU_ERF")


def silu(a):
    return _unary(a, "SILU")


def scale(a, s):
    t = T(a.type, a.ne, op="SCALE", src=[a])
    t.params[0], t.params[1] = _f(s), _f(0.0)
    return t


def norm(a, eps):
    t = T(a.type, a.ne, op="NORM", src=[a])
    t.params[0] = _f(eps)
    return t


def rms_norm(a, eps):
    t = T(a.type, a.ne, op="RMS_NORM", src=[a])
    t.params[0] = _f(eps)
    return t


# The native-bf16 patch's fused constructors (native-bf16.patch:594-678).
def gated_residual_bf16(hidden, branch, gate):
    return T(hidden.type, hidden.ne, op="ADD", src=[hidden, branch, gate])


def bias_gelu_bf16(x, bias):
    t = T(x.type, x.ne, op="UNARY", src=[x, bias])
    t.unary = "GELU"
    return t


def norm_modulation_bf16(x, scale_t, shift_t, eps):
    t = T(x.type, x.ne, op="NORM", src=[x, scale_t, shift_t])
    t.params[0] = _f(eps)
    return t


def layer_norm_bf16(x, w, b, eps):
    return norm_modulation_bf16(x, w, b, eps)


def rms_norm_bf16_f32(x, w, eps):
    t = T("f32", x.ne, op="RMS_NORM", src=[x, w])
    t.params[0] = _f(eps)
    return t


def im2col(kernel, inp, s0, s1, p0, p1, d0, d1, is_2d, dst_type):
    KW, KH, IC = kernel.ne[0], kernel.ne[1], inp.ne[2]
    OW = (inp.ne[0] + 2 * p0 - d0 * (KW - 1) - 1) // s0 + 1
    OH = (inp.ne[1] + 2 * p1 - d1 * (KH - 1) - 1) // s1 + 1
    t = T(dst_type, [IC * KH * KW, OW, OH, inp.ne[3]], op="IM2COL", src=[kernel, inp])
    t.params[0:7] = [s0, s1, p0, p1, d0, d1, 1 if is_2d else 0]
    return t


def conv_2d_direct(kernel, inp, s0, s1, p0, p1, d0, d1):
    KW, KH = kernel.ne[0], kernel.ne[1]
    OW = (inp.ne[0] + 2 * p0 - d0 * (KW - 1) - 1) // s0 + 1
    OH = (inp.ne[1] + 2 * p1 - d1 * (KH - 1) - 1) // s1 + 1
    t = T(inp.type, [OW, OH, kernel.ne[3], inp.ne[3]], op="CONV_2D", src=[kernel, inp])
    t.params[0:6] = [s0, s1, p0, p1, d0, d1]
    return t


# --- graphs ------------------------------------------------------------------
class Graph:
    """ggml_cgraph: nodes in post-order of ggml_build_forward_expand (sources
    left to right), leafs are tensors without an op."""

    def __init__(self):
        self.nodes: list[T] = []
        self.leafs: list[T] = []
        self._seen: set[int] = set()

    def expand(self, t: T) -> None:
        stack = [(t, 0)]
        if id(t) in self._seen:
            return
        self._seen.add(id(t))
        while stack:
            cur, i = stack.pop()
            pushed = False
            while i < 10:
                s = cur.src[i]
                i += 1
                if s is not None and id(s) not in self._seen:
                    self._seen.add(id(s))
                    stack.append((cur, i))
                    stack.append((s, 0))
                    pushed = True
                    break
            if pushed:
                continue
            (self.leafs if cur.op == "NONE" else self.nodes).append(cur)

    def tensors(self) -> list[T]:
        """Every tensor the graph reaches, view roots included."""
        out, seen = [], set()

        def add_t(x):
            if x is not None and id(x) not in seen:
                seen.add(id(x))
                out.append(x)
                add_t(x.view_src)
                for s in x.src:
                    add_t(s)

        for x in self.leafs + self.nodes:
            add_t(x)
        return out


def place(tensors, base: int, capacity: int, align: int = 256) -> int:
    """Give every non-view tensor without data an address in [base, base +
    capacity) (no reuse: the ggml-side allocator's job is not under test),
    then resolve views.  Returns the bytes used."""
    off = 0
    for t in tensors:
        if t.data is None and t.view_src is None:
            t.data = base + off
            off += (t.nbytes() + align - 1) // align * align
            assert off <= capacity, "mirror arena too small"
    for t in tensors:
        if t.view_src is not None:
            t.data = t.view_src.data + t.view_offs
    return off


def describe(graph: Graph):
    """Descriptors for wamx_graph_from_ggml: (array, node indices, keepalive)."""
    ts = graph.tensors()
    index = {id(t): i for i, t in enumerate(ts)}
    arr = (Desc * len(ts))()
    keep = []
    for i, t in enumerate(ts):
        d = arr[i]
        for s in (t.op, t.unary, t.type, t.name):
            keep.append(s.encode() if s is not None else None)
        d.op, d.unary_op, d.type, d.name = keep[-4], keep[-3], keep[-2], keep[-1]
        for k in range(4):
            d.ne[k], d.nb[k] = t.ne[k], t.nb[k]
        for k in range(16):
            d.op_params[k] = t.params[k]
        d.flags = t.flags
        for k in range(10):
            d.src[k] = index[id(t.src[k])] if t.src[k] is not None else -1
        d.view_src = index[id(t.view_src)] if t.view_src is not None else -1
        d.view_offs = t.view_offs
        d.data = t.data
    nodes = (C.c_int32 * len(graph.nodes))(*[index[id(t)] for t in graph.nodes])
    return arr, nodes, keep
