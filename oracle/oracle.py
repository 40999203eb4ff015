"""ctypes wrapper of oracle/liboracle.so — the CPU restatement of the
reference arithmetic (test infrastructure: imported only by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg).

Arrays are numpy; bf16 arrays are uint16 bit patterns.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

F32, BF16 = 0, 30
EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_GATED, EPI_BIAS_RESIDUAL = 0, 1, 2, 3, 4

_lib = None


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
    lib = C.CDLL(str(LIB_PATH))
    vp, i64, f32 = C.c_void_p, C.c_int64, C.c_float
    sig = {
        "orc_f32_to_bf16": (C.c_uint16, [f32]),
        "orc_bf16_to_f32": (f32, [C.c_uint16]),
        "orc_num_threads": (C.c_int, []),
        "orc_gelu_tanh": (f32, [f32]),
        "orc_gelu_erf": (f32, [f32]),
        "orc_mul_mat": (None, [vp, i64, vp, C.c_int, i64, vp, C.c_int, i64, i64, i64, i64]),
        "orc_linear": (None, [vp, vp, C.c_int, vp, C.c_int, vp, vp, vp, i64, i64, i64]),
        "orc_norm_mod_bf16": (None, [vp, i64, vp, vp, i64, vp, i64, i64, f32]),
        "orc_layer_norm_bf16": (None, [vp, i64, vp, vp, vp, i64, i64, f32]),
        "orc_rms_norm_bf16_f32": (None, [vp, i64, vp, vp, i64, i64, f32]),
        "orc_norm_mod_f32": (None, [vp, i64, vp, vp, i64, vp, i64, i64, f32]),
        "orc_gated_residual_bf16": (None, [vp, vp, vp, C.c_int, i64, vp, i64, i64]),
        "orc_gated_residual_f32": (None, [vp, vp, vp, i64, vp, i64, i64]),
        "orc_bias_gelu_bf16": (None, [vp, vp, vp, i64, i64]),
        "orc_rope_f32": (None, [vp, vp, vp, i64, i64, i64, C.c_int, f32]),
        "orc_qk_norm_rope": (None, [vp, i64, vp, vp, i64, i64, i64, i64, i64, C.c_int, vp, vp, vp, f32, f32]),
        "orc_softmax_f32": (None, [vp, vp, i64, i64, f32]),
        "orc_attention": (None, [vp, vp, vp, i64, i64, vp, vp, i64, i64, i64, vp, i64, i64, i64, f32]),
        "orc_modulation": (None, [vp, vp, vp, i64, i64]),
        "orc_flow_schedule": (None, [C.c_int, f32, vp, vp]),
        "orc_timestep_embedding": (None, [f32, i64, vp]),
        "orc_fill_normal": (None, [vp, C.c_int, i64, C.c_uint64, f32, f32]),
        "orc_set_port": (None, [C.c_int]),
        "orc_get_port": (C.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def num_threads() -> int:
    return int(load().orc_num_threads())


def set_port(on: bool) -> None:
    """Route the products and attentions through the fp32 CPU port
    (cpu_port.c), for timing; off for parity."""
    load().orc_set_port(1 if on else 0)


def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    f = load().orc_f32_to_bf16
    flat, of = x.reshape(-1), out.reshape(-1)
    for i in range(flat.size):
        of[i] = f(float(flat[i]))
    return out


def gelu_tanh(x: float) -> float:
    return float(load().orc_gelu_tanh(x))


def gelu_erf(x: float) -> float:
    return float(load().orc_gelu_erf(x))


def mul_mat(w_bf16, x, y_type=F32) -> np.ndarray:
    """w bf16 [M][K], x f32|bf16(uint16) [N][K] -> y [N][M] (f32 or bf16 bits)."""
    w = _c(w_bf16, np.uint16)
    M, K = w.shape
    x_type = BF16 if x.dtype == np.uint16 else F32
    x = _c(x, np.uint16 if x_type == BF16 else np.float32)
    N = x.shape[0]
    y = np.empty((N, M), np.float32 if y_type == F32 else np.uint16)
    load().orc_mul_mat(_p(w), K, _p(x), x_type, K, _p(y), y_type, M, M, N, K)
    return y


def linear(w, x, bias=None, epi=EPI_NONE, residual=None, gate=None) -> np.ndarray:
    w = _c(w, np.uint16)
    M, K = w.shape
    x_type = BF16 if x.dtype == np.uint16 else F32
    x = _c(x, np.uint16 if x_type == BF16 else np.float32)
    N = x.shape[0]
    b = None if bias is None else _c(bias, np.uint16)
    r = None if residual is None else _c(residual, np.uint16)
    g = None if gate is None else _c(gate, np.float32)
    y = np.empty((N, M), np.uint16)
    load().orc_linear(_p(w), _p(x), x_type, _p(b), epi, _p(r), _p(g), _p(y), M, N, K)
    return y


def norm_mod_bf16(x, scale, shift, eps) -> np.ndarray:
    x = _c(x, np.uint16)
    rows, cols = x.shape
    scale, shift = _c(scale, np.float32), _c(shift, np.float32)
    ss = 0 if scale.ndim == 1 else cols
    y = np.empty_like(x)
    load().orc_norm_mod_bf16(_p(x), cols, _p(scale), _p(shift), ss, _p(y), rows, cols, eps)
    return y


def layer_norm_bf16(x, w, b, eps) -> np.ndarray:
    x = _c(x, np.uint16)
    rows, cols = x.shape
    y = np.empty_like(x)
    load().orc_layer_norm_bf16(_p(x), cols, _p(_c(w, np.uint16)), _p(_c(b, np.uint16)), _p(y), rows, cols, eps)
    return y


def rms_norm_bf16_f32(x, w, eps) -> np.ndarray:
    x = _c(x, np.uint16)
    rows, cols = x.shape
    y = np.empty((rows, cols), np.float32)
    load().orc_rms_norm_bf16_f32(_p(x), cols, _p(_c(w, np.uint16)), _p(y), rows, cols, eps)
    return y


def norm_mod_f32(x, scale, shift, eps) -> np.ndarray:
    x = _c(x, np.float32)
    rows, cols = x.shape
    scale, shift = _c(scale, np.float32), _c(shift, np.float32)
    ss = 0 if scale.ndim == 1 else cols
    y = np.empty_like(x)
    load().orc_norm_mod_f32(_p(x), cols, _p(scale), _p(shift), ss, _p(y), rows, cols, eps)
    return y


def gated_residual_bf16(h, b, g) -> np.ndarray:
    h, b = _c(h, np.uint16), _c(b, np.uint16)
    rows, cols = h.shape
    g_type = BF16 if g.dtype == np.uint16 else F32
    g = _c(g, np.uint16 if g_type == BF16 else np.float32)
    gs = 0 if g.ndim == 1 else cols
    y = np.empty_like(h)
    load().orc_gated_residual_bf16(_p(h), _p(b), _p(g), g_type, gs, _p(y), rows, cols)
    return y


def gated_residual_f32(r, b, g) -> np.ndarray:
    r, b, g = _c(r, np.float32), _c(b, np.float32), _c(g, np.float32)
    rows, cols = r.shape
    gs = 0 if g.ndim == 1 else cols
    y = np.empty_like(r)
    load().orc_gated_residual_f32(_p(r), _p(b), _p(g), gs, _p(y), rows, cols)
    return y


def bias_gelu_bf16(x, bias) -> np.ndarray:
    x, bias = _c(x, np.uint16), _c(bias, np.uint16)
    y = np.empty_like(x)
    load().orc_bias_gelu_bf16(_p(x), _p(bias), _p(y), x.size, bias.size)
    return y


def rope_f32(x, pos, n_dims, base=10000.0) -> np.ndarray:
    """x f32 [tokens][heads][head_dim]."""
    x = _c(x, np.float32)
    T, H, D = x.shape
    y = np.empty_like(x)
    load().orc_rope_f32(_p(x), _p(_c(pos, np.int32)), _p(y), D, H, T, n_dims, base)
    return y


def qk_norm_rope(x, w, heads, head_dim, rope_mode, pos0=None, pos1=None, pos2=None, eps=1e-6, base=10000.0,
                 dst=None, tok0=0) -> np.ndarray:
    """x bf16 [T][heads*head_dim] -> dst bf16 [heads][dst_tokens][head_dim]."""
    x = _c(x, np.uint16)
    T = x.shape[0]
    if dst is None:
        dst = np.zeros((heads, T, head_dim), np.uint16)
    ps = [None if p is None else _c(p, np.int32) for p in (pos0, pos1, pos2)]
    load().orc_qk_norm_rope(_p(x), x.shape[1], _p(_c(w, np.uint16)), _p(dst), heads, head_dim, T, dst.shape[1], tok0,
                            rope_mode, _p(ps[0]), _p(ps[1]), _p(ps[2]), eps, base)
    return dst


def softmax_f32(x, scale=1.0) -> np.ndarray:
    x = _c(x, np.float32)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    y = np.empty_like(x)
    load().orc_softmax_f32(_p(x), _p(y), rows, cols, scale)
    return y


def attention(q, k_a, vt_a, k_b=None, vt_b=None, na_split=0, scale=None) -> np.ndarray:
    """q [H][tq][dh], k_a [H][na][dh], vt_a [H][dh][ld_a] (bf16) -> out bf16 [tq][H*dh]."""
    q, k_a, vt_a = _c(q, np.uint16), _c(k_a, np.uint16), _c(vt_a, np.uint16)
    H, tq, dh = q.shape
    na = k_a.shape[1]
    nb = 0 if k_b is None else k_b.shape[1]
    kb = None if k_b is None else _c(k_b, np.uint16)
    vb = None if vt_b is None else _c(vt_b, np.uint16)
    scale = 1.0 / np.sqrt(dh) if scale is None else scale
    out = np.empty((tq, H * dh), np.uint16)
    load().orc_attention(_p(q), _p(k_a), _p(vt_a), na, vt_a.shape[2], _p(kb), _p(vb), nb,
                         0 if vb is None else vb.shape[2], na_split, _p(out), H, dh, tq, float(scale))
    return out


def modulation(mod, tables) -> np.ndarray:
    mod, tables = _c(mod, np.uint16), _c(tables, np.uint16)
    per = mod.size
    layers = tables.size // per
    out = np.empty((layers, per), np.float32)
    load().orc_modulation(_p(mod), _p(tables), _p(out), per, layers)
    return out


def flow_schedule(steps: int, shift: float):
    t = np.empty(steps, np.float32)
    s = np.empty(steps + 1, np.float32)
    load().orc_flow_schedule(steps, shift, _p(t), _p(s))
    return t, s


def timestep_embedding(t: float, dim: int = 256) -> np.ndarray:
    out = np.empty(dim, np.float32)
    load().orc_timestep_embedding(t, dim, _p(out))
    return out


def fill_normal(n: int, seed: int, mean=0.0, std=1.0, dtype=F32) -> np.ndarray:
    out = np.empty(n, np.float32 if dtype == F32 else np.uint16)
    load().orc_fill_normal(_p(out), dtype, n, seed & (2**64 - 1), mean, std)
    return out


# ---------------------------------------------------------------------------
# Full MoT step (oracle_mot.c)
# ---------------------------------------------------------------------------
class GwpConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "hidden", "n_heads", "head_dim", "ffn_dim", "action_hidden", "action_ffn_dim",
        "action_chunk", "action_dim", "grid_h", "grid_w", "n_lang", "t5_hidden", "z_dim",
        "num_steps", "enc_hidden")] + [("shift", C.c_float), ("eps", C.c_float)]


_WEIGHT_FN = C.CFUNCTYPE(C.c_void_p, C.c_void_p, C.c_char_p)


class Gwp:
    """CPU restatement of the synthetic GWP-0.5 MoT over named bf16 weights."""

    def __init__(self, cfg: dict, weights: dict):
        lib = load()
        for name, res, args in (
                ("orc_gwp_new", C.c_void_p, [C.POINTER(GwpConfig), _WEIGHT_FN, C.c_void_p]),
                ("orc_gwp_free", None, [C.c_void_p]),
                ("orc_gwp_prompt", C.c_int, [C.c_void_p, C.c_void_p, C.c_int]),
                ("orc_gwp_prefix", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]),
                ("orc_gwp_denoise", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]),
                ("orc_gwp_prefix_key", C.c_void_p, [C.c_void_p, C.c_int]),
                ("orc_gwp_prefix_value", C.c_void_p, [C.c_void_p, C.c_int]),
                ("orc_gwp_prompt_key", C.c_void_p, [C.c_void_p, C.c_int]),
                ("orc_gwp_prompt_value", C.c_void_p, [C.c_void_p, C.c_int]),
                ("orc_gwp_prefix_hidden_in", C.c_void_p, [C.c_void_p, C.c_int]),
                ("orc_gwp_set_visual_positions", C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
                ("orc_gwp_action_prompt", C.c_void_p, [C.c_void_p]),
                ("orc_gwp_velocity", C.c_void_p, [C.c_void_p, C.c_int])):
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        self.lib = lib
        self.cfg = dict(cfg)
        self.weights = {k.encode(): np.ascontiguousarray(v, np.uint16) for k, v in weights.items()}

        def lookup(_user, name):
            a = self.weights.get(name)
            return None if a is None else a.ctypes.data

        self._cb = _WEIGHT_FN(lookup)
        c = GwpConfig(**{k: self.cfg[k] for k, _ in GwpConfig._fields_})
        self.ptr = lib.orc_gwp_new(C.byref(c), self._cb, None)
        c_ = self.cfg
        self.d = c_["n_heads"] * c_["head_dim"]
        self.P = 1 + c_["grid_h"] * c_["grid_w"]

    def close(self):
        if self.ptr:
            self.lib.orc_gwp_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def prompt(self, prompt, layers=0):
        p = _c(prompt, np.float32)
        if self.lib.orc_gwp_prompt(self.ptr, _p(p), layers) != 0:
            raise RuntimeError("oracle prompt projection failed (missing weight)")

    def prefix(self, state, latent, prompt, layers=0):
        s, lt, p = _c(state, np.float32), _c(latent, np.float32), _c(prompt, np.float32)
        if self.lib.orc_gwp_prefix(self.ptr, _p(s), _p(lt), _p(p), layers) != 0:
            raise RuntimeError("oracle prefix failed (missing weight)")

    def denoise(self, noise, layers=0, steps=0):
        n = _c(noise, np.float32)
        out = np.empty_like(n)
        if self.lib.orc_gwp_denoise(self.ptr, _p(n), _p(out), layers, steps) != 0:
            raise RuntimeError("oracle denoise failed (missing weight)")
        return out

    def velocity(self, step):
        """The decoder output (velocity) of denoise step `step` of the last
        denoise, f32 [T * A]."""
        c = self.cfg
        ptr = self.lib.orc_gwp_velocity(self.ptr, step)
        if not ptr:
            raise RuntimeError(f"oracle velocity of step {step} unavailable")
        n = c["action_chunk"] * c["action_dim"]
        return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_float)), shape=(n,)).copy()

    def _arr(self, ptr, shape):
        n = int(np.prod(shape))
        return np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_uint16)), shape=(n,)).reshape(shape).copy()

    def prefix_key(self, layer):
        c = self.cfg
        return self._arr(self.lib.orc_gwp_prefix_key(self.ptr, layer), (c["n_heads"], self.P, c["head_dim"]))

    def prefix_value(self, layer):
        c = self.cfg
        return self._arr(self.lib.orc_gwp_prefix_value(self.ptr, layer), (c["n_heads"], c["head_dim"], self.P))

    def prompt_key(self, layer):
        c = self.cfg
        return self._arr(self.lib.orc_gwp_prompt_key(self.ptr, layer), (c["n_heads"], c["n_lang"], c["head_dim"]))

    def action_prompt(self):
        c = self.cfg
        return self._arr(self.lib.orc_gwp_action_prompt(self.ptr), (c["n_lang"], c["action_hidden"]))

    def prompt_value(self, layer):
        c = self.cfg
        return self._arr(self.lib.orc_gwp_prompt_value(self.ptr, layer), (c["n_heads"], c["head_dim"], c["n_lang"]))

    def prefix_hidden_in(self, which):
        """0: the state encoder's output [1][action_hidden]; 1: the patch
        embedding's output [nimg][hidden] (the prefix pass's layer-0 inputs)."""
        c = self.cfg
        shape = (1, c["action_hidden"]) if which == 0 else (c["grid_h"] * c["grid_w"], self.d)
        return self._arr(self.lib.orc_gwp_prefix_hidden_in(self.ptr, which), shape)

    def set_visual_positions(self, t=None, h=None, w=None):
        """(t, h, w) positions of the visual tokens for the next prefix pass
        (None: the grid's own, semantics.cpp:235-257)."""
        if t is None:
            self.lib.orc_gwp_set_visual_positions(self.ptr, None, None, None)
            return
        self._pos = [_c(a, np.int32) for a in (t, h, w)]
        self.lib.orc_gwp_set_visual_positions(self.ptr, *[_p(a) for a in self._pos])


# ---------------------------------------------------------------------------
# The synthetic weights of the model driver (wamx_gwp_create /
# wamx_gwp_init_synthetic), generated on the host with fill_normal.
# ---------------------------------------------------------------------------
def fnv1a(s: str) -> int:
    h = 1469598103934665603
    for ch in s.encode():
        h ^= ch
        h = (h * 1099511628211) & (2**64 - 1)
    return h


def gwp_weight_specs(cfg: dict):
    """[(name, elements)] of every named weight of the synthetic GWP-0.5
    model, with the reference's GGUF names (weights.cpp:116-167)."""
    c = cfg
    d = c["n_heads"] * c["head_dim"]
    da, E, A, L = c["action_hidden"], c["enc_hidden"], c["action_dim"], c["n_layers"]
    out = [("gwp.patch_embedding.weight", 4 * c["z_dim"] * d), ("gwp.patch_embedding.bias", d)]

    def lin(name, i, o):
        out.extend([(name + ".weight", i * o), (name + ".bias", o)])

    for p, i, o in (("gwp.state_encoder", A, da), ("gwp.action_encoder", A, da), ("gwp.action_decoder", da, A)):
        lin(p + ".in_proj", i, E)
        lin(p + ".mid_proj", E, E)
        lin(p + ".out_proj", E, o)
    for p, w in (("gwp.action_condition_embedder", da), ("gwp.condition_embedder", d)):
        lin(p + ".time_embedder.linear_1", 256, w)
        lin(p + ".time_embedder.linear_2", w, w)
        lin(p + ".time_proj", w, 6 * w)
        lin(p + ".text_embedder.linear_1", c["t5_hidden"], w)
        lin(p + ".text_embedder.linear_2", w, w)
    out.append(("gwp.action_scale_shift_table", 2 * da))
    out.append(("gwp.blocks.action_expert.scale_shift_table", 6 * da * L))
    out.append(("gwp.blocks.visual_expert.scale_shift_table", 6 * d * L))
    for l in range(L):
        for ex, w, f in (("action_expert", da, c["action_ffn_dim"]), ("visual_expert", d, c["ffn_dim"])):
            p = f"gwp.blocks.{l}.{ex}"
            lin(p + ".attn1.to_qkv", w, 3 * d)
            out.extend([(p + ".attn1.norm_q.weight", d), (p + ".attn1.norm_k.weight", d)])
            lin(p + ".attn1.to_out.0", d, w)
            out.extend([(p + ".norm2.weight", w), (p + ".norm2.bias", w)])
            lin(p + ".attn2.to_q", w, d)
            lin(p + ".attn2.to_k", w, d)
            lin(p + ".attn2.to_v", w, d)
            out.extend([(p + ".attn2.norm_q.weight", d), (p + ".attn2.norm_k.weight", d)])
            lin(p + ".attn2.to_out.0", d, w)
            lin(p + ".ffn.net.0.proj", w, f)
            lin(p + ".ffn.net.2", f, w)
    return out


def gwp_fill_rule(name: str, wstd: float):
    """(mean, std) of a weight in the synthetic fill: biases N(0, 0.02), norm
    weights 1 + N(0, 0.02), scale/shift tables N(0, 0.1), matrices N(0, wstd)."""
    if name.endswith(".bias"):
        return 0.0, 0.02
    if name.endswith(("norm_q.weight", "norm_k.weight", "norm2.weight")):
        return 1.0, 0.02
    if "scale_shift_table" in name:
        return 0.0, 0.1
    return 0.0, wstd


def gwp_synthetic_weight(name: str, n: int, seed: int, wstd: float = 0.02) -> np.ndarray:
    mean, std = gwp_fill_rule(name, wstd)
    return fill_normal(n, (seed ^ fnv1a(name)) & (2**64 - 1), mean, std, BF16)


def gwp_synthetic_weights(cfg: dict, seed: int, wstd: float = 0.02) -> dict:
    return {n: gwp_synthetic_weight(n, k, seed, wstd) for n, k in gwp_weight_specs(cfg)}


# ---------------------------------------------------------------------------
# UMT5 text encoder (src/models/gwp05/engine/text_encoder.cpp:13-24, :26-73,
# :112-204), restated in numpy with float64 accumulation and the reference's
# rounding points: activations rounded to bf16 where a bf16 weight multiplies
# them (stock MUL_MAT converts src1 to the weight's vec-dot type), f32 K.Q and
# V.P kept unrounded, bf16 weights widened exactly.
# ---------------------------------------------------------------------------
_libm = None


def _logf(x: float) -> float:
    """The C library's single-precision log (the reference's std::log(float))."""
    global _libm
    if _libm is None:
        import ctypes.util
        _libm = C.CDLL(ctypes.util.find_library("m"))
        _libm.logf.restype, _libm.logf.argtypes = C.c_float, [C.c_float]
    return _libm.logf(x)


def t5_relative_bucket(relative: int, buckets: int = 32, max_distance: int = 128) -> int:
    """text_encoder.cpp:13-24: half the buckets per direction (key after the
    query: upper half), exact below half/2, logarithmic up to max_distance,
    in single precision."""
    half = buckets // 2
    base = half if relative > 0 else 0
    d = abs(relative)
    exact = half // 2
    if d < exact:
        return base + d
    r = np.float32(_logf(np.float32(d) / np.float32(exact))) / np.float32(_logf(np.float32(max_distance) / np.float32(exact)))
    return base + min(half - 1, exact + int(np.float32(r) * np.float32(half - exact)))


def t5_weight_specs(c: dict):
    """[(name, ggml ne)] of the UMT5 encoder's weights (reference names)."""
    d, inner, F, H = c["hidden"], c["heads"] * c["head_dim"], c["ffn_dim"], c["heads"]
    out = [("t5.shared.weight", (d, c["vocab"]))]
    for l in range(c["layers"]):
        p = f"t5.encoder.block.{l}.layer"
        a = p + ".0.SelfAttention"
        out += [(a + ".q.weight", (d, inner)), (a + ".k.weight", (d, inner)), (a + ".v.weight", (d, inner)),
                (a + ".o.weight", (inner, d)), (a + ".relative_attention_bias.weight", (H, 32)),
                (p + ".0.layer_norm.weight", (d,)), (p + ".1.DenseReluDense.wi_0.weight", (d, F)),
                (p + ".1.DenseReluDense.wi_1.weight", (d, F)), (p + ".1.DenseReluDense.wo.weight", (F, d)),
                (p + ".1.layer_norm.weight", (d,))]
    out.append(("t5.encoder.final_layer_norm.weight", (d,)))
    return out


def _bf(a) -> np.ndarray:
    """bf16 bit patterns -> float64."""
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def bf16_rne(x) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even, NaN kept quiet: the
    element rule of orc_f32_to_bf16, vectorised (tests check the two agree)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    return np.where(nan, (u >> 16) | 0x40, r).astype(np.uint16)


def _r(x) -> np.ndarray:
    """Round to bf16 (RNE) and widen: a bf16-weight MUL_MAT's view of its f32 input."""
    return _bf(bf16_rne(np.asarray(x, np.float32)))


def _rms(x, w, eps):
    """ggml_rms_norm over the row, then MUL by the widened weight (weights.cpp:904-917)."""
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * w


def _gelu(x):
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def t5_encode(c: dict, weights: dict, tokens, mask=None, eps: float = 1e-6) -> np.ndarray:
    """run_t5 (text_encoder.cpp:112-204): f32 [max_tokens][hidden], rows past
    the mask's valid prefix zero.  weights: name -> bf16 bit patterns in the
    ggml layout of t5_weight_specs (row-major [ne1][ne0])."""
    tokens = np.asarray(tokens, np.int64)
    n = tokens.size if mask is None else int(np.sum(mask))
    d, H, dh, F = c["hidden"], c["heads"], c["head_dim"], c["ffn_dim"]
    W = {k: _bf(v).reshape(tuple(reversed(s))) for (k, s), v in ((ks, weights[ks[0]]) for ks in t5_weight_specs(c))}
    h = W["t5.shared.weight"][tokens[:n]]                                   # get_rows: [n, d]
    bucket = np.array([[t5_relative_bucket(k - q) for k in range(n)] for q in range(n)])  # [query, key]
    for l in range(c["layers"]):
        p = f"t5.encoder.block.{l}.layer"
        a = p + ".0.SelfAttention"
        bias = W[a + ".relative_attention_bias.weight"][bucket]           # [query, key, head]
        x = _rms(h, W[p + ".0.layer_norm.weight"], eps)
        xr = _r(x)
        q, k, v = (xr @ W[a + f".{m}.weight"].T for m in "qkv")          # [n, H*dh] f32 outputs
        q, k, v = (t.reshape(n, H, dh).transpose(1, 0, 2) for t in (q, k, v))
        s = q @ k.transpose(0, 2, 1) + bias.transpose(2, 0, 1)              # scale 1, bias as the mask
        s = s - s.max(axis=-1, keepdims=True)
        pr = np.exp(s)
        pr /= pr.sum(axis=-1, keepdims=True)
        att = (pr @ v).transpose(1, 0, 2).reshape(n, H * dh)
        h = h + _r(att) @ W[a + ".o.weight"].T
        f = p + ".1.DenseReluDense"
        xr = _r(_rms(h, W[p + ".1.layer_norm.weight"], eps))
        g = _gelu(xr @ W[f + ".wi_0.weight"].T) * (xr @ W[f + ".wi_1.weight"].T)
        h = h + _r(g) @ W[f + ".wo.weight"].T
    y = _rms(h, W["t5.encoder.final_layer_norm.weight"], eps)
    out = np.zeros((c["max_tokens"], d))
    out[:n] = y
    return out


# ---------------------------------------------------------------------------
# Vision front-end: the three-view canvas and its 2x2 patchify
# (src/models/gwp05/engine/vae.cpp:1-133, compose_and_patchify and
# resize_center_crop), and ggml_conv_2d_direct (the VAE convolution,
# vae.cpp:140-157).  Filter parameters in float32 as the reference computes
# them; the resampling sums in float64.
# ---------------------------------------------------------------------------
def _resize_axis(src: int, resized: int, dst: int):
    """Taps of every output position of one axis (vae.cpp:17-44): the
    triangle filter of support max(1, 1/scale) around the source centre of
    the cropped output position, zero taps dropped, indices clamped to the
    image, weights normalised to sum 1.  Returns (indices, weights) lists."""
    f = np.float32
    crop = (resized - dst) // 2
    scale = f(resized) / f(src)
    support = max(f(1.0), f(1.0) / scale)
    out = []
    for o in range(dst):
        center = (f(o + crop) + f(0.5)) / scale - f(0.5)
        first, last = int(np.ceil(center - support)), int(np.floor(center + support))
        idx, wts = [], []
        for s in range(first, last + 1):
            w = max(f(0.0), f(1.0) - f(abs(f(s) - center)) / support)
            if w == 0.0:
                continue
            idx.append(min(max(s, 0), src - 1))
            wts.append(w)
        total = f(0.0)
        for w in wts:
            total = f(total + w)
        out.append((np.array(idx), np.array([f(w / total) for w in wts], np.float64)))
    return out


def resize_center_crop(img: np.ndarray, dst_w: int, dst_h: int) -> np.ndarray:
    """One view [h][w][3] (float, in [0, 1]) resized to cover dst_w x dst_h
    (scale = max of the axis ratios, sizes rounded half away from zero) and
    centre-cropped: x first, then y (vae.cpp:1-87)."""
    h, w = img.shape[:2]
    f = np.float32
    scale = max(f(dst_w) / f(w), f(dst_h) / f(h))
    rw = int(np.floor(np.float64(f(w) * scale) + 0.5))
    rh = int(np.floor(np.float64(f(h) * scale) + 0.5))
    ax, ay = _resize_axis(w, rw, dst_w), _resize_axis(h, rh, dst_h)
    src = np.asarray(img, np.float64)
    horiz = np.stack([np.einsum("hkc,k->hc", src[:, i, :], wt) for i, wt in ax], axis=1)   # [h][dst_w][3]
    return np.stack([np.einsum("kwc,k->wc", horiz[i], wt) for i, wt in ay], axis=0)     # [dst_h][dst_w][3]


def view_pixels(data: np.ndarray) -> np.ndarray:
    """A camera view as the reference reads it: u8 -> v / 255 (in float32), f32 as is."""
    a = np.asarray(data)
    return (a.astype(np.float32) * np.float32(1.0 / 255.0)) if a.dtype == np.uint8 else a.astype(np.float32)


def compose_and_patchify(views, width: int, height: int) -> np.ndarray:
    """vae.cpp:89-133: the high camera on the top half, the two wrist cameras
    on the bottom-left / bottom-right, the canvas 2x2 pixel-unshuffled to
    f32 [12][height/2][width/2] (channel 4c + 2dx + dy), mapped v * 2 - 1."""
    top, left = height // 2, width // 2
    canvas = np.zeros((height, width, 3))
    canvas[:top, :] = resize_center_crop(view_pixels(views[0]), width, top)
    canvas[top:, :left] = resize_center_crop(view_pixels(views[1]), left, height - top)
    canvas[top:, left:] = resize_center_crop(view_pixels(views[2]), width - left, height - top)
    ow, oh = width // 2, height // 2
    c = canvas[:2 * oh, :2 * ow].reshape(oh, 2, ow, 2, 3)                # [y][dy][x][dx][c]
    out = c.transpose(4, 3, 1, 0, 2).reshape(12, oh, ow)                 # channel (c, dx, dy)
    return out * 2.0 - 1.0


def conv_2d(kernel: np.ndarray, inp: np.ndarray, s0=1, s1=1, p0=0, p1=0, d0=1, d1=1) -> np.ndarray:
    """ggml_conv_2d_direct: kernel [OC][IC][KH][KW], input [N][IC][IH][IW]
    (float arrays: bf16 operands widened exactly), out [N][OC][OH][OW] in
    float64; out = sum over ic, ky, kx of kernel * input at
    (oy*s1 - p1 + ky*d1, ox*s0 - p0 + kx*d0), zero outside the image."""
    k = np.asarray(kernel, np.float64)
    x = np.asarray(inp, np.float64)
    OC, IC, KH, KW = k.shape
    N, _, IH, IW = x.shape
    OW = (IW + 2 * p0 - d0 * (KW - 1) - 1) // s0 + 1
    OH = (IH + 2 * p1 - d1 * (KH - 1) - 1) // s1 + 1
    xp = np.zeros((N, IC, IH + 2 * p1, IW + 2 * p0))
    xp[:, :, p1:p1 + IH, p0:p0 + IW] = x
    out = np.zeros((N, OC, OH, OW))
    for ky in range(KH):
        for kx in range(KW):
            y0, x0 = ky * d1, kx * d0
            patch = xp[:, :, y0:y0 + s1 * (OH - 1) + 1:s1, x0:x0 + s0 * (OW - 1) + 1:s0]   # [N][IC][OH][OW]
            out += np.einsum("nchw,oc->nohw", patch, k[:, :, ky, kx], optimize=True)
    return out
