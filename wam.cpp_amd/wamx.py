"""ctypes binding of libwamx.so (the C ABI declared in include/wamx/wamx.h).

Used by the parity tests and bench.py.  Device memory is owned by the library
(wamx_device_malloc / backend buffers); numpy arrays cross the boundary through
explicit host<->device copies.  bf16 tensors are carried as numpy uint16 bit
patterns.
"""
from __future__ import annotations

import ctypes as C
import os
import re
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent
LIB_PATH = HERE / "libwamx.so"
HEADER = REPO / "include" / "wamx" / "wamx.h"

TYPE_F32, TYPE_F16, TYPE_I32, TYPE_BF16 = 0, 1, 26, 30
STATUS_SUCCESS = 0
EPI_NONE, EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_GATED, EPI_BIAS_RESIDUAL = 0, 1, 2, 3, 4
UNARY_GELU, UNARY_SILU, UNARY_GELU_ERF = 8, 10, 14

OP_NAMES = ["NONE", "DUP", "ADD", "MUL", "SCALE", "CPY", "CONT", "RESHAPE", "VIEW", "PERMUTE",
            "TRANSPOSE", "CONCAT", "REPEAT", "NORM", "RMS_NORM", "MUL_MAT", "SOFT_MAX", "ROPE",
            "UNARY", "GET_ROWS", "IM2COL", "CONV_2D", "LINEAR", "QK_NORM_ROPE", "JOINT_ATTN", "MODULATION",
            "EULER_STEP", "MLP_SMALL"]
OP = {name: i for i, name in enumerate(OP_NAMES)}


class Tensor(C.Structure):
    pass


Tensor._fields_ = [
    ("type", C.c_int32),
    ("buffer", C.c_void_p),
    ("ne", C.c_int64 * 4),
    ("nb", C.c_size_t * 4),
    ("op", C.c_int32),
    ("op_params", C.c_int32 * 16),
    ("flags", C.c_int32),
    ("src", C.POINTER(Tensor) * 10),
    ("view_src", C.POINTER(Tensor)),
    ("view_offs", C.c_size_t),
    ("data", C.c_void_p),
    ("name", C.c_char * 64),
    ("extra", C.c_void_p),
    ("lane", C.c_int32),
]
TensorP = C.POINTER(Tensor)


class GwpConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_layers", "hidden", "n_heads", "head_dim", "ffn_dim", "action_hidden", "action_ffn_dim",
        "action_chunk", "action_dim", "grid_h", "grid_w", "n_lang", "t5_hidden", "z_dim",
        "num_steps", "enc_hidden")] + [("shift", C.c_float), ("eps", C.c_float), ("batch", C.c_int32)]


class ImageView(C.Structure):
    _fields_ = [("data", C.c_void_p), ("w", C.c_int32), ("h", C.c_int32), ("format", C.c_int32)]


class T5Config(C.Structure):
    _fields_ = [(k, C.c_int32) for k in ("vocab", "hidden", "ffn_dim", "heads", "head_dim", "layers", "max_tokens")] + \
               [("eps", C.c_float)]


class PromptCacheStats(C.Structure):
    _fields_ = [("enabled", C.c_int32), ("last_hit", C.c_int32)] + \
               [(k, C.c_uint64) for k in ("capacity", "hits", "misses", "entries", "bytes")]


class GwpTiming(C.Structure):
    _fields_ = [("prompt_ms", C.c_float), ("prefix_ms", C.c_float), ("denoise_ms", C.c_float),
                ("total_ms", C.c_float)]


def declared_symbols() -> list[str]:
    """Every function name declared WAMX_API in the public header."""
    text = HEADER.read_text()
    return sorted(set(re.findall(r"WAMX_API\s+[^;(]*?\b(wamx_\w+)\s*\(", text)))


_lib = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libwamx.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build it with `make -C wam.cpp_amd` or __graft_entry__.build()")
    lib = C.CDLL(str(p))
    vp, i64, i32, f32, sz = C.c_void_p, C.c_int64, C.c_int32, C.c_float, C.c_size_t
    sig = {
        "wamx_last_error": (C.c_char_p, []),
        "wamx_get_device_count": (C.c_int, []),
        "wamx_backend_init": (vp, [C.c_int]),
        "wamx_backend_free": (None, [vp]),
        "wamx_backend_name": (C.c_char_p, [vp]),
        "wamx_backend_synchronize": (None, [vp]),
        "wamx_backend_stream": (vp, [vp]),
        "wamx_device_malloc": (vp, [vp, sz]),
        "wamx_device_free": (None, [vp, vp]),
        "wamx_memcpy_h2d": (C.c_int, [vp, vp, vp, sz]),
        "wamx_memcpy_d2h": (C.c_int, [vp, vp, vp, sz]),
        "wamx_op_mul_mat": (C.c_int, [vp, vp, i64, vp, i32, i64, vp, i32, i64, i64, i64, i64]),
        "wamx_op_linear": (C.c_int, [vp, vp, vp, i32, vp, i32, vp, vp, vp, i64, i64, i64]),
        "wamx_op_linear_tiled": (C.c_int, [vp, vp, vp, i32, vp, i32, vp, vp, vp, i64, i64, i64]),
        "wamx_op_linear_noalloc": (C.c_int, [vp, vp, vp, i32, vp, i32, vp, vp, vp, i64, i64, i64]),
        "wamx_op_norm_modulation_bf16": (C.c_int, [vp, vp, i64, vp, vp, i64, vp, i64, i64, f32]),
        "wamx_op_layer_norm_bf16": (C.c_int, [vp, vp, i64, vp, vp, vp, i64, i64, f32]),
        "wamx_op_rms_norm_bf16_f32": (C.c_int, [vp, vp, i64, vp, vp, i64, i64, f32]),
        "wamx_op_norm_modulation_f32": (C.c_int, [vp, vp, i64, vp, vp, i64, vp, i64, i64, f32]),
        "wamx_op_gated_residual_bf16": (C.c_int, [vp, vp, vp, vp, i32, i64, vp, i64, i64]),
        "wamx_op_gated_residual_f32": (C.c_int, [vp, vp, vp, vp, i64, vp, i64, i64]),
        "wamx_op_bias_gelu_bf16": (C.c_int, [vp, vp, vp, vp, i64, i64]),
        "wamx_op_rope_f32": (C.c_int, [vp, vp, vp, vp, i64, i64, i64, C.c_int, f32]),
        "wamx_op_qk_norm_rope": (C.c_int, [vp, vp, i64, vp, vp, i64, i64, i64, i64, i64, C.c_int,
                                           vp, vp, vp, f32, f32]),
        "wamx_op_joint_attn": (C.c_int, [vp, vp, vp, vp, i64, vp, vp, i64, i64, vp, i64, i64, i64, f32]),
        "wamx_op_qk_norm_rope_hilo": (C.c_int, [vp, vp, i64, vp, vp, vp, i64, i64, i64, i64, i64, C.c_int,
                                                vp, vp, vp, f32, f32]),
        "wamx_op_joint_attn_hilo": (C.c_int, [vp, vp, vp, vp, vp, vp, i64, i64, vp, i64, i64, i64, f32]),
        "wamx_qk_norm_rope_hilo": (TensorP, [vp, TensorP, TensorP, TensorP, i64, C.c_int, TensorP, TensorP,
                                             TensorP, f32, f32]),
        "wamx_joint_attn_hilo": (TensorP, [vp, TensorP, TensorP, TensorP, f32]),
        "wamx_euler_step": (TensorP, [vp, TensorP, TensorP, TensorP]),
        "wamx_op_rope_table": (C.c_int, [vp, C.c_int, vp, vp, vp, i64, i64, f32, vp]),
        "wamx_op_qk_norm_rope_table": (C.c_int, [vp, vp, i64, vp, vp, i64, i64, i64, i64, i64, vp, f32]),
        "wamx_mlp_small": (TensorP, [vp, TensorP, TensorP, TensorP, TensorP, TensorP, i32]),
        "wamx_op_soft_max_f32": (C.c_int, [vp, vp, vp, i64, i64, f32]),
        "wamx_fill_normal": (C.c_int, [vp, vp, i32, i64, C.c_uint64, f32, f32]),
        "wamx_timer_new": (vp, [vp]),
        "wamx_timer_start": (None, [vp]),
        "wamx_timer_stop_ms": (f32, [vp]),
        "wamx_timer_free": (None, [vp]),
        # IR
        "wamx_init": (vp, [sz]),
        "wamx_free": (None, [vp]),
        "wamx_type_size": (sz, [i32]),
        "wamx_nbytes": (sz, [TensorP]),
        "wamx_nelements": (i64, [TensorP]),
        "wamx_is_contiguous": (C.c_bool, [TensorP]),
        "wamx_set_name": (None, [TensorP, C.c_char_p]),
        "wamx_set_input": (None, [TensorP]),
        "wamx_set_output": (None, [TensorP]),
        "wamx_set_lane": (None, [vp, C.c_int]),
        "wamx_new_tensor_1d": (TensorP, [vp, i32, i64]),
        "wamx_new_tensor_2d": (TensorP, [vp, i32, i64, i64]),
        "wamx_new_tensor_3d": (TensorP, [vp, i32, i64, i64, i64]),
        "wamx_new_tensor_4d": (TensorP, [vp, i32, i64, i64, i64, i64]),
        "wamx_view_1d": (TensorP, [vp, TensorP, i64, sz]),
        "wamx_view_2d": (TensorP, [vp, TensorP, i64, i64, sz, sz]),
        "wamx_view_3d": (TensorP, [vp, TensorP, i64, i64, i64, sz, sz, sz]),
        "wamx_view_4d": (TensorP, [vp, TensorP, i64, i64, i64, i64, sz, sz, sz, sz]),
        "wamx_reshape_2d": (TensorP, [vp, TensorP, i64, i64]),
        "wamx_reshape_3d": (TensorP, [vp, TensorP, i64, i64, i64]),
        "wamx_permute": (TensorP, [vp, TensorP, C.c_int, C.c_int, C.c_int, C.c_int]),
        "wamx_transpose": (TensorP, [vp, TensorP]),
        "wamx_cont": (TensorP, [vp, TensorP]),
        "wamx_cast": (TensorP, [vp, TensorP, i32]),
        "wamx_cpy": (TensorP, [vp, TensorP, TensorP]),
        "wamx_concat": (TensorP, [vp, TensorP, TensorP, C.c_int]),
        "wamx_repeat": (TensorP, [vp, TensorP, TensorP]),
        "wamx_add": (TensorP, [vp, TensorP, TensorP]),
        "wamx_mul": (TensorP, [vp, TensorP, TensorP]),
        "wamx_scale": (TensorP, [vp, TensorP, f32]),
        "wamx_gelu": (TensorP, [vp, TensorP]),
        "wamx_gelu_erf": (TensorP, [vp, TensorP]),
        "wamx_silu": (TensorP, [vp, TensorP]),
        "wamx_norm": (TensorP, [vp, TensorP, f32]),
        "wamx_rms_norm": (TensorP, [vp, TensorP, f32]),
        "wamx_mul_mat": (TensorP, [vp, TensorP, TensorP]),
        "wamx_mul_mat_out_type": (TensorP, [vp, TensorP, TensorP, i32]),
        "wamx_mul_mat_set_prec": (None, [TensorP, i32]),
        "wamx_soft_max_ext": (TensorP, [vp, TensorP, TensorP, f32, f32]),
        "wamx_rope_ext": (TensorP, [vp, TensorP, TensorP, TensorP, C.c_int, C.c_int, C.c_int,
                                    f32, f32, f32, f32, f32, f32]),
        "wamx_get_rows": (TensorP, [vp, TensorP, TensorP]),
        "wamx_im2col": (TensorP, [vp, TensorP, TensorP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, i32]),
        "wamx_gated_residual_bf16": (TensorP, [vp, TensorP, TensorP, TensorP]),
        "wamx_bias_gelu_bf16": (TensorP, [vp, TensorP, TensorP]),
        "wamx_norm_modulation_bf16": (TensorP, [vp, TensorP, TensorP, TensorP, f32]),
        "wamx_layer_norm_bf16": (TensorP, [vp, TensorP, TensorP, TensorP, f32]),
        "wamx_rms_norm_bf16_f32": (TensorP, [vp, TensorP, TensorP, f32]),
        "wamx_linear": (TensorP, [vp, TensorP, TensorP, TensorP, i32, TensorP, TensorP]),
        "wamx_qk_norm_rope": (TensorP, [vp, TensorP, TensorP, TensorP, i64, C.c_int, TensorP, TensorP,
                                        TensorP, f32, f32]),
        "wamx_joint_attn": (TensorP, [vp, TensorP, TensorP, TensorP, TensorP, TensorP, i64, f32]),
        "wamx_modulation": (TensorP, [vp, TensorP, TensorP]),
        "wamx_new_graph": (vp, [vp, sz]),
        "wamx_build_forward_expand": (None, [vp, TensorP]),
        "wamx_graph_n_nodes": (C.c_int, [vp]),
        "wamx_graph_node": (TensorP, [vp, C.c_int]),
        "wamx_graph_assign_uid": (None, [vp]),
        "wamx_graph_uid": (C.c_uint64, [vp]),
        "wamx_backend_supports_op": (C.c_bool, [vp, TensorP]),
        "wamx_backend_graph_compute": (C.c_int, [vp, vp]),
        "wamx_backend_alloc_ctx_tensors": (vp, [vp, vp]),
        "wamx_backend_alloc_ctx_tensors_from_buft": (vp, [vp, vp]),
        "wamx_backend_tiled_buffer_type": (vp, [C.c_int]),
        "wamx_backend_buffer_type": (vp, [C.c_int]),
        "wamx_buffer_free": (None, [vp]),
        "wamx_gallocr_new": (vp, [vp]),
        "wamx_gallocr_alloc_graph": (C.c_bool, [vp, vp]),
        "wamx_gallocr_get_buffer_size": (sz, [vp]),
        "wamx_gallocr_free": (None, [vp]),
        "wamx_backend_tensor_set": (C.c_int, [TensorP, vp, sz, sz]),
        "wamx_backend_tensor_get": (C.c_int, [TensorP, vp, sz, sz]),
        "wamx_backend_tensor_copy": (C.c_int, [TensorP, TensorP]),
        "wamx_backend_tensor_memset": (C.c_int, [TensorP, C.c_uint8, sz, sz]),
        "wamx_ggml_op_count": (C.c_int, []),
        "wamx_ggml_op_name": (C.c_char_p, [C.c_int]),
        "wamx_ggml_op_to_wamx": (i32, [C.c_int]),
        "wamx_graph_from_ggml": (vp, [vp, vp, C.c_int, vp, C.c_int]),
        # model driver
        "wamx_gwp_default_config": (GwpConfig, []),
        "wamx_gwp_create": (vp, [vp, C.POINTER(GwpConfig)]),
        "wamx_gwp_free": (None, [vp]),
        "wamx_gwp_n_weights": (C.c_int, [vp]),
        "wamx_gwp_weight_name": (C.c_char_p, [vp, C.c_int]),
        "wamx_gwp_weight": (TensorP, [vp, C.c_char_p]),
        "wamx_gwp_param_count": (C.c_uint64, [vp]),
        "wamx_gwp_init_synthetic": (C.c_int, [vp, C.c_uint64, f32]),
        "wamx_gwp_set_inputs": (C.c_int, [vp, vp, vp, vp, vp]),
        "wamx_gwp_predict": (C.c_int, [vp, C.POINTER(GwpTiming)]),
        "wamx_gwp_run_prompt": (C.c_int, [vp]),
        "wamx_gwp_set_prompt_cache": (C.c_int, [vp, sz]),
        "wamx_gwp_prompt_cache_stats": (C.c_int, [vp, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
        "wamx_gwp_run_prefix": (C.c_int, [vp]),
        "wamx_gwp_run_denoise": (C.c_int, [vp]),
        "wamx_gwp_get_action": (C.c_int, [vp, vp]),
        "wamx_gwp_get_velocity": (C.c_int, [vp, C.c_int, vp]),
        "wamx_check_finite_f32": (C.c_int, [vp, sz, C.c_char_p]),
        "wamx_gwp_prefix_key": (TensorP, [vp, C.c_int]),
        "wamx_gwp_prefix_value": (TensorP, [vp, C.c_int]),
        "wamx_gwp_graph_nodes": (C.c_int, [vp, C.c_int]),
        "wamx_gguf_open": (vp, [C.c_char_p]),
        "wamx_gguf_close": (None, [vp]),
        "wamx_gguf_version": (C.c_uint32, [vp]),
        "wamx_gguf_data_offset": (C.c_uint64, [vp]),
        "wamx_gguf_n_keys": (i64, [vp]),
        "wamx_gguf_key": (C.c_char_p, [vp, i64]),
        "wamx_gguf_key_type": (i32, [vp, C.c_char_p]),
        "wamx_gguf_has": (C.c_bool, [vp, C.c_char_p]),
        "wamx_gguf_get_u32": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_uint32)]),
        "wamx_gguf_get_u64": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_uint64)]),
        "wamx_gguf_get_f32": (C.c_int, [vp, C.c_char_p, C.POINTER(C.c_float)]),
        "wamx_gguf_get_str": (C.c_char_p, [vp, C.c_char_p]),
        "wamx_gguf_get_f32_array": (i64, [vp, C.c_char_p, C.POINTER(C.c_float), i64]),
        "wamx_gguf_n_tensors": (i64, [vp]),
        "wamx_gguf_find_tensor": (i64, [vp, C.c_char_p]),
        "wamx_gguf_tensor_name": (C.c_char_p, [vp, i64]),
        "wamx_gguf_tensor_type": (i32, [vp, i64]),
        "wamx_gguf_tensor_n_dims": (i32, [vp, i64]),
        "wamx_gguf_tensor_ne": (i64, [vp, i64, i32]),
        "wamx_gguf_tensor_offset": (C.c_uint64, [vp, i64]),
        "wamx_gguf_tensor_bytes": (C.c_uint64, [vp, i64]),
        "wamx_gguf_read_tensor": (C.c_int, [vp, i64, vp, C.c_uint64]),
        "wamx_gguf_compact_name": (i32, [C.c_char_p, C.c_char_p, i32]),
        "wamx_gwp_create_from_gguf": (vp, [vp, vp, i32, i32]),
        "wamx_t5_create": (vp, [vp, vp]),
        "wamx_conv_2d_direct": (TensorP, [vp, TensorP, TensorP, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
        "wamx_preprocessor_create": (vp, [vp]),
        "wamx_preprocessor_free": (None, [vp]),
        "wamx_preprocess_views": (C.c_int, [vp, vp, i32, i32, i32, vp]),
        "wamx_t5_free": (None, [vp]),
        "wamx_t5_n_weights": (C.c_int, [vp]),
        "wamx_t5_weight_name": (C.c_char_p, [vp, C.c_int]),
        "wamx_t5_weight": (TensorP, [vp, C.c_char_p]),
        "wamx_t5_load_gguf": (C.c_int, [vp, vp]),
        "wamx_t5_create_from_gguf": (vp, [vp, vp]),
        "wamx_t5_encode": (C.c_int, [vp, vp, vp, i32, vp]),
        "wamx_t5_set_prompt_cache": (C.c_int, [vp, C.c_size_t]),
        "wamx_t5_prompt_cache_stats": (C.c_int, [vp, vp]),
        "wamx_t5_fix_prompt": (C.c_int, [vp, vp, vp, i32]),
        "wamx_t5_relative_bucket": (i32, [i32, i32, i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().wamx_last_error().decode()


def check(status: int, what: str = "wamx call") -> None:
    if status != STATUS_SUCCESS:
        raise RuntimeError(f"{what} failed ({status}): {last_error()}")


# ---------------------------------------------------------------------------
# bf16 helpers (round-to-nearest-even, NaN kept quiet)
# ---------------------------------------------------------------------------
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return bf16_to_f32(f32_to_bf16(x))


# ---------------------------------------------------------------------------
# Device objects
# ---------------------------------------------------------------------------
class Backend:
    def __init__(self, device: int = 0):
        self.lib = load()
        self.ptr = self.lib.wamx_backend_init(device)
        if not self.ptr:
            raise RuntimeError(f"wamx_backend_init({device}) failed: {last_error()}")

    @property
    def name(self) -> str:
        return self.lib.wamx_backend_name(self.ptr).decode()

    def sync(self) -> None:
        self.lib.wamx_backend_synchronize(self.ptr)

    def close(self) -> None:
        if self.ptr:
            self.lib.wamx_backend_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def array(self, host: np.ndarray) -> "DeviceArray":
        d = DeviceArray(self, host.nbytes)
        d.upload(host)
        return d

    def empty(self, nbytes: int) -> "DeviceArray":
        return DeviceArray(self, nbytes)


class DeviceArray:
    def __init__(self, be: Backend, nbytes: int):
        self.be = be
        self.nbytes = int(nbytes)
        self.ptr = be.lib.wamx_device_malloc(be.ptr, max(self.nbytes, 1))
        if not self.ptr:
            raise RuntimeError(f"device malloc of {nbytes} bytes failed: {last_error()}")

    def upload(self, host: np.ndarray) -> None:
        h = np.ascontiguousarray(host)
        assert h.nbytes <= self.nbytes
        check(self.be.lib.wamx_memcpy_h2d(self.be.ptr, self.ptr, h.ctypes.data, h.nbytes), "h2d")

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        check(self.be.lib.wamx_memcpy_d2h(self.be.ptr, out.ctypes.data, self.ptr, out.nbytes), "d2h")
        return out

    def free(self) -> None:
        if self.ptr:
            self.be.lib.wamx_device_free(self.be.ptr, self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Timer:
    """hipEvent timing on the backend's stream."""

    def __init__(self, be: Backend):
        self.be = be
        self.ptr = be.lib.wamx_timer_new(be.ptr)

    def start(self) -> None:
        self.be.lib.wamx_timer_start(self.ptr)

    def stop_ms(self) -> float:
        return float(self.be.lib.wamx_timer_stop_ms(self.ptr))

    def __del__(self):
        try:
            self.be.lib.wamx_timer_free(self.ptr)
        except Exception:
            pass
