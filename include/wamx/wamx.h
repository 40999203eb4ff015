/*
 * wamx — MI355X (gfx950) compute backend for the GWP-0.5 Mixture-of-Transformers
 * action path of wam.cpp.
 *
 * This header is the whole C ABI of libwamx.so.  It has four parts:
 *
 *   1. A tensor/graph IR shaped like ggml's (ne[]/nb[] strides, op + op_params,
 *      src[] slots, views).  The engine in wam.cpp builds ggml graphs through
 *      src/models/gwp05/engine/{mot,cache,weights}.cpp and submits them with
 *      ggml_backend_graph_compute; the constructors below mirror the ggml entry
 *      points those files call, including the ones added by
 *      patches/llama-b9866-native-bf16.patch:7-51.
 *   2. A backend plugin interface mirroring ggml-backend-impl.h of llama.cpp b9866
 *      (ggml_backend_i / ggml_backend_device_i / buffer types / buffers).  ggml is
 *      not vendored in the reference (cmake/Dependencies.cmake:73-89), so the
 *      struct layouts are restated, not copied.  Graphs cross the boundary by
 *      name (wamx_graph_from_ggml: ggml_op_name / ggml_unary_op_name /
 *      ggml_type_name strings and ggml's op_params layouts), so no ggml enum
 *      value is read: UNARY's sub-op comes by its name as well.  The internal
 *      unary codes (GELU 8, SILU 10, GELU_ERF 14) are the GGML_UNARY_OP_*
 *      values of b9866 as restated (unverified against its headers), so a
 *      UNARY's op_params mean the same on both sides.
 *   3. Single-op entry points on device pointers (wamx_op_*), used by the parity
 *      tests and by callers that do not build graphs.
 *   4. A synthetic GWP-0.5-shaped model driver (wamx_gwp_*) that builds the
 *      prompt-projection, prefix and unrolled-denoise graphs the way
 *      src/models/gwp05/engine/cache.cpp:53-485 and mot.cpp:358-594 do, and runs
 *      them through the backend above.
 *
 * Conventions: every call returns a status or NULL, never aborts.  The last
 * error message of the calling thread is available from wamx_last_error().
 * One backend instance is not re-entrant: callers serialise, as wam.cpp does
 * (src/models/gwp05/model.cpp:61).
 */
#ifndef WAMX_WAMX_H
#define WAMX_WAMX_H

#include <stddef.h>
#include <stdint.h>
#include <stdbool.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WAMX_API __attribute__((visibility("default")))

#define WAMX_MAX_DIMS      4
#define WAMX_MAX_SRC       10
#define WAMX_MAX_OP_PARAMS 16   /* int32 slots, 64 bytes like ggml's GGML_MAX_OP_PARAMS */
#define WAMX_MAX_NAME      64

/* ---------------------------------------------------------------------------
 * Enums.  Values of wamx_type follow enum ggml_type (F32=0, F16=1, I32=26,
 * BF16=30).  wamx_status follows enum ggml_status.
 * ------------------------------------------------------------------------- */
typedef enum wamx_type {
    WAMX_TYPE_F32  = 0,
    WAMX_TYPE_F16  = 1,
    WAMX_TYPE_I32  = 26,
    WAMX_TYPE_BF16 = 30,
} wamx_type;

typedef enum wamx_status {
    WAMX_STATUS_ALLOC_FAILED = -2,
    WAMX_STATUS_FAILED       = -1,
    WAMX_STATUS_SUCCESS      = 0,
    WAMX_STATUS_ABORTED      = 1,
} wamx_status;

typedef enum wamx_op {
    WAMX_OP_NONE = 0,
    WAMX_OP_DUP,
    WAMX_OP_ADD,        /* src[2] set: gated residual bf16 (native-bf16.patch:594-612) */
    WAMX_OP_MUL,
    WAMX_OP_SCALE,
    WAMX_OP_CPY,        /* also ggml_cast */
    WAMX_OP_CONT,
    WAMX_OP_RESHAPE,
    WAMX_OP_VIEW,
    WAMX_OP_PERMUTE,
    WAMX_OP_TRANSPOSE,
    WAMX_OP_CONCAT,
    WAMX_OP_REPEAT,
    WAMX_OP_NORM,       /* src[1..2] set: bf16 norm + modulation / affine LN (patch:630-663) */
    WAMX_OP_RMS_NORM,   /* src[1] set: bf16 in, bf16 weight, f32 out (patch:665-678) */
    WAMX_OP_MUL_MAT,
    WAMX_OP_SOFT_MAX,
    WAMX_OP_ROPE,
    WAMX_OP_UNARY,      /* GELU with src[1]: bias + GELU-tanh bf16 (patch:614-628) */
    WAMX_OP_GET_ROWS,
    WAMX_OP_IM2COL,
    WAMX_OP_CONV_2D,    /* ggml_conv_2d_direct (bf16: the patch's cuDNN path, native-bf16.patch:174-218) */
    /* Fused ops with no single ggml counterpart.  They are what the engine's
     * attention hook native_attention_context (mot.cpp:269-282) and a fused
     * linear would emit.  Each one documents the unfused ggml subgraph it
     * replaces, with identical rounding points. */
    WAMX_OP_LINEAR,           /* MUL_MAT(bf16 out) [+ bf16 bias ADD] [+ GELU] [+ residual] */
    WAMX_OP_QK_NORM_ROPE,     /* RMS_NORM(bf16->f32) + ROPE + CAST(bf16) + PERMUTE/CONT */
    WAMX_OP_JOINT_ATTN,       /* CONCAT(K,V) + MUL_MAT(K,Q) + SOFT_MAX + MUL_MAT(V,P) + PERMUTE */
    WAMX_OP_MODULATION,       /* CAST(f32) + ADD of the adaLN modulation and table */
    WAMX_OP_EULER_STEP,       /* CAST(f32) x2 + MUL(dt) + ADD + CAST(bf16): scheduler_step */
    WAMX_OP_MLP_SMALL,        /* [GELU_ERF] + (MUL_MAT + ADD bias [+ GELU_ERF]) x2, widths <= 128 */
    WAMX_OP_COUNT
} wamx_op;

/* UNARY sub-op in op_params[0].  The values restate enum ggml_unary_op of
 * ggml b9866 (GELU 8, SILU 10, GELU_ERF 14; not verified against its header),
 * so the codes ggml writes (native-bf16.patch:626) read the same here; every
 * other code is refused by supports_op.  wamx_graph_from_ggml translates by
 * name (ggml_unary_op_name) and does not depend on these values. */
typedef enum wamx_unary_op {
    WAMX_UNARY_GELU     = 8,   /* tanh approximation, ggml_gelu */
    WAMX_UNARY_SILU     = 10,
    WAMX_UNARY_GELU_ERF = 14,
} wamx_unary_op;

typedef enum wamx_prec {
    WAMX_PREC_DEFAULT = 0,
    WAMX_PREC_F32     = 10,   /* ggml_prec: GGML_PREC_F32 = 10 */
} wamx_prec;

/* Epilogue selector for WAMX_OP_LINEAR (op_params[0]). */
typedef enum wamx_linear_epilogue {
    WAMX_EPI_NONE          = 0, /* y = bf16(acc)                                        */
    WAMX_EPI_BIAS          = 1, /* y = bf16(bf16(acc) + b)                              */
    WAMX_EPI_BIAS_GELU     = 2, /* y = bf16(gelu_tanh(bf16(acc) + b))                   */
    WAMX_EPI_BIAS_GATED    = 3, /* y = bf16(h + bf16(bf16(acc) + b) * g)   g f32 [M]    */
    WAMX_EPI_BIAS_RESIDUAL = 4, /* y = bf16(h + bf16(bf16(acc) + b))                    */
} wamx_linear_epilogue;

/* Tensor flags (ggml_tensor_flag). */
#define WAMX_TENSOR_FLAG_INPUT  1
#define WAMX_TENSOR_FLAG_OUTPUT 2
#define WAMX_TENSOR_FLAG_PARAM  4

/* ---------------------------------------------------------------------------
 * IR: tensors, contexts, graphs.
 * ------------------------------------------------------------------------- */
typedef struct wamx_buffer wamx_buffer;

typedef struct wamx_tensor {
    int32_t  type;                         /* wamx_type */
    wamx_buffer * buffer;                  /* owning buffer, NULL until allocated */
    int64_t  ne[WAMX_MAX_DIMS];            /* elements per dim, ne[0] innermost */
    size_t   nb[WAMX_MAX_DIMS];            /* byte strides */
    int32_t  op;                           /* wamx_op */
    int32_t  op_params[WAMX_MAX_OP_PARAMS];
    int32_t  flags;
    struct wamx_tensor * src[WAMX_MAX_SRC];
    struct wamx_tensor * view_src;
    size_t   view_offs;
    void *   data;                         /* device address once allocated */
    char     name[WAMX_MAX_NAME];
    void *   extra;
    int32_t  lane;                         /* execution lane (0 or 1), set by wamx_set_lane */
} wamx_tensor;

typedef struct wamx_context wamx_context;
typedef struct wamx_cgraph  wamx_cgraph;

/* A context owns tensor metadata only (ggml no_alloc=true contexts). */
WAMX_API wamx_context * wamx_init(size_t max_tensors);
WAMX_API void           wamx_free(wamx_context * ctx);

WAMX_API size_t  wamx_type_size(int32_t type);
WAMX_API const char * wamx_type_name(int32_t type);
WAMX_API const char * wamx_op_name(int32_t op);
WAMX_API int64_t wamx_nelements(const wamx_tensor * t);
WAMX_API int64_t wamx_nrows(const wamx_tensor * t);
WAMX_API size_t  wamx_nbytes(const wamx_tensor * t);
WAMX_API bool    wamx_is_contiguous(const wamx_tensor * t);
WAMX_API bool    wamx_are_same_shape(const wamx_tensor * a, const wamx_tensor * b);
WAMX_API void    wamx_set_name(wamx_tensor * t, const char * name);
WAMX_API void    wamx_set_input(wamx_tensor * t);
WAMX_API void    wamx_set_output(wamx_tensor * t);

WAMX_API wamx_tensor * wamx_new_tensor(wamx_context * ctx, int32_t type, int n_dims, const int64_t * ne);
WAMX_API wamx_tensor * wamx_new_tensor_1d(wamx_context * ctx, int32_t type, int64_t ne0);
WAMX_API wamx_tensor * wamx_new_tensor_2d(wamx_context * ctx, int32_t type, int64_t ne0, int64_t ne1);
WAMX_API wamx_tensor * wamx_new_tensor_3d(wamx_context * ctx, int32_t type, int64_t ne0, int64_t ne1, int64_t ne2);
WAMX_API wamx_tensor * wamx_new_tensor_4d(wamx_context * ctx, int32_t type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3);

/* Views (no compute; data aliases the source). */
WAMX_API wamx_tensor * wamx_view_1d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, size_t offset);
WAMX_API wamx_tensor * wamx_view_2d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, size_t nb1, size_t offset);
WAMX_API wamx_tensor * wamx_view_3d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1, size_t nb2, size_t offset);
WAMX_API wamx_tensor * wamx_view_4d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3, size_t nb1, size_t nb2, size_t nb3, size_t offset);
WAMX_API wamx_tensor * wamx_reshape_2d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1);
WAMX_API wamx_tensor * wamx_reshape_3d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2);
WAMX_API wamx_tensor * wamx_reshape_4d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3);
WAMX_API wamx_tensor * wamx_permute(wamx_context * ctx, wamx_tensor * a, int axis0, int axis1, int axis2, int axis3);
WAMX_API wamx_tensor * wamx_transpose(wamx_context * ctx, wamx_tensor * a);

/* Compute ops mirroring ggml constructors. */
WAMX_API wamx_tensor * wamx_dup(wamx_context * ctx, wamx_tensor * a);
WAMX_API wamx_tensor * wamx_cont(wamx_context * ctx, wamx_tensor * a);
WAMX_API wamx_tensor * wamx_cast(wamx_context * ctx, wamx_tensor * a, int32_t type);
WAMX_API wamx_tensor * wamx_cpy(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b);
WAMX_API wamx_tensor * wamx_concat(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b, int dim);
WAMX_API wamx_tensor * wamx_repeat(wamx_context * ctx, wamx_tensor * a, wamx_tensor * shape);
WAMX_API wamx_tensor * wamx_add(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b);
WAMX_API wamx_tensor * wamx_mul(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b);
WAMX_API wamx_tensor * wamx_scale(wamx_context * ctx, wamx_tensor * a, float s);
WAMX_API wamx_tensor * wamx_gelu(wamx_context * ctx, wamx_tensor * a);
WAMX_API wamx_tensor * wamx_gelu_erf(wamx_context * ctx, wamx_tensor * a);
WAMX_API wamx_tensor * wamx_silu(wamx_context * ctx, wamx_tensor * a);
WAMX_API wamx_tensor * wamx_norm(wamx_context * ctx, wamx_tensor * a, float eps);
WAMX_API wamx_tensor * wamx_rms_norm(wamx_context * ctx, wamx_tensor * a, float eps);
WAMX_API wamx_tensor * wamx_mul_mat(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b);
WAMX_API wamx_tensor * wamx_mul_mat_out_type(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b, int32_t type);
WAMX_API void          wamx_mul_mat_set_prec(wamx_tensor * a, int32_t prec);
/* ggml_soft_max_ext: y = softmax(a*scale + mask) over ne0, f32.  mask (may be
 * NULL) is F32 or F16 with ne0 == a->ne0, ne1 >= a->ne1, broadcast over dims 2
 * and 3 by modulo (the complete-MoT mask of mot.cpp:1025-1027); -inf entries
 * drop a key.  max_bias (ALiBi) must be 0.  op_params = {scale, max_bias}. */
WAMX_API wamx_tensor * wamx_soft_max_ext(wamx_context * ctx, wamx_tensor * a, wamx_tensor * mask, float scale, float max_bias);
WAMX_API wamx_tensor * wamx_rope_ext(wamx_context * ctx, wamx_tensor * a, wamx_tensor * positions, wamx_tensor * freq_factors,
                                     int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale,
                                     float ext_factor, float attn_factor, float beta_fast, float beta_slow);
WAMX_API wamx_tensor * wamx_get_rows(wamx_context * ctx, wamx_tensor * a, wamx_tensor * rows);
/* ggml_im2col, 2-D: kernel ne={KW,KH,IC,OC} (shape only), input f32 ne={IW,IH,IC,N};
 * result ne={IC*KH*KW, OW, OH, N} of dst_type (F32 or BF16), inner index
 * ic*KH*KW + kh*KW + kw (the patch embedding of cache.cpp:203-218). */
WAMX_API wamx_tensor * wamx_im2col(wamx_context * ctx, wamx_tensor * kernel, wamx_tensor * input, int s0, int s1,
                                   int p0, int p1, int d0, int d1, int32_t dst_type);

/* ggml_conv_2d_direct: kernel ne={KW,KH,IC,OC}, input ne={IW,IH,IC,N} (both
 * bf16, or both f32); result ne={OW,OH,OC,N} of the input's type,
 * op_params {s0, s1, p0, p1, d0, d1} (ggml's layout).  BF16 is the VAE's
 * convolution (vae.cpp:139-157; native-bf16.patch:174-218: f32 accumulation,
 * bf16 out). */
WAMX_API wamx_tensor * wamx_conv_2d_direct(wamx_context * ctx, wamx_tensor * kernel, wamx_tensor * input, int s0,
                                           int s1, int p0, int p1, int d0, int d1);

/* The fused ops of patches/llama-b9866-native-bf16.patch:566-678. */
WAMX_API wamx_tensor * wamx_gated_residual_bf16(wamx_context * ctx, wamx_tensor * hidden, wamx_tensor * branch, wamx_tensor * gate);
WAMX_API wamx_tensor * wamx_bias_gelu_bf16(wamx_context * ctx, wamx_tensor * input, wamx_tensor * bias);
WAMX_API wamx_tensor * wamx_norm_modulation_bf16(wamx_context * ctx, wamx_tensor * input, wamx_tensor * scale, wamx_tensor * shift, float eps);
WAMX_API wamx_tensor * wamx_layer_norm_bf16(wamx_context * ctx, wamx_tensor * input, wamx_tensor * weight, wamx_tensor * bias, float eps);
WAMX_API wamx_tensor * wamx_rms_norm_bf16_f32(wamx_context * ctx, wamx_tensor * input, wamx_tensor * weight, float eps);

/* Fused ops of this backend (see wamx_op).
 *
 * wamx_linear: y[N][M] bf16 from weight w bf16 [ne={K,M}], x bf16|f32 [ne={K,N}],
 *   bias bf16 [M] (may be NULL for WAMX_EPI_NONE), residual bf16 [ne={M,N}] and
 *   gate f32 [M] (row broadcast) as the epilogue needs.  Replaces
 *   linear_with_activation / linear_gelu_with_activation (weights.cpp:819-849)
 *   followed by gated_residual (mot.cpp:161-173) or the plain add of mot.cpp:338.
 *
 * wamx_qk_norm_rope: from a packed projection x bf16 [ne={d, T}] (row stride
 *   nb[1]) computes RMSNorm over the full d (weights.cpp:904-917), rotates it
 *   with NORMAL RoPE and writes bf16 into dst laid out [ne={head_dim, T_total, H}]
 *   starting at token offset tok0 (the head-major layout mot.cpp:395-396 builds
 *   with permute+cont).  rope_mode 0: 1-D rope over head_dim with pos0[T];
 *   rope_mode 1: 3-section {44,42,42} rope with pos0/pos1/pos2 (mot.cpp:182-202);
 *   rope_mode 2: no rope (cross-attention queries, mot.cpp:301-306);
 *   rope_mode 3: the rotation of mode 0 or 1 from a precomputed table: pos0
 *   is an f32 tensor [ne={head_dim, T}] holding (cos, sin) of every pair of
 *   each token (wamx_op_rope_table; computed with the same angle and sincos
 *   as modes 0 and 1, so the result is the same bit for bit).  For fixed
 *   positions (the visual grid) it is built once and saves the
 *   transcendental work of every layer.
 *   Chunks: dst [ne={head_dim, T_total, H, C}] takes C chunks (the batch of
 *   chunks of a request, or the layers of a cache), each a contiguous block
 *   at its own nb[3].  x is then [ne={d, C*T}] (the chunks' rows one after
 *   another, positions restarting per chunk) or [ne={d, T, C}] with chunk c's
 *   rows at x + c * nb[2] (for example layer c's column range of a packed
 *   projection of every layer), and weight is [d] or one norm weight per
 *   chunk [ne={d, C}] (the layers' own norm weights).
 *   Writes into an existing tensor (dst), returned as a node that depends on it.
 *
 * wamx_joint_attn: softmax(scale * Q K^T) V per head over the key set
 *   [kv_a rows 0..na_split), kv_b, kv_a rows [na_split..)] i.e. the complete-MoT
 *   order [state, action, reference] of mot.cpp:402-431 without the CONCAT copies.
 *   Q bf16 [ne={dh, Tq, H}], K tensors bf16 [ne={dh, n, H}], V tensors bf16
 *   transposed [ne={n, dh, H}] (cache.cpp:22-25).  kv_b may be NULL.  Output bf16
 *   [ne={dh*H, Tq}], the layout the output projection consumes (mot.cpp:437-445).
 *
 * wamx_qk_norm_rope_hilo / wamx_joint_attn_hilo: the f32-score attention of
 *   build_attention (src/models/gwp05/engine/text_encoder.cpp:26-73), used by
 *   the prefix's visual cross-attention (mot.cpp:326-337): there RMSNorm keeps
 *   Q and K in f32 (rms_norm_bf16_f32) and the scores are an f32 x f32
 *   MUL_MAT at GGML_PREC_F32.  wamx_qk_norm_rope_hilo writes dst
 *   [ne={head_dim, T_total, H, 2}]: plane 0 the bf16 rounding of the f32
 *   result, plane 1 its remainder bf16(v - plane0); with C chunks (x and
 *   weight as for wamx_qk_norm_rope) dst is [ne={head_dim, T_total, H, 2C}],
 *   planes 2c and 2c + 1 for chunk c, contiguous.  wamx_joint_attn_hilo
 *   takes q [ne={dh, Tq, H, 2}] and k [ne={dh, n, H, 2}] in that form, V^T
 *   bf16 [ne={n, dh, H}] (rows a multiple of 8 keys, n >= 8), and forms
 *   every score as K.Q + K.Q_lo + K_lo.Q with fp32 accumulation (the
 *   dropped K_lo.Q_lo is below 2^-16 of the product); softmax and P.V as
 *   wamx_joint_attn.  Output bf16 [ne={dh*H, Tq}].
 *
 * wamx_modulation: f32 [ne={d, 6, L}] = f32(mod [ne={d,6}]) + f32(table_l) for the
 *   L per-layer tables packed in `tables` [ne={d, 6, L}] (mot.cpp:137-145, 380-393).
 *   A mod of S columns ([ne={6d, S}], S timesteps) gives [ne={d, 6, L, S}]:
 *   column s against every table.
 *
 * wamx_euler_step: bf16 [ne={A, N}] = bf16(f32(action) + f32(velocity) * dt),
 *   the flow-matching update of scheduler_step (weights.cpp:885-902: two
 *   casts to f32, MUL by the f32 dt [1], ADD, cast to bf16), with the
 *   product and the sum rounded separately as those two ggml ops do.
 *
 * wamx_mlp_small: two linear layers of at most 128 features on at most 128
 *   inputs, as the action/state encoder and the action decoder chain them
 *   (mot.cpp:16-55): optionally GELU_ERF of x first (flag
 *   WAMX_MLP_GELU_IN), then h = bf16(bf16(W1 x) + b1) (the bf16-output
 *   MUL_MAT and bf16 bias ADD of linear_with_activation, weights.cpp:819-831)
 *   with GELU_ERF after it (WAMX_MLP_GELU_MID), then y = bf16(bf16(W2 h) +
 *   b2) with GELU_ERF after it (WAMX_MLP_GELU_OUT).  x bf16 [ne={K0, N}],
 *   W1 bf16 [ne={K0, M1}], b1 bf16 [M1], W2 bf16 [ne={M1, M2}], b2 bf16 [M2];
 *   y bf16 [ne={M2, N}].  Each GELU_ERF rounds to bf16.  fp32 accumulation
 *   (in k order).
 */
WAMX_API wamx_tensor * wamx_linear(wamx_context * ctx, wamx_tensor * w, wamx_tensor * x, wamx_tensor * bias,
                                   int32_t epilogue, wamx_tensor * residual, wamx_tensor * gate);
WAMX_API wamx_tensor * wamx_qk_norm_rope(wamx_context * ctx, wamx_tensor * x, wamx_tensor * weight, wamx_tensor * dst,
                                         int64_t tok0, int rope_mode, wamx_tensor * pos0, wamx_tensor * pos1,
                                         wamx_tensor * pos2, float eps, float freq_base);
WAMX_API wamx_tensor * wamx_joint_attn(wamx_context * ctx, wamx_tensor * q, wamx_tensor * k_a, wamx_tensor * v_a,
                                       wamx_tensor * k_b, wamx_tensor * v_b, int64_t na_split, float scale);
WAMX_API wamx_tensor * wamx_modulation(wamx_context * ctx, wamx_tensor * mod, wamx_tensor * tables);
WAMX_API wamx_tensor * wamx_qk_norm_rope_hilo(wamx_context * ctx, wamx_tensor * x, wamx_tensor * weight,
                                              wamx_tensor * dst, int64_t tok0, int rope_mode, wamx_tensor * pos0,
                                              wamx_tensor * pos1, wamx_tensor * pos2, float eps, float freq_base);
WAMX_API wamx_tensor * wamx_joint_attn_hilo(wamx_context * ctx, wamx_tensor * q, wamx_tensor * k, wamx_tensor * v,
                                            float scale);
WAMX_API wamx_tensor * wamx_euler_step(wamx_context * ctx, wamx_tensor * action, wamx_tensor * velocity,
                                       wamx_tensor * dt);
enum { WAMX_MLP_GELU_IN = 1, WAMX_MLP_GELU_MID = 2, WAMX_MLP_GELU_OUT = 4 };
WAMX_API wamx_tensor * wamx_mlp_small(wamx_context * ctx, wamx_tensor * x, wamx_tensor * w1, wamx_tensor * b1,
                                      wamx_tensor * w2, wamx_tensor * b2, int32_t flags);

/* Graphs. */
WAMX_API wamx_cgraph * wamx_new_graph(wamx_context * ctx, size_t max_nodes);
WAMX_API void          wamx_build_forward_expand(wamx_cgraph * g, wamx_tensor * t);
WAMX_API int           wamx_graph_n_nodes(const wamx_cgraph * g);
WAMX_API wamx_tensor * wamx_graph_node(wamx_cgraph * g, int i);
WAMX_API void          wamx_graph_assign_uid(wamx_cgraph * g);   /* native-bf16.patch:700-703 */
WAMX_API uint64_t      wamx_graph_uid(const wamx_cgraph * g);
/* Execution lane of the tensors `ctx` creates from now on (0 or 1).  No
 * counterpart in the reference (ggml schedules a graph on one stream): a
 * graph whose nodes use both lanes runs lane 1 on a second stream, ordered
 * against lane 0 only where one lane's node reads or writes memory the other
 * lane's earlier nodes wrote or read.  Intermediates touched by both lanes are
 * not recycled by the graph allocator. */
WAMX_API void          wamx_set_lane(wamx_context * ctx, int lane);

/* ---------------------------------------------------------------------------
 * Backend plugin interface (restating ggml-backend-impl.h, b9866).
 * ------------------------------------------------------------------------- */
typedef struct wamx_backend        * wamx_backend_t;
typedef struct wamx_buffer_type    * wamx_buffer_type_t;
typedef struct wamx_buffer         * wamx_buffer_t;
typedef struct wamx_device         * wamx_device_t;
typedef struct wamx_backend_reg    * wamx_backend_reg_t;

typedef struct wamx_buffer_type_i {
    const char *  (*get_name)      (wamx_buffer_type_t buft);
    wamx_buffer_t (*alloc_buffer)  (wamx_buffer_type_t buft, size_t size);
    size_t        (*get_alignment) (wamx_buffer_type_t buft);
    size_t        (*get_max_size)  (wamx_buffer_type_t buft);
    size_t        (*get_alloc_size)(wamx_buffer_type_t buft, const wamx_tensor * t);
    bool          (*is_host)       (wamx_buffer_type_t buft);
} wamx_buffer_type_i;

typedef struct wamx_buffer_i {
    void          (*free_buffer)  (wamx_buffer_t buf);
    void *        (*get_base)     (wamx_buffer_t buf);
    wamx_status   (*init_tensor)  (wamx_buffer_t buf, wamx_tensor * t);
    void          (*memset_tensor)(wamx_buffer_t buf, wamx_tensor * t, uint8_t value, size_t offset, size_t size);
    void          (*set_tensor)   (wamx_buffer_t buf, wamx_tensor * t, const void * data, size_t offset, size_t size);
    void          (*get_tensor)   (wamx_buffer_t buf, const wamx_tensor * t, void * data, size_t offset, size_t size);
    bool          (*cpy_tensor)   (wamx_buffer_t buf, const wamx_tensor * src, wamx_tensor * dst);
    void          (*clear)        (wamx_buffer_t buf, uint8_t value);
    void          (*reset)        (wamx_buffer_t buf);
} wamx_buffer_i;

typedef struct wamx_backend_i {
    const char * (*get_name)        (wamx_backend_t backend);
    void         (*free)            (wamx_backend_t backend);
    void         (*set_tensor_async)(wamx_backend_t backend, wamx_tensor * t, const void * data, size_t offset, size_t size);
    void         (*get_tensor_async)(wamx_backend_t backend, const wamx_tensor * t, void * data, size_t offset, size_t size);
    bool         (*cpy_tensor_async)(wamx_backend_t src, wamx_backend_t dst, const wamx_tensor * a, wamx_tensor * b);
    void         (*synchronize)     (wamx_backend_t backend);
    wamx_status  (*graph_compute)   (wamx_backend_t backend, wamx_cgraph * g);
} wamx_backend_i;

typedef struct wamx_device_i {
    const char *        (*get_name)       (wamx_device_t dev);
    const char *        (*get_description)(wamx_device_t dev);
    void                (*get_memory)     (wamx_device_t dev, size_t * free, size_t * total);
    wamx_backend_t      (*init_backend)   (wamx_device_t dev, const char * params);
    wamx_buffer_type_t  (*get_buffer_type)(wamx_device_t dev);
    bool                (*supports_op)    (wamx_device_t dev, const wamx_tensor * op);
    bool                (*supports_buft)  (wamx_device_t dev, wamx_buffer_type_t buft);
    bool                (*offload_op)     (wamx_device_t dev, const wamx_tensor * op);
} wamx_device_i;

typedef struct wamx_backend_reg_i {
    const char *  (*get_name)        (wamx_backend_reg_t reg);
    size_t        (*get_device_count)(wamx_backend_reg_t reg);
    wamx_device_t (*get_device)      (wamx_backend_reg_t reg, size_t index);
    void *        (*get_proc_address)(wamx_backend_reg_t reg, const char * name);
} wamx_backend_reg_i;

/* Registry / device / backend lifetime (ggml_backend_cuda_init, weights.cpp:582-596). */
WAMX_API wamx_backend_reg_t  wamx_backend_reg(void);
WAMX_API const wamx_backend_reg_i * wamx_backend_reg_iface(void);
WAMX_API const wamx_device_i      * wamx_device_iface(void);
WAMX_API const wamx_backend_i     * wamx_backend_iface(void);
WAMX_API const wamx_buffer_type_i * wamx_buffer_type_iface(void);
WAMX_API const wamx_buffer_i      * wamx_buffer_iface(void);

WAMX_API int             wamx_get_device_count(void);
WAMX_API wamx_backend_t  wamx_backend_init(int device);
WAMX_API void            wamx_backend_free(wamx_backend_t backend);
WAMX_API const char *    wamx_backend_name(wamx_backend_t backend);
WAMX_API void *          wamx_backend_stream(wamx_backend_t backend);   /* hipStream_t */
WAMX_API wamx_buffer_type_t wamx_backend_get_default_buffer_type(wamx_backend_t backend);
WAMX_API wamx_buffer_type_t wamx_backend_buffer_type(int device);
/* The tiled weight buffer type of a device, in the role of ggml's repacking
 * "extra" buffer types (ggml_backend_dev_get_extra_bufts / the CPU backend's
 * weight repack, ggml b9866): a 2-D bf16 weight [K][M] with M % 16 == 0 and
 * K % 32 == 0 allocated here is stored MFMA-tiled and is read by the few-token
 * (<= 64) MUL_MAT/LINEAR path only (supports_op says so); tensor set/get/copy
 * convert to and from the row-major layout, and a set writes the whole tensor.
 * wam.cpp would place the action expert's projection weights here. */
WAMX_API wamx_buffer_type_t wamx_backend_tiled_buffer_type(int device);

/* Buffers (ggml_backend_buft_alloc_buffer, ggml_backend_alloc_ctx_tensors). */
WAMX_API wamx_buffer_t wamx_buft_alloc_buffer(wamx_buffer_type_t buft, size_t size);
WAMX_API size_t        wamx_buft_get_alignment(wamx_buffer_type_t buft);
WAMX_API size_t        wamx_buft_get_alloc_size(wamx_buffer_type_t buft, const wamx_tensor * t);
WAMX_API wamx_buffer_t wamx_backend_alloc_buffer(wamx_backend_t backend, size_t size);
WAMX_API void          wamx_buffer_free(wamx_buffer_t buf);
WAMX_API void *        wamx_buffer_get_base(wamx_buffer_t buf);
WAMX_API size_t        wamx_buffer_get_size(wamx_buffer_t buf);
WAMX_API wamx_status   wamx_tensor_alloc(wamx_buffer_t buf, wamx_tensor * t, void * addr);
WAMX_API wamx_buffer_t wamx_backend_alloc_ctx_tensors(wamx_context * ctx, wamx_backend_t backend);
/* ggml_backend_alloc_ctx_tensors_from_buft (ggml-alloc.h, b9866). */
WAMX_API wamx_buffer_t wamx_backend_alloc_ctx_tensors_from_buft(wamx_context * ctx, wamx_buffer_type_t buft);

/* Tensor data movement (ggml_backend_tensor_set/get/copy). */
WAMX_API wamx_status wamx_backend_tensor_set(wamx_tensor * t, const void * data, size_t offset, size_t size);
WAMX_API wamx_status wamx_backend_tensor_get(const wamx_tensor * t, void * data, size_t offset, size_t size);
WAMX_API wamx_status wamx_backend_tensor_copy(const wamx_tensor * src, wamx_tensor * dst);
WAMX_API wamx_status wamx_backend_tensor_memset(wamx_tensor * t, uint8_t value, size_t offset, size_t size);
WAMX_API void        wamx_backend_synchronize(wamx_backend_t backend);

/* Graph allocation (ggml_gallocr): allocates every unallocated tensor of the
 * graph in one device buffer with liveness-based reuse. */
typedef struct wamx_gallocr * wamx_gallocr_t;
WAMX_API wamx_gallocr_t wamx_gallocr_new(wamx_backend_t backend);
WAMX_API bool           wamx_gallocr_alloc_graph(wamx_gallocr_t galloc, wamx_cgraph * g);
WAMX_API size_t         wamx_gallocr_get_buffer_size(wamx_gallocr_t galloc);
WAMX_API void           wamx_gallocr_free(wamx_gallocr_t galloc);

/* Compute.  graph_compute replays a captured HIP graph when the same graph
 * (uid, node count and tensor addresses) was computed before; set
 * WAMX_DISABLE_HIP_GRAPHS=1 to launch eagerly every time. */
WAMX_API wamx_status wamx_backend_graph_compute(wamx_backend_t backend, wamx_cgraph * g);
WAMX_API bool        wamx_backend_supports_op(wamx_backend_t backend, const wamx_tensor * op);

/* ---------------------------------------------------------------------------
 * Single-op entry points on device pointers (no graph).  All run on the
 * backend's stream and return immediately (asynchronous).  Sizes are in
 * elements; leading dimensions are row strides in elements.
 * ------------------------------------------------------------------------- */

/* GGML_OP_MUL_MAT semantics (native-bf16.patch:566-592): y[n][m] = sum_k w[m][k]*x[n][k]
 * with x rounded to bf16 (round-to-nearest-even) when x_type is F32, fp32
 * accumulation, output F32 or rounded BF16. */
WAMX_API wamx_status wamx_op_mul_mat(wamx_backend_t be, const void * w, int64_t ldw,
                                     const void * x, int32_t x_type, int64_t ldx,
                                     void * y, int32_t y_type, int64_t ldy,
                                     int64_t M, int64_t N, int64_t K);
/* WAMX_OP_LINEAR on device pointers. */
WAMX_API wamx_status wamx_op_linear(wamx_backend_t be, const void * w, const void * x, int32_t x_type,
                                    const void * bias, int32_t epilogue, const void * residual,
                                    const float * gate, void * y, int64_t M, int64_t N, int64_t K);
/* wamx_op_linear with w in the MFMA-tiled layout of the tiled buffer type
 * (the data pointer of a tensor placed by wamx_backend_tiled_buffer_type);
 * M % 16 == 0, K % 32 == 0, N <= 64.  Plays the part of the matmul over a
 * repacked weight in ggml's CPU extra buffer types (ggml-cpu repack). */
WAMX_API wamx_status wamx_op_linear_tiled(wamx_backend_t be, const void * w, const void * x, int32_t x_type,
                                          const void * bias, int32_t epilogue, const void * residual,
                                          const float * gate, void * y, int64_t M, int64_t N, int64_t K);
/* wamx_op_linear that allocates nothing: no counterpart in the reference; it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, hosts that forbid hipMalloc).  stream is a
 * hipStream_t (NULL: the null stream); the caller owns w, x, bias, residual,
 * gate and y.  The split-K partials of every product that takes a K split
 * (products on <= 64 tokens, and products on more tokens whose grid is too
 * small for the large tiles, e.g. 384 x 3072 x 3072) live in a library-owned
 * device array of 32 MiB per GPU, held until the process ends.  The split is
 * planned as wamx_op_linear plans it; a product whose partials would not fit
 * the array is refused (status FAILED, reason in wamx_last_error) before
 * anything runs.  Every call on one GPU shares that array: calls that overlap
 * on one GPU race and must be serialised by the caller.  Same kernels, same
 * K slices, same bits as wamx_op_linear. */
WAMX_API wamx_status wamx_op_linear_noalloc(void * stream, const void * w, const void * x, int32_t x_type,
                                            const void * bias, int32_t epilogue, const void * residual,
                                            const float * gate, void * y, int64_t M, int64_t N, int64_t K);
/* norm_bf16_fused<bs,false> (native-bf16.patch:368-409): y = bf16(n*(1+scale)+shift).
 * scale/shift f32, row stride ss (0 = broadcast). */
WAMX_API wamx_status wamx_op_norm_modulation_bf16(wamx_backend_t be, const void * x, int64_t ldx,
                                                  const float * scale, const float * shift, int64_t ss,
                                                  void * y, int64_t rows, int64_t cols, float eps);
/* norm_bf16_fused<bs,true>: y = bf16(n*w+b), w/b bf16 [cols]. */
WAMX_API wamx_status wamx_op_layer_norm_bf16(wamx_backend_t be, const void * x, int64_t ldx,
                                             const void * w, const void * b, void * y,
                                             int64_t rows, int64_t cols, float eps);
/* rms_norm_bf16_f32 (native-bf16.patch:411-430): y f32 = x*rsqrt(mean(x^2)+eps)*w. */
WAMX_API wamx_status wamx_op_rms_norm_bf16_f32(wamx_backend_t be, const void * x, int64_t ldx,
                                               const void * w, float * y, int64_t rows, int64_t cols, float eps);
/* norm_modulation_f32 (p7-fusions.patch:19-51): one-pass variance, no FMA. */
WAMX_API wamx_status wamx_op_norm_modulation_f32(wamx_backend_t be, const float * x, int64_t ldx,
                                                 const float * scale, const float * shift, int64_t ss,
                                                 float * y, int64_t rows, int64_t cols, float eps);
/* gated_residual_bf16<gate_t> (native-bf16.patch:79-91): y = bf16(h + b*g). gate_type F32|BF16,
 * gs row stride of gate (0 = broadcast). */
WAMX_API wamx_status wamx_op_gated_residual_bf16(wamx_backend_t be, const void * h, const void * b,
                                                 const void * g, int32_t gate_type, int64_t gs,
                                                 void * y, int64_t rows, int64_t cols);
/* gated_residual_f32 (p7-fusions.patch:122-134): y = r + b*g, no FMA. */
WAMX_API wamx_status wamx_op_gated_residual_f32(wamx_backend_t be, const float * r, const float * b,
                                                const float * g, int64_t gs, float * y,
                                                int64_t rows, int64_t cols);
/* bias_gelu_bf16_kernel (native-bf16.patch:507-514): y = bf16(gelu_tanh(x + bias[i % width])). */
WAMX_API wamx_status wamx_op_bias_gelu_bf16(wamx_backend_t be, const void * x, const void * bias,
                                            void * y, int64_t n, int64_t width);
/* ROPE NORMAL on f32 [ne={head_dim, heads, tokens}] contiguous, rotating the first n_dims. */
WAMX_API wamx_status wamx_op_rope_f32(wamx_backend_t be, const float * x, const int32_t * pos,
                                      float * y, int64_t head_dim, int64_t heads, int64_t tokens,
                                      int n_dims, float freq_base);
/* Fused QK RMSNorm + RoPE + bf16 + head-major write (WAMX_OP_QK_NORM_ROPE). */
WAMX_API wamx_status wamx_op_qk_norm_rope(wamx_backend_t be, const void * x, int64_t ldx,
                                          const void * w, void * dst, int64_t heads, int64_t head_dim,
                                          int64_t tokens, int64_t dst_tokens, int64_t tok0,
                                          int rope_mode, const int32_t * pos0, const int32_t * pos1,
                                          const int32_t * pos2, float eps, float freq_base);
/* Joint attention (WAMX_OP_JOINT_ATTN) on device pointers.  q [H][Tq][dh], k_a [H][na][dh],
 * vt_a [H][dh][na], k_b [H][nb][dh], vt_b [H][dh][nb], out bf16 [Tq][H*dh]. */
WAMX_API wamx_status wamx_op_joint_attn(wamx_backend_t be, const void * q, const void * k_a,
                                        const void * vt_a, int64_t na, const void * k_b,
                                        const void * vt_b, int64_t nb, int64_t na_split,
                                        void * out, int64_t heads, int64_t head_dim, int64_t tq,
                                        float scale);
/* The hi/lo forms on device pointers (f32-score attention of build_attention,
 * text_encoder.cpp:26-73).  wamx_op_qk_norm_rope_hilo: as wamx_op_qk_norm_rope,
 * plus the remainder plane at dst_lo (16-byte aligned offset from dst_hi).
 * wamx_op_joint_attn_hilo: q / q_lo [H][Tq][dh], k / k_lo [H][nk][dh], vt
 * [H][dh][vt_ld] (vt_ld % 8 == 0, nk >= 8), out bf16 [Tq][H*dh]. */
WAMX_API wamx_status wamx_op_qk_norm_rope_hilo(wamx_backend_t be, const void * x, int64_t ldx, const void * w,
                                               void * dst_hi, void * dst_lo, int64_t heads, int64_t head_dim,
                                               int64_t tokens, int64_t dst_tokens, int64_t tok0, int rope_mode,
                                               const int32_t * pos0, const int32_t * pos1, const int32_t * pos2,
                                               float eps, float freq_base);
WAMX_API wamx_status wamx_op_joint_attn_hilo(wamx_backend_t be, const void * q, const void * q_lo, const void * k,
                                             const void * k_lo, const void * vt, int64_t nk, int64_t vt_ld,
                                             void * out, int64_t heads, int64_t head_dim, int64_t tq, float scale);
/* The rope table of rope mode 3 for positions of mode 0 or 1: out f32
 * [tokens][head_dim], (cos, sin) of pair i at 2i, 2i+1. */
WAMX_API wamx_status wamx_op_rope_table(wamx_backend_t be, int rope_mode, const int32_t * pos0,
                                        const int32_t * pos1, const int32_t * pos2, int64_t tokens,
                                        int64_t head_dim, float freq_base, float * out);
/* wamx_op_qk_norm_rope with rope mode 3 (rotation from `table`). */
WAMX_API wamx_status wamx_op_qk_norm_rope_table(wamx_backend_t be, const void * x, int64_t ldx, const void * w,
                                                void * dst, int64_t heads, int64_t head_dim, int64_t tokens,
                                                int64_t dst_tokens, int64_t tok0, const float * table, float eps);
/* SOFT_MAX_EXT without mask: y[r][:] = softmax(scale * x[r][:]) over ne0=cols, f32. */
WAMX_API wamx_status wamx_op_soft_max_f32(wamx_backend_t be, const float * x, float * y,
                                          int64_t rows, int64_t cols, float scale);

/* Fill a device array with a seeded synthetic normal sample: splitmix64 on
 * (seed, index) -> Box-Muller -> mean + std*z, stored as type (F32 or BF16, RNE). */
WAMX_API wamx_status wamx_fill_normal(wamx_backend_t be, void * dst, int32_t type, int64_t n,
                                      uint64_t seed, float mean, float std);

/* Device memory helpers for callers without another allocator. */
WAMX_API void *      wamx_device_malloc(wamx_backend_t be, size_t size);
WAMX_API void        wamx_device_free(wamx_backend_t be, void * p);
WAMX_API wamx_status wamx_memcpy_h2d(wamx_backend_t be, void * dst, const void * src, size_t size);
WAMX_API wamx_status wamx_memcpy_d2h(wamx_backend_t be, void * dst, const void * src, size_t size);

/* HIP event timing on the backend's stream. */
typedef struct wamx_timer * wamx_timer_t;
WAMX_API wamx_timer_t wamx_timer_new(wamx_backend_t be);
WAMX_API void         wamx_timer_start(wamx_timer_t t);
WAMX_API float        wamx_timer_stop_ms(wamx_timer_t t);   /* synchronises */
WAMX_API void         wamx_timer_free(wamx_timer_t t);

/* ---------------------------------------------------------------------------
 * Synthetic GWP-0.5-shaped MoT driver.
 * ------------------------------------------------------------------------- */
typedef struct wamx_gwp_config {
    int32_t n_layers;        /* gwp05.n_layers */
    int32_t hidden;          /* visual expert width d = n_heads * head_dim */
    int32_t n_heads;
    int32_t head_dim;
    int32_t ffn_dim;         /* visual expert FFN */
    int32_t action_hidden;   /* action expert width */
    int32_t action_ffn_dim;
    int32_t action_chunk;    /* T */
    int32_t action_dim;      /* max_action_dim == max_state_dim */
    int32_t grid_h;          /* visual token grid (n_img = grid_h * grid_w) */
    int32_t grid_w;
    int32_t n_lang;          /* prompt tokens */
    int32_t t5_hidden;       /* prompt embedding width */
    int32_t z_dim;           /* latent channels (patch embedding input) */
    int32_t num_steps;       /* flow-matching steps */
    int32_t enc_hidden;      /* action/state encoder and decoder MLP width (128) */
    float   shift;           /* flow-matching shift */
    float   eps;             /* norm eps */
    int32_t batch;           /* independent action chunks per request (0 or 1: one).  Each chunk has
                                its own inputs and prompt / prefix caches; the denoise graph runs all
                                chunks' 48 tokens through each projection together (batch x chunk
                                tokens) and each chunk's queries attend its own caches. */
} wamx_gwp_config;

typedef struct wamx_gwp_model * wamx_gwp_t;

/* Phase timings of the last predict, milliseconds (hipEvent on the stream). */
typedef struct wamx_gwp_timing {
    float prompt_ms;
    float prefix_ms;
    float denoise_ms;
    float total_ms;
} wamx_gwp_timing;

WAMX_API wamx_gwp_config wamx_gwp_default_config(void);
WAMX_API wamx_gwp_t  wamx_gwp_create(wamx_backend_t be, const wamx_gwp_config * cfg);
WAMX_API void        wamx_gwp_free(wamx_gwp_t m);
WAMX_API int         wamx_gwp_n_weights(wamx_gwp_t m);
WAMX_API const char * wamx_gwp_weight_name(wamx_gwp_t m, int i);
WAMX_API wamx_tensor * wamx_gwp_weight(wamx_gwp_t m, const char * name);
WAMX_API uint64_t    wamx_gwp_param_count(wamx_gwp_t m);
/* Random-init every weight on the device: bf16 matrices ~N(0, wstd), biases
 * ~N(0, 0.02), norm weights 1 + N(0, 0.02), scale/shift tables ~N(0, 0.1). */
WAMX_API wamx_status wamx_gwp_init_synthetic(wamx_gwp_t m, uint64_t seed, float wstd);
/* Inputs, chunk-major for batch > 1: state f32 [batch][action_dim], latent f32
 * [batch][z_dim][2*grid_h][2*grid_w] (CHW), prompt f32 [batch][n_lang][t5_hidden],
 * noise f32 [batch][action_chunk][action_dim].  A NaN or Inf anywhere is
 * refused (WAMX_STATUS_FAILED) before anything is uploaded, as the reference
 * refuses state, latent, prompt and noise (src/models/gwp05/engine/engine.cpp
 * :238-247, :274, :320, :350-357). */
WAMX_API wamx_status wamx_gwp_set_inputs(wamx_gwp_t m, const float * state, const float * latent,
                                         const float * prompt, const float * noise);
/* Run the three graphs (prompt projection, prefix, unrolled denoise). */
WAMX_API wamx_status wamx_gwp_predict(wamx_gwp_t m, wamx_gwp_timing * timing);
WAMX_API wamx_status wamx_gwp_run_prompt(wamx_gwp_t m);
/* Projected-prompt reuse across requests, replacing wam.cpp's
 * update_projected_prompt_cache (src/models/gwp05/engine/cache.cpp:53-67,
 * :131) as enabled by ModelOptions::prompt_cache_capacity (include/wam/types.h:193,
 * default 0; apps/wam-bench.cpp:83 sets 4 in --mode steady, 0 in raw).  With a
 * nonzero capacity, set_inputs keeps a host copy of the prompt it uploads;
 * a later request whose prompt has the same bytes skips the prompt upload,
 * and predict skips the prompt graphs (the prompt K/V caches already hold its
 * projection).  0 (the default) projects every request's prompt and drops
 * the copy.  The prefix pass still reads the resident prompt every request. */
WAMX_API wamx_status wamx_gwp_set_prompt_cache(wamx_gwp_t m, size_t capacity);
/* Projected-prompt hits and misses counted by set_inputs while enabled
 * (the reference's projected_prompt_hits / _misses, cache.cpp:61-68). */
WAMX_API wamx_status wamx_gwp_prompt_cache_stats(wamx_gwp_t m, uint64_t * hits, uint64_t * misses);
WAMX_API wamx_status wamx_gwp_run_prefix(wamx_gwp_t m);
WAMX_API wamx_status wamx_gwp_run_denoise(wamx_gwp_t m);
/* Final action chunks (bf16 state widened to f32) [batch][action_chunk][action_dim].
 * Waits for the request.  A non-finite element returns WAMX_STATUS_FAILED
 * with wamx_last_error() naming it, as the reference's prediction check
 * (src/models/gwp05/model.cpp:246-251) fails the request; out is still
 * written. */
WAMX_API wamx_status wamx_gwp_get_action(wamx_gwp_t m, float * out);
/* The velocity of denoise step `step` of the last request: the action
 * decoder's bf16 output widened to f32, [batch][action_chunk][action_dim],
 * the tensor the scheduler step adds as dt * v.  It replaces the reference's
 * velocity_step0 / denoise_%02d_velocity debug dumps
 * (src/models/gwp05/engine/engine.cpp:416-421, gwp-f32-dump-v1 format
 * weights.cpp:13-104), which exist there only on its stepwise path; here the
 * velocities are outputs of the unrolled denoise graph.  Waits for the
 * request. */
WAMX_API wamx_status wamx_gwp_get_velocity(wamx_gwp_t m, int step, float * out);
/* First non-finite element check of a host f32 array, the finite-value test
 * of the reference's copy_f32_tensor (src/models/common/input_validation.cpp
 * :37-42).  WAMX_STATUS_FAILED and wamx_last_error() "<field> contains NaN or
 * Inf (element i)" on the first one; no GPU call.  wamx_gwp_set_inputs
 * applies it to state, latent, prompt and noise before uploading anything,
 * wamx_gwp_get_action and wamx_t5_encode to their outputs. */
WAMX_API wamx_status wamx_check_finite_f32(const float * values, size_t n, const char * field);
/* Prefix K/V cache of one layer as stored: K bf16 [batch][H][P][dh] (ggml ne
 * {dh, P, H, batch}), V^T bf16 [batch][H][dh][Ppad] viewed as ne {P, dh, H, batch}. */
WAMX_API wamx_tensor * wamx_gwp_prefix_key(wamx_gwp_t m, int layer);
WAMX_API wamx_tensor * wamx_gwp_prefix_value(wamx_gwp_t m, int layer);
WAMX_API int         wamx_gwp_graph_nodes(wamx_gwp_t m, int which);  /* 0 prompt, 1 prefix (chunk 0's), 2 denoise */

/* ---------------------------------------------------------------------------
 * GGUF artifacts.  wamx_gguf_* replaces wam.cpp's GgufReader
 * (src/models/common/gguf_reader.h:26-66, .cpp:26-227), which parses through
 * ggml's gguf library; this one reads the GGUF v2/v3 container directly.
 * Opening reads the header (metadata and tensor descriptors) and checks every
 * count, length and offset against the file; payloads are read on request.
 * No GPU is needed.
 * ------------------------------------------------------------------------- */
typedef struct wamx_gguf * wamx_gguf_t;

WAMX_API wamx_gguf_t  wamx_gguf_open(const char * path);          /* GgufReader::open; NULL + wamx_last_error() */
WAMX_API void         wamx_gguf_close(wamx_gguf_t g);
WAMX_API uint32_t     wamx_gguf_version(wamx_gguf_t g);
WAMX_API uint64_t     wamx_gguf_data_offset(wamx_gguf_t g);       /* GgufReader::data_offset */
WAMX_API int64_t      wamx_gguf_n_keys(wamx_gguf_t g);
WAMX_API const char * wamx_gguf_key(wamx_gguf_t g, int64_t i);
/* GGUF value type of a key (0 u8 .. 12 f64, 9 array), -1 when absent (GgufReader::has). */
WAMX_API int32_t      wamx_gguf_key_type(wamx_gguf_t g, const char * key);
WAMX_API bool         wamx_gguf_has(wamx_gguf_t g, const char * key);
/* GgufReader::require_u32 / require_u64 / require_f32 / require_string /
 * require_f32_array: FAILED (NULL, -1) with a message when the key is missing
 * or of another type.  The f32 array getter copies up to cap values (F32 or
 * F64 elements) and returns the array length. */
WAMX_API wamx_status  wamx_gguf_get_u32(wamx_gguf_t g, const char * key, uint32_t * out);
WAMX_API wamx_status  wamx_gguf_get_u64(wamx_gguf_t g, const char * key, uint64_t * out);
WAMX_API wamx_status  wamx_gguf_get_f32(wamx_gguf_t g, const char * key, float * out);
WAMX_API const char * wamx_gguf_get_str(wamx_gguf_t g, const char * key);
WAMX_API int64_t      wamx_gguf_get_f32_array(wamx_gguf_t g, const char * key, float * out, int64_t cap);
/* Tensor descriptors (GgufTensorInfo): name, ggml type (0 F32, 1 F16, 30 BF16,
 * ...), n_dims, ne[dim] (1 past n_dims), absolute file offset, payload bytes
 * (0 for a type this reader does not size).  find returns -1 when absent. */
WAMX_API int64_t      wamx_gguf_n_tensors(wamx_gguf_t g);
WAMX_API int64_t      wamx_gguf_find_tensor(wamx_gguf_t g, const char * name);
WAMX_API const char * wamx_gguf_tensor_name(wamx_gguf_t g, int64_t i);
WAMX_API int32_t      wamx_gguf_tensor_type(wamx_gguf_t g, int64_t i);
WAMX_API int32_t      wamx_gguf_tensor_n_dims(wamx_gguf_t g, int64_t i);
WAMX_API int64_t      wamx_gguf_tensor_ne(wamx_gguf_t g, int64_t i, int32_t dim);
WAMX_API uint64_t     wamx_gguf_tensor_offset(wamx_gguf_t g, int64_t i);
WAMX_API uint64_t     wamx_gguf_tensor_bytes(wamx_gguf_t g, int64_t i);
/* GgufReader::read_tensor: the payload of tensor i into dst (bytes must equal
 * its size). */
WAMX_API wamx_status  wamx_gguf_read_tensor(wamx_gguf_t g, int64_t i, void * dst, uint64_t bytes);

/* The GGUF tensor-name ABI: the compact name under which a GWP artifact
 * stores a weight the engine addresses by its framework name (weights.cpp
 * compact_tensor_name, :116-167; scripts/convert/convert_gwp05.py:57-140),
 * e.g. "gwp.blocks.3.action_expert.attn1.to_qkv.weight" ->
 * "gwp.blk.3.a.sa.qkv.weight".  Writes at most cap bytes (NUL included);
 * returns the full length, -1 for an unknown component. */
WAMX_API int32_t      wamx_gguf_compact_name(const char * name, char * out, int32_t cap);

/* A GWP-0.5 model from a GGUF artifact, with its weights resident on the
 * backend (the MoT component of wam.cpp's load_resident_weights,
 * weights.cpp:702-770, and the geometry / schema checks of inspect_artifact,
 * artifact.cpp:20-120, 232-292).  The geometry comes from the gwp05.* keys:
 * grid = image_height/32 x image_width/32 (semantics.cpp:58-66), latent
 * channels vae_z_dim, flow steps / shift, norm eps; n_lang prompt tokens (0:
 * the reference's 64, semantics.h:11) and batch are the caller's.  The
 * artifact's policy must store the MoT in BF16 (mot-bf16-v1, mot-vae-bf16-v1,
 * mot-vae-bf16-qkv-v1): this backend runs the BF16 latency profile only.
 * Weights are repacked as the model holds them: the per-layer adaLN tables
 * into [width, 6, L], the embodiment_id slice of the category-specific
 * encoder / decoder projections transposed to [out][in] (mot.cpp:1-53), and
 * separate attn1 q / k / v into the packed QKV when the artifact is not
 * packed.  T5, VAE and statistic tensors are not read. */
WAMX_API wamx_gwp_t  wamx_gwp_create_from_gguf(wamx_backend_t be, wamx_gguf_t g, int32_t n_lang, int32_t batch);

/* ---------------------------------------------------------------------------
 * Camera views -> VAE input (gwp05_cuda_preprocessor_create / _destroy /
 * gwp05_cuda_preprocess, src/models/gwp05/kernels/cuda_preprocess.h:8-15,
 * .cu:45-200): three host images (camera_high, camera_left_wrist,
 * camera_right_wrist) composed into an out_w x out_h canvas (top half; bottom
 * left; bottom right), each resized to cover its region with an antialiased
 * triangle filter and centre-cropped, written 2x2 pixel-unshuffled as f32
 * [12][out_h/2][out_w/2] in [-1, 1] to device memory.  The preprocessor keeps
 * the per-view device staging buffers; the call is synchronous.
 * ------------------------------------------------------------------------- */
typedef struct wamx_image_view {
    const void * data;   /* host RGB, row-major [h][w][3] */
    int32_t w, h;
    int32_t format;      /* 0: u8 (value / 255), 1: f32 in [0, 1] (PixelFormat U8 / F32_RGB_01) */
} wamx_image_view;
typedef struct wamx_preprocessor * wamx_preprocessor_t;
WAMX_API wamx_preprocessor_t wamx_preprocessor_create(wamx_backend_t be);
WAMX_API void                wamx_preprocessor_free(wamx_preprocessor_t p);
WAMX_API wamx_status         wamx_preprocess_views(wamx_preprocessor_t p, const wamx_image_view * views,
                                                   int32_t n_views, int32_t out_w, int32_t out_h, float * out_device);

/* ---------------------------------------------------------------------------
 * UMT5 text encoder: prompt tokens -> the f32 prompt embedding [max_tokens]
 * [hidden] (the reference's run_t5, src/models/gwp05/engine/text_encoder.cpp
 * :112-204, for its `resident` / `fixed` language policies).  Built on this
 * backend's IR op for op and run through wamx_backend_graph_compute: token
 * rows by GET_ROWS, per layer RMSNorm x weight, self-attention with a
 * relative-position bias (32 buckets, max distance 128) as the SOFT_MAX mask
 * and scale 1, gated-GELU FFN, residual adds; a final RMSNorm.  Weights are
 * bf16 with the reference's names ("t5.shared.weight",
 * "t5.encoder.block.{l}.layer.0.SelfAttention.{q,k,v,o}.weight", ...).
 * ------------------------------------------------------------------------- */
typedef struct wamx_t5_config {
    int32_t vocab;       /* gwp05.t5_vocab_size */
    int32_t hidden;      /* gwp05.t5_hidden */
    int32_t ffn_dim;     /* gwp05.t5_ffn_dim */
    int32_t heads;       /* gwp05.t5_heads */
    int32_t head_dim;    /* gwp05.t5_head_dim */
    int32_t layers;      /* gwp05.t5_layers */
    int32_t max_tokens;  /* prompt rows returned (the GWP prompt: 64) */
    float   eps;         /* RMSNorm eps (1e-6) */
} wamx_t5_config;
typedef struct wamx_t5 * wamx_t5_t;

WAMX_API wamx_t5_t    wamx_t5_create(wamx_backend_t be, const wamx_t5_config * cfg);  /* weights allocated, unset */
WAMX_API void         wamx_t5_free(wamx_t5_t t);
WAMX_API int          wamx_t5_n_weights(wamx_t5_t t);
WAMX_API const char * wamx_t5_weight_name(wamx_t5_t t, int i);
WAMX_API wamx_tensor * wamx_t5_weight(wamx_t5_t t, const char * name);
/* The t5.* tensors of a GWP artifact (BF16, compact names). */
WAMX_API wamx_status  wamx_t5_load_gguf(wamx_t5_t t, wamx_gguf_t g);
/* Configuration from the gwp05.t5_* keys, 64 prompt tokens, weights loaded. */
WAMX_API wamx_t5_t    wamx_t5_create_from_gguf(wamx_backend_t be, wamx_gguf_t g);
/* Encode n (1..max_tokens) tokens; mask (nullable) holds 0/1 with the valid
 * tokens a contiguous prefix, as validate_prompt_mask requires
 * (text_encoder.cpp:75-110).  out: f32 [max_tokens][hidden], rows past the
 * valid prefix zero.  Synchronous.  A non-finite embedding returns
 * WAMX_STATUS_FAILED (the engine's check, engine.cpp:314-320); out is still
 * written. */
WAMX_API wamx_status  wamx_t5_encode(wamx_t5_t t, const int32_t * tokens, const int32_t * mask, int32_t n,
                                     float * out);
/* Prompt-embedding cache of wamx_t5_encode, the reference engine's LRU
 * (src/models/gwp05/engine/weights.cpp:305-317, :394-451; engine.cpp:306-331):
 * a request whose tokens and mask (all ones when null) equal a cached
 * entry's gets that embedding without encoding and moves it to the front; a
 * miss that encodes to a finite embedding is added at the front and the
 * oldest entry dropped past the capacity.  Misses are counted only with the
 * cache on.  The initial capacity is WAM_GWP05_PROMPT_CACHE_SIZE as the
 * reference reads it (unset or empty: 4; any '-', a non-number or trailing
 * characters: 0, off).  Setting the capacity drops the oldest entries past
 * it (0 empties and disables).  wamx_t5_weight and wamx_t5_load_gguf empty
 * the cache, since its embeddings were made with the weights they change. */
WAMX_API wamx_status  wamx_t5_set_prompt_cache(wamx_t5_t t, size_t capacity);
typedef struct wamx_prompt_cache_stats {
    int32_t  enabled;   /* capacity != 0 (stats.prompt_cache_enabled) */
    int32_t  last_hit;  /* the last encode was served by the cache or the fixed prompt */
    uint64_t capacity;
    uint64_t hits;      /* stats.prompt_cache_hits */
    uint64_t misses;    /* stats.prompt_cache_misses */
    uint64_t entries;   /* stats.prompt_cache_entries */
    uint64_t bytes;     /* f32 embedding bytes held (stats.prompt_cache_bytes) */
} wamx_prompt_cache_stats;
WAMX_API wamx_status  wamx_t5_prompt_cache_stats(wamx_t5_t t, wamx_prompt_cache_stats * out);
/* The `fixed` language policy (engine.cpp:180-199, :290-300): encode this one
 * prompt now, release the encoder weights (unload_component), and from then
 * on answer wamx_t5_encode only for exactly these tokens and mask, with the
 * stored embedding; any other prompt is refused ("does not match the fixed
 * prompt").  wamx_t5_weight then returns NULL. */
WAMX_API wamx_status  wamx_t5_fix_prompt(wamx_t5_t t, const int32_t * tokens, const int32_t * mask, int32_t n);
/* T5's bidirectional relative-position bucket of key - query
 * (text_encoder.cpp:13-24); -1 for invalid bucket parameters. */
WAMX_API int32_t      wamx_t5_relative_bucket(int32_t relative, int32_t buckets, int32_t max_distance);

/* Last error message of the calling thread ("" when none). */
WAMX_API const char * wamx_last_error(void);

/* ggml op correspondence by name: wamx_ggml_op_name(i) is the string
 * ggml_op_name() returns for a ggml op ("MUL_MAT", "SOFT_MAX", ...) and
 * wamx_ggml_op_to_wamx(i) the wamx_op it runs as.  Numeric ggml values are
 * not reproduced because b9866 headers are not available.  The fused ops of
 * this backend (LINEAR, QK_NORM_ROPE, JOINT_ATTN, MODULATION) have no ggml
 * name. */
WAMX_API int          wamx_ggml_op_count(void);
WAMX_API const char * wamx_ggml_op_name(int i);
WAMX_API int32_t      wamx_ggml_op_to_wamx(int i);

/* ---------------------------------------------------------------------------
 * Graph import from ggml (the drop-in path of ggml_backend_i::graph_compute).
 *
 * The ggml side of the shim fills one descriptor per tensor of a ggml graph
 * (every node and every leaf or view source it reaches) straight from the
 * ggml_tensor fields, with names instead of enum values:
 *   op       = ggml_op_name(t->op)            ("NONE" for leaves)
 *   unary_op = ggml_unary_op_name(ggml_get_unary_op(t)) for UNARY, else NULL
 *   type     = ggml_type_name(t->type)        ("f32", "f16", "bf16", "i32")
 *   ne, nb, op_params, flags, data, name      copied verbatim
 *   src[i], view_src                           indices into the array, -1 = none
 * op_params are read in ggml's layouts (ROPE, SOFT_MAX, SCALE, IM2COL, NORM,
 * RMS_NORM, CONCAT, PERMUTE, MUL_MAT precision, the native-bf16 patch's
 * src[] extensions of ADD/NORM/RMS_NORM/UNARY).  IM2COL takes its kernel size
 * from src[0]->ne as ggml does.
 *
 * wamx_graph_from_ggml mirrors the tensors into ctx and returns a graph whose
 * nodes are graph_nodes[0..n_graph_nodes) in ggml's order, or NULL with
 * wamx_last_error() naming the first tensor it cannot represent (an unknown
 * op, unary op or type).  Replaces the body of ggml_backend_cuda's
 * graph_compute (ggml b9866, ggml-cuda.cu) as the engine reaches it from
 * mot.cpp:589, cache.cpp:121, :440. */
typedef struct wamx_ggml_tensor {
    const char * op;
    const char * unary_op;
    const char * type;
    int64_t ne[WAMX_MAX_DIMS];
    size_t  nb[WAMX_MAX_DIMS];
    int32_t op_params[WAMX_MAX_OP_PARAMS];
    int32_t flags;
    int32_t src[WAMX_MAX_SRC];
    int32_t view_src;
    size_t  view_offs;
    void *  data;
    const char * name;
} wamx_ggml_tensor;

WAMX_API wamx_cgraph * wamx_graph_from_ggml(wamx_context * ctx, const wamx_ggml_tensor * tensors, int n_tensors,
                                            const int32_t * graph_nodes, int n_graph_nodes);

#ifdef __cplusplus
}
#endif

#endif /* WAMX_WAMX_H */
