/*
 * oracle — CPU restatement of the reference's arithmetic for the GWP-0.5 MoT
 * hot path (test infrastructure only).
 *
 * This library is the checker: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it.  libwamx never links or calls it.
 *
 * Each function states the reference source it restates.  Semantics follow
 * the reference's BF16 latency profile: ggml MUL_MAT converts src1 to the
 * weight's type (bf16, round-to-nearest-even) and accumulates; the patch
 * kernels of patches/llama-b9866-native-bf16.patch and
 * patches/llama-b9866-p7-fusions.patch define the fused ops.  Reductions here
 * accumulate in double (the exact value of the bf16-rounded operands up to
 * double rounding) and round once where the reference stores.
 *
 * Layouts are plain C row-major: a ggml tensor ne={K, M} is w[M][K].
 * bf16 values are uint16 bit patterns.
 */
#ifndef WAMX_ORACLE_H
#define WAMX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_BF16 = 30 };
enum { ORC_EPI_NONE = 0, ORC_EPI_BIAS = 1, ORC_EPI_BIAS_GELU = 2, ORC_EPI_BIAS_GATED = 3, ORC_EPI_BIAS_RESIDUAL = 4 };

uint16_t orc_f32_to_bf16(float f);
float    orc_bf16_to_f32(uint16_t h);
void     orc_round_bf16(const float * x, uint16_t * y, int64_t n);
int      orc_num_threads(void);

/* GELU-tanh (Hendrycks & Gimpel) and GELU-erf in double, rounded to f32. */
float orc_gelu_tanh(float x);
float orc_gelu_erf(float x);

/* MUL_MAT: y[n][m] = sum_k w[m][k] * bf16(x[n][k]); y F32 or BF16 (RNE). */
void orc_mul_mat(const uint16_t * w, int64_t ldw, const void * x, int x_type, int64_t ldx, void * y, int y_type,
                 int64_t ldy, int64_t M, int64_t N, int64_t K);

/* linear_with_activation / linear_gelu_with_activation (weights.cpp:819-849)
 * followed by gated_residual / the plain residual add (mot.cpp:161-173, 338),
 * with the rounding points of the unfused graph.  y bf16 [N][M]. */
void orc_linear(const uint16_t * w, const void * x, int x_type, const uint16_t * bias, int epi,
                const uint16_t * residual, const float * gate, uint16_t * y, int64_t M, int64_t N, int64_t K);

/* norm_bf16_fused<.,false> (native-bf16.patch:368-409): two-pass LayerNorm,
 * y = bf16(n*(1+scale)+shift) with f32 scale/shift (row stride ss, 0 = broadcast). */
void orc_norm_mod_bf16(const uint16_t * x, int64_t ldx, const float * scale, const float * shift, int64_t ss,
                       uint16_t * y, int64_t rows, int64_t cols, float eps);
/* norm_bf16_fused<.,true>: y = bf16(n*w+b) with bf16 w/b. */
void orc_layer_norm_bf16(const uint16_t * x, int64_t ldx, const uint16_t * w, const uint16_t * b, uint16_t * y,
                         int64_t rows, int64_t cols, float eps);
/* rms_norm_bf16_f32 (native-bf16.patch:411-430): y = x*rsqrt(mean(x^2)+eps)*w, f32. */
void orc_rms_norm_bf16_f32(const uint16_t * x, int64_t ldx, const uint16_t * w, float * y, int64_t rows,
                           int64_t cols, float eps);
/* norm_modulation_f32 (p7-fusions.patch:19-51): var = E[x^2]-mean^2,
 * y = (n + n*scale) + shift, each op rounded separately. */
void orc_norm_mod_f32(const float * x, int64_t ldx, const float * scale, const float * shift, int64_t ss,
                      float * y, int64_t rows, int64_t cols, float eps);
/* gated_residual_bf16<gate_t> (native-bf16.patch:79-91): y = bf16(h + b*g). */
void orc_gated_residual_bf16(const uint16_t * h, const uint16_t * b, const void * g, int g_type, int64_t gs,
                             uint16_t * y, int64_t rows, int64_t cols);
/* gated_residual_f32 (p7-fusions.patch:122-134): y = r + b*g, unfused. */
void orc_gated_residual_f32(const float * r, const float * b, const float * g, int64_t gs, float * y,
                            int64_t rows, int64_t cols);
/* bias_gelu_bf16_kernel (native-bf16.patch:507-514). */
void orc_bias_gelu_bf16(const uint16_t * x, const uint16_t * bias, uint16_t * y, int64_t n, int64_t width);

/* GGML_OP_ROPE mode NORMAL (ggml b9866, as called by mot.cpp:175-202):
 * x f32 [tokens][heads][head_dim]; pair (2i, 2i+1), 2i < n_dims, rotated by
 * theta = pos[token] * base^(-2i/n_dims). */
void orc_rope_f32(const float * x, const int32_t * pos, float * y, int64_t head_dim, int64_t heads, int64_t tokens,
                  int n_dims, float freq_base);
/* expert_qkv's Q/K chain (mot.cpp:245-265, 395-396): rms_norm_bf16_f32 over the
 * full row, RoPE (rope_mode 0: 1-D over head_dim; 1: sections {44,42,42} with
 * pos0/pos1/pos2; 2: none), bf16 cast, written to dst [H][dst_tokens][head_dim]
 * at token offset tok0. */
void orc_qk_norm_rope(const uint16_t * x, int64_t ldx, const uint16_t * w, uint16_t * dst, int64_t heads,
                      int64_t head_dim, int64_t tokens, int64_t dst_tokens, int64_t tok0, int rope_mode,
                      const int32_t * pos0, const int32_t * pos1, const int32_t * pos2, float eps, float freq_base);
/* SOFT_MAX_EXT without mask over rows of length cols. */
void orc_softmax_f32(const float * x, float * y, int64_t rows, int64_t cols, float scale);

/* The joint attention of build_cached_action_body (mot.cpp:402-445): keys in
 * the order [a[0, na_split), b, a[na_split, na)], S = K.Q in f32
 * (GGML_PREC_F32), P = softmax(scale*S) in f32, P rounded to bf16 for the
 * V.P MUL_MAT, output f32 rounded to bf16 (the O projection's input cast).
 * q [H][tq][dh]; k_a [H][na][dh]; vt_a [H][dh][vt_ld_a]; same for b;
 * out bf16 [tq][H*dh]. */
void orc_attention(const uint16_t * q, const uint16_t * k_a, const uint16_t * vt_a, int64_t na, int64_t vt_ld_a,
                   const uint16_t * k_b, const uint16_t * vt_b, int64_t nb, int64_t vt_ld_b, int64_t na_split,
                   uint16_t * out, int64_t heads, int64_t head_dim, int64_t tq, float scale);

/* modulation_add (mot.cpp:137-145): out[l][j] = f32(mod[j]) + f32(tab[l][j]). */
void orc_modulation(const uint16_t * mod, const uint16_t * tables, float * out, int64_t per_layer, int64_t layers);

/* Flow-match Euler schedule (src/models/common/scheduler.cpp:26-55). */
void orc_flow_schedule(int steps, float shift, float * timesteps, float * sigmas);
/* Sinusoidal timestep embedding, cos first (text_encoder.cpp:1-12). */
void orc_timestep_embedding(float timestep, int64_t dim, float * out);

/* Seeded N(mean, std) sample: splitmix64(seed + (i+1)*0x9E3779B97F4A7C15),
 * Box-Muller over two 24-bit uniforms.  type ORC_F32 or ORC_BF16. */
void orc_fill_normal(void * dst, int type, int64_t n, uint64_t seed, float mean, float std);

/* CPU port (cpu_port.c): the same algorithm with fp32 accumulation in a
 * blocked, vectorised order, for bench.py's cpu_baseline timing only.
 * orc_set_port(1) routes orc_mul_mat, orc_linear, orc_attention and the MoT
 * path's attentions through it; parity tests leave it off. */
void orc_set_port(int on);
int  orc_get_port(void);
void orc_port_gemm(const uint16_t * w, int64_t ldw, const float * xf, int64_t N, int64_t K, float * y, int64_t M);
void orc_port_attention(const uint16_t * q, const uint16_t * k_a, const uint16_t * vt_a, int64_t na, int64_t vt_ld_a,
                        const uint16_t * k_b, const uint16_t * vt_b, int64_t nb, int64_t vt_ld_b, int64_t na_split,
                        uint16_t * out, int64_t heads, int64_t head_dim, int64_t tq, float scale);
void orc_port_attention_f32qk(const float * q, int64_t T, const float * k, int64_t NL, const uint16_t * vt,
                              int64_t H, int64_t dh, float scale, uint16_t * out);

#ifdef __cplusplus
}
#endif

#endif
