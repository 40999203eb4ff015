/*
 * oracle — CPU restatement of the reference's hot-path arithmetic.
 * Test infrastructure only: see oracle.h.  Built by oracle/Makefile into
 * oracle/liboracle.so (gcc, OpenMP).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------------------
 * bf16: round-to-nearest-even on the f32 bit pattern, NaN kept quiet
 * (ggml_fp32_to_bf16 / __float2bfloat16 semantics).
 * ------------------------------------------------------------------------- */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t) ((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t) (u >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t) h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float rb(float f) { return orc_bf16_to_f32(orc_f32_to_bf16(f)); }
static inline float b2f(uint16_t h) { return orc_bf16_to_f32(h); }

void orc_round_bf16(const float * x, uint16_t * y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_bf16(x[i]);
}

int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* GELU, tanh form: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))). */
float orc_gelu_tanh(float x) {
    const double xd = x;
    return (float) (0.5 * xd * (1.0 + tanh(sqrt(2.0 / M_PI) * (xd + 0.044715 * xd * xd * xd))));
}

float orc_gelu_erf(float x) {
    const double xd = x;
    return (float) (0.5 * xd * (1.0 + erf(xd / sqrt(2.0))));
}

/* ---------------------------------------------------------------------------
 * MUL_MAT core: exact-in-double dot products of bf16-rounded operands.
 * Blocked as 4 activation rows x 16 weight rows with the weight block
 * transposed so the inner loop runs over independent accumulators (no
 * reassociation of any single sum: each sum is accumulated in k order).
 * ------------------------------------------------------------------------- */
static float x_as_bf16(const void * x, int x_type, int64_t i) {
    return x_type == ORC_F32 ? rb(((const float *) x)[i]) : b2f(((const uint16_t *) x)[i]);
}

static void gemm_f64(const uint16_t * w, int64_t ldw, const void * x, int x_type, int64_t ldx, double * acc_out,
                     int64_t M, int64_t N, int64_t K) {
    const int64_t MB = 16, NB = 4;
    const int64_t nmb = (M + MB - 1) / MB, nnb = (N + NB - 1) / NB;
    float * xf = (float *) malloc(sizeof(float) * (size_t) N * (size_t) K);
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) xf[n * K + k] = x_as_bf16(x, x_type, n * ldx + k);
#pragma omp parallel
    {
        float * wt = (float *) malloc(sizeof(float) * (size_t) K * MB);
#pragma omp for schedule(dynamic, 1)
        for (int64_t mb = 0; mb < nmb; ++mb) {
            const int64_t m0 = mb * MB;
            const int64_t mcount = (M - m0) < MB ? (M - m0) : MB;
            for (int64_t k = 0; k < K; ++k)
                for (int64_t j = 0; j < MB; ++j) wt[k * MB + j] = j < mcount ? b2f(w[(m0 + j) * ldw + k]) : 0.0f;
            for (int64_t nb = 0; nb < nnb; ++nb) {
                const int64_t n0 = nb * NB;
                const int64_t ncount = (N - n0) < NB ? (N - n0) : NB;
                double acc[4][16];
                memset(acc, 0, sizeof acc);
                const float * x0 = xf + (n0 + 0) * K;
                const float * x1 = xf + (n0 + (ncount > 1 ? 1 : 0)) * K;
                const float * x2 = xf + (n0 + (ncount > 2 ? 2 : 0)) * K;
                const float * x3 = xf + (n0 + (ncount > 3 ? 3 : 0)) * K;
                for (int64_t k = 0; k < K; ++k) {
                    const float * wk = wt + k * MB;
                    const double a0 = x0[k], a1 = x1[k], a2 = x2[k], a3 = x3[k];
                    for (int j = 0; j < 16; ++j) {
                        const double wv = wk[j];
                        acc[0][j] += a0 * wv;
                        acc[1][j] += a1 * wv;
                        acc[2][j] += a2 * wv;
                        acc[3][j] += a3 * wv;
                    }
                }
                for (int64_t i = 0; i < ncount; ++i)
                    for (int64_t j = 0; j < mcount; ++j) acc_out[(n0 + i) * M + m0 + j] = acc[i][j];
            }
        }
        free(wt);
    }
    free(xf);
}

/* The CPU-port switch (cpu_port.c): products and attention accumulate in
 * fp32 in blocked order, for timing only. */
static int g_port = 0;
void orc_set_port(int on) { g_port = on != 0; }
int orc_get_port(void) { return g_port; }

/* acc[n][m] for either mode: the exact double sums or the fp32 port. */
static void gemm_acc(const uint16_t * w, int64_t ldw, const void * x, int x_type, int64_t ldx, double * acc,
                     int64_t M, int64_t N, int64_t K) {
    if (!g_port) {
        gemm_f64(w, ldw, x, x_type, ldx, acc, M, N, K);
        return;
    }
    float * xf = (float *) malloc(sizeof(float) * (size_t) N * (size_t) K);
    float * yf = (float *) malloc(sizeof(float) * (size_t) N * (size_t) M);
#pragma omp parallel for
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) xf[n * K + k] = x_as_bf16(x, x_type, n * ldx + k);
    orc_port_gemm(w, ldw, xf, N, K, yf, M);
    for (int64_t i = 0; i < N * M; ++i) acc[i] = yf[i];
    free(xf);
    free(yf);
}

void orc_mul_mat(const uint16_t * w, int64_t ldw, const void * x, int x_type, int64_t ldx, void * y, int y_type,
                 int64_t ldy, int64_t M, int64_t N, int64_t K) {
    double * acc = (double *) malloc(sizeof(double) * (size_t) M * (size_t) N);
    gemm_acc(w, ldw, x, x_type, ldx, acc, M, N, K);
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m) {
            const float v = (float) acc[n * M + m];
            if (y_type == ORC_F32) ((float *) y)[n * ldy + m] = v;
            else ((uint16_t *) y)[n * ldy + m] = orc_f32_to_bf16(v);
        }
    free(acc);
}

/* The GEMM writes bf16 (native-bf16.patch:273-275); ADD(bias) is bf16+bf16
 * (weights.cpp:826-828); bias_gelu_bf16 (patch:507-514);
 * gated_residual_bf16 (patch:79-91, h + b*g contracted to one fma by nvcc);
 * the cross-attention residual is a plain bf16 ADD (mot.cpp:338). */
void orc_linear(const uint16_t * w, const void * x, int x_type, const uint16_t * bias, int epi,
                const uint16_t * residual, const float * gate, uint16_t * y, int64_t M, int64_t N, int64_t K) {
    double * acc = (double *) malloc(sizeof(double) * (size_t) M * (size_t) N);
    gemm_acc(w, K, x, x_type, K, acc, M, N, K);
    for (int64_t n = 0; n < N; ++n)
        for (int64_t m = 0; m < M; ++m) {
            const float g = rb((float) acc[n * M + m]);
            float out;
            switch (epi) {
                case ORC_EPI_NONE: out = g; break;
                case ORC_EPI_BIAS: out = g + b2f(bias[m]); break;
                case ORC_EPI_BIAS_GELU: out = orc_gelu_tanh(g + b2f(bias[m])); break;
                case ORC_EPI_BIAS_GATED: {
                    const float o = rb(g + b2f(bias[m]));
                    out = fmaf(o, gate[m], b2f(residual[n * M + m]));
                    break;
                }
                default: {
                    const float o = rb(g + b2f(bias[m]));
                    out = b2f(residual[n * M + m]) + o;
                    break;
                }
            }
            y[n * M + m] = orc_f32_to_bf16(out);
        }
    free(acc);
}

/* ---------------------------------------------------------------------------
 * Norms.  Row statistics in double, rounded to f32 where the kernel holds
 * them in f32; the per-element formula is the kernel's f32 expression.
 * ------------------------------------------------------------------------- */
static void row_stats_bf16(const uint16_t * xr, int64_t cols, float eps, float * mean_out, float * inv_out) {
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += b2f(xr[c]);
    const float mean = (float) (s / (double) cols);
    double v = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
        const double d = (double) (b2f(xr[c]) - mean);
        v += d * d;
    }
    const float var = (float) (v / (double) cols);
    *mean_out = mean;
    *inv_out = (float) (1.0 / sqrt((double) var + (double) eps));
}

void orc_norm_mod_bf16(const uint16_t * x, int64_t ldx, const float * scale, const float * shift, int64_t ss,
                       uint16_t * y, int64_t rows, int64_t cols, float eps) {
#pragma omp parallel for
    for (int64_t r = 0; r < rows; ++r) {
        float mean, inv;
        row_stats_bf16(x + r * ldx, cols, eps, &mean, &inv);
        for (int64_t c = 0; c < cols; ++c) {
            const float n = (b2f(x[r * ldx + c]) - mean) * inv;
            y[r * cols + c] = orc_f32_to_bf16(fmaf(n, 1.0f + scale[r * ss + c], shift[r * ss + c]));
        }
    }
}

void orc_layer_norm_bf16(const uint16_t * x, int64_t ldx, const uint16_t * w, const uint16_t * b, uint16_t * y,
                         int64_t rows, int64_t cols, float eps) {
#pragma omp parallel for
    for (int64_t r = 0; r < rows; ++r) {
        float mean, inv;
        row_stats_bf16(x + r * ldx, cols, eps, &mean, &inv);
        for (int64_t c = 0; c < cols; ++c) {
            const float n = (b2f(x[r * ldx + c]) - mean) * inv;
            y[r * cols + c] = orc_f32_to_bf16(fmaf(n, b2f(w[c]), b2f(b[c])));
        }
    }
}

static float rms_inv(const uint16_t * xr, int64_t cols, float eps) {
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
        const double v = b2f(xr[c]);
        s += v * v;
    }
    const float ms = (float) (s / (double) cols);
    return (float) (1.0 / sqrt((double) ms + (double) eps));
}

void orc_rms_norm_bf16_f32(const uint16_t * x, int64_t ldx, const uint16_t * w, float * y, int64_t rows,
                           int64_t cols, float eps) {
#pragma omp parallel for
    for (int64_t r = 0; r < rows; ++r) {
        const float inv = rms_inv(x + r * ldx, cols, eps);
        for (int64_t c = 0; c < cols; ++c) y[r * cols + c] = b2f(x[r * ldx + c]) * inv * b2f(w[c]);
    }
}

/* p7-fusions.patch:19-51, no contraction of the output expression. */
void orc_norm_mod_f32(const float * x, int64_t ldx, const float * scale, const float * shift, int64_t ss,
                      float * y, int64_t rows, int64_t cols, float eps) {
#pragma omp parallel for
    for (int64_t r = 0; r < rows; ++r) {
        const float * xr = x + r * ldx;
        double s1 = 0.0, s2 = 0.0;
        for (int64_t c = 0; c < cols; ++c) {
            s1 += xr[c];
            s2 += (double) xr[c] * (double) xr[c];
        }
        const float mean = (float) (s1 / (double) cols);
        const float var = (float) (s2 / (double) cols - (s1 / (double) cols) * (s1 / (double) cols));
        const float inv = (float) (1.0 / sqrt((double) var + (double) eps));
        for (int64_t c = 0; c < cols; ++c) {
            volatile float n = (xr[c] - mean) * inv;
            volatile float scaled = n * scale[r * ss + c];
            volatile float t = n + scaled;
            y[r * cols + c] = t + shift[r * ss + c];
        }
    }
}

void orc_gated_residual_bf16(const uint16_t * h, const uint16_t * b, const void * g, int g_type, int64_t gs,
                             uint16_t * y, int64_t rows, int64_t cols) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < cols; ++c) {
            const float gv = g_type == ORC_F32 ? ((const float *) g)[r * gs + c] : b2f(((const uint16_t *) g)[r * gs + c]);
            y[r * cols + c] = orc_f32_to_bf16(fmaf(b2f(b[r * cols + c]), gv, b2f(h[r * cols + c])));
        }
}

void orc_gated_residual_f32(const float * r, const float * b, const float * g, int64_t gs, float * y, int64_t rows,
                            int64_t cols) {
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t c = 0; c < cols; ++c) {
            volatile float scaled = b[i * cols + c] * g[i * gs + c];
            y[i * cols + c] = r[i * cols + c] + scaled;
        }
}

void orc_bias_gelu_bf16(const uint16_t * x, const uint16_t * bias, uint16_t * y, int64_t n, int64_t width) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_bf16(orc_gelu_tanh(b2f(x[i]) + b2f(bias[i % width])));
}

/* ---------------------------------------------------------------------------
 * RoPE NORMAL, angles in double.
 * ------------------------------------------------------------------------- */
static void rotate_pair(float a, float b, double theta, float * ra, float * rb_) {
    const double c = cos(theta), s = sin(theta);
    *ra = (float) (a * c - b * s);
    *rb_ = (float) (a * s + b * c);
}

void orc_rope_f32(const float * x, const int32_t * pos, float * y, int64_t head_dim, int64_t heads, int64_t tokens,
                  int n_dims, float freq_base) {
    for (int64_t t = 0; t < tokens; ++t)
        for (int64_t h = 0; h < heads; ++h) {
            const float * xr = x + (t * heads + h) * head_dim;
            float * yr = y + (t * heads + h) * head_dim;
            for (int64_t e = 0; e + 1 < head_dim; e += 2) {
                if (e < n_dims) {
                    const double theta = (double) pos[t] * pow((double) freq_base, -(double) e / (double) n_dims);
                    rotate_pair(xr[e], xr[e + 1], theta, &yr[e], &yr[e + 1]);
                } else {
                    yr[e] = xr[e];
                    yr[e + 1] = xr[e + 1];
                }
            }
            if (head_dim & 1) yr[head_dim - 1] = xr[head_dim - 1];
        }
}

void orc_qk_norm_rope(const uint16_t * x, int64_t ldx, const uint16_t * w, uint16_t * dst, int64_t heads,
                      int64_t head_dim, int64_t tokens, int64_t dst_tokens, int64_t tok0, int rope_mode,
                      const int32_t * pos0, const int32_t * pos1, const int32_t * pos2, float eps, float freq_base) {
    const int64_t d = heads * head_dim;
#pragma omp parallel for
    for (int64_t t = 0; t < tokens; ++t) {
        const uint16_t * xr = x + t * ldx;
        const float inv = rms_inv(xr, d, eps);
        for (int64_t e = 0; e < d; e += 2) {
            float a = b2f(xr[e]) * inv * b2f(w[e]);
            float b = b2f(xr[e + 1]) * inv * b2f(w[e + 1]);
            const int64_t h = e / head_dim, dd = e % head_dim;
            if (rope_mode != 2) {
                double theta;
                if (rope_mode == 0) {
                    theta = (double) pos0[t] * pow((double) freq_base, -(double) dd / (double) head_dim);
                } else if (dd < 44) {
                    theta = (double) pos0[t] * pow((double) freq_base, -(double) dd / 44.0);
                } else if (dd < 86) {
                    theta = (double) pos1[t] * pow((double) freq_base, -(double) (dd - 44) / 42.0);
                } else {
                    theta = (double) pos2[t] * pow((double) freq_base, -(double) (dd - 86) / 42.0);
                }
                float ra, rbv;
                rotate_pair(a, b, theta, &ra, &rbv);
                a = ra;
                b = rbv;
            }
            uint16_t * o = dst + (h * dst_tokens + tok0 + t) * head_dim + dd;
            o[0] = orc_f32_to_bf16(a);
            o[1] = orc_f32_to_bf16(b);
        }
    }
}

void orc_softmax_f32(const float * x, float * y, int64_t rows, int64_t cols, float scale) {
    for (int64_t r = 0; r < rows; ++r) {
        const float * xr = x + r * cols;
        float * yr = y + r * cols;
        float mx = -INFINITY;
        for (int64_t c = 0; c < cols; ++c) mx = fmaxf(mx, xr[c] * scale);
        double sum = 0.0;
        for (int64_t c = 0; c < cols; ++c) {
            yr[c] = expf(xr[c] * scale - mx);
            sum += yr[c];
        }
        const float inv = (float) (1.0 / sum);
        for (int64_t c = 0; c < cols; ++c) yr[c] *= inv;
    }
}

/* ---------------------------------------------------------------------------
 * Attention (mot.cpp:402-445), key order [a[0,na_split), b, a[na_split,na)].
 * ------------------------------------------------------------------------- */
void orc_attention(const uint16_t * q, const uint16_t * k_a, const uint16_t * vt_a, int64_t na, int64_t vt_ld_a,
                   const uint16_t * k_b, const uint16_t * vt_b, int64_t nb, int64_t vt_ld_b, int64_t na_split,
                   uint16_t * out, int64_t heads, int64_t head_dim, int64_t tq, float scale) {
    if (g_port) {
        orc_port_attention(q, k_a, vt_a, na, vt_ld_a, k_b, vt_b, nb, vt_ld_b, na_split, out, heads, head_dim, tq, scale);
        return;
    }
    const int64_t nbk = k_b ? nb : 0;
    const int64_t nk = na + nbk;
#pragma omp parallel for collapse(2)
    for (int64_t h = 0; h < heads; ++h)
        for (int64_t i = 0; i < tq; ++i) {
            float * s = (float *) malloc(sizeof(float) * (size_t) nk);
            const uint16_t ** krow = (const uint16_t **) malloc(sizeof(void *) * (size_t) nk);
            const uint16_t ** vcol = (const uint16_t **) malloc(sizeof(void *) * (size_t) nk);
            int64_t * vld = (int64_t *) malloc(sizeof(int64_t) * (size_t) nk);
            int64_t j = 0;
            for (int64_t a = 0; a < na_split; ++a, ++j) {
                krow[j] = k_a + (h * na + a) * head_dim;
                vcol[j] = vt_a + h * head_dim * vt_ld_a + a;
                vld[j] = vt_ld_a;
            }
            for (int64_t b = 0; b < nbk; ++b, ++j) {
                krow[j] = k_b + (h * nb + b) * head_dim;
                vcol[j] = vt_b + h * head_dim * vt_ld_b + b;
                vld[j] = vt_ld_b;
            }
            for (int64_t a = na_split; a < na; ++a, ++j) {
                krow[j] = k_a + (h * na + a) * head_dim;
                vcol[j] = vt_a + h * head_dim * vt_ld_a + a;
                vld[j] = vt_ld_a;
            }
            const uint16_t * qr = q + (h * tq + i) * head_dim;
            for (int64_t jj = 0; jj < nk; ++jj) {
                double acc = 0.0;
                for (int64_t d = 0; d < head_dim; ++d) acc += (double) b2f(qr[d]) * (double) b2f(krow[jj][d]);
                s[jj] = (float) acc;
            }
            orc_softmax_f32(s, s, 1, nk, scale);
            for (int64_t d = 0; d < head_dim; ++d) {
                double acc = 0.0;
                for (int64_t jj = 0; jj < nk; ++jj) acc += (double) rb(s[jj]) * (double) b2f(vcol[jj][d * vld[jj]]);
                out[i * heads * head_dim + h * head_dim + d] = orc_f32_to_bf16((float) acc);
            }
            free(s);
            free(krow);
            free(vcol);
            free(vld);
        }
}

void orc_modulation(const uint16_t * mod, const uint16_t * tables, float * out, int64_t per_layer, int64_t layers) {
    for (int64_t l = 0; l < layers; ++l)
        for (int64_t j = 0; j < per_layer; ++j) out[l * per_layer + j] = b2f(mod[j]) + b2f(tables[l * per_layer + j]);
}

/* ---------------------------------------------------------------------------
 * Schedule and timestep embedding.
 * ------------------------------------------------------------------------- */
void orc_flow_schedule(int steps, float shift, float * timesteps, float * sigmas) {
    /* Endpoint from the f32 training schedule (sigma_min = 1/1000 shifted),
     * then linspace and the shift transform in double
     * (src/models/common/scheduler.cpp:36-53). */
    const float train_sigma = 1.0f / 1000.0f;
    const float shifted_min = shift * train_sigma / (1.0f + (shift - 1.0f) * train_sigma);
    const double t_min = (double) shifted_min * 1000.0;
    for (int i = 0; i < steps; ++i) {
        const double t = steps == 1 ? 1000.0 : 1000.0 + (t_min - 1000.0) * i / (steps - 1);
        const double sg = t / 1000.0;
        const double sh = (double) shift * sg / (1.0 + ((double) shift - 1.0) * sg);
        sigmas[i] = (float) sh;
        timesteps[i] = sigmas[i] * 1000.0f;
    }
    sigmas[steps] = 0.0f;
}

void orc_timestep_embedding(float timestep, int64_t dim, float * out) {
    const int64_t half = dim / 2;
    for (int64_t i = 0; i < half; ++i) {
        const float freq = expf(-logf(10000.0f) * (float) i / (float) half);
        const float v = timestep * freq;
        out[i] = cosf(v);
        out[i + half] = sinf(v);
    }
    if (dim & 1) out[dim - 1] = 0.0f;
}

/* ---------------------------------------------------------------------------
 * Seeded normal sample (splitmix64 + Box-Muller).
 * ------------------------------------------------------------------------- */
static inline uint64_t splitmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

void orc_fill_normal(void * dst, int type, int64_t n, uint64_t seed, float mean, float std) {
#pragma omp parallel for
    for (int64_t i = 0; i < n; ++i) {
        const uint64_t z = splitmix64(seed + (uint64_t) (i + 1) * 0x9E3779B97F4A7C15ull);
        const double u1 = ((double) (z >> 40) + 0.5) / 16777216.0;
        const double u2 = ((double) ((z >> 16) & 0xFFFFFFull) + 0.5) / 16777216.0;
        const double r = sqrt(-2.0 * log(u1));
        const float v = (float) (mean + std * r * cos(2.0 * M_PI * u2));
        if (type == ORC_F32) ((float *) dst)[i] = v;
        else ((uint16_t *) dst)[i] = orc_f32_to_bf16(v);
    }
}
