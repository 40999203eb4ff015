/*
 * cpu_port — the oracle's two heavy loops restated for speed, for the
 * cpu_baseline leg of bench.py (test infrastructure, like the rest of
 * oracle/; libwamx never links or calls it).
 *
 * The algorithm is the oracle's (same operands, same rounding points of the
 * reference's BF16 latency profile), but the reductions accumulate in fp32 in
 * a blocked order instead of in double in k order, as a CPU implementation of
 * the path would:
 *   - orc_port_gemm: y[n][m] = sum_k x[n][k] w[m][k] for bf16 weights and f32
 *     activations (already bf16-rounded), register-blocked 6 rows x 16
 *     features with AVX2 FMA (x86-64-v3), K in cache blocks of 256, weight
 *     panels converted to f32 once per block, OpenMP over feature blocks; up
 *     to 64 tokens, each weight row streamed once against the token rows;
 *   - orc_port_attention: softmax(scale K.Q) V per head with K and V^T
 *     converted to f32 once, the scores of four queries at a time in
 *     register tiles over keys, P rounded to bf16 before P.V as in the
 *     oracle.
 * Results agree with the exact oracle to fp32 accumulation error (checked in
 * tests/test_oracle.py); parity tests never use this path.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

static inline float pb2f(uint16_t h) {
    const uint32_t u = (uint32_t) h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

enum { kMB = 16, kNB = 6, kKC = 256 };

/* c[i][0..16) += sum_{k < kc} x_i[k] * wt[k][0..16) for six rows. */
static inline void micro_6x16(const float * const x[kNB], const float * wt, int kc, float * c, int ldc) {
    __m256 c0[kNB], c1[kNB];
    for (int i = 0; i < kNB; ++i) {
        c0[i] = _mm256_loadu_ps(c + i * ldc);
        c1[i] = _mm256_loadu_ps(c + i * ldc + 8);
    }
    for (int k = 0; k < kc; ++k) {
        const __m256 w0 = _mm256_load_ps(wt + k * kMB), w1 = _mm256_load_ps(wt + k * kMB + 8);
        for (int i = 0; i < kNB; ++i) {
            const __m256 a = _mm256_broadcast_ss(x[i] + k);
            c0[i] = _mm256_fmadd_ps(a, w0, c0[i]);
            c1[i] = _mm256_fmadd_ps(a, w1, c1[i]);
        }
    }
    for (int i = 0; i < kNB; ++i) {
        _mm256_storeu_ps(c + i * ldc, c0[i]);
        _mm256_storeu_ps(c + i * ldc + 8, c1[i]);
    }
}

static inline float hsum8(__m256 v);

/* Few tokens (N <= 64, the denoise step's products): each weight row is
 * streamed once, converted to f32 eight values at a time, and dotted with
 * the token rows eight at a time (eight-lane partial sums, then summed). */
static void port_gemm_skinny(const uint16_t * w, int64_t ldw, const float * xf, int64_t N, int64_t K, float * y,
                             int64_t M) {
#pragma omp parallel
    {
        float * wf = (float *) aligned_alloc(64, sizeof(float) * (size_t) ((K + 7) / 8 * 8));
#pragma omp for schedule(static)
        for (int64_t m = 0; m < M; ++m) {
            const uint16_t * wr = w + m * ldw;
            int64_t k = 0;
            for (; k + 8 <= K; k += 8) {
                const __m128i h = _mm_loadu_si128((const __m128i *) (wr + k));
                _mm256_store_ps(wf + k, _mm256_castsi256_ps(_mm256_slli_epi32(_mm256_cvtepu16_epi32(h), 16)));
            }
            for (; k < K; ++k) wf[k] = pb2f(wr[k]);
            const int64_t K8 = K / 8 * 8;
            for (int64_t n0 = 0; n0 < N; n0 += 8) {
                const int nc = (int) (N - n0 < 8 ? N - n0 : 8);
                __m256 acc[8];
                for (int i = 0; i < 8; ++i) acc[i] = _mm256_setzero_ps();
                for (int64_t kk = 0; kk < K8; kk += 8) {
                    const __m256 wv = _mm256_load_ps(wf + kk);
                    for (int i = 0; i < 8; ++i) {
                        const int64_t n = n0 + (i < nc ? i : 0);
                        acc[i] = _mm256_fmadd_ps(_mm256_loadu_ps(xf + n * K + kk), wv, acc[i]);
                    }
                }
                for (int i = 0; i < nc; ++i) {
                    float t = hsum8(acc[i]);
                    for (int64_t kk = K8; kk < K; ++kk) t += xf[(n0 + i) * K + kk] * wf[kk];
                    y[(n0 + i) * M + m] = t;
                }
            }
        }
        free(wf);
    }
}

void orc_port_gemm(const uint16_t * w, int64_t ldw, const float * xf, int64_t N, int64_t K, float * y, int64_t M) {
    if (N <= 64) {
        port_gemm_skinny(w, ldw, xf, N, K, y, M);
        return;
    }
    const int64_t nmb = (M + kMB - 1) / kMB;
    const int64_t npad = (N + kNB - 1) / kNB * kNB;
#pragma omp parallel
    {
        float * wt = (float *) aligned_alloc(64, sizeof(float) * kKC * kMB);
        float * ct = (float *) aligned_alloc(64, sizeof(float) * (size_t) npad * kMB);
#pragma omp for schedule(dynamic, 1)
        for (int64_t mb = 0; mb < nmb; ++mb) {
            const int64_t m0 = mb * kMB, mc = M - m0 < kMB ? M - m0 : kMB;
            memset(ct, 0, sizeof(float) * (size_t) npad * kMB);
            for (int64_t k0 = 0; k0 < K; k0 += kKC) {
                const int kc = (int) (K - k0 < kKC ? K - k0 : kKC);
                for (int k = 0; k < kc; ++k)
                    for (int j = 0; j < kMB; ++j) wt[k * kMB + j] = j < mc ? pb2f(w[(m0 + j) * ldw + k0 + k]) : 0.0f;
                for (int64_t n0 = 0; n0 < N; n0 += kNB) {
                    const float * x[kNB];
                    for (int i = 0; i < kNB; ++i) x[i] = xf + (n0 + i < N ? n0 + i : N - 1) * K + k0;
                    micro_6x16(x, wt, kc, ct + n0 * kMB, kMB);
                }
            }
            for (int64_t n = 0; n < N; ++n)
                for (int64_t j = 0; j < mc; ++j) y[n * M + m0 + j] = ct[n * kMB + j];
        }
        free(wt);
        free(ct);
    }
}

static inline float hsum8(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    s = _mm_add_ps(s, _mm_movehl_ps(s, s));
    s = _mm_add_ss(s, _mm_shuffle_ps(s, s, 1));
    return _mm_cvtss_f32(s);
}

static inline float prb(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
    memcpy(&f, &u, 4);
    return f;
}

enum { kQB = 4 };

/* One head: queries q[tq][dh] (f32), keys kT[dh][nkp] and values vT[dh][nkp]
 * (f32, keys padded to a multiple of 16 with zeros), out[tq][dh] f32.  Four
 * queries at a time: scores in register tiles of 4 queries x 16 keys over
 * all dims, softmax per query, P rounded to bf16, then P.V two dims at a
 * time. */
static void head_attention(const float * q, int64_t tq, const float * kT, const float * vT, int64_t nk, int64_t nkp,
                           int64_t dh, float scale, float * out, float * s /* [kQB][nkp] */) {
    for (int64_t i0 = 0; i0 < tq; i0 += kQB) {
        const int qb = (int) (tq - i0 < kQB ? tq - i0 : kQB);
        const float * qr[kQB];
        for (int r = 0; r < kQB; ++r) qr[r] = q + (i0 + (r < qb ? r : 0)) * dh;
        for (int64_t j0 = 0; j0 < nkp; j0 += 16) {
            __m256 c0[kQB], c1[kQB];
            for (int r = 0; r < kQB; ++r) c0[r] = c1[r] = _mm256_setzero_ps();
            for (int64_t d = 0; d < dh; ++d) {
                const __m256 k0 = _mm256_loadu_ps(kT + d * nkp + j0), k1 = _mm256_loadu_ps(kT + d * nkp + j0 + 8);
                for (int r = 0; r < kQB; ++r) {
                    const __m256 a = _mm256_broadcast_ss(qr[r] + d);
                    c0[r] = _mm256_fmadd_ps(a, k0, c0[r]);
                    c1[r] = _mm256_fmadd_ps(a, k1, c1[r]);
                }
            }
            for (int r = 0; r < kQB; ++r) {
                _mm256_storeu_ps(s + r * nkp + j0, c0[r]);
                _mm256_storeu_ps(s + r * nkp + j0 + 8, c1[r]);
            }
        }
        for (int r = 0; r < kQB; ++r) {
            float * sr = s + r * nkp;
            float mx = -INFINITY;
            for (int64_t j = 0; j < nk; ++j) mx = sr[j] * scale > mx ? sr[j] * scale : mx;
            float sum = 0.0f;
            for (int64_t j = 0; j < nk; ++j) {
                sr[j] = expf(sr[j] * scale - mx);
                sum += sr[j];
            }
            const float inv = 1.0f / sum;
            for (int64_t j = 0; j < nk; ++j) sr[j] = prb(sr[j] * inv);
            for (int64_t j = nk; j < nkp; ++j) sr[j] = 0.0f;
        }
        for (int64_t d = 0; d < dh; d += 2) {
            const float * v0 = vT + d * nkp, * v1 = vT + (d + 1 < dh ? d + 1 : d) * nkp;
            __m256 a0[kQB], a1[kQB];
            for (int r = 0; r < kQB; ++r) a0[r] = a1[r] = _mm256_setzero_ps();
            for (int64_t j = 0; j < nkp; j += 8) {
                const __m256 x0 = _mm256_loadu_ps(v0 + j), x1 = _mm256_loadu_ps(v1 + j);
                for (int r = 0; r < kQB; ++r) {
                    const __m256 p = _mm256_loadu_ps(s + r * nkp + j);
                    a0[r] = _mm256_fmadd_ps(p, x0, a0[r]);
                    a1[r] = _mm256_fmadd_ps(p, x1, a1[r]);
                }
            }
            for (int r = 0; r < qb; ++r) {
                out[(i0 + r) * dh + d] = hsum8(a0[r]);
                if (d + 1 < dh) out[(i0 + r) * dh + d + 1] = hsum8(a1[r]);
            }
        }
    }
}

/* orc_attention's contract (keys: source a's first na_split, then source b,
 * then the rest of a), q bf16 head-major, out bf16 [tq][heads * head_dim]. */
void orc_port_attention(const uint16_t * q, const uint16_t * k_a, const uint16_t * vt_a, int64_t na, int64_t vt_ld_a,
                        const uint16_t * k_b, const uint16_t * vt_b, int64_t nb, int64_t vt_ld_b, int64_t na_split,
                        uint16_t * out, int64_t heads, int64_t head_dim, int64_t tq, float scale) {
    const int64_t nbk = k_b ? nb : 0, nk = na + nbk, nkp = (nk + 15) / 16 * 16, dh = head_dim;
    float * kT = (float *) calloc((size_t) heads * dh * nkp, sizeof(float));
    float * vT = (float *) calloc((size_t) heads * dh * nkp, sizeof(float));
    float * qf = (float *) malloc(sizeof(float) * (size_t) heads * tq * dh);
#pragma omp parallel for collapse(2)
    for (int64_t h = 0; h < heads; ++h)
        for (int64_t d = 0; d < dh; ++d) {
            float * kr = kT + (h * dh + d) * nkp;
            float * vr = vT + (h * dh + d) * nkp;
            int64_t j = 0;
            for (int64_t a = 0; a < na_split; ++a, ++j) {
                kr[j] = pb2f(k_a[(h * na + a) * dh + d]);
                vr[j] = pb2f(vt_a[(h * dh + d) * vt_ld_a + a]);
            }
            for (int64_t b = 0; b < nbk; ++b, ++j) {
                kr[j] = pb2f(k_b[(h * nb + b) * dh + d]);
                vr[j] = pb2f(vt_b[(h * dh + d) * vt_ld_b + b]);
            }
            for (int64_t a = na_split; a < na; ++a, ++j) {
                kr[j] = pb2f(k_a[(h * na + a) * dh + d]);
                vr[j] = pb2f(vt_a[(h * dh + d) * vt_ld_a + a]);
            }
        }
    for (int64_t i = 0; i < heads * tq * dh; ++i) qf[i] = pb2f(q[i]);
    const int64_t qblocks = (tq + 63) / 64;
#pragma omp parallel
    {
        float * s = (float *) malloc(sizeof(float) * (size_t) kQB * nkp);
        float * o = (float *) malloc(sizeof(float) * (size_t) 64 * dh);
#pragma omp for collapse(2) schedule(dynamic, 1)
        for (int64_t h = 0; h < heads; ++h)
            for (int64_t qb = 0; qb < qblocks; ++qb) {
                const int64_t i0 = qb * 64, n = tq - i0 < 64 ? tq - i0 : 64;
                head_attention(qf + (h * tq + i0) * dh, n, kT + h * dh * nkp, vT + h * dh * nkp, nk, nkp, dh, scale,
                               o, s);
                for (int64_t i = 0; i < n; ++i)
                    for (int64_t d = 0; d < dh; ++d)
                        out[(i0 + i) * heads * dh + h * dh + d] = orc_f32_to_bf16(o[i * dh + d]);
            }
        free(s);
        free(o);
    }
    free(kT);
    free(vT);
    free(qf);
}

/* The visual cross-attention's form: f32 q [T][H*dh] and k [NL][H*dh], bf16
 * V^T [H*dh][NL], out bf16 [T][H*dh]. */
void orc_port_attention_f32qk(const float * q, int64_t T, const float * k, int64_t NL, const uint16_t * vt,
                              int64_t H, int64_t dh, float scale, uint16_t * out) {
    const int64_t d = H * dh, nkp = (NL + 15) / 16 * 16;
    float * kT = (float *) calloc((size_t) H * dh * nkp, sizeof(float));
    float * vT = (float *) calloc((size_t) H * dh * nkp, sizeof(float));
    float * qh = (float *) malloc(sizeof(float) * (size_t) H * T * dh);
#pragma omp parallel for collapse(2)
    for (int64_t h = 0; h < H; ++h)
        for (int64_t e = 0; e < dh; ++e)
            for (int64_t j = 0; j < NL; ++j) {
                kT[(h * dh + e) * nkp + j] = k[j * d + h * dh + e];
                vT[(h * dh + e) * nkp + j] = pb2f(vt[(h * dh + e) * NL + j]);
            }
    for (int64_t h = 0; h < H; ++h)
        for (int64_t i = 0; i < T; ++i)
            for (int64_t e = 0; e < dh; ++e) qh[(h * T + i) * dh + e] = q[i * d + h * dh + e];
    const int64_t qblocks = (T + 63) / 64;
#pragma omp parallel
    {
        float * s = (float *) malloc(sizeof(float) * (size_t) kQB * nkp);
        float * o = (float *) malloc(sizeof(float) * (size_t) 64 * dh);
#pragma omp for collapse(2) schedule(dynamic, 1)
        for (int64_t h = 0; h < H; ++h)
            for (int64_t qb = 0; qb < qblocks; ++qb) {
                const int64_t i0 = qb * 64, n = T - i0 < 64 ? T - i0 : 64;
                head_attention(qh + (h * T + i0) * dh, n, kT + h * dh * nkp, vT + h * dh * nkp, NL, nkp, dh, scale, o,
                               s);
                for (int64_t i = 0; i < n; ++i)
                    for (int64_t e = 0; e < dh; ++e) out[(i0 + i) * d + h * dh + e] = orc_f32_to_bf16(o[i * dh + e]);
            }
        free(s);
        free(o);
    }
    free(kT);
    free(vT);
    free(qh);
}
