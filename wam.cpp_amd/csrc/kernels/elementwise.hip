// Strided glue kernels for the ggml ops the engine's graphs contain besides
// the fused hot path (CPY/CONT/DUP, ADD/MUL with broadcast, SCALE, unary
// GELU/GELU_ERF/SILU, CONCAT, GET_ROWS, SOFT_MAX, ROPE), the per-layer adaLN
// modulation sum, and the seeded synthetic-weight generator.
//
// Tensors are 4-D strided views (ne[], byte strides nb[]); one thread per
// destination element, index decomposed in ne[0]-fastest order so consecutive
// threads touch consecutive destination elements.
#include "../internal.h"
#include "device.h"

#include <algorithm>

namespace wamx {

struct Ref4 {
    char * data;
    int32_t type;
    int64_t ne0, ne1, ne2, ne3;
    int64_t nb0, nb1, nb2, nb3;
};

static Ref4 to_ref4(const TensorRef & t) {
    return Ref4{(char *) t.data, t.type, t.ne[0], t.ne[1], t.ne[2], t.ne[3], t.nb[0], t.nb[1], t.nb[2], t.nb[3]};
}

__device__ __forceinline__ void unravel(int64_t i, const Ref4 & r, int64_t & i0, int64_t & i1, int64_t & i2,
                                        int64_t & i3) {
    i0 = i % r.ne0;
    i /= r.ne0;
    i1 = i % r.ne1;
    i /= r.ne1;
    i2 = i % r.ne2;
    i3 = i / r.ne2;
}

__device__ __forceinline__ char * at(const Ref4 & r, int64_t i0, int64_t i1, int64_t i2, int64_t i3) {
    return r.data + i0 * r.nb0 + i1 * r.nb1 + i2 * r.nb2 + i3 * r.nb3;
}

__device__ __forceinline__ float ld(const Ref4 & r, const char * p) {
    switch (r.type) {
        case WAMX_TYPE_F32: return *(const float *) p;
        case WAMX_TYPE_BF16: return bf16_to_f32(*(const uint16_t *) p);
        case WAMX_TYPE_I32: return (float) *(const int32_t *) p;
        default: return (float) *(const _Float16 *) p;
    }
}
__device__ __forceinline__ void st(const Ref4 & r, char * p, float v) {
    switch (r.type) {
        case WAMX_TYPE_F32: *(float *) p = v; break;
        case WAMX_TYPE_BF16: *(uint16_t *) p = f32_to_bf16(v); break;
        case WAMX_TYPE_I32: *(int32_t *) p = (int32_t) v; break;
        default: *(_Float16 *) p = (_Float16) v; break;
    }
}

// Element k of src (in its own ne0-fastest order) goes to element k of dst.
__global__ void copy_kernel(Ref4 src, Ref4 dst, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t a0, a1, a2, a3, b0, b1, b2, b3;
    unravel(i, src, a0, a1, a2, a3);
    unravel(i, dst, b0, b1, b2, b3);
    const char * ps = at(src, a0, a1, a2, a3);
    char * pd = at(dst, b0, b1, b2, b3);
    if (src.type == dst.type) {
        if (src.type == WAMX_TYPE_F32 || src.type == WAMX_TYPE_I32) *(uint32_t *) pd = *(const uint32_t *) ps;
        else *(uint16_t *) pd = *(const uint16_t *) ps;
    } else {
        st(dst, pd, ld(src, ps));
    }
}

// A copy between two same-shape views of 2-byte elements that transposes
// dims 0 and 1 in memory: dst's dim 0 and src's dim 1 are contiguous (the
// V^T store of the attention caches: token-major V -> [head][dim][token]).
// 64 x 64 tiles through LDS, so both the reads (along dim 1) and the writes
// (along dim 0) are consecutive addresses across consecutive threads.
// transpose01_kernel with 16-byte global accesses: src dim 1 and dst dim 0
// contiguous, ne1 % 8 == 0 and 16-byte aligned row strides.  The destination
// may start `mis` elements past a 16-byte boundary (a cache written from token
// 1): `dst` is then the aligned view `mis` elements earlier, and destination
// element j holds source row j - mis.  A 64 x 64 tile of the destination's
// 16-byte grid per workgroup: 512 source chunks of 8 elements are loaded (two
// per thread, both issued before the LDS stores), transposed through LDS and
// stored as 512 destination chunks; chunks that are not whole inside
// [mis, ne0 of dst) are written element by element.
__global__ __launch_bounds__(256) void transpose01_vec_kernel(Ref4 src, Ref4 dst, int mis) {
    __shared__ uint32_t tile[64][33];  // tile[r][j]: elements 2j, 2j+1 of source row b0 + r - mis
    const int64_t b0 = (int64_t) blockIdx.x * 64, b1 = (int64_t) blockIdx.y * 64;
    const int64_t i2 = blockIdx.z % src.ne2, i3 = blockIdx.z / src.ne2;
    const int t = threadIdx.x;
    uint4 v[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int q = k * 256 + t, r = q >> 3, c8 = q & 7;
        const int64_t sr = b0 + r - mis;
        const bool ok = sr >= 0 && sr < src.ne0 && b1 + 8 * c8 < src.ne1;
        v[k] = ok ? *(const uint4 *) at(src, sr, b1 + 8 * c8, i2, i3) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int q = k * 256 + t, r = q >> 3, c8 = q & 7;
        tile[r][4 * c8] = v[k].x;
        tile[r][4 * c8 + 1] = v[k].y;
        tile[r][4 * c8 + 2] = v[k].z;
        tile[r][4 * c8 + 3] = v[k].w;
    }
    __syncthreads();
    const uint16_t * tl = (const uint16_t *) &tile[0][0];  // element (r, c) at r * 66 + c
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int q = k * 256 + t, d = q >> 3, c8 = q & 7;  // destination row b1 + d, elements b0 + 8 c8 ..
        if (b1 + d >= dst.ne1) continue;
        uint16_t e[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) e[i] = tl[(8 * c8 + i) * 66 + d];
        const int64_t j0 = b0 + 8 * c8;
        if (j0 >= mis && j0 + 8 <= dst.ne0) {
            *(uint4 *) at(dst, j0, b1 + d, i2, i3) =
                make_uint4(e[0] | (uint32_t) e[1] << 16, e[2] | (uint32_t) e[3] << 16, e[4] | (uint32_t) e[5] << 16,
                           e[6] | (uint32_t) e[7] << 16);
        } else {
            for (int i = 0; i < 8; ++i)
                if (j0 + i >= mis && j0 + i < dst.ne0) *(uint16_t *) at(dst, j0 + i, b1 + d, i2, i3) = e[i];
        }
    }
}

__global__ __launch_bounds__(256) void transpose01_kernel(Ref4 src, Ref4 dst) {
    __shared__ uint16_t tile[64][66];
    const int64_t b0 = (int64_t) blockIdx.x * 64, b1 = (int64_t) blockIdx.y * 64;
    const int64_t i2 = blockIdx.z % src.ne2, i3 = blockIdx.z / src.ne2;
    const int t = threadIdx.x;
#pragma unroll 4
    for (int k = 0; k < 16; ++k) {
        const int idx = k * 256 + t, r = idx >> 6, c = idx & 63;  // r: dim 0, c: dim 1
        if (b0 + r < src.ne0 && b1 + c < src.ne1) tile[r][c] = *(const uint16_t *) at(src, b0 + r, b1 + c, i2, i3);
    }
    __syncthreads();
#pragma unroll 4
    for (int k = 0; k < 16; ++k) {
        const int idx = k * 256 + t, r = idx >> 6, c = idx & 63;  // r: dim 1, c: dim 0
        if (b0 + c < dst.ne0 && b1 + r < dst.ne1) *(uint16_t *) at(dst, b0 + c, b1 + r, i2, i3) = tile[c][r];
    }
}

__global__ void binary_kernel(int op, Ref4 a, Ref4 b, Ref4 dst, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t i0, i1, i2, i3;
    unravel(i, dst, i0, i1, i2, i3);
    const float y = ld(b, at(b, i0 % b.ne0, i1 % b.ne1, i2 % b.ne2, i3 % b.ne3));
    if (op == 2) {  // REPEAT: dst = b broadcast
        st(dst, at(dst, i0, i1, i2, i3), y);
        return;
    }
    const float x = ld(a, at(a, i0, i1, i2, i3));
    st(dst, at(dst, i0, i1, i2, i3), op == 0 ? x + y : x * y);
}

__global__ void unary_kernel(int op, Ref4 a, Ref4 dst, float scale, float bias, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t i0, i1, i2, i3;
    unravel(i, dst, i0, i1, i2, i3);
    const float x = ld(a, at(a, i0, i1, i2, i3));
    float y;
    switch (op) {
        case WAMX_UNARY_GELU: y = gelu_tanh(x); break;
        case WAMX_UNARY_GELU_ERF: y = gelu_erf(x); break;
        case WAMX_UNARY_SILU: y = silu(x); break;
        default: y = x * scale + bias; break;
    }
    st(dst, at(dst, i0, i1, i2, i3), y);
}

__global__ void concat_kernel(Ref4 a, Ref4 b, Ref4 dst, int dim, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t c[4];
    unravel(i, dst, c[0], c[1], c[2], c[3]);
    const int64_t ane[4] = {a.ne0, a.ne1, a.ne2, a.ne3};
    const char * src;
    if (c[dim] < ane[dim]) {
        src = at(a, c[0], c[1], c[2], c[3]);
    } else {
        c[dim] -= ane[dim];
        src = at(b, c[0], c[1], c[2], c[3]);
        c[dim] += ane[dim];
    }
    char * d = at(dst, c[0], c[1], c[2], c[3]);
    if (dst.type == WAMX_TYPE_F32 || dst.type == WAMX_TYPE_I32) *(uint32_t *) d = *(const uint32_t *) src;
    else *(uint16_t *) d = *(const uint16_t *) src;
}

// dst[i0, i1, i2] = a[i0, rows[i1, i2], i2 % a.ne2]
__global__ void get_rows_kernel(Ref4 a, const int32_t * rows, int64_t rows_ld, Ref4 dst, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t i0, i1, i2, i3;
    unravel(i, dst, i0, i1, i2, i3);
    const int64_t r = rows[i1 + i2 * rows_ld];
    st(dst, at(dst, i0, i1, i2, i3), ld(a, at(a, i0, r, i2 % a.ne2, i3 % a.ne3)));
}

// SOFT_MAX_EXT: y = exp(w - max) / sum over ne0 with w = scale * x + mask
// (mask row i1 of plane (i2 % ne2, i3 % ne3); no mask when m.data is null).
// One workgroup per row.
__global__ __launch_bounds__(256) void softmax_kernel(Ref4 x, Ref4 m, Ref4 y, float scale) {
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int64_t r1 = row % x.ne1, r2 = (row / x.ne1) % x.ne2, r3 = row / (x.ne1 * x.ne2);
    const char * xr = at(x, 0, r1, r2, r3);
    const char * mr = m.data ? at(m, 0, r1, r2 % m.ne2, r3 % m.ne3) : nullptr;
    char * yr = at(y, 0, r1, r2, r3);
    auto w_at = [&](int64_t c) {
        const float v = *(const float *) (xr + c * x.nb0) * scale;
        return mr ? v + ld(m, mr + c * m.nb0) : v;
    };
    float mx = -INFINITY;
    for (int64_t c = threadIdx.x; c < x.ne0; c += 256) mx = fmaxf(mx, w_at(c));
    mx = wave_max(mx);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sum = 0.0f;
    for (int64_t c = threadIdx.x; c < x.ne0; c += 256) {
        const float e = expf(w_at(c) - mx);
        *(float *) (yr + c * y.nb0) = e;
        sum += e;
    }
    sum = block_sum(sum, red);
    const float inv = 1.0f / sum;
    for (int64_t c = threadIdx.x; c < x.ne0; c += 256) *(float *) (yr + c * y.nb0) *= inv;
}

// ROPE mode NORMAL on [head_dim, heads, tokens(, ne3)]: pairs (2i, 2i+1) for
// 2i < n_dims rotate by pos[token] * theta_scale^i; the rest is copied.
__global__ void rope_kernel(Ref4 x, const int32_t * pos, Ref4 y, int n_dims, float theta_scale, int64_t npairs) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= npairs) return;
    const int64_t half = (x.ne0 + 1) / 2;
    const int64_t ip = i % half;
    int64_t rest = i / half;
    const int64_t i1 = rest % x.ne1;
    rest /= x.ne1;
    const int64_t i2 = rest % x.ne2, i3 = rest / x.ne2;
    const int64_t e = 2 * ip;
    const char * px = at(x, e, i1, i2, i3);
    char * py = at(y, e, i1, i2, i3);
    const float a = *(const float *) px;
    if (e + 1 >= x.ne0) {
        *(float *) py = a;
        return;
    }
    const float b = *(const float *) (px + x.nb0);
    if (e < n_dims) {
        const float theta = (float) pos[i2] * powf(theta_scale, (float) ip);
        float sn, cs;
        sincosf(theta, &sn, &cs);
        *(float *) py = a * cs - b * sn;
        *(float *) (py + y.nb0) = a * sn + b * cs;
    } else {
        *(float *) py = a;
        *(float *) (py + y.nb0) = b;
    }
}

// ggml_im2col, 2-D: dst[n][oh][ow][ic*KH*KW + kh*KW + kw] =
// src[n][ic][oh*s1 + kh*d1 - p1][ow*s0 + kw*d0 - p0] (zero outside).
__global__ void im2col_kernel(Ref4 src, Ref4 dst, int KW, int KH, int s0, int s1, int p0, int p1, int d0, int d1,
                              int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    int64_t c, ow, oh, b;
    unravel(i, dst, c, ow, oh, b);
    const int64_t kw = c % KW, kh = (c / KW) % KH, ic = c / (KW * KH);
    const int64_t iw = ow * s0 + kw * d0 - p0, ih = oh * s1 + kh * d1 - p1;
    float v = 0.0f;
    if (iw >= 0 && iw < src.ne0 && ih >= 0 && ih < src.ne1) v = ld(src, at(src, iw, ih, ic, b));
    st(dst, at(dst, c, ow, oh, b), v);
}

// out[l][j] = f32(mod[j]) + f32(tables[l][j])  (modulation_add, mot.cpp:137-145).
// out[s][r] = f32(mod[s][r % per_layer]) + f32(tables[r]) for the S columns
// (timesteps) of mod, r over the per_step = per_layer * layers table values.
__global__ void modulation_kernel(const void * mod, int32_t mod_type, const void * tables, int32_t tab_type, float * out,
                                  int64_t per_layer, int64_t per_step, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int64_t st = i / per_step, r = i - st * per_step, j = r % per_layer;
    out[i] = load_as_f32(mod, mod_type, st * per_layer + j) + load_as_f32(tables, tab_type, r);
}

// scheduler_step (weights.cpp:885-902): bf16(f32(a) + f32(v) * dt), the
// product and the sum rounded separately as the MUL and ADD nodes do.
#pragma clang fp contract(off)
__global__ void euler_step_kernel(const uint16_t * __restrict__ a, const uint16_t * __restrict__ v,
                                  const float * __restrict__ dt, uint16_t * __restrict__ out, int64_t n) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float t = bf16_to_f32(v[i]) * dt[0];
    out[i] = f32_to_bf16(bf16_to_f32(a[i]) + t);
}
#pragma clang fp contract(on)

// Two small linear layers (widths <= kMlpMax) for 16 tokens per workgroup:
// the tokens' inputs transposed into LDS as f32 [k][16], one layer's weight
// staged as bf16 [m][k] (rows padded by one element); thread t owns feature
// t % 128 for tokens 8 (t / 128) .. +8 and accumulates in k order in f32.
// Each layer: bf16(bf16(acc) + bias), then GELU_ERF rounded to bf16 where
// its flag is set; layer 1's output is layer 2's input in LDS.
constexpr int kMlpMax = 128, kMlpTok = 16;
__global__ __launch_bounds__(256) void mlp_small_kernel(const uint16_t * __restrict__ x, const uint16_t * __restrict__ w1,
                                                        const uint16_t * __restrict__ b1,
                                                        const uint16_t * __restrict__ w2,
                                                        const uint16_t * __restrict__ b2, uint16_t * __restrict__ y,
                                                        int64_t N, int K0, int M1, int M2, int flags) {
    __shared__ __align__(16) float xt[kMlpMax][kMlpTok];
    __shared__ __align__(16) float ht[kMlpMax][kMlpTok];
    __shared__ uint16_t ws[kMlpMax * (kMlpMax + 1)];
    const int tid = threadIdx.x;
    const int64_t n0 = (int64_t) blockIdx.x * kMlpTok;
    for (int e = tid; e < kMlpTok * K0; e += 256) {
        const int n = e / K0, k = e % K0;
        float v = n0 + n < N ? bf16_to_f32(x[(n0 + n) * K0 + k]) : 0.0f;
        if (flags & WAMX_MLP_GELU_IN) v = round_bf16(gelu_erf(v));
        xt[k][n] = v;
    }
    const int m = tid % kMlpMax, g = tid / kMlpMax;  // feature, token group of 8
    auto layer = [&](const uint16_t * __restrict__ w, const uint16_t * __restrict__ b, int K, int M, bool gelu,
                     float (*in)[kMlpTok], float (*out)[kMlpTok], bool last) {
        const int pitch = K + 1;
        __syncthreads();  // the previous layer is done with the weight tile and has written `in`
        for (int e = tid; e < M * K; e += 256) ws[(e / K) * pitch + e % K] = w[e];
        __syncthreads();
        if (m >= M) return;
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
        for (int k = 0; k < K; ++k) {
            const float wv = bf16_to_f32(ws[m * pitch + k]);
            const float4 xa = *(const float4 *) &in[k][8 * g], xb = *(const float4 *) &in[k][8 * g + 4];
            acc[0] = fmaf(wv, xa.x, acc[0]);
            acc[1] = fmaf(wv, xa.y, acc[1]);
            acc[2] = fmaf(wv, xa.z, acc[2]);
            acc[3] = fmaf(wv, xa.w, acc[3]);
            acc[4] = fmaf(wv, xb.x, acc[4]);
            acc[5] = fmaf(wv, xb.y, acc[5]);
            acc[6] = fmaf(wv, xb.z, acc[6]);
            acc[7] = fmaf(wv, xb.w, acc[7]);
        }
        const float bias = bf16_to_f32(b[m]);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float v = round_bf16(round_bf16(acc[j]) + bias);
            if (gelu) v = round_bf16(gelu_erf(v));
            const int64_t n = n0 + 8 * g + j;
            if (last) {
                if (n < N) y[n * M + m] = f32_to_bf16(v);
            } else {
                out[m][8 * g + j] = v;
            }
        }
    };
    layer(w1, b1, K0, M1, flags & WAMX_MLP_GELU_MID, xt, ht, false);
    layer(w2, b2, M1, M2, flags & WAMX_MLP_GELU_OUT, ht, nullptr, true);
}

// mlp_small_kernel's arithmetic (each output an f32 FMA chain over k in
// ascending order, then the same roundings, so the same bits) spread over
// more CUs: kMlpRegTok tokens per workgroup, thread t owning feature t % 128
// for tokens 2 (t / 128) .. +2.  The FMAs are VALU work (16 tokens x 128 x
// 128 per layer is 8k cycles of one CU), so the 16-token workgroups of
// mlp_small_kernel ran 19-21 us on 3 CUs.  Each thread's weight rows of both
// layers are loaded into registers up front as 16-byte chunks and the k loop
// is unrolled over them, so the only LDS traffic is the broadcast activation
// reads.  K0, M1 and M2 multiples of 8, weights 16-byte aligned.
constexpr int kMlpChunks = kMlpMax / 8, kMlpRegTok = 4, kMlpTpt = kMlpRegTok / 2;
__device__ __forceinline__ void mlp_row_load(const uint16_t * __restrict__ w, int K, int m, int M, uint4 (&r)[kMlpChunks]) {
#pragma unroll
    for (int c = 0; c < kMlpChunks; ++c)
        r[c] = (m < M && 8 * c < K) ? *(const uint4 *) (w + (int64_t) m * K + 8 * c) : make_uint4(0, 0, 0, 0);
}
__device__ __forceinline__ void mlp_row_dot(const uint4 (&r)[kMlpChunks], int K, const float (*in)[kMlpRegTok], int g,
                                            float (&acc)[kMlpTpt]) {
#pragma unroll
    for (int c = 0; c < kMlpChunks; ++c) {
        if (8 * c >= K) break;
        const uint32_t wp[4] = {r[c].x, r[c].y, r[c].z, r[c].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float wv = __uint_as_float(e & 1 ? wp[e >> 1] & 0xffff0000u : wp[e >> 1] << 16);
            const float2 xv = *(const float2 *) &in[8 * c + e][kMlpTpt * g];
            acc[0] = fmaf(wv, xv.x, acc[0]);
            acc[1] = fmaf(wv, xv.y, acc[1]);
        }
    }
}
__global__ __launch_bounds__(256) void mlp_small_reg_kernel(const uint16_t * __restrict__ x,
                                                            const uint16_t * __restrict__ w1,
                                                            const uint16_t * __restrict__ b1,
                                                            const uint16_t * __restrict__ w2,
                                                            const uint16_t * __restrict__ b2, uint16_t * __restrict__ y,
                                                            int64_t N, int K0, int M1, int M2, int flags) {
    static_assert(kMlpTpt == 2, "two tokens per thread");
    __shared__ __align__(16) float xt[kMlpMax][kMlpRegTok];
    __shared__ __align__(16) float ht[kMlpMax][kMlpRegTok];
    const int tid = threadIdx.x;
    const int m = tid % kMlpMax, g = tid / kMlpMax;  // feature, token pair
    const int64_t n0 = (int64_t) blockIdx.x * kMlpRegTok;
    uint4 r1[kMlpChunks], r2[kMlpChunks];
    mlp_row_load(w1, K0, m, M1, r1);
    mlp_row_load(w2, M1, m, M2, r2);
    const float bias1 = m < M1 ? bf16_to_f32(b1[m]) : 0.0f, bias2 = m < M2 ? bf16_to_f32(b2[m]) : 0.0f;
    for (int e = tid; e < kMlpRegTok * K0; e += 256) {
        const int n = e / K0, k = e % K0;
        float v = n0 + n < N ? bf16_to_f32(x[(n0 + n) * K0 + k]) : 0.0f;
        if (flags & WAMX_MLP_GELU_IN) v = round_bf16(gelu_erf(v));
        xt[k][n] = v;
    }
    __syncthreads();
    float acc[kMlpTpt];
    if (m < M1) {
        acc[0] = acc[1] = 0.0f;
        mlp_row_dot(r1, K0, xt, g, acc);
#pragma unroll
        for (int j = 0; j < kMlpTpt; ++j) {
            float v = round_bf16(round_bf16(acc[j]) + bias1);
            if (flags & WAMX_MLP_GELU_MID) v = round_bf16(gelu_erf(v));
            ht[m][kMlpTpt * g + j] = v;
        }
    }
    __syncthreads();
    if (m >= M2) return;
    acc[0] = acc[1] = 0.0f;
    mlp_row_dot(r2, M1, ht, g, acc);
#pragma unroll
    for (int j = 0; j < kMlpTpt; ++j) {
        float v = round_bf16(round_bf16(acc[j]) + bias2);
        if (flags & WAMX_MLP_GELU_OUT) v = round_bf16(gelu_erf(v));
        const int64_t n = n0 + kMlpTpt * g + j;
        if (n < N) y[n * M2 + m] = f32_to_bf16(v);
    }
}

// splitmix64 (Steele, Lea, Flood: "Fast splittable pseudorandom number
// generators", OOPSLA 2014) on seed + (i+1)*golden gamma, then Box-Muller
// with two 24-bit uniforms in (0, 1).
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void fill_normal_kernel(void * dst, int32_t type, int64_t n, uint64_t seed, float mean, float stdv) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t z = splitmix64(seed + (uint64_t) (i + 1) * 0x9E3779B97F4A7C15ull);
    const float u1 = ((float) (z >> 40) + 0.5f) * (1.0f / 16777216.0f);
    const float u2 = ((float) ((z >> 16) & 0xFFFFFFull) + 0.5f) * (1.0f / 16777216.0f);
    const float r = sqrtf(-2.0f * logf(u1));
    const float v = mean + stdv * r * cosf(6.283185307179586f * u2);
    if (type == WAMX_TYPE_F32) ((float *) dst)[i] = v;
    else ((uint16_t *) dst)[i] = f32_to_bf16(v);
}

__global__ void fill_f32_kernel(float * dst, int64_t n, float v) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) dst[i] = v;
}

// ---------------------------------------------------------------------------
static int64_t nel(const TensorRef & t) { return t.ne[0] * t.ne[1] * t.ne[2] * t.ne[3]; }
static dim3 grid1d(int64_t n) { return dim3((unsigned) ((n + 255) / 256)); }

hipError_t launch_copy(const TensorRef & src, const TensorRef & dst, hipStream_t s) {
    const int64_t n = nel(dst);
    if (n <= 0) return hipSuccess;
    if (nel(src) != n) return hipErrorInvalidValue;
    const bool two_byte = src.type == dst.type && (src.type == WAMX_TYPE_BF16 || src.type == WAMX_TYPE_F16);
    const bool same_shape =
        src.ne[0] == dst.ne[0] && src.ne[1] == dst.ne[1] && src.ne[2] == dst.ne[2] && src.ne[3] == dst.ne[3];
    if (two_byte && same_shape && dst.nb[0] == 2 && src.nb[1] == 2 && src.nb[0] != 2 && src.ne[0] >= 64 &&
        src.ne[1] >= 16) {
        const dim3 grid((unsigned) ((src.ne[0] + 63) / 64), (unsigned) ((src.ne[1] + 63) / 64),
                        (unsigned) (src.ne[2] * src.ne[3]));
        auto a16 = [](const void * p, int64_t a, int64_t b, int64_t c) {
            return (((uintptr_t) p | (uintptr_t) a | (uintptr_t) b | (uintptr_t) c) & 15) == 0;
        };
        const int mis = (int) (((uintptr_t) dst.data & 15) / 2);  // elements past the 16-byte boundary
        if (src.ne[1] % 8 == 0 && ((uintptr_t) dst.data & 1) == 0 && a16(src.data, src.nb[0], src.nb[2], src.nb[3]) &&
            a16(nullptr, dst.nb[1], dst.nb[2], dst.nb[3])) {
            Ref4 dv = to_ref4(dst);
            dv.data -= 2 * mis;
            dv.ne0 += mis;
            const dim3 vgrid((unsigned) ((dv.ne0 + 63) / 64), grid.y, grid.z);
            hipLaunchKernelGGL(transpose01_vec_kernel, vgrid, dim3(256), 0, s, to_ref4(src), dv, mis);
        } else
            hipLaunchKernelGGL(transpose01_kernel, grid, dim3(256), 0, s, to_ref4(src), to_ref4(dst));
        return hipGetLastError();
    }
    hipLaunchKernelGGL(copy_kernel, grid1d(n), dim3(256), 0, s, to_ref4(src), to_ref4(dst), n);
    return hipGetLastError();
}

hipError_t launch_binary(int op, const TensorRef & a, const TensorRef & b, const TensorRef & dst, hipStream_t s) {
    const int64_t n = nel(dst);
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(binary_kernel, grid1d(n), dim3(256), 0, s, op, to_ref4(a), to_ref4(b), to_ref4(dst), n);
    return hipGetLastError();
}

hipError_t launch_unary(int op, const TensorRef & a, const TensorRef & dst, float scale, float bias, hipStream_t s) {
    const int64_t n = nel(dst);
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(unary_kernel, grid1d(n), dim3(256), 0, s, op, to_ref4(a), to_ref4(dst), scale, bias, n);
    return hipGetLastError();
}

hipError_t launch_concat(const TensorRef & a, const TensorRef & b, const TensorRef & dst, int dim, hipStream_t s) {
    const int64_t n = nel(dst);
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(concat_kernel, grid1d(n), dim3(256), 0, s, to_ref4(a), to_ref4(b), to_ref4(dst), dim, n);
    return hipGetLastError();
}

hipError_t launch_get_rows(const TensorRef & a, const int32_t * rows, const TensorRef & dst, hipStream_t s) {
    const int64_t n = nel(dst);
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(get_rows_kernel, grid1d(n), dim3(256), 0, s, to_ref4(a), rows, dst.ne[1], to_ref4(dst), n);
    return hipGetLastError();
}

hipError_t launch_softmax_f32(const TensorRef & x, const TensorRef & mask, const TensorRef & y, float scale,
                              hipStream_t s) {
    const int64_t rows = x.ne[1] * x.ne[2] * x.ne[3];
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(softmax_kernel, dim3((unsigned) rows), dim3(256), 0, s, to_ref4(x), to_ref4(mask), to_ref4(y),
                       scale);
    return hipGetLastError();
}

hipError_t launch_rope_f32(const TensorRef & x, const int32_t * pos, const TensorRef & y, int n_dims, float freq_base,
                           hipStream_t s) {
    const int64_t npairs = (x.ne[0] + 1) / 2 * x.ne[1] * x.ne[2] * x.ne[3];
    if (npairs <= 0) return hipSuccess;
    const float theta_scale = powf(freq_base, -2.0f / (float) n_dims);
    hipLaunchKernelGGL(rope_kernel, grid1d(npairs), dim3(256), 0, s, to_ref4(x), pos, to_ref4(y), n_dims, theta_scale,
                       npairs);
    return hipGetLastError();
}

hipError_t launch_im2col(const TensorRef & src, const TensorRef & dst, int KW, int KH, int s0, int s1, int p0, int p1,
                         int d0, int d1, hipStream_t s) {
    const int64_t n = nel(dst);
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(im2col_kernel, grid1d(n), dim3(256), 0, s, to_ref4(src), to_ref4(dst), KW, KH, s0, s1, p0, p1,
                       d0, d1, n);
    return hipGetLastError();
}

hipError_t launch_modulation(const void * mod, int32_t mod_type, const void * tables, int32_t tab_type, float * out,
                             int64_t per_layer, int64_t layers, hipStream_t s, int64_t steps) {
    const int64_t per_step = per_layer * layers, n = per_step * steps;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(modulation_kernel, grid1d(n), dim3(256), 0, s, mod, mod_type, tables, tab_type, out, per_layer,
                       per_step, n);
    return hipGetLastError();
}

// Smallest index of an Inf or NaN of p[0, n) into *first (left as is when
// there is none; the caller starts it at UINT32_MAX).
__global__ void nonfinite_scan_kernel(const float * __restrict__ p, int64_t n, uint32_t * first) {
    for (int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t) gridDim.x * blockDim.x) {
        uint32_t u;
        memcpy(&u, p + i, sizeof u);
        if ((u & 0x7f800000u) == 0x7f800000u) atomicMin(first, (uint32_t) i);
    }
}

hipError_t launch_nonfinite_scan(const float * p, int64_t n, uint32_t * first, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (n >= (int64_t) UINT32_MAX) return hipErrorInvalidValue;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 2048);
    hipLaunchKernelGGL(nonfinite_scan_kernel, dim3((unsigned) blocks), dim3(256), 0, s, p, n, first);
    return hipGetLastError();
}

hipError_t launch_euler_step(const void * a, const void * v, const float * dt, void * out, int64_t n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(euler_step_kernel, grid1d(n), dim3(256), 0, s, (const uint16_t *) a, (const uint16_t *) v, dt,
                       (uint16_t *) out, n);
    return hipGetLastError();
}

hipError_t launch_mlp_small(const void * x, const void * w1, const void * b1, const void * w2, const void * b2, void * y,
                            int64_t N, int64_t K0, int64_t M1, int64_t M2, int32_t flags, hipStream_t s) {
    if (N <= 0) return hipSuccess;
    if (K0 < 1 || M1 < 1 || M2 < 1 || K0 > kMlpMax || M1 > kMlpMax || M2 > kMlpMax) return hipErrorInvalidValue;
    const bool reg = K0 % 8 == 0 && M1 % 8 == 0 && M2 % 8 == 0 && (((uintptr_t) w1 | (uintptr_t) w2) & 15) == 0;
    const int tok = reg ? kMlpRegTok : kMlpTok;
    hipLaunchKernelGGL(reg ? mlp_small_reg_kernel : mlp_small_kernel, dim3((unsigned) ((N + tok - 1) / tok)), dim3(256), 0, s,
                       (const uint16_t *) x, (const uint16_t *) w1, (const uint16_t *) b1, (const uint16_t *) w2,
                       (const uint16_t *) b2, (uint16_t *) y, N, (int) K0, (int) M1, (int) M2, (int) flags);
    return hipGetLastError();
}

hipError_t launch_fill_normal(void * dst, int32_t type, int64_t n, uint64_t seed, float mean, float stdv, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    if (type != WAMX_TYPE_F32 && type != WAMX_TYPE_BF16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(fill_normal_kernel, grid1d(n), dim3(256), 0, s, dst, type, n, seed, mean, stdv);
    return hipGetLastError();
}

hipError_t launch_fill_f32(float * dst, int64_t n, float v, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(fill_f32_kernel, grid1d(n), dim3(256), 0, s, dst, n, v);
    return hipGetLastError();
}

TensorRef ref_of(const wamx_tensor * t) {
    TensorRef r;
    r.data = t->data;
    r.type = t->type;
    for (int i = 0; i < 4; ++i) {
        r.ne[i] = t->ne[i];
        r.nb[i] = (int64_t) t->nb[i];
    }
    return r;
}

}  // namespace wamx
