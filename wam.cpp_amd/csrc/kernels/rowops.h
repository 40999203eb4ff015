// Row arithmetic shared by the standalone row kernels (norm.hip, attention.hip)
// and the split-K reduce kernels that apply the same row op to a GEMM output
// (gemm.hip), so both produce identical bits.  A row of `cols` values is held
// as CPT chunks of 8 per thread: chunk c = threadIdx.x + i * blockDim.x.
#pragma once

#include "device.h"

namespace wamx {

// Eight bf16 values (one 16-byte chunk) <-> f32.
__device__ __forceinline__ void unpack8(const uint4 & u, float (&f)[8]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        f[2 * e] = __uint_as_float(w[e] << 16);
        f[2 * e + 1] = __uint_as_float(w[e] & 0xFFFF0000u);
    }
}
__device__ __forceinline__ uint4 pack8(const float (&f)[8]) {
    return make_uint4(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]), pack_bf16x2(f[4], f[5]),
                      pack_bf16x2(f[6], f[7]));
}
__device__ __forceinline__ void load8_f32(const float * p, float (&f)[8]) {
    const float4 a = *(const float4 *) p, b = *(const float4 *) (p + 4);
    f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
    f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
}

// Mean and 1/sqrt(var + eps) of a row (two-pass, centred variance), as the
// LayerNorm of norm_bf16_fused (native-bf16.patch:368-409).  Chunks past
// nchunk must hold zeros.  Every thread of the block gets the result.
template <int CPT>
__device__ __forceinline__ void row_mean_istd(const float (&v)[CPT][8], int nchunk, int cols, float eps, float * red,
                                              float & mean, float & inv_std) {
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < CPT; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += v[i][e];
    mean = block_sum(sum, red) / (float) cols;
    float var = 0.0f;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        if ((int) threadIdx.x + i * (int) blockDim.x >= nchunk) continue;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float d = v[i][e] - mean;
            var = fmaf(d, d, var);
        }
    }
    var = block_sum(var, red) / (float) cols;
    inv_std = rsqrtf(var + eps);
}

// Normalised and modulated chunk: affine n*a+b, otherwise n*(1+a)+b.
template <bool AFFINE>
__device__ __forceinline__ uint4 norm_chunk(const float (&v)[8], float mean, float inv_std, const float (&a)[8],
                                            const float (&b)[8]) {
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float n = (v[e] - mean) * inv_std;
        o[e] = AFFINE ? fmaf(n, a[e], b[e]) : fmaf(n, 1.0f + a[e], b[e]);
    }
    return pack8(o);
}

// 1/rms of a row (sum of squares over cols, then + eps), as rms_norm_bf16_f32
// (native-bf16.patch:411-430).  Chunks past nchunk must hold zeros.
template <int CPT>
__device__ __forceinline__ float row_inv_rms(const float (&v)[CPT][8], int cols, float eps, float * red) {
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < CPT; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e) sum = fmaf(v[i][e], v[i][e], sum);
    return rsqrtf(block_sum(sum, red) / (float) cols + eps);
}

// RoPE parameters of one token: positions and log2 of the per-section
// theta scales (NORMAL rope over head_dim, or the {44, 42, 42} 3-D split).
struct RopeTok {
    int mode;  // 0: 1-D over head_dim, 1: 3-D sections, 2: none
    float p0, p1, p2;
    float l2ts128, l2ts44, l2ts42;
};

__device__ __forceinline__ RopeTok rope_tok(int mode, const int32_t * pos0, const int32_t * pos1,
                                            const int32_t * pos2, int64_t t, float l2ts128, float l2ts44,
                                            float l2ts42) {
    RopeTok r;
    r.mode = mode;
    r.p0 = mode == 2 ? 0.0f : (float) pos0[t];
    r.p1 = mode == 1 ? (float) pos1[t] : 0.0f;
    r.p2 = mode == 1 ? (float) pos2[t] : 0.0f;
    r.l2ts128 = l2ts128;
    r.l2ts44 = l2ts44;
    r.l2ts42 = l2ts42;
    return r;
}

// Rotation angle of the pair at element dd of a head: theta = pos *
// base^(-2i/n) for pair i of its rope section (mode 0: 1-D over head_dim;
// mode 1: the {44, 42, 42} sections on positions p0, p1, p2).
__device__ __forceinline__ float rope_theta(const RopeTok & r, int dd) {
    if (r.mode == 0) return r.p0 * exp2f((float) (dd >> 1) * r.l2ts128);
    if (dd < 44) return r.p0 * exp2f((float) (dd >> 1) * r.l2ts44);
    if (dd < 86) return r.p1 * exp2f((float) ((dd - 44) >> 1) * r.l2ts42);
    return r.p2 * exp2f((float) ((dd - 86) >> 1) * r.l2ts42);
}

// (a, b) rotated by the angle with cosine cs and sine sn, in one fixed
// rounding sequence (each output one fma over a rounded product), so every
// kernel that rotates gives the same bits whatever the compiler would
// contract in `a * cs - b * sn`.
__device__ __forceinline__ void rotate_pair(float & a, float & b, float cs, float sn) {
    const float ra = fmaf(a, cs, -(b * sn));
    const float rb = fmaf(a, sn, b * cs);
    a = ra;
    b = rb;
}

// RMSNorm-scaled chunk (x * inv_rms * w, f32) rotated in (even, odd) pairs by
// rope_theta, f32 sincos; or (cs_tab non-null) by the (cos, sin) pairs of a
// precomputed table row, cs_tab[dd] = cos, cs_tab[dd + 1] = sin (built by the
// same rope_theta and sincosf, so the bits are the same).  e0 is the chunk's
// first element within the head (head_dim % 8 == 0).  The f32 values, before
// the bf16 cast.
__device__ __forceinline__ void qk_chunk_f32(const float (&v)[8], float inv_rms, const uint4 & wv, int dd0,
                                             const RopeTok & r, float (&o)[8], const float * cs_tab = nullptr) {
    const uint32_t wu[4] = {wv.x, wv.y, wv.z, wv.w};
    float4 ct[2];
    if (cs_tab) {
        ct[0] = *(const float4 *) (cs_tab + dd0);
        ct[1] = *(const float4 *) (cs_tab + dd0 + 4);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float a = v[2 * j] * inv_rms * __uint_as_float(wu[j] << 16);
        float b = v[2 * j + 1] * inv_rms * __uint_as_float(wu[j] & 0xFFFF0000u);
        if (cs_tab || r.mode != 2) {
            float sn, cs;
            if (cs_tab) {
                const float4 & c = ct[j >> 1];
                cs = (j & 1) ? c.z : c.x;
                sn = (j & 1) ? c.w : c.y;
            } else {
                sincosf(rope_theta(r, dd0 + 2 * j), &sn, &cs);
            }
            rotate_pair(a, b, cs, sn);
        }
        o[2 * j] = a;
        o[2 * j + 1] = b;
    }
}
__device__ __forceinline__ uint4 qk_chunk(const float (&v)[8], float inv_rms, const uint4 & wv, int dd0,
                                          const RopeTok & r, const float * cs_tab = nullptr) {
    float o[8];
    qk_chunk_f32(v, inv_rms, wv, dd0, r, o, cs_tab);
    return pack8(o);
}
// The same chunk as two bf16 planes: hi = bf16(o) and lo = bf16(o - hi), so
// hi + lo carries the f32 value to about 2^-17 relative (o - hi is exact in
// f32).  Products of hi and lo parts are exact in fp32, which lets bf16 MFMA
// form f32-accurate dot products as hi*hi + hi*lo + lo*hi.
__device__ __forceinline__ void qk_chunk_hilo(const float (&v)[8], float inv_rms, const uint4 & wv, int dd0,
                                              const RopeTok & r, uint4 & hi, uint4 & lo, const float * cs_tab = nullptr) {
    float o[8], l[8];
    qk_chunk_f32(v, inv_rms, wv, dd0, r, o, cs_tab);
    hi = pack8(o);
    float h[8];
    unpack8(hi, h);
#pragma unroll
    for (int e = 0; e < 8; ++e) l[e] = o[e] - h[e];
    lo = pack8(l);
}

}  // namespace wamx
