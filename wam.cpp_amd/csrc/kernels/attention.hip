// Attention-side kernels of the MoT layer.
//
// qk_norm_rope: RMSNorm over the full hidden width (rms_norm_bf16_f32,
//   native-bf16.patch:411-430; weights.cpp:904-917), NORMAL RoPE in f32
//   (ggml_rope_ext mode 0 as called by mot.cpp:175-202) and the bf16 cast +
//   head-major permute/cont of mot.cpp:262-265, 395-396 in one pass.  Reads
//   the row once, writes bf16 once into [H][tokens][head_dim] at token tok0.
//
// joint_attn: softmax(scale * Q K^T) V per head over keys taken from two
//   sources without concatenating them (mot.cpp:402-445 builds the CONCAT and
//   three GEMM/softmax nodes; the math here is the same with fp32 scores and
//   bf16 probabilities).  Split-KV ("flash-decoding"): every wave streams its
//   32-key blocks of K and V^T once from HBM, keeps an online softmax per
//   query, waves of a workgroup merge in LDS, and the last workgroup of a
//   (head, query group) merges the split partials in split order.
#include "../internal.h"
#include "device.h"

namespace wamx {

// ---------------------------------------------------------------------------
// qk_norm_rope
// ---------------------------------------------------------------------------
constexpr int kQkThreads = 256;
constexpr int kQkMaxPairs = 16;  // pairs per thread held in registers (row width up to 8192)

__global__ __launch_bounds__(kQkThreads) void qk_norm_rope_kernel(const uint16_t * __restrict__ x, int64_t ldx,
                                                                   const uint16_t * __restrict__ w,
                                                                   uint16_t * __restrict__ dst, int heads, int head_dim,
                                                                   int64_t dst_tokens, int64_t tok0, int rope_mode,
                                                                   const int32_t * __restrict__ pos0,
                                                                   const int32_t * __restrict__ pos1,
                                                                   const int32_t * __restrict__ pos2, float eps,
                                                                   float ts128, float ts44, float ts42) {
    __shared__ float red[kQkThreads / 64];
    const int64_t t = blockIdx.x;
    const int d = heads * head_dim;
    const int npairs = d / 2;
    const uint32_t * xr = (const uint32_t *) (x + t * ldx);
    float2 v[kQkMaxPairs];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kQkMaxPairs; ++j) {
        const int p = threadIdx.x + j * kQkThreads;
        if (p < npairs) {
            const uint32_t u = xr[p];
            v[j] = make_float2(bf16_to_f32((uint16_t) (u & 0xffff)), bf16_to_f32((uint16_t) (u >> 16)));
            sum = fmaf(v[j].x, v[j].x, sum);
            sum = fmaf(v[j].y, v[j].y, sum);
        }
    }
    const float inv_rms = rsqrtf(block_sum(sum, red) / (float) d + eps);
    const uint32_t * wr = (const uint32_t *) w;
#pragma unroll
    for (int j = 0; j < kQkMaxPairs; ++j) {
        const int p = threadIdx.x + j * kQkThreads;
        if (p >= npairs) continue;
        const uint32_t wu = wr[p];
        // rms_norm_bf16_f32: y = x * inv_rms * w, f32.
        float a = v[j].x * inv_rms * bf16_to_f32((uint16_t) (wu & 0xffff));
        float b = v[j].y * inv_rms * bf16_to_f32((uint16_t) (wu >> 16));
        const int e = 2 * p;  // element index within the row
        const int h = e / head_dim, dd = e % head_dim;
        if (rope_mode != 2) {
            float theta;
            if (rope_mode == 0) {
                theta = (float) pos0[t] * powf(ts128, (float) (dd >> 1));
            } else if (dd < 44) {
                theta = (float) pos0[t] * powf(ts44, (float) (dd >> 1));
            } else if (dd < 86) {
                theta = (float) pos1[t] * powf(ts42, (float) ((dd - 44) >> 1));
            } else {
                theta = (float) pos2[t] * powf(ts42, (float) ((dd - 86) >> 1));
            }
            float sn, cs;
            sincosf(theta, &sn, &cs);
            const float ra = a * cs - b * sn;
            const float rb = a * sn + b * cs;
            a = ra;
            b = rb;
        }
        uint32_t * out = (uint32_t *) (dst + ((int64_t) h * dst_tokens + tok0 + t) * head_dim + dd);
        *out = pack_bf16x2(a, b);
    }
}

hipError_t launch_qk_norm_rope(const void * x, int64_t ldx, const void * w, void * dst, int64_t heads, int64_t head_dim,
                               int64_t tokens, int64_t dst_tokens, int64_t tok0, int rope_mode, const int32_t * pos0,
                               const int32_t * pos1, const int32_t * pos2, float eps, float freq_base, hipStream_t s) {
    if (tokens <= 0) return hipSuccess;
    if ((heads * head_dim) / 2 > (int64_t) kQkThreads * kQkMaxPairs || (head_dim & 1) || (ldx & 1))
        return hipErrorInvalidValue;
    // theta_i = pos * theta_scale^i with theta_scale = base^(-2/n_dims) per rope section.
    const float ts128 = powf(freq_base, -2.0f / (float) head_dim);
    const float ts44 = powf(freq_base, -2.0f / 44.0f);
    const float ts42 = powf(freq_base, -2.0f / 42.0f);
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned) tokens), dim3(kQkThreads), 0, s, (const uint16_t *) x, ldx,
                       (const uint16_t *) w, (uint16_t *) dst, (int) heads, (int) head_dim, dst_tokens, tok0, rope_mode,
                       pos0, pos1, pos2, eps, ts128, ts44, ts42);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// joint_attn
// ---------------------------------------------------------------------------
constexpr int kDh = 128;         // head_dim
constexpr int kQG = 48;          // queries per workgroup (3 MFMA column tiles of 16)
constexpr int kQT = kQG / 16;
constexpr int kKB = 32;          // keys per block
constexpr int kAttnWaves = 4;
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
    const uint16_t * q;
    const uint16_t * k[2];   // key sources: a (prefix cache) and b (current tokens)
    const uint16_t * vt[2];
    int64_t vt_ld[2];        // V^T row stride (elements, multiple of 4)
    int64_t seg_len[2];
    int64_t seg_blocks[2];
    int64_t nblocks;
    uint16_t * out;
    float * ws;              // partials [H][qgroups][splits][kQG][kDh + 2]
    unsigned * counters;     // [H][qgroups]
    int64_t heads, tq, qgroups;
    int splits;
    float scale_log2;
};

// Unpack 4 bf16 packed in a uint2 with keys >= valid replaced by zero.
__device__ __forceinline__ uint2 mask4(uint2 v, int first_key, int valid) {
    uint32_t lo = v.x, hi = v.y;
    if (first_key + 0 >= valid) lo &= 0xffff0000u;
    if (first_key + 1 >= valid) lo &= 0x0000ffffu;
    if (first_key + 2 >= valid) hi &= 0xffff0000u;
    if (first_key + 3 >= valid) hi &= 0x0000ffffu;
    return make_uint2(lo, hi);
}

__global__ __launch_bounds__(256) void joint_attn_kernel(AttnParams p) {
    __shared__ float s_m[kAttnWaves][kQG];
    __shared__ float s_l[kAttnWaves][kQG];
    __shared__ float s_o[kQG][kDh + 1];
    __shared__ int s_last;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int split = blockIdx.x;
    const int64_t h = blockIdx.y, qg = blockIdx.z;
    const int64_t q0 = qg * kQG;

    // Q fragments: B operand of S^T = K Q^T.  Lane (query c16 of tile t,
    // group g) holds dims [32g, 32g+32) as four 8-element k-steps.
    bf16x8_t qf[kQT][4];
#pragma unroll
    for (int t = 0; t < kQT; ++t) {
        const int64_t qi = q0 + 16 * t + c16;
        const bool ok = qi < p.tq;
        const uint4 * src = (const uint4 *) (p.q + (h * p.tq + (ok ? qi : 0)) * kDh + 32 * g);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            uint4 u = ok ? src[c] : make_uint4(0, 0, 0, 0);
            qf[t][c] = __builtin_bit_cast(bf16x8_t, u);
        }
    }

    f32x4_t o[kQT][8];
#pragma unroll
    for (int t = 0; t < kQT; ++t)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[t][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run[kQT], l_run[kQT];
#pragma unroll
    for (int t = 0; t < kQT; ++t) {
        m_run[t] = -INFINITY;
        l_run[t] = 0.0f;
    }

    const int64_t stride = (int64_t) p.splits * kAttnWaves;
    for (int64_t b = (int64_t) split * kAttnWaves + wave; b < p.nblocks; b += stride) {
        const int seg = b < p.seg_blocks[0] ? 0 : 1;
        const int64_t lb = seg == 0 ? b : b - p.seg_blocks[0];
        const int64_t k0 = lb * kKB;
        const int valid = (int) min((int64_t) kKB, p.seg_len[seg] - k0);
        const uint16_t * kbase = p.k[seg] + (h * p.seg_len[seg] + k0) * kDh;
        const uint16_t * vbase = p.vt[seg] + h * kDh * p.vt_ld[seg] + k0;
        const int64_t vld = p.vt_ld[seg];

        // S^T tiles: two 16-key tiles x kQT query tiles.
        f32x4_t st[2][kQT];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
            const int key = 16 * kt + c16;
            const bool ok = key < valid;
            const uint4 * ksrc = (const uint4 *) (kbase + (int64_t) (ok ? key : 0) * kDh + 32 * g);
            uint4 kr[4];
#pragma unroll
            for (int c = 0; c < 4; ++c) kr[c] = ok ? ksrc[c] : make_uint4(0, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < kQT; ++t) {
                f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[c]), qf[t][c], acc, 0,
                                                                  0, 0);
                st[kt][t] = acc;
            }
        }
        // V^T fragments: lane (dim row c16 of dim tile dt, group g) holds keys
        // 4g..4g+3 and 16+4g..16+4g+3, matching the S^T accumulator layout.
        uint2 va[8], vb[8];
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const uint16_t * row = vbase + (int64_t) (16 * dt + c16) * vld;
            const bool full = valid == kKB;
            const int ka = 4 * g, kb = 16 + 4 * g;
            va[dt] = (full || ka < valid) ? *(const uint2 *) (row + ka) : make_uint2(0, 0);
            vb[dt] = (full || kb < valid) ? *(const uint2 *) (row + kb) : make_uint2(0, 0);
            if (!full) {
                va[dt] = mask4(va[dt], ka, valid);
                vb[dt] = mask4(vb[dt], kb, valid);
            }
        }
        // Online softmax per query (lane's query c16 of tile t; its 8 keys are
        // keys 4g+r and 16+4g+r; the rest of the block lives in lanes ^16, ^32).
#pragma unroll
        for (int t = 0; t < kQT; ++t) {
            float sv[8];
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool oka = 4 * g + r < valid, okb = 16 + 4 * g + r < valid;
                sv[r] = oka ? st[0][t][r] * p.scale_log2 : -INFINITY;
                sv[4 + r] = okb ? st[1][t][r] * p.scale_log2 : -INFINITY;
                mx = fmaxf(mx, fmaxf(sv[r], sv[4 + r]));
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_run[t], mx);
            const float corr = exp2f(m_run[t] - m_new);
            float ps = 0.0f;
            uint32_t pk[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pa = exp2f(sv[r] - m_new);
                const float pb = exp2f(sv[4 + r] - m_new);
                sv[r] = round_bf16(pa);
                sv[4 + r] = round_bf16(pb);
                ps += sv[r] + sv[4 + r];
            }
            pk[0] = pack_bf16x2(sv[0], sv[1]);
            pk[1] = pack_bf16x2(sv[2], sv[3]);
            pk[2] = pack_bf16x2(sv[4], sv[5]);
            pk[3] = pack_bf16x2(sv[6], sv[7]);
            ps += __shfl_xor(ps, 16, 64);
            ps += __shfl_xor(ps, 32, 64);
            l_run[t] = l_run[t] * corr + ps;
            m_run[t] = m_new;
            const bf16x8_t pfrag = __builtin_bit_cast(bf16x8_t, make_uint4(pk[0], pk[1], pk[2], pk[3]));
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
                for (int r = 0; r < 4; ++r) o[t][dt][r] *= corr;
                const bf16x8_t vfrag = __builtin_bit_cast(bf16x8_t, make_uint4(va[dt].x, va[dt].y, vb[dt].x, vb[dt].y));
                o[t][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vfrag, pfrag, o[t][dt], 0, 0, 0);
            }
        }
    }

    // --- merge the four waves of this workgroup (in wave order) ------------
    // O^T accumulator: lane holds query c16 of tile t, dims 16dt + 4g + r.
#pragma unroll
    for (int t = 0; t < kQT; ++t) {
        if (g == 0) {
            s_m[wave][16 * t + c16] = m_run[t];
            s_l[wave][16 * t + c16] = l_run[t];
        }
    }
    __syncthreads();
    float fac[kQT];
#pragma unroll
    for (int t = 0; t < kQT; ++t) {
        const int q = 16 * t + c16;
        float mstar = -INFINITY;
        for (int w = 0; w < kAttnWaves; ++w) mstar = fmaxf(mstar, s_m[w][q]);
        fac[t] = (m_run[t] == -INFINITY) ? 0.0f : exp2f(m_run[t] - mstar);
    }
    for (int w = 0; w < kAttnWaves; ++w) {
        if (wave == w) {
#pragma unroll
            for (int t = 0; t < kQT; ++t)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        float * cell = &s_o[16 * t + c16][16 * dt + 4 * g + r];
                        const float add = o[t][dt][r] * fac[t];
                        *cell = (w == 0) ? add : *cell + add;
                    }
        }
        __syncthreads();
    }
    // Per-query merged max and denominator (thread q < kQG computes them).
    __shared__ float s_mstar[kQG], s_lstar[kQG];
    if (tid < kQG) {
        float mstar = -INFINITY;
        for (int w = 0; w < kAttnWaves; ++w) mstar = fmaxf(mstar, s_m[w][tid]);
        float l = 0.0f;
        for (int w = 0; w < kAttnWaves; ++w)
            if (s_m[w][tid] != -INFINITY) l += s_l[w][tid] * exp2f(s_m[w][tid] - mstar);
        s_mstar[tid] = mstar;
        s_lstar[tid] = l;
    }
    __syncthreads();

    const int64_t nq = min((int64_t) kQG, p.tq - q0);
    if (p.splits == 1) {
        for (int e = tid; e < nq * kDh; e += 256) {
            const int q = e / kDh, d = e % kDh;
            const float l = s_lstar[q];
            p.out[(q0 + q) * (p.heads * kDh) + h * kDh + d] = f32_to_bf16(l > 0.0f ? s_o[q][d] / l : 0.0f);
        }
        return;
    }

    // --- split-KV: publish the partial, last workgroup merges -------------
    const int64_t slot = (h * p.qgroups + qg) * p.splits;
    float * part = p.ws + (slot + split) * (int64_t) kQG * (kDh + 2);
    for (int e = tid; e < kQG * kDh; e += 256) part[e] = s_o[e / kDh][e % kDh];
    if (tid < kQG) {
        part[kQG * kDh + tid] = s_mstar[tid];
        part[kQG * kDh + kQG + tid] = s_lstar[tid];
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = atomicAdd(&p.counters[h * p.qgroups + qg], 1u);
        s_last = prev == (unsigned) (p.splits - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    const float * base = p.ws + slot * (int64_t) kQG * (kDh + 2);
    const int64_t pstride = (int64_t) kQG * (kDh + 2);
    for (int e = tid; e < nq * kDh; e += 256) {
        const int q = e / kDh, d = e % kDh;
        float mstar = -INFINITY;
        for (int sp = 0; sp < p.splits; ++sp) mstar = fmaxf(mstar, base[sp * pstride + kQG * kDh + q]);
        float acc = 0.0f, l = 0.0f;
        for (int sp = 0; sp < p.splits; ++sp) {
            const float ms = base[sp * pstride + kQG * kDh + q];
            if (ms == -INFINITY) continue;
            const float f = exp2f(ms - mstar);
            acc += base[sp * pstride + q * kDh + d] * f;
            l += base[sp * pstride + kQG * kDh + kQG + q] * f;
        }
        p.out[(q0 + q) * (p.heads * kDh) + h * kDh + d] = f32_to_bf16(l > 0.0f ? acc / l : 0.0f);
    }
    if (tid == 0) atomicExch(&p.counters[h * p.qgroups + qg], 0u);
}

// Softmax is order-free, so the keys are visited per source in 32-key blocks
// aligned to each source's start: source a ([state, reference] prefix cache,
// na keys) and source b (the current action tokens, nb keys).  The complete
// MoT order [state, action, reference] (mot.cpp:402-403) only fixes the
// reference's fp32 summation order, which split-KV reassociates anyway.
static void attn_plan(const AttnArgs & a, int64_t & nblocks, int64_t & qgroups, int & splits) {
    const int64_t seg1 = a.k_b ? a.nb : 0;
    nblocks = (a.na + kKB - 1) / kKB + (seg1 + kKB - 1) / kKB;
    qgroups = (a.tq + kQG - 1) / kQG;
    // Enough workgroups to cover the chip, at least two key blocks per wave.
    const int64_t wgs = a.heads * qgroups;
    int64_t sp = 1;
    while (wgs * sp < 256 && (nblocks + (sp * 2 * kAttnWaves) - 1) / (sp * 2 * kAttnWaves) >= 2) sp *= 2;
    splits = (int) sp;
}

size_t attn_workspace_bytes(const AttnArgs & a) {
    int64_t nblocks, qgroups;
    int splits;
    attn_plan(a, nblocks, qgroups, splits);
    if (splits == 1) return 0;
    return (size_t) a.heads * qgroups * splits * kQG * (kDh + 2) * sizeof(float);
}

hipError_t launch_joint_attn(const AttnArgs & a, void * ws, hipStream_t s) {
    if (a.head_dim != kDh) return hipErrorInvalidValue;
    if (a.tq <= 0) return hipSuccess;
    AttnParams p{};
    p.q = (const uint16_t *) a.q;
    p.k[0] = (const uint16_t *) a.k_a;
    p.vt[0] = (const uint16_t *) a.vt_a;
    p.vt_ld[0] = a.vt_ld_a ? a.vt_ld_a : a.na;
    p.seg_len[0] = a.na;
    p.k[1] = (const uint16_t *) a.k_b;
    p.vt[1] = (const uint16_t *) a.vt_b;
    p.vt_ld[1] = a.vt_ld_b ? a.vt_ld_b : a.nb;
    p.seg_len[1] = a.k_b ? a.nb : 0;
    p.seg_blocks[0] = (p.seg_len[0] + kKB - 1) / kKB;
    p.seg_blocks[1] = (p.seg_len[1] + kKB - 1) / kKB;
    int64_t nblocks, qgroups;
    int splits;
    attn_plan(a, nblocks, qgroups, splits);
    p.nblocks = nblocks;
    p.out = (uint16_t *) a.out;
    p.heads = a.heads;
    p.tq = a.tq;
    p.qgroups = qgroups;
    p.splits = splits;
    p.scale_log2 = a.scale * kLog2e;
    p.ws = (float *) ws;
    p.counters = a.counters;
    if (splits > 1 && (!ws || !a.counters || a.heads * qgroups > a.max_counters)) return hipErrorInvalidValue;
    // 8-byte V^T loads of 4 keys need rows padded to a multiple of 4 keys.
    for (int i = 0; i < 2; ++i)
        if (p.seg_len[i] > 0 &&
            (p.vt_ld[i] % 4 != 0 || p.vt_ld[i] < p.seg_len[i] || ((uintptr_t) p.vt[i] & 7) || ((uintptr_t) p.k[i] & 15)))
            return hipErrorInvalidValue;
    hipLaunchKernelGGL(joint_attn_kernel, dim3((unsigned) splits, (unsigned) a.heads, (unsigned) qgroups), dim3(256), 0,
                       s, p);
    return hipGetLastError();
}

}  // namespace wamx
