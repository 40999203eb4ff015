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
//   bf16 probabilities).  Every wave streams its 32-key blocks of K and V^T
//   once, keeps an online softmax per query, and the waves of the workgroup
//   merge their states in LDS in wave order.
#include "../internal.h"
#include "device.h"
#include "rowops.h"

#include <algorithm>
#include <type_traits>

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
                                                                   float ts128, float ts44, float ts42,
                                                                   int64_t chunk_tokens, int64_t chunk_stride,
                                                                   int64_t lo_off) {
    __shared__ float red[kQkThreads / 64];
    const int64_t t = blockIdx.x;
    // Row t is token tl of chunk cb: positions by tl, output in chunk cb's slice.
    const int64_t cb = t / chunk_tokens, tl = t - cb * chunk_tokens;
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
                theta = (float) pos0[tl] * powf(ts128, (float) (dd >> 1));
            } else if (dd < 44) {
                theta = (float) pos0[tl] * powf(ts44, (float) (dd >> 1));
            } else if (dd < 86) {
                theta = (float) pos1[tl] * powf(ts42, (float) ((dd - 44) >> 1));
            } else {
                theta = (float) pos2[tl] * powf(ts42, (float) ((dd - 86) >> 1));
            }
            float sn, cs;
            sincosf(theta, &sn, &cs);
            rotate_pair(a, b, cs, sn);
        }
        uint32_t * out = (uint32_t *) (dst + cb * chunk_stride + ((int64_t) h * dst_tokens + tok0 + tl) * head_dim + dd);
        const uint32_t hi = pack_bf16x2(a, b);
        *out = hi;
        // lo plane: the f32 value less its bf16 rounding (exact in f32).
        if (lo_off)
            *(uint32_t *) ((uint16_t *) out + lo_off) =
                pack_bf16x2(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
    }
}

// Vectorised qk_norm_rope for 16-byte aligned rows (width % 8 == 0, head_dim
// % 8 == 0): thread i owns CPT chunks of 8 elements (4 rotation pairs of one
// head); the row and weight chunks are loaded before the reduction, and each
// chunk is stored as one 16-byte write.  theta = pos * 2^(i * log2(ts)).
template <int CPT>
__global__ __launch_bounds__(1024) void qk_norm_rope_vec(const uint16_t * __restrict__ x, int64_t ldx,
                                                          const uint16_t * __restrict__ w, uint16_t * __restrict__ dst,
                                                          int heads, int head_dim, int64_t dst_tokens, int64_t tok0,
                                                          int rope_mode, const int32_t * __restrict__ pos0,
                                                          const int32_t * __restrict__ pos1,
                                                          const int32_t * __restrict__ pos2, float eps, float l2ts128,
                                                          float l2ts44, float l2ts42, int64_t chunk_tokens,
                                                          int64_t chunk_stride, int64_t lo_off,
                                                          const float * __restrict__ tab, int64_t x_cs, int64_t w_cs) {
    __shared__ float red[16];
    const int64_t t = blockIdx.x;
    const int64_t b = t / chunk_tokens, tl = t - b * chunk_tokens;
    const int d = heads * head_dim;
    const int nchunk = d >> 3;
    const uint16_t * xr = x + b * x_cs + tl * ldx;
    const uint16_t * wr = w + b * w_cs;
    uint4 xv[CPT], wv[CPT];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = min((int) threadIdx.x + i * (int) blockDim.x, nchunk - 1);
        xv[i] = *(const uint4 *) (xr + 8 * c);
        wv[i] = *(const uint4 *) (wr + 8 * c);
    }
    // Rope mode 3: the (cos, sin) of every pair from the table row of the token.
    const RopeTok rt = rope_tok(tab ? 2 : rope_mode, pos0, pos1, pos2, tl, l2ts128, l2ts44, l2ts42);
    const float * cs = tab ? tab + tl * head_dim : nullptr;
    float v[CPT][8];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        unpack8(xv[i], v[i]);
        if ((int) threadIdx.x + i * (int) blockDim.x >= nchunk)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
    }
    const float inv_rms = row_inv_rms<CPT>(v, d, eps, red);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = (int) threadIdx.x + i * (int) blockDim.x;
        if (c >= nchunk) continue;
        const int e0 = 8 * c, h = e0 / head_dim, dd0 = e0 % head_dim;
        uint16_t * o = dst + b * chunk_stride + ((int64_t) h * dst_tokens + tok0 + tl) * head_dim + dd0;
        if (lo_off) {
            uint4 hi, lo;
            qk_chunk_hilo(v[i], inv_rms, wv[i], dd0, rt, hi, lo, cs);
            *(uint4 *) o = hi;
            *(uint4 *) (o + lo_off) = lo;
        } else {
            *(uint4 *) o = qk_chunk(v[i], inv_rms, wv[i], dd0, rt, cs);
        }
    }
}

hipError_t launch_qk_norm_rope(const void * x, int64_t ldx, const void * w, void * dst, int64_t heads, int64_t head_dim,
                               int64_t tokens, int64_t dst_tokens, int64_t tok0, int rope_mode, const int32_t * pos0,
                               const int32_t * pos1, const int32_t * pos2, float eps, float freq_base, hipStream_t s,
                               int64_t chunk_tokens, int64_t chunk_stride, int64_t lo_off, const float * tab,
                               int64_t x_cs, int64_t w_cs) {
    if (tokens <= 0) return hipSuccess;
    // Rope mode 3: the rotation comes from tab [tokens][head_dim] (cos, sin
    // per pair), 16-byte aligned; only the vectorised kernel reads it.
    if ((rope_mode == 3) != (tab != nullptr) || (tab && (((uintptr_t) tab & 15) || (head_dim % 8)))) return hipErrorInvalidValue;
    if (lo_off & 7) return hipErrorInvalidValue;
    if (chunk_tokens <= 0) chunk_tokens = tokens;
    if (tokens % chunk_tokens != 0) return hipErrorInvalidValue;
    // Chunk b's rows start b * x_cs elements into x and use norm weight row b
    // (w + b * w_cs); by default the rows follow each other and share w.
    if (x_cs < 0) x_cs = chunk_tokens * ldx;
    const bool layered = x_cs != chunk_tokens * ldx || w_cs != 0;
    const int64_t d = heads * head_dim;
    if (d % 8 == 0 && head_dim % 8 == 0 && d / 8 <= 4096 && ldx % 8 == 0 && x_cs % 8 == 0 && w_cs % 8 == 0 &&
        ((uintptr_t) x & 15) == 0 && ((uintptr_t) w & 15) == 0 && ((uintptr_t) dst & 15) == 0) {
        const int64_t nchunk = d / 8;
        const int cpt = nchunk <= 1024 ? 1 : nchunk <= 2048 ? 2 : 4;
        const int threads = (int) std::min<int64_t>(1024, ((nchunk + cpt - 1) / cpt + 63) / 64 * 64);
        const float l2ts128 = -2.0f / (float) head_dim * log2f(freq_base);
        const float l2ts44 = -2.0f / 44.0f * log2f(freq_base);
        const float l2ts42 = -2.0f / 42.0f * log2f(freq_base);
#define WAMX_QK_VEC(CPT)                                                                                            \
    hipLaunchKernelGGL(qk_norm_rope_vec<CPT>, dim3((unsigned) tokens), dim3((unsigned) threads), 0, s,            \
                       (const uint16_t *) x, ldx, (const uint16_t *) w, (uint16_t *) dst, (int) heads, (int) head_dim, \
                       dst_tokens, tok0, rope_mode, pos0, pos1, pos2, eps, l2ts128, l2ts44, l2ts42, chunk_tokens,    \
                       chunk_stride, lo_off, tab, x_cs, w_cs)
        if (cpt == 1) WAMX_QK_VEC(1);
        else if (cpt == 2) WAMX_QK_VEC(2);
        else WAMX_QK_VEC(4);
#undef WAMX_QK_VEC
        return hipGetLastError();
    }
    if ((heads * head_dim) / 2 > (int64_t) kQkThreads * kQkMaxPairs || (head_dim & 1) || (ldx & 1) || tab || layered)
        return hipErrorInvalidValue;
    // theta_i = pos * theta_scale^i with theta_scale = base^(-2/n_dims) per rope section.
    const float ts128 = powf(freq_base, -2.0f / (float) head_dim);
    const float ts44 = powf(freq_base, -2.0f / 44.0f);
    const float ts42 = powf(freq_base, -2.0f / 42.0f);
    hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned) tokens), dim3(kQkThreads), 0, s, (const uint16_t *) x, ldx,
                       (const uint16_t *) w, (uint16_t *) dst, (int) heads, (int) head_dim, dst_tokens, tok0, rope_mode,
                       pos0, pos1, pos2, eps, ts128, ts44, ts42, chunk_tokens, chunk_stride, lo_off);
    return hipGetLastError();
}

// The rope table of rope mode 3: out[t][dd] = cos, out[t][dd + 1] = sin of
// rope_theta for token t's positions, every even dd < head_dim, with the
// section scales launch_qk_norm_rope uses, so a table-driven rotation equals
// the computed one bit for bit.
__global__ void rope_table_kernel(int mode, const int32_t * __restrict__ pos0, const int32_t * __restrict__ pos1,
                                  const int32_t * __restrict__ pos2, int64_t tokens, int head_dim, float l2ts128,
                                  float l2ts44, float l2ts42, float * __restrict__ out) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    const int half = head_dim / 2;
    if (i >= tokens * half) return;
    const int64_t t = i / half;
    const int dd = 2 * (int) (i - t * half);
    const RopeTok r = rope_tok(mode, pos0, pos1, pos2, t, l2ts128, l2ts44, l2ts42);
    float sn, cs;
    sincosf(rope_theta(r, dd), &sn, &cs);
    out[t * head_dim + dd] = cs;
    out[t * head_dim + dd + 1] = sn;
}

hipError_t launch_rope_table(int rope_mode, const int32_t * pos0, const int32_t * pos1, const int32_t * pos2,
                             int64_t tokens, int64_t head_dim, float freq_base, float * out, hipStream_t s) {
    if (tokens <= 0) return hipSuccess;
    if ((rope_mode != 0 && rope_mode != 1) || !pos0 || (rope_mode == 1 && (!pos1 || !pos2 || head_dim != 128)) ||
        (head_dim & 1))
        return hipErrorInvalidValue;
    const float l2ts128 = -2.0f / (float) head_dim * log2f(freq_base);
    const float l2ts44 = -2.0f / 44.0f * log2f(freq_base);
    const float l2ts42 = -2.0f / 42.0f * log2f(freq_base);
    const int64_t n = tokens * (head_dim / 2);
    hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, s, rope_mode, pos0, pos1,
                       pos2, tokens, (int) head_dim, l2ts128, l2ts44, l2ts42, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// joint_attn
// ---------------------------------------------------------------------------

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// s_waitcnt immediate: at most n vector-memory operations outstanding, other
// counters untouched (vmcnt in bits [3:0] and [15:14]).
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (((n >> 4) & 3) << 14) | (7 << 4) | (0xF << 8); }

__device__ __forceinline__ void cta_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

constexpr int kDh = 128;         // head_dim
constexpr int kKB = 32;          // keys per block
constexpr float kLog2e = 1.4426950408889634f;

struct AttnParams {
    const uint16_t * q;
    const uint16_t * k[2];   // key sources: a (prefix cache) and b (current tokens)
    const uint16_t * vt[2];
    int64_t vt_ld[2];        // V^T row stride (elements, multiple of 4)
    int64_t seg_len[2];
    int64_t seg_blocks[2];
    int64_t nblocks;
    uint16_t * out;          // bf16 [batch][tq][hb * kDh]
    int64_t heads, tq;       // heads: batch x hb (chunk b's head h is head b * hb + h)
    int64_t hb;              // heads per chunk
    float scale_log2;
    // Key-split mode: workgroup z of gridDim.z covers key blocks
    // [z * split_blocks, (z + 1) * split_blocks) and writes fp32 partials.
    int64_t split_blocks;
    float * part_o;          // [split][head][query][kDh], unnormalised, scaled to part_m
    float * part_m;          // [split][head][query] running max (log2 domain)
    float * part_l;          // [split][head][query] running sum
    // Unit-mapped attn_prefill launches (units > 0): workgroup x takes unit
    // unit0 + x, i.e. head u % heads and query block u / heads; key-split
    // partials are then indexed [split][x][query of the block] and
    // joint_attn_merge maps its rows the same way.
    int64_t unit0, units;
    // f32-accurate scores (attn_prefill_kernel<., true>): the remainders of
    // Q and of source a's K, laid out as q and k[0].
    const uint16_t * q_lo;
    const uint16_t * k_lo;
};

// attn_prefill's workgroup: 4 waves x 32 queries of one head.
constexpr int kPfWaves = 4;
constexpr int kPfQueries = 32 * kPfWaves;

// Output row of query q of head h: chunk b = h / hb writes rows [b * tq, (b + 1) * tq).
__device__ __forceinline__ uint16_t * out_row(const AttnParams & p, int64_t h, int64_t q) {
    const int64_t b = h / p.hb;
    return p.out + ((b * p.tq + q) * p.hb + (h - b * p.hb)) * kDh;
}

// Zero the bf16 values of keys >= valid in 4 packed keys starting at first_key.
__device__ __forceinline__ uint2 mask4(uint2 v, int first_key, int valid) {
    uint32_t lo = v.x, hi = v.y;
    if (first_key + 0 >= valid) lo &= 0xffff0000u;
    if (first_key + 1 >= valid) lo &= 0x0000ffffu;
    if (first_key + 2 >= valid) hi &= 0xffff0000u;
    if (first_key + 3 >= valid) hi &= 0x0000ffffu;
    return make_uint2(lo, hi);
}

// One 32-key block's operands in registers: K as two 16-key A fragments
// (lane = key c16 of the tile, dims [32g, 32g+32) as four k-steps) and V^T as
// 8 dim tiles of keys {4g..4g+3} and {16+4g..16+4g+3} (the S^T accumulator
// layout, so P needs no shuffle before the PV MFMA).
struct KvBlock {
    uint4 k[2][4];
    uint2 va[8], vb[8];
    int valid;
};

// Branch-free loads: rows and columns are clamped into the segment and the
// out-of-range keys are masked (scores to -inf, V to zero) by the consumer.
__device__ __forceinline__ void load_block(const AttnParams & p, int64_t b, int64_t h, int g, int c16, KvBlock & kv) {
    const int seg = b < p.seg_blocks[0] ? 0 : 1;
    const int64_t lb = seg == 0 ? b : b - p.seg_blocks[0];
    const int64_t k0 = lb * kKB;
    const int valid = (int) min((int64_t) kKB, p.seg_len[seg] - k0);
    kv.valid = valid;
    const uint16_t * kbase = p.k[seg] + (h * p.seg_len[seg] + k0) * kDh;
    const uint16_t * vbase = p.vt[seg] + h * kDh * p.vt_ld[seg] + k0;
    const int64_t vld = p.vt_ld[seg];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
        const int key = min(16 * kt + c16, valid - 1);
        const uint4 * src = (const uint4 *) (kbase + (int64_t) key * kDh + 32 * g);
#pragma unroll
        for (int c = 0; c < 4; ++c) kv.k[kt][c] = src[c];
    }
    const int last = ((valid - 1) >> 2) << 2;  // last 4-aligned chunk inside the block
    const int ka = min(4 * g, last), kb = min(16 + 4 * g, last);
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
        const uint16_t * row = vbase + (int64_t) (16 * dt + c16) * vld;
        kv.va[dt] = *(const uint2 *) (row + ka);
        kv.vb[dt] = *(const uint2 *) (row + kb);
    }
}

// softmax(scale * Q K^T) V for one (head, group of 16*QT queries) per
// workgroup; the NW waves take key blocks round-robin, each with one block of
// prefetch, and merge their online-softmax states in LDS in wave order.  With
// SPLIT the workgroup covers one key range (blockIdx.z) and writes its merged
// state as fp32 partials for joint_attn_merge instead of the output.
template <int QT, int NW, bool SPLIT>
__global__ __launch_bounds__(NW * 64) void joint_attn_kernel(AttnParams p) {
    constexpr int QG = 16 * QT;
    __shared__ float s_m[NW][QG];
    __shared__ float s_l[NW][QG];
    __shared__ float s_o[QG][kDh + 1];
    __shared__ float s_lstar[QG];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t h = blockIdx.x, qg = blockIdx.y;
    const int64_t q0 = qg * QG;

    // Q fragments: B operand of S^T = K Q^T.  Lane (query c16 of tile t,
    // group g) holds dims [32g, 32g+32) as four 8-element k-steps.
    bf16x8_t qf[QT][4];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        const int64_t qi = min(q0 + 16 * t + c16, p.tq - 1);
        const uint4 * src = (const uint4 *) (p.q + (h * p.tq + qi) * kDh + 32 * g);
#pragma unroll
        for (int c = 0; c < 4; ++c) qf[t][c] = __builtin_bit_cast(bf16x8_t, src[c]);
    }

    f32x4_t o[QT][8];
#pragma unroll
    for (int t = 0; t < QT; ++t)
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[t][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float m_run[QT], l_run[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        m_run[t] = -INFINITY;
        l_run[t] = 0.0f;
    }

    const int64_t b_begin = SPLIT ? (int64_t) blockIdx.z * p.split_blocks : 0;
    const int64_t b_end = SPLIT ? min(p.nblocks, b_begin + p.split_blocks) : p.nblocks;
    KvBlock cur, nxt;
    int64_t b = b_begin + wave;
    if (b < b_end) load_block(p, b, h, g, c16, cur);
    for (; b < b_end; b += NW) {
        if (b + NW < b_end) load_block(p, b + NW, h, g, c16, nxt);
        const int valid = cur.valid;
        // S^T tiles: two 16-key tiles x QT query tiles.
        f32x4_t st[2][QT];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int t = 0; t < QT; ++t) {
                f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, cur.k[kt][c]),
                                                                  qf[t][c], acc, 0, 0, 0);
                st[kt][t] = acc;
            }
        uint2 va[8], vb[8];
        const bool full = valid == kKB;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            va[dt] = full ? cur.va[dt] : mask4(cur.va[dt], 4 * g, valid);
            vb[dt] = full ? cur.vb[dt] : mask4(cur.vb[dt], 16 + 4 * g, valid);
        }
        // Online softmax per query (lane's query c16 of tile t; its 8 keys are
        // keys 4g+r and 16+4g+r; the rest of the block lives in lanes ^16, ^32).
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            float sv[8];
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sv[r] = (4 * g + r < valid) ? st[0][t][r] * p.scale_log2 : -INFINITY;
                sv[4 + r] = (16 + 4 * g + r < valid) ? st[1][t][r] * p.scale_log2 : -INFINITY;
                mx = fmaxf(mx, fmaxf(sv[r], sv[4 + r]));
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = fmaxf(m_run[t], mx);
            const float corr = exp2f(m_run[t] - m_new);
            float ps = 0.0f;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                sv[r] = round_bf16(exp2f(sv[r] - m_new));
                ps += sv[r];
            }
            ps += __shfl_xor(ps, 16, 64);
            ps += __shfl_xor(ps, 32, 64);
            l_run[t] = l_run[t] * corr + ps;
            m_run[t] = m_new;
            const bf16x8_t pfrag = __builtin_bit_cast(
                bf16x8_t, make_uint4(pack_bf16x2(sv[0], sv[1]), pack_bf16x2(sv[2], sv[3]), pack_bf16x2(sv[4], sv[5]),
                                     pack_bf16x2(sv[6], sv[7])));
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
                for (int r = 0; r < 4; ++r) o[t][dt][r] *= corr;
                const bf16x8_t vfrag = __builtin_bit_cast(bf16x8_t, make_uint4(va[dt].x, va[dt].y, vb[dt].x, vb[dt].y));
                o[t][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vfrag, pfrag, o[t][dt], 0, 0, 0);
            }
        }
        cur = nxt;
    }

    // --- merge the waves of this workgroup (in wave order) ----------------
    // O^T accumulator: lane holds query c16 of tile t, dims 16dt + 4g + r.
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        if (g == 0) {
            s_m[wave][16 * t + c16] = m_run[t];
            s_l[wave][16 * t + c16] = l_run[t];
        }
    }
    __syncthreads();
    float fac[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        const int q = 16 * t + c16;
        float mstar = -INFINITY;
        for (int w = 0; w < NW; ++w) mstar = fmaxf(mstar, s_m[w][q]);
        fac[t] = (m_run[t] == -INFINITY) ? 0.0f : exp2f(m_run[t] - mstar);
    }
    for (int w = 0; w < NW; ++w) {
        if (wave == w) {
#pragma unroll
            for (int t = 0; t < QT; ++t)
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
    const int64_t nq = min((int64_t) QG, p.tq - q0);
    if (tid < QG) {
        float mstar = -INFINITY;
        for (int w = 0; w < NW; ++w) mstar = fmaxf(mstar, s_m[w][tid]);
        float l = 0.0f;
        for (int w = 0; w < NW; ++w)
            if (s_m[w][tid] != -INFINITY) l += s_l[w][tid] * exp2f(s_m[w][tid] - mstar);
        s_lstar[tid] = l;
        if (SPLIT && tid < nq) {
            const int64_t pi = ((int64_t) blockIdx.z * p.heads + h) * p.tq + q0 + tid;
            p.part_m[pi] = mstar;
            p.part_l[pi] = l;
        }
    }
    __syncthreads();
    for (int e = tid; e < nq * kDh; e += NW * 64) {
        const int q = e / kDh, d = e % kDh;
        if constexpr (SPLIT) {
            p.part_o[(((int64_t) blockIdx.z * p.heads + h) * p.tq + q0 + q) * kDh + d] = s_o[q][d];
        } else {
            const float l = s_lstar[q];
            out_row(p, h, q0 + q)[d] = f32_to_bf16(l > 0.0f ? s_o[q][d] / l : 0.0f);
        }
    }
}

// Combines the key-split partials of (head, query) rows, splits in order:
// m* = max m_z, l* = sum l_z 2^(m_z - m*), out = sum o_z 2^(m_z - m*) / l*.
// A workgroup takes kMergeRows rows, 32 lanes per row and 4 head dims per
// lane (16-byte partial loads, 8-byte output stores); all loads of a batch of
// eight splits are issued before they are combined.
constexpr int kMergeRows = 8;
__global__ __launch_bounds__(32 * kMergeRows) void joint_attn_merge(AttnParams p, int nsplit, int64_t rows) {
    const int64_t hq = (int64_t) blockIdx.x * kMergeRows + (threadIdx.x >> 5);
    if (hq >= rows) return;
    int64_t h = hq / p.tq, q = hq % p.tq, stride = p.heads * p.tq;
    if (p.units) {  // row hq = query hq % 128 of unit unit0 + hq / 128
        const int64_t u = p.unit0 + hq / kPfQueries;
        h = u % p.heads;
        q = u / p.heads * kPfQueries + hq % kPfQueries;
        stride = p.units * kPfQueries;
        if (q >= p.tq) return;
    }
    const int d = 4 * (threadIdx.x & 31);
    constexpr int kB = 8;
    float mstar = -INFINITY;
    for (int z0 = 0; z0 < nsplit; z0 += kB) {
        float m[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) m[u] = p.part_m[min(z0 + u, nsplit - 1) * stride + hq];
#pragma unroll
        for (int u = 0; u < kB; ++u) mstar = fmaxf(mstar, m[u]);
    }
    float l = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int z0 = 0; z0 < nsplit; z0 += kB) {
        float m[kB], lz[kB];
        float4 oz[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            const int64_t z = min(z0 + u, nsplit - 1);
            m[u] = p.part_m[z * stride + hq];
            lz[u] = p.part_l[z * stride + hq];
            oz[u] = *(const float4 *) (p.part_o + (z * stride + hq) * kDh + d);
        }
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            if (z0 + u >= nsplit || m[u] == -INFINITY) continue;
            const float w = exp2f(m[u] - mstar);
            l += lz[u] * w;
            o[0] += oz[u].x * w;
            o[1] += oz[u].y * w;
            o[2] += oz[u].z * w;
            o[3] += oz[u].w * w;
        }
    }
    uint2 out;
    out.x = pack_bf16x2(l > 0.0f ? o[0] / l : 0.0f, l > 0.0f ? o[1] / l : 0.0f);
    out.y = pack_bf16x2(l > 0.0f ? o[2] / l : 0.0f, l > 0.0f ? o[3] / l : 0.0f);
    *(uint2 *) (out_row(p, h, q) + d) = out;
}


// ---------------------------------------------------------------------------
// attn_prefill: softmax(scale * Q K^T) V for many queries over one key source
// (the prefix self-attention, 3073 x 3073 keys per head, and the visual
// cross-attention over the 512 prompt keys).
//
// Workgroup: 4 waves x 32 queries of one head.  Key blocks of 64: the K tile
// [64 keys][128] and the V^T tile [128][64 keys] are copied into LDS with
// global_load_lds_dwordx4 through a 2-stage ring (separate LDS objects, loop
// unrolled by 2, so only the stage being read is waited for), shared by the
// four waves.  Per block and wave: S^T = K Q^T with MFMA 32x32x16 (Q^T
// fragments held in registers for the whole key loop), online softmax in the
// log2 domain with P rounded to bf16, then O^T += V^T P^T with the P operand
// taken straight from the S^T accumulators: the key slots of a PV k-step are
// the keys that accumulator layout gives each lane half, and the V^T operand
// reads the same keys as two 8-byte pieces.  Keys past the source length are
// masked (scores to -inf, V^T values to zero).  The normalised O^T goes
// through LDS so the output rows are written as 16-byte pieces.
//
// LDS rows are XOR-swizzled by 16-byte chunk: K chunk c of key r at
// c ^ (r & 15), V^T chunk c of row d at c ^ ((d >> 1) & 7).
// ---------------------------------------------------------------------------
constexpr int kPfKeys = 64;
constexpr int kPfStageElems = kPfKeys * kDh + kDh * kPfKeys;  // K tile + V^T tile

__device__ __forceinline__ int pf_kswz(int key, int c) { return c ^ (key & 15); }
__device__ __forceinline__ int pf_vswz(int d, int c) { return c ^ ((d >> 1) & 7); }

// Key block `blk` of head h: source a's 64-key blocks come first, then
// source b's (each source's last block partial).
struct PfBlk {
    const uint16_t * kb;
    const uint16_t * vb;
    const uint16_t * klb;  // K remainder (f32-accurate scores), source a only
    int64_t vld, k0, nk;
};
template <bool HILO = false>
__device__ __forceinline__ PfBlk pf_locate(const AttnParams & p, int64_t h, int nblk_a, int blk) {
    const int seg = blk < nblk_a ? 0 : 1;
    PfBlk r;
    r.nk = p.seg_len[seg];
    r.vld = p.vt_ld[seg];
    r.k0 = (int64_t) (blk - (seg ? nblk_a : 0)) * kPfKeys;
    r.kb = p.k[seg] + h * r.nk * kDh;
    r.vb = p.vt[seg] + h * kDh * r.vld;
    r.klb = HILO ? p.k_lo + h * r.nk * kDh : nullptr;
    return r;
}

// One block's K tile and V^T tile into an LDS stage by a workgroup of
// kPfWaves waves: 8 global_load_lds_dwordx4 per thread.  DMA slots: K tile
// 1024 chunks (key = s / 16), V^T tile 1024 chunks (row = s / 8).  Rows past
// the source end are clamped to its last key (the consumer masks them).
__device__ __forceinline__ void pf_dma(const PfBlk & bl, uint16_t * stage, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int slot = (i * kPfWaves + wave) * 64 + lane;
        const int key = slot >> 4, c = pf_kswz(key, slot & 15);
        const int64_t kr = min(bl.k0 + key, bl.nk - 1);
        __builtin_amdgcn_global_load_lds((glb_void_t *) (bl.kb + kr * kDh + 8 * c),
                                         (lds_void_t *) (stage + (i * kPfWaves + wave) * 512), 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int slot = (i * kPfWaves + wave) * 64 + lane;
        const int d = slot >> 3, c = pf_vswz(d, slot & 7);
        const int64_t kc = min(bl.k0 + 8 * c, bl.vld - 8);
        __builtin_amdgcn_global_load_lds((glb_void_t *) (bl.vb + (int64_t) d * bl.vld + kc),
                                         (lds_void_t *) (stage + kPfKeys * kDh + (i * kPfWaves + wave) * 512), 16, 0,
                                         0);
    }
}
constexpr int kPfDmaPerBlock = 8;  // global_load_lds per thread per block

// A full block's copies (pf_dma's slots without the clamping of a source's
// partial last block): 32-bit byte offsets of this thread's K and V^T chunks
// from the block's first key row / first V^T column (V^T rows vld apart; the
// launcher keeps 128 rows within 2^31 bytes) on 64-bit block base addresses.
__device__ __forceinline__ void pf_dma_full(const PfBlk & bl, uint16_t * stage, int wave, int lane) {
    const char * kb = (const char *) (bl.kb + bl.k0 * kDh);
    const char * vb = (const char *) (bl.vb + bl.k0);
    const uint32_t vld = (uint32_t) bl.vld;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t slot = (uint32_t) ((i * kPfWaves + wave) * 64 + lane), key = slot >> 4;
        const uint32_t off = (key * kDh + 8 * (uint32_t) pf_kswz((int) key, (int) (slot & 15))) * 2;
        __builtin_amdgcn_global_load_lds((glb_void_t *) (kb + off),
                                         (lds_void_t *) (stage + (i * kPfWaves + wave) * 512), 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t slot = (uint32_t) ((i * kPfWaves + wave) * 64 + lane), d = slot >> 3;
        const uint32_t off = (d * vld + 8 * (uint32_t) pf_vswz((int) d, (int) (slot & 7))) * 2;
        __builtin_amdgcn_global_load_lds((glb_void_t *) (vb + off),
                                         (lds_void_t *) (stage + kPfKeys * kDh + (i * kPfWaves + wave) * 512), 16, 0,
                                         0);
    }
}

// The K remainder tile of a block (f32-accurate scores), as pf_dma's K tile
// (clamped rows) into its own LDS tile.
__device__ __forceinline__ void pf_dma_klo(const PfBlk & bl, uint16_t * tile, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int slot = (i * kPfWaves + wave) * 64 + lane;
        const int key = slot >> 4, c = pf_kswz(key, slot & 15);
        const int64_t kr = min(bl.k0 + key, bl.nk - 1);
        __builtin_amdgcn_global_load_lds((glb_void_t *) (bl.klb + kr * kDh + 8 * c),
                                         (lds_void_t *) (tile + (i * kPfWaves + wave) * 512), 16, 0, 0);
    }
}

// HILO: f32-accurate scores from bf16 hi/lo planes of Q and K (q_lo, k_lo):
// S^T = K Q^T + K Q_lo^T + K_lo Q^T with fp32 accumulation.  The K remainder
// has one LDS tile (16 KB; 80 KB per workgroup, two per CU): block b+1's is
// copied in after a barrier that follows block b's score MFMAs, and lands
// during its softmax and P.V.  One key source; no key split.
template <bool SPLIT, bool HILO = false>
__global__ __launch_bounds__(kPfWaves * 64, 2) void attn_prefill_kernel(AttnParams p) {
    __shared__ __align__(16) uint16_t st0[kPfStageElems];
    __shared__ __align__(16) uint16_t st1[kPfStageElems];
    __shared__ __align__(16) uint16_t klo[HILO ? kPfKeys * kDh : 8];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, hl = lane >> 5;
    // Work of this workgroup: head h, queries from q0 (and key range
    // blockIdx.z with SPLIT).
    const int64_t unit = p.unit0 + blockIdx.x;
    const int64_t h = p.units ? unit % p.heads : (int64_t) blockIdx.x;
    const int64_t q0 = (p.units ? unit / p.heads : (int64_t) blockIdx.y) * kPfQueries;
    const int nblk_a = (int) ((p.seg_len[0] + kPfKeys - 1) / kPfKeys);
    const int nblk = nblk_a + (int) ((p.seg_len[1] + kPfKeys - 1) / kPfKeys);
    const int b_begin = SPLIT ? (int) blockIdx.z * (int) p.split_blocks : 0;
    const int b_end = SPLIT ? min(nblk, b_begin + (int) p.split_blocks) : nblk;
    auto locate = [&](int blk) { return pf_locate<HILO>(p, h, nblk_a, blk); };
    // Copies of block blk into a stage: full blocks by pf_dma_full, a
    // source's partial last block by pf_dma, which clamps its rows.  Both
    // issue kPfDmaPerBlock copies.
    auto dma = [&](int blk, uint16_t * stage) {
        blk = min(blk, b_end - 1);
        const PfBlk bl = locate(blk);
        if (bl.k0 + kPfKeys <= bl.nk) pf_dma_full(bl, stage, wave, lane);
        else pf_dma(bl, stage, wave, lane);
    };
    auto dma_lo = [&](int blk) { pf_dma_klo(locate(min(blk, b_end - 1)), klo, wave, lane); };

    // Q^T fragments (B operand of S^T = K Q^T): lane holds query l32 of the
    // wave, dims 16s + 8hl .. +8 for k-step s.
    bf16x8_t qf[8], ql[HILO ? 8 : 1];
    {
        const int64_t qi = min(q0 + 32 * wave + l32, p.tq - 1);
        const uint16_t * qrow = p.q + (h * p.tq + qi) * kDh + 8 * hl;
#pragma unroll
        for (int s = 0; s < 8; ++s) qf[s] = *(const bf16x8_t *) (qrow + 16 * s);
        if constexpr (HILO) {
            const uint16_t * qlrow = p.q_lo + (h * p.tq + qi) * kDh + 8 * hl;
#pragma unroll
            for (int s = 0; s < 8; ++s) ql[s] = *(const bf16x8_t *) (qlrow + 16 * s);
        }
    }
    // This lane's operand positions in a stage (elements): the K fragment of
    // k-step s is row l32 of key tile t (t adds 32 rows), chunk 2s + hl; the
    // V^T operand of PV k-step g = 2t + hh is row l32 of dim tile i (i adds
    // 32 rows), chunk 2g + hl: keys 32t + 16hh + 8hl .. +8.
    int kro[8], vro[4];
#pragma unroll
    for (int s = 0; s < 8; ++s) kro[s] = l32 * kDh + 8 * pf_kswz(l32, 2 * s + hl);
#pragma unroll
    for (int g = 0; g < 4; ++g) vro[g] = kPfKeys * kDh + l32 * kPfKeys + 8 * pf_vswz(l32, 2 * g + hl);

    f32x16_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) o[i][v] = 0.0f;
    float m_run = -INFINITY, l_run = 0.0f;
    const bf16x2_t ones = __builtin_bit_cast(bf16x2_t, 0x3f803f80u);

    // Softmax state per lane (its query): m_run is the running max of
    // scale*log2(e)*s used as the exponent offset.  It is raised lazily, only
    // when a block's max exceeds it by more than kPfSlack, so most blocks skip
    // rescaling O; probabilities stay <= 2^kPfSlack and O / l is unchanged.
    //
    // The block is written out in its issue order, fenced by scheduling
    // barriers so the LDS reads run ahead of the MFMAs that use them: K
    // fragments two k-steps per batch with two batches in flight, the S^T
    // MFMAs (the two key tiles' chains interleaved), the first PV k-step's
    // V^T reads, the softmax, then per PV k-step the next one's reads and
    // this one's MFMAs.  A source's partial last block also masks the scores
    // of keys past its end (a uniform branch around that step only, so the
    // block body exists once); its V^T columns there are zeroed in the stage
    // before the block.
    constexpr float kPfSlack = 8.0f;
    auto block = [&](int valid, const uint16_t * stage, int next) __attribute__((always_inline)) {
        // S^T tiles: key tile t (32 keys) x the wave's 32 queries.  K
        // fragments in batches of two k-steps (both tiles), two batches in
        // flight ahead of the MFMAs.
        f32x16_t sacc[2];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) sacc[t][v] = 0.0f;
        bf16x8_t kf[2][2][2];  // [batch buffer][k-step of the batch][tile]
        auto kread = [&](int b, bf16x8_t (&kb)[2][2]) __attribute__((always_inline)) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int t = 0; t < 2; ++t) kb[j][t] = *(const bf16x8_t *) (stage + 32 * t * kDh + kro[2 * b + j]);
        };
        if constexpr (HILO) {
            // Half-batch x = 2b + lo: k-steps 2b, 2b+1 of the K tile (lo = 0:
            // K Q^T and K Q_lo^T) or of the K remainder tile (lo = 1: K_lo
            // Q^T), through the same two fragment buffers.
            auto kread_x = [&](int x, bf16x8_t (&kb)[2][2]) __attribute__((always_inline)) {
                const uint16_t * base = (x & 1) ? klo : stage;
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
                        kb[j][t] = *(const bf16x8_t *) (base + 32 * t * kDh + kro[2 * (x >> 1) + j]);
            };
            kread_x(0, kf[0]);
            kread_x(1, kf[1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int x = 0; x < 8; ++x) {
                const int b = x >> 1;
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int t = 0; t < 2; ++t) {
                        sacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[x & 1][j][t], qf[2 * b + j], sacc[t], 0,
                                                                          0, 0);
                        if (!(x & 1))
                            sacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[x & 1][j][t], ql[2 * b + j], sacc[t],
                                                                              0, 0, 0);
                    }
                __builtin_amdgcn_sched_barrier(0);
                if (x + 2 < 8) kread_x(x + 2, kf[x & 1]);
            }
            // Every wave has read this block's K remainder: the tile takes the
            // next block's.
            cta_barrier();
            if (next < b_end) dma_lo(next);
        } else {
            kread(0, kf[0]);
            kread(1, kf[1]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int b = 0; b < 4; ++b) {
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int t = 0; t < 2; ++t)
                        sacc[t] =
                            __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[b & 1][j][t], qf[2 * b + j], sacc[t], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (b + 2 < 4) kread(b + 2, kf[b & 1]);
            }
        }
        // V^T operands of PV k-step g = 2t + hh (dim tile i), one k-step read
        // ahead.
        uint4 vbuf[2][4];
        auto vread = [&](int g, uint4 (&vb)[4]) __attribute__((always_inline)) {
#pragma unroll
            for (int i = 0; i < 4; ++i) vb[i] = *(const uint4 *) (stage + 32 * i * kPfKeys + vro[g]);
        };
        vread(0, vbuf[0]);
        __builtin_amdgcn_sched_barrier(0);
        // Lane holds query l32, keys 32t + 8(v/4) + 4hl + v%4; the other keys
        // of its query are in lane ^ 32.
        if (valid < kPfKeys) {
            // Scores of keys >= valid to -inf (bit masks, computed in place).
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const uint32_t m = (uint32_t) ((valid - 1 - (32 * t + 8 * (v >> 2) + 4 * hl + (v & 3))) >> 31);
                    sacc[t][v] = __uint_as_float((__float_as_uint(sacc[t][v]) & ~m) | (0xff800000u & m));
                }
        }
        float mx = sacc[0][0];
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int v = 0; v < 16; ++v) mx = fmaxf(mx, sacc[t][v]);
        mx = max_xor32(mx) * p.scale_log2;
        if (__builtin_amdgcn_read_exec() & __ballot(mx > m_run + kPfSlack)) {
            const float m_new = mx > m_run + kPfSlack ? mx : m_run;
            const float corr = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= corr;
            m_run = m_new;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 16; ++v) o[i][v] *= corr;
        }
        // P = bf16(2^(scale*log2e*s - m)), packed in pairs for the PV operand;
        // the row sum adds the rounded values (a bf16 dot with 1.0 per pair).
        uint32_t pk[2][8];
        float ps[2] = {0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float e0 = __builtin_amdgcn_exp2f(fmaf(sacc[t][2 * j], p.scale_log2, -m_run));
                const float e1 = __builtin_amdgcn_exp2f(fmaf(sacc[t][2 * j + 1], p.scale_log2, -m_run));
                pk[t][j] = pack_bf16x2(e0, e1);
                ps[t] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk[t][j]), ones, ps[t], false);
            }
        l_run += sum_xor32(ps[0] + ps[1]);
        // O^T += V^T P^T, k-step g = (t, hh) over keys 32t + 16hh + 0..15:
        // lane half hl takes key slots 8hl..8hl+7 = keys 32t + 16hh + 8hl ..
        // +8, one 16-byte V^T chunk.  The S^T layout gives lane half hl keys
        // 16hh + 4hl + {0..3} (pk[4hh], pk[4hh+1]) and 16hh + 8 + 4hl + {0..3}
        // (pk[4hh+2], pk[4hh+3]); v_permlane32_swap (upper 32 lanes of the
        // first operand with lower 32 lanes of the second) trades the middle
        // two 4-key groups between the halves, so each half holds its 8 keys
        // in order.
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int t = g >> 1, hh = g & 1;
            if (g + 1 < 4) vread(g + 1, vbuf[(g + 1) & 1]);
            __builtin_amdgcn_sched_barrier(0);
            const auto s0 = __builtin_amdgcn_permlane32_swap(pk[t][4 * hh], pk[t][4 * hh + 2], false, false);
            const auto s1 = __builtin_amdgcn_permlane32_swap(pk[t][4 * hh + 1], pk[t][4 * hh + 3], false, false);
            const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, make_uint4(s0[0], s1[0], s0[1], s1[1]));
#pragma unroll
            for (int i = 0; i < 4; ++i)
                o[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vbuf[g & 1][i]), pf, o[i],
                                                               0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto step = [&](int blk, const uint16_t * cur, uint16_t * nxt) __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        cta_barrier();
        if (blk + 1 < b_end) dma(blk + 1, nxt);
        const PfBlk bl = locate(blk);
        if (bl.k0 + kPfKeys > bl.nk) {
            // A source's partial last block: the V^T columns of keys past its
            // end (clamped or padding data) are zeroed in the stage, so the
            // masked keys' P = 0 meets V^T = 0, and their scores are masked.
            const int valid = (int) (bl.nk - bl.k0);
            uint16_t * vt = (uint16_t *) cur + kPfKeys * kDh;
            for (int e = tid; e < kDh * kPfKeys; e += kPfWaves * 64) {
                const int d = e / kPfKeys, key = e % kPfKeys;
                if (key >= valid) vt[d * kPfKeys + 8 * pf_vswz(d, key >> 3) + (key & 7)] = 0;
            }
            __syncthreads();
        }
        block((int) min((int64_t) kPfKeys, bl.nk - bl.k0), cur, blk + 1);
    };

    dma(b_begin, st0);
    if constexpr (HILO) dma_lo(b_begin);
    for (int blk = b_begin; blk < b_end; blk += 2) {
        step(blk, st0, st1);
        if (blk + 1 < b_end) step(blk + 1, st1, st0);
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    cta_barrier();

    if constexpr (SPLIT) {
        // Unnormalised O^T with its running max (log2 domain) and sum, for
        // joint_attn_merge: part_o [split][head][query][dh] (unit-mapped:
        // [split][workgroup][query of the block][dh]).
        const int64_t z = blockIdx.z, qi = q0 + 32 * wave + l32;
        if (qi < p.tq) {
            const int64_t pi = p.units ? (z * p.units + blockIdx.x) * kPfQueries + (qi - q0) : (z * p.heads + h) * p.tq + qi;
            if (hl == 0) {
                p.part_m[pi] = m_run;
                p.part_l[pi] = l_run;
            }
            float * po = p.part_o + pi * kDh;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 16; v += 4)
                    *(float4 *) (po + 32 * i + 8 * (v >> 2) + 4 * hl) =
                        make_float4(o[i][v], o[i][v + 1], o[i][v + 2], o[i][v + 3]);
        }
        return;
    }

    // Normalise and stage O (bf16, [query][dh]) in LDS, then write whole rows.
    uint16_t * ot = st0;  // 128 queries x 128 dims = 32 KB <= one stage
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const int d = 32 * i + 8 * (v >> 2) + 4 * hl + (v & 3);
            ot[(32 * wave + l32) * kDh + d] = f32_to_bf16(o[i][v] * inv);
        }
    // A full workgroup fence: the LDS writes above must complete before other
    // waves read them (a bare s_barrier does not wait for them).
    __syncthreads();
    const int64_t nq = min((int64_t) kPfQueries, p.tq - q0);
    for (int c = tid; c < nq * (kDh / 8); c += kPfWaves * 64) {
        const int q = c / (kDh / 8), dc = c % (kDh / 8);
        *(uint4 *) (out_row(p, h, q0 + q) + 8 * dc) = *(const uint4 *) (ot + q * kDh + 8 * dc);
    }
}

// ---------------------------------------------------------------------------
// attn_decode: softmax(scale * Q K^T) V for at most 64 queries (the 48-token
// denoise step) over long key sources, one workgroup per (head, group of
// 16*QT queries, key range).
//
// All four waves work on real queries: in every 64-key block (the attn_prefill
// K / V^T tiles, same LDS layout and swizzle) wave w takes keys 16w..16w+15
// for all 16*QT queries.  S^T = K Q^T with MFMA 16x16x32 (one 16-key x
// 16-query tile per query tile, Q^T fragments in registers), online softmax
// per (wave, query) in the log2 domain with P rounded to bf16, then O^T +=
// V^T P^T with MFMA 16x16x16, whose P operand is the S^T accumulator as it
// stands (lane: query l%16, keys 4(l/16)..+4) and whose V^T operand is one
// 8-byte LDS read of the same four keys.  Blocks stream through an S-stage
// LDS ring with S-1 in flight: S = 2 (64 KB) runs two workgroups per CU, so
// one workgroup's softmax and waits overlap the other's copies and MFMAs.  At
// the end the waves' states merge in LDS in wave order, one half of the head
// dims at a time, and the workgroup writes its key range's partial
// (unnormalised O, max, sum) for attn_merge_kernel, or the output when the
// range is all keys.
// ---------------------------------------------------------------------------
constexpr int kDecHalf = kDh / 2;  // fp32 merge rows of 64 dims, 16-byte chunks XOR-swizzled by query

__device__ __forceinline__ uint32_t lds_addr(const void * ptr) {
    return (uint32_t) (uintptr_t) (const __attribute__((address_space(3))) void *) ptr;
}

template <int QT, int S>
__global__ __launch_bounds__(kPfWaves * 64, S == 2 ? 2 : 1) void attn_decode_kernel(AttnParams p) {
    static_assert(QT >= 1 && QT <= 4 && (S == 2 || S == 4), "query tiles / ring stages");
    static_assert(kPfWaves * 16 * QT * kDecHalf * 4 <= S * kPfStageElems * 2, "the merge rows fit in the ring");
    __shared__ __align__(16) uint16_t ring[S][kPfStageElems];
    __shared__ float s_m[kPfWaves][16 * QT];
    __shared__ float s_l[kPfWaves][16 * QT];
    __shared__ float s_mstar[16 * QT], s_lstar[16 * QT];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 4, c16 = lane & 15;
    const int64_t h = blockIdx.x;
    const int64_t q0 = (int64_t) blockIdx.y * 16 * QT;  // first query of this workgroup's group
    const int nblk_a = (int) ((p.seg_len[0] + kPfKeys - 1) / kPfKeys);
    const int nblk = nblk_a + (int) ((p.seg_len[1] + kPfKeys - 1) / kPfKeys);
    const int b_begin = (int) blockIdx.z * (int) p.split_blocks;
    const int b_end = min(nblk, b_begin + (int) p.split_blocks);
    // Only the range's own blocks are loaded (no clamped repeats past its end).
    auto dma = [&](int blk, int stage) {
        if (blk < b_end) pf_dma(pf_locate(p, h, nblk_a, blk), &ring[stage][0], wave, lane);
    };

    // Q^T fragments (B operand of S^T = K Q^T): lane holds query 16t + c16,
    // dims 32c + 8g .. +8 for k-step c.
    bf16x8_t qf[QT][4];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        const int64_t qi = min(q0 + 16 * t + c16, p.tq - 1);
        const uint16_t * qrow = p.q + (h * p.tq + qi) * kDh + 8 * g;
#pragma unroll
        for (int c = 0; c < 4; ++c) qf[t][c] = *(const bf16x8_t *) (qrow + 32 * c);
    }
    f32x4_t o[QT][8];
    float m_run[QT], l_run[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        m_run[t] = -INFINITY;
        l_run[t] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[t][dt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    // LDS byte offsets of this lane's operands within a stage: K row `key`
    // (16-byte chunk 4c + g) and V^T rows 16dt + c16 (keys k4 .. k4+3).
    const int key = 16 * wave + c16, k4 = 16 * wave + 4 * g;
    uint32_t koff[4], voff[8];
#pragma unroll
    for (int c = 0; c < 4; ++c) koff[c] = (uint32_t) (key * kDh + 8 * pf_kswz(key, 4 * c + g)) * 2;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
        const int d = 16 * dt + c16;
        voff[dt] = (uint32_t) (kPfKeys * kDh + d * kPfKeys + 8 * pf_vswz(d, k4 >> 3) + (k4 & 7)) * 2;
    }

    // Lazy rescaling as in attn_prefill: the exponent offset is raised only
    // when a block's max exceeds it by more than kSlack.
    constexpr float kSlack = 8.0f;
    auto block = [&](int stage, int valid) __attribute__((always_inline)) {
        // The operand reads are issued as LDS instructions the compiler's
        // wait insertion does not track against the ring's in-flight DMA
        // (which it would otherwise drain); the explicit wait below covers
        // them, and the barrier before this block covers the DMA.
        const uint32_t base = lds_addr(&ring[stage][0]);
        bf16x8_t kf[4];
        uint2 va[8];
#pragma unroll
        for (int c = 0; c < 4; ++c) asm volatile("ds_read_b128 %0, %1" : "=v"(kf[c]) : "v"(base + koff[c]));
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) asm volatile("ds_read_b64 %0, %1" : "=v"(va[dt]) : "v"(base + voff[dt]));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int c = 0; c < 4; ++c) asm volatile("" : "+v"(kf[c]));
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            asm volatile("" : "+v"(va[dt]));
            if (valid < kPfKeys) va[dt] = mask4(va[dt], k4, valid);
        }
        // S^T for every query tile first: QT independent MFMA chains.
        f32x4_t sacc[QT];
#pragma unroll
        for (int t = 0; t < QT; ++t) sacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int t = 0; t < QT; ++t) sacc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[c], qf[t][c], sacc[t], 0, 0, 0);
        // Online softmax: lane holds query 16t + c16, keys k4 + r; the wave's
        // other keys of the query are in lanes ^16, ^32.
        bf16x4_t pf[QT];
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            bool ok[4];
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                ok[r] = k4 + r < valid;
                if (ok[r]) mx = fmaxf(mx, sacc[t][r]);
            }
            mx = max_xor32(max_xor16(mx)) * p.scale_log2;
            if (__builtin_amdgcn_read_exec() & __ballot(mx > m_run[t] + kSlack)) {
                const float m_new = mx > m_run[t] + kSlack ? mx : m_run[t];
                const float corr = __builtin_amdgcn_exp2f(m_run[t] - m_new);
                l_run[t] *= corr;
                m_run[t] = m_new;
#pragma unroll
                for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                    for (int r = 0; r < 4; ++r) o[t][dt][r] *= corr;
            }
            float e[4];
#pragma unroll
            for (int r = 0; r < 4; ++r)
                e[r] = ok[r] ? __builtin_amdgcn_exp2f(fmaf(sacc[t][r], p.scale_log2, -m_run[t])) : 0.0f;
            const uint32_t p01 = pack_bf16x2(e[0], e[1]), p23 = pack_bf16x2(e[2], e[3]);
            const float ps = __uint_as_float(p01 << 16) + __uint_as_float(p01 & 0xffff0000u) +
                             __uint_as_float(p23 << 16) + __uint_as_float(p23 & 0xffff0000u);
            l_run[t] += sum_xor32(sum_xor16(ps));
            pf[t] = __builtin_bit_cast(bf16x4_t, make_uint2(p01, p23));
        }
        // O^T += V^T P^T: 8 x QT independent MFMAs.
#pragma unroll
        for (int dt = 0; dt < 8; ++dt)
#pragma unroll
            for (int t = 0; t < QT; ++t)
                o[t][dt] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4_t, va[dt]), pf[t], o[t][dt],
                                                                     0, 0, 0);
    };
    // Block i: wait for it (blocks i+1 .. i+S-2 may stay in flight), barrier
    // (every wave is past block i-1), refill block i-1's stage with block i+S-1.
#pragma unroll
    for (int i = 0; i < S - 1; ++i) dma(b_begin + i, i);
    for (int blk = b_begin; blk < b_end; ++blk) {
        const int stage = (blk - b_begin) & (S - 1);
        // Blocks issued after this one: min(S - 2, b_end - 1 - blk).
        const int younger = min(S - 2, b_end - 1 - blk);
        if (younger >= 2) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kPfDmaPerBlock));
        else if (younger == 1) __builtin_amdgcn_s_waitcnt(vmcnt_imm(kPfDmaPerBlock));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        cta_barrier();
        dma(blk + S - 1, (stage + S - 1) & (S - 1));
        const PfBlk bl = pf_locate(p, h, nblk_a, blk);
        block(stage, (int) min((int64_t) kPfKeys, bl.nk - bl.k0));
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    __syncthreads();

    // Merge the waves in LDS, one half of the head dims at a time: wave w's
    // O^T (scaled to the common max) goes to region w as fp32 rows [query][64
    // dims], 16-byte chunk j of query q at j ^ (q & 15); every thread then sums
    // four dims of one query over the waves in wave order.
#pragma unroll
    for (int t = 0; t < QT; ++t)
        if (g == 0) {
            s_m[wave][16 * t + c16] = m_run[t];
            s_l[wave][16 * t + c16] = l_run[t];
        }
    __syncthreads();
    if (tid < 16 * QT) {
        float mstar = -INFINITY, l = 0.0f;
#pragma unroll
        for (int w = 0; w < kPfWaves; ++w) mstar = fmaxf(mstar, s_m[w][tid]);
#pragma unroll
        for (int w = 0; w < kPfWaves; ++w)
            if (s_m[w][tid] != -INFINITY) l += s_l[w][tid] * __builtin_amdgcn_exp2f(s_m[w][tid] - mstar);
        s_mstar[tid] = mstar;
        s_lstar[tid] = l;
    }
    float fac[QT];
#pragma unroll
    for (int t = 0; t < QT; ++t) {
        float mstar = -INFINITY;
#pragma unroll
        for (int w = 0; w < kPfWaves; ++w) mstar = fmaxf(mstar, s_m[w][16 * t + c16]);
        fac[t] = m_run[t] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run[t] - mstar);
    }
    constexpr int kRegion = 16 * QT * kDecHalf;  // floats per wave
    float * const rows = (float *) &ring[0][0];
    const int nq = (int) min((int64_t) (16 * QT), p.tq - q0);
    const bool split = gridDim.z > 1;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        if (half) __syncthreads();  // the previous half's rows have been read
#pragma unroll
        for (int t = 0; t < QT; ++t) {
            const int q = 16 * t + c16;
#pragma unroll
            for (int dd = 0; dd < 4; ++dd) {
                const int dt = 4 * half + dd;
                *(float4 *) (rows + wave * kRegion + q * kDecHalf + 4 * ((4 * dd + g) ^ c16)) =
                    make_float4(o[t][dt][0] * fac[t], o[t][dt][1] * fac[t], o[t][dt][2] * fac[t], o[t][dt][3] * fac[t]);
            }
        }
        __syncthreads();
        for (int e = tid; e < nq * (kDecHalf / 4); e += kPfWaves * 64) {
            const int q = e / (kDecHalf / 4), j = e % (kDecHalf / 4);
            const int off = q * kDecHalf + 4 * (j ^ (q & 15));
            const int d = kDecHalf * half + 4 * j;
            float4 acc = *(const float4 *) (rows + off);
#pragma unroll
            for (int w = 1; w < kPfWaves; ++w) {
                const float4 v = *(const float4 *) (rows + w * kRegion + off);
                acc.x += v.x;
                acc.y += v.y;
                acc.z += v.z;
                acc.w += v.w;
            }
            if (split) {
                const int64_t pi = ((int64_t) blockIdx.z * p.heads + h) * p.tq + q0 + q;
                *(float4 *) (p.part_o + pi * kDh + d) = acc;
                if (d == 0) {
                    p.part_m[pi] = s_mstar[q];
                    p.part_l[pi] = s_lstar[q];
                }
            } else {
                const float l = s_lstar[q], inv = l > 0.0f ? 1.0f / l : 0.0f;
                *(uint2 *) (out_row(p, h, q0 + q) + d) =
                    make_uint2(pack_bf16x2(acc.x * inv, acc.y * inv), pack_bf16x2(acc.z * inv, acc.w * inv));
            }
        }
    }
}

// Combines the key-range partials of one (head, query) per 128-thread
// workgroup, ranges in order: m* = max m_z, l* = sum l_z 2^(m_z - m*),
// out = sum o_z 2^(m_z - m*) / l*.  Every partial is requested before the
// first is combined (nsplit <= MAXS), so the merge costs one memory latency.
template <int MAXS>
__global__ __launch_bounds__(32 * kMergeRows) void attn_merge_kernel(AttnParams p, int nsplit) {
    // kMergeRows (head, query) rows per workgroup, 32 lanes per row, 4 head
    // dims per lane: 16-byte partial loads, all issued before they combine.
    const int64_t hq = (int64_t) blockIdx.x * kMergeRows + (threadIdx.x >> 5), stride = p.heads * p.tq;
    if (hq >= stride) return;
    const int d = 4 * (threadIdx.x & 31);
    const int64_t h = hq / p.tq, q = hq % p.tq;
    float m[MAXS], lz[MAXS];
    float4 oz[MAXS];
#pragma unroll
    for (int u = 0; u < MAXS; ++u) {
        const int64_t z = min(u, nsplit - 1);
        m[u] = p.part_m[z * stride + hq];
        lz[u] = p.part_l[z * stride + hq];
        oz[u] = *(const float4 *) (p.part_o + (z * stride + hq) * kDh + d);
    }
    float mstar = -INFINITY;
#pragma unroll
    for (int u = 0; u < MAXS; ++u)
        if (u < nsplit) mstar = fmaxf(mstar, m[u]);
    float l = 0.0f, o[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int u = 0; u < MAXS; ++u) {
        if (u >= nsplit || m[u] == -INFINITY) continue;
        const float w = __builtin_amdgcn_exp2f(m[u] - mstar);
        l += lz[u] * w;
        o[0] += oz[u].x * w;
        o[1] += oz[u].y * w;
        o[2] += oz[u].z * w;
        o[3] += oz[u].w * w;
    }
    uint2 out;
    out.x = pack_bf16x2(l > 0.0f ? o[0] / l : 0.0f, l > 0.0f ? o[1] / l : 0.0f);
    out.y = pack_bf16x2(l > 0.0f ? o[2] / l : 0.0f, l > 0.0f ? o[3] / l : 0.0f);
    *(uint2 *) (out_row(p, h, q) + d) = out;
}
constexpr int kDecMaxSplits = 32;
// About one workgroup per CU in all: more ranges shorten each workgroup's
// stream but add partial traffic and merge work (measured best on the
// 24-head, 3121-key denoise shape at 10 ranges).
constexpr int kDecTargetWgs = 256;
// Sources of at most this many 64-key blocks (the 512-key prompt) are split
// by query tile as well: measured on 24 heads x 48 queries x 512 keys, 16-query
// workgroups in 4 key ranges take 10.3 us against 12.3 us for 48-query
// workgroups in 8 ranges (decode + merge).
constexpr int64_t kDecShortBlocks = 16;

// Softmax is order-free, so the keys are visited per source in 32-key blocks
// aligned to each source's start: source a ([state, reference] prefix cache,
// na keys) and source b (the current action tokens, nb keys).  The complete
// MoT order [state, action, reference] (mot.cpp:402-403) only fixes the
// reference's fp32 summation order, which the online softmax reassociates.
// Within a workgroup the waves split the key blocks and merge in LDS; across
// workgroups (key-split mode) the merge is a second kernel, so no partial
// state crosses workgroups inside a kernel and no device-scope fence is used.
constexpr int64_t kSplitBlocks = 8;   // key blocks (of 32) per split workgroup
constexpr int64_t kMaxSplits = 32;
constexpr int64_t kFlashSplitBlocks = 4;  // 64-key blocks per split of the LDS-tiled decode
constexpr int kSplitWaves = 4;
// Compute units of the current device, per device.
static int device_cus() {
    static int cus[64] = {0};
    int d = 0;
    if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= 64) return 0;
    if (!cus[d]) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, d) != hipSuccess) n = 0;
        cus[d] = n > 0 ? n : -1;
    }
    return cus[d] > 0 ? cus[d] : 0;
}

hipError_t launch_joint_attn(const AttnArgs & a, hipStream_t s) {
    if (a.head_dim != kDh) return hipErrorInvalidValue;
    if (a.tq <= 0) return hipSuccess;
    // Every path below plans key ranges over the key blocks: at least one key.
    if (a.na < 0 || a.nb < 0 || a.na + (a.k_b ? a.nb : 0) <= 0 || a.heads <= 0) return hipErrorInvalidValue;
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
    p.nblocks = p.seg_blocks[0] + p.seg_blocks[1];
    p.out = (uint16_t *) a.out;
    p.heads = a.heads;
    p.hb = a.hb > 0 ? a.hb : a.heads;
    if (p.heads % p.hb != 0) return hipErrorInvalidValue;
    p.tq = a.tq;
    p.scale_log2 = a.scale * kLog2e;
    // 8-byte V^T loads of 4 keys need rows padded to a multiple of 4 keys.
    for (int i = 0; i < 2; ++i)
        if (p.seg_len[i] > 0 &&
            (p.vt_ld[i] % 4 != 0 || p.vt_ld[i] < p.seg_len[i] || ((uintptr_t) p.vt[i] & 7) || ((uintptr_t) p.k[i] & 15)))
            return hipErrorInvalidValue;
    // Many queries over one key source (the prefix self-attention, the
    // visual cross-attention): the LDS-tiled flash kernel.
    auto flash_ok = [&](int i) {
        return p.seg_len[i] == 0 || (p.seg_len[i] >= 8 && p.vt_ld[i] % 8 == 0 && p.vt_ld[i] < (1 << 20) &&
                                     ((uintptr_t) p.vt[i] & 15) == 0 &&
                                     ((uintptr_t) p.k[i] & 15) == 0);
    };
    const bool flash = flash_ok(0) && flash_ok(1) && p.seg_len[0] > 0 && ((uintptr_t) p.q & 15) == 0 &&
                       ((uintptr_t) p.out & 15) == 0;
    // f32-accurate scores from hi/lo planes (one source, the prefix's
    // visual cross-attention): the flash kernel's HILO form.
    const bool hilo = a.q_lo || a.k_lo;
    if (hilo) {
        if (!a.q_lo || !a.k_lo || p.seg_len[1] != 0 || !flash || ((uintptr_t) a.q_lo & 15) ||
            ((uintptr_t) a.k_lo & 15) || p.heads != p.hb)
            return hipErrorInvalidValue;
        p.q_lo = (const uint16_t *) a.q_lo;
        p.k_lo = (const uint16_t *) a.k_lo;
    }
    if (flash && (a.tq > 64 || hilo) && p.seg_len[1] == 0) {
        const int64_t qblocks = (a.tq + kPfQueries - 1) / kPfQueries;
        // The (head, query block) units fill rounds of two workgroups per CU.
        // When the last round would run at most a quarter full (3072 queries
        // x 24 heads: 576 units on 512 slots), its units are split into key
        // ranges that fill it instead, with their partials merged after: as
        // many ranges as give one workgroup per CU (the 64 units of the prefix
        // self-attention in 4 ranges of 13 blocks; 7 ranges filling both
        // slots of every CU made the chunk 0.2 ms slower).
        // Sources of fewer than 16 blocks (the 512-key prompt) keep the plain
        // grid with bf16 scores (their ranges would be one or two blocks
        // long); the hi/lo form, with three times the score MFMAs per block,
        // splits them too (measured: 3072 x 512 x 24, 72 us plain).
        const int64_t units = a.heads * qblocks, slots = 2 * (int64_t) device_cus();
        const int64_t tail = slots > 0 ? units % slots : 0;
        const int64_t nblk = (p.seg_len[0] + kPfKeys - 1) / kPfKeys;
        if (units > slots && tail > 0 && 4 * tail <= slots && (nblk >= 16 || (hilo && nblk >= 2))) {
            int64_t nsplit = std::min<int64_t>({slots / (2 * tail), nblk / 2, (int64_t) kMaxSplits});
            p.split_blocks = (nblk + nsplit - 1) / nsplit;
            nsplit = (nblk + p.split_blocks - 1) / p.split_blocks;
            const size_t rows = (size_t) tail * kPfQueries;
            if (nsplit >= 2 && a.ws && (size_t) nsplit * rows * (kDh + 2) * sizeof(float) <= a.ws_bytes) {
                p.unit0 = 0;
                p.units = units - tail;
                if (hilo)
                    hipLaunchKernelGGL((attn_prefill_kernel<false, true>), dim3((unsigned) p.units),
                                       dim3(kPfWaves * 64), 0, s, p);
                else
                    hipLaunchKernelGGL(attn_prefill_kernel<false>, dim3((unsigned) p.units), dim3(kPfWaves * 64), 0,
                                       s, p);
                p.unit0 = units - tail;
                p.units = tail;
                p.part_o = (float *) a.ws;
                p.part_m = p.part_o + (size_t) nsplit * rows * kDh;
                p.part_l = p.part_m + (size_t) nsplit * rows;
                if (hilo)
                    hipLaunchKernelGGL((attn_prefill_kernel<true, true>), dim3((unsigned) tail, 1, (unsigned) nsplit),
                                       dim3(kPfWaves * 64), 0, s, p);
                else
                    hipLaunchKernelGGL(attn_prefill_kernel<true>, dim3((unsigned) tail, 1, (unsigned) nsplit),
                                       dim3(kPfWaves * 64), 0, s, p);
                hipLaunchKernelGGL(joint_attn_merge, dim3((unsigned) ((rows + kMergeRows - 1) / kMergeRows)),
                                   dim3(32 * kMergeRows), 0, s, p, (int) nsplit, (int64_t) rows);
                return hipGetLastError();
            }
        }
        if (hilo)
            hipLaunchKernelGGL((attn_prefill_kernel<false, true>), dim3((unsigned) a.heads, (unsigned) qblocks),
                               dim3(kPfWaves * 64), 0, s, p);
        else
            hipLaunchKernelGGL(attn_prefill_kernel<false>, dim3((unsigned) a.heads, (unsigned) qblocks),
                               dim3(kPfWaves * 64), 0, s, p);
        return hipGetLastError();
    }
    if (hilo) return hipErrorInvalidValue;
    // At most 64 queries (the 48-token denoise step) over long key sources:
    // attn_decode, one workgroup per (head, key range) with about one
    // workgroup per CU in all, every key read once; the ranges' fp32 partials
    // are merged by attn_merge_kernel.
    if (flash && a.tq <= 16 * 4) {
        const int64_t nblk = (p.seg_len[0] + kPfKeys - 1) / kPfKeys + (p.seg_len[1] + kPfKeys - 1) / kPfKeys;
        // Query tiles of 16 per workgroup: all queries (<= 3: 2-stage ring at
        // two workgroups per CU), or one tile per workgroup when the source is
        // short (few key ranges per head would leave most CUs idle, and the
        // per-block cost falls with the query count).
        const int qt = nblk <= kDecShortBlocks ? 1 : (int) ((a.tq + 15) / 16);
        const int64_t qg = (a.tq + 16 * qt - 1) / (16 * qt);
        int64_t nsplit =
            std::min<int64_t>({(kDecTargetWgs + a.heads * qg - 1) / (a.heads * qg), nblk, (int64_t) kDecMaxSplits});
        p.split_blocks = (nblk + nsplit - 1) / nsplit;
        nsplit = (nblk + p.split_blocks - 1) / p.split_blocks;
        const size_t part_bytes = (size_t) nsplit * a.heads * a.tq * (kDh + 2) * sizeof(float);
        if (nsplit > 1 && (!a.ws || part_bytes > a.ws_bytes)) {
            nsplit = 1;
            p.split_blocks = nblk;
        }
        if (nsplit > 1) {
            p.part_o = (float *) a.ws;
            p.part_m = p.part_o + (size_t) nsplit * a.heads * a.tq * kDh;
            p.part_l = p.part_m + (size_t) nsplit * a.heads * a.tq;
        }
        const dim3 grid((unsigned) a.heads, (unsigned) qg, (unsigned) nsplit), block(kPfWaves * 64);
        switch (qt) {
            case 1: hipLaunchKernelGGL((attn_decode_kernel<1, 2>), grid, block, 0, s, p); break;
            case 2: hipLaunchKernelGGL((attn_decode_kernel<2, 2>), grid, block, 0, s, p); break;
            case 3: hipLaunchKernelGGL((attn_decode_kernel<3, 2>), grid, block, 0, s, p); break;
            default: hipLaunchKernelGGL((attn_decode_kernel<4, 4>), grid, block, 0, s, p); break;
        }
        const dim3 mgrid((unsigned) ((a.heads * a.tq + kMergeRows - 1) / kMergeRows)), mblock(32 * kMergeRows);
        if (nsplit > 16) hipLaunchKernelGGL(attn_merge_kernel<kDecMaxSplits>, mgrid, mblock, 0, s, p, (int) nsplit);
        else if (nsplit > 8) hipLaunchKernelGGL(attn_merge_kernel<16>, mgrid, mblock, 0, s, p, (int) nsplit);
        else if (nsplit > 1) hipLaunchKernelGGL(attn_merge_kernel<8>, mgrid, mblock, 0, s, p, (int) nsplit);
        return hipGetLastError();
    }
    // Up to 128 queries over long key sources: the LDS-tiled prefill kernel,
    // one workgroup per (head, key range), every key read once; fp32 partials
    // merged by joint_attn_merge.
    if (flash && a.tq <= kPfQueries) {
        const int64_t nblk = (p.seg_len[0] + kPfKeys - 1) / kPfKeys + (p.seg_len[1] + kPfKeys - 1) / kPfKeys;
        // About kFlashSplitBlocks blocks per split, but at least 8 splits (short
        // sources such as the 512-key prompt would otherwise leave most CUs idle).
        int64_t nsplit = std::min<int64_t>(
            nblk, std::max<int64_t>((nblk + kFlashSplitBlocks - 1) / kFlashSplitBlocks, 8));
        nsplit = std::min<int64_t>(nsplit, kMaxSplits);
        p.split_blocks = (nblk + nsplit - 1) / nsplit;
        nsplit = (nblk + p.split_blocks - 1) / p.split_blocks;
        const size_t part_bytes = (size_t) nsplit * a.heads * a.tq * (kDh + 2) * sizeof(float);
        if (a.ws && part_bytes <= a.ws_bytes) {
            p.part_o = (float *) a.ws;
            p.part_m = p.part_o + (size_t) nsplit * a.heads * a.tq * kDh;
            p.part_l = p.part_m + (size_t) nsplit * a.heads * a.tq;
            hipLaunchKernelGGL(attn_prefill_kernel<true>, dim3((unsigned) a.heads, 1, (unsigned) nsplit),
                               dim3(kPfWaves * 64), 0, s, p);
            const int64_t rows = a.heads * a.tq;
            hipLaunchKernelGGL(joint_attn_merge, dim3((unsigned) ((rows + kMergeRows - 1) / kMergeRows)),
                               dim3(32 * kMergeRows), 0, s, p, (int) nsplit, rows);
            return hipGetLastError();
        }
    }
    // Other many-query cases: 48-query groups, 4 waves, one workgroup per
    // (head, group).
    if (a.tq > 64) {
        const int64_t qgroups = (a.tq + 47) / 48;
        hipLaunchKernelGGL((joint_attn_kernel<3, 4, false>), dim3((unsigned) a.heads, (unsigned) qgroups), dim3(256), 0,
                           s, p);
        return hipGetLastError();
    }
    // Few queries (the 48-token denoise step): heads x 16-query groups alone
    // would occupy a fraction of the CUs, so the keys are also split into
    // ranges of about kSplitBlocks blocks, each workgroup writing fp32
    // partials that joint_attn_merge combines.
    const int64_t qgroups = (a.tq + 15) / 16;
    int64_t nsplit = (p.nblocks + kSplitBlocks - 1) / kSplitBlocks;
    nsplit = std::min<int64_t>(nsplit, kMaxSplits);
    const size_t part_bytes = (size_t) nsplit * a.heads * a.tq * (kDh + 2) * sizeof(float);
    if (nsplit <= 1 || !a.ws || part_bytes > a.ws_bytes) {
        hipLaunchKernelGGL((joint_attn_kernel<1, 8, false>), dim3((unsigned) a.heads, (unsigned) qgroups), dim3(512), 0,
                           s, p);
        return hipGetLastError();
    }
    p.split_blocks = (p.nblocks + nsplit - 1) / nsplit;
    nsplit = (p.nblocks + p.split_blocks - 1) / p.split_blocks;
    p.part_o = (float *) a.ws;
    p.part_m = p.part_o + (size_t) nsplit * a.heads * a.tq * kDh;
    p.part_l = p.part_m + (size_t) nsplit * a.heads * a.tq;
    hipLaunchKernelGGL((joint_attn_kernel<1, kSplitWaves, true>),
                       dim3((unsigned) a.heads, (unsigned) qgroups, (unsigned) nsplit), dim3(kSplitWaves * 64), 0, s, p);
    const int64_t rows = a.heads * a.tq;
    hipLaunchKernelGGL(joint_attn_merge, dim3((unsigned) ((rows + kMergeRows - 1) / kMergeRows)),
                       dim3(32 * kMergeRows), 0, s, p, (int) nsplit, rows);
    return hipGetLastError();
}

}  // namespace wamx
