// BF16 GEMMs for GGML_OP_MUL_MAT / WAMX_OP_LINEAR on gfx950.
//
//   y[b][n][m] = epilogue( sum_k w[b/r][m][k] * x[b][n][k] )
//
// w is the packed-BF16 weight ([out][in], K-contiguous, the GGUF layout of
// src/models/gwp05/artifact.cpp:115-116), x the activation (bf16, or f32
// rounded to bf16 on load: ggml converts src1 to the weight's vec-dot type).
//
// Three kernels:
//  * gemm_tile   — MFMA 32x32x16 bf16, LDS double-buffered 128x128x64 tiles,
//                  128-bit global loads, for token counts above 64.
//  * gemm_skinny — N <= 64 tokens (the 48-token action expert): HBM-bound
//                  weight streaming with MFMA 16x16x32, K split across the
//                  waves of a workgroup and reduced in LDS.
//  * gemm_simt   — f32 weights (generic MUL_MAT only), plain FMA.
#include "../internal.h"
#include "device.h"

#include <algorithm>

namespace wamx {

struct GemmParams {
    const uint16_t * w;
    const void * x;
    void * y;
    const uint16_t * bias;
    const uint16_t * res;
    const float * gate;
    int64_t ldw, w_bs2, w_bs3;
    int64_t ldx, x_bs2, x_bs3;
    int64_t ldy, y_bs2, y_bs3;
    int64_t ldres;
    int64_t M, N, K;
    int64_t B2, r2, r3;
    int32_t y_type, epi;
};

// Epilogue for one output element (row n, col m) from the fp32 accumulator.
// Rounding points follow the unfused reference graph: the GEMM writes bf16
// (native-bf16.patch:273-275), the bias ADD is a bf16 + bf16 -> bf16 op
// (weights.cpp:826-828), bias_gelu_bf16 (patch:507-514) and
// gated_residual_bf16 (patch:79-91) read bf16 and round once.
__device__ __forceinline__ void store_out(const GemmParams & p, void * yb, const uint16_t * resb, int64_t n, int64_t m,
                                          float acc) {
    const int64_t yi = n * p.ldy + m;
    switch (p.epi) {
        case WAMX_EPI_NONE:
            if (p.y_type == WAMX_TYPE_F32) ((float *) yb)[yi] = acc;
            else ((uint16_t *) yb)[yi] = f32_to_bf16(acc);
            return;
        case WAMX_EPI_BIAS: {
            const float v = round_bf16(acc) + bf16_to_f32(p.bias[m]);
            ((uint16_t *) yb)[yi] = f32_to_bf16(v);
            return;
        }
        case WAMX_EPI_BIAS_GELU: {
            const float v = round_bf16(acc) + bf16_to_f32(p.bias[m]);
            ((uint16_t *) yb)[yi] = f32_to_bf16(gelu_tanh(v));
            return;
        }
        case WAMX_EPI_BIAS_GATED: {
            const float o = round_bf16(round_bf16(acc) + bf16_to_f32(p.bias[m]));
            const float h = bf16_to_f32(resb[n * p.ldres + m]);
            ((uint16_t *) yb)[yi] = f32_to_bf16(fmaf(o, p.gate[m], h));
            return;
        }
        default: {  // WAMX_EPI_BIAS_RESIDUAL
            const float o = round_bf16(round_bf16(acc) + bf16_to_f32(p.bias[m]));
            const float h = bf16_to_f32(resb[n * p.ldres + m]);
            ((uint16_t *) yb)[yi] = f32_to_bf16(h + o);
            return;
        }
    }
}

// 8 consecutive activations as packed bf16 (f32 sources rounded RNE).
template <bool XF32>
__device__ __forceinline__ uint4 load_x8(const void * x, int64_t idx) {
    if constexpr (XF32) {
        const float4 a = *(const float4 *) ((const float *) x + idx);
        const float4 b = *(const float4 *) ((const float *) x + idx + 4);
        uint4 r;
        r.x = pack_bf16x2(a.x, a.y);
        r.y = pack_bf16x2(a.z, a.w);
        r.z = pack_bf16x2(b.x, b.y);
        r.w = pack_bf16x2(b.z, b.w);
        return r;
    } else {
        return *(const uint4 *) ((const uint16_t *) x + idx);
    }
}

template <bool XF32>
__device__ __forceinline__ uint16_t load_x1(const void * x, int64_t idx) {
    if constexpr (XF32) return f32_to_bf16(((const float *) x)[idx]);
    else return ((const uint16_t *) x)[idx];
}

// ---------------------------------------------------------------------------
// gemm_tile: TR tokens x TC features per 256-thread workgroup, BK = 64.
// Four waves in a 2x2 grid; each wave owns (TR/2) x (TC/2) built from 32x32
// MFMA fragments.  LDS rows are padded by 16 bytes so the 128-bit fragment
// reads of 32 consecutive rows hit distinct banks.
// ---------------------------------------------------------------------------
constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;  // elements per LDS row

template <int TR, int TC, bool XF32, bool VEC>
__global__ __launch_bounds__(256) void gemm_tile(GemmParams p) {
    constexpr int FR = TR / 64;  // 32-row fragments per wave
    constexpr int FC = TC / 64;
    constexpr int CPR = kBK / 8;  // 16-byte chunks per row per K tile
    constexpr int A_PER = TR * CPR / 256;
    constexpr int B_PER = TC * CPR / 256;
    static_assert(A_PER * 256 == TR * CPR && B_PER * 256 == TC * CPR, "tile/thread mismatch");

    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t * buf0 = lds;
    uint16_t * buf1 = lds + (TR + TC) * kPitch;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave >> 1, wc = wave & 1;
    const int64_t bz = blockIdx.z;
    const int64_t b2 = bz % p.B2, b3 = bz / p.B2;
    const uint16_t * w = p.w + (b2 / p.r2) * p.w_bs2 + (b3 / p.r3) * p.w_bs3;
    const char * x = (const char *) p.x + (b2 * p.x_bs2 + b3 * p.x_bs3) * (XF32 ? 4 : 2);
    char * y = (char *) p.y + (b2 * p.y_bs2 + b3 * p.y_bs3) * (p.y_type == WAMX_TYPE_F32 ? 4 : 2);
    const int64_t n0 = (int64_t) blockIdx.y * TR, m0 = (int64_t) blockIdx.x * TC;
    const int64_t N = p.N, M = p.M, K = p.K;

    uint4 ra[A_PER], rb[B_PER];
    float4 raf[XF32 && VEC ? 2 * A_PER : 1];  // raw f32 activations, rounded at LDS store

    auto gload = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + 256 * i, r = c / CPR, kc = c % CPR;
            const int64_t n = n0 + r, k = k0 + kc * 8;
            if constexpr (VEC && XF32) {
                const bool ok = n < N && k < K;
                const float * src = (const float *) x + n * p.ldx + k;
                raf[2 * i] = ok ? *(const float4 *) src : make_float4(0.f, 0.f, 0.f, 0.f);
                raf[2 * i + 1] = ok ? *(const float4 *) (src + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
            } else if constexpr (VEC) {
                ra[i] = (n < N && k < K) ? load_x8<XF32>(x, n * p.ldx + k) : make_uint4(0, 0, 0, 0);
            } else {
                uint16_t e[8];
#pragma unroll
                for (int v = 0; v < 8; ++v) e[v] = (n < N && k + v < K) ? load_x1<XF32>(x, n * p.ldx + k + v) : 0;
                ra[i] = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + 256 * i, r = c / CPR, kc = c % CPR;
            const int64_t m = m0 + r, k = k0 + kc * 8;
            if constexpr (VEC) {
                rb[i] = (m < M && k < K) ? *(const uint4 *) (w + m * p.ldw + k) : make_uint4(0, 0, 0, 0);
            } else {
                uint16_t e[8];
#pragma unroll
                for (int v = 0; v < 8; ++v) e[v] = (m < M && k + v < K) ? w[m * p.ldw + k + v] : 0;
                rb[i] = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
            }
        }
    };
    auto sstore = [&](uint16_t * buf) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + 256 * i, r = c / CPR, kc = c % CPR;
            if constexpr (VEC && XF32) {
                const float4 a = raf[2 * i], b = raf[2 * i + 1];
                ra[i] = make_uint4(pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w), pack_bf16x2(b.x, b.y),
                                   pack_bf16x2(b.z, b.w));
            }
            *(uint4 *) (buf + r * kPitch + kc * 8) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + 256 * i, r = c / CPR, kc = c % CPR;
            *(uint4 *) (buf + (TR + r) * kPitch + kc * 8) = rb[i];
        }
    };

    f32x16_t acc[FR][FC];
#pragma unroll
    for (int i = 0; i < FR; ++i)
#pragma unroll
        for (int j = 0; j < FC; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int64_t nk = (K + kBK - 1) / kBK;
    gload(0);
    sstore(buf0);
    __syncthreads();

    const int arow = wr * (TR / 2) + (lane & 31);
    const int brow = TR + wc * (TC / 2) + (lane & 31);
    const int koff = 8 * (lane >> 5);

    for (int64_t kt = 0; kt < nk; ++kt) {
        uint16_t * cur = (kt & 1) ? buf1 : buf0;
        uint16_t * nxt = (kt & 1) ? buf0 : buf1;
        if (kt + 1 < nk) gload((kt + 1) * kBK);
#pragma unroll
        for (int s = 0; s < kBK / 16; ++s) {
            bf16x8_t a[FR], b[FC];
#pragma unroll
            for (int i = 0; i < FR; ++i) a[i] = *(const bf16x8_t *) (cur + (arow + 32 * i) * kPitch + 16 * s + koff);
#pragma unroll
            for (int j = 0; j < FC; ++j) b[j] = *(const bf16x8_t *) (cur + (brow + 32 * j) * kPitch + 16 * s + koff);
#pragma unroll
            for (int i = 0; i < FR; ++i)
#pragma unroll
                for (int j = 0; j < FC; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) sstore(nxt);
        __syncthreads();
    }

    // Stage the fp32 tile through LDS (the K loop ended with a barrier, so
    // both operand buffers are free), then write rows with consecutive threads
    // on consecutive columns.  32x32 fragment: lane holds column (lane & 31);
    // register v holds row 8*(v/4) + 4*(lane/32) + (v%4).
    constexpr int kOutPitch = TC + 4;
    static_assert(TR * kOutPitch * 4 <= 2 * (TR + TC) * kPitch * 2, "epilogue tile must fit the operand buffers");
    float * otile = (float *) lds;
#pragma unroll
    for (int i = 0; i < FR; ++i)
#pragma unroll
        for (int j = 0; j < FC; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = wr * (TR / 2) + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                const int c = wc * (TC / 2) + 32 * j + (lane & 31);
                otile[r * kOutPitch + c] = acc[i][j][v];
            }
    __syncthreads();
    const uint16_t * resb = p.res ? p.res + (b2 * p.y_bs2 + b3 * p.y_bs3) : nullptr;
    for (int e = tid; e < TR * TC; e += 256) {
        const int r = e / TC, c = e % TC;
        const int64_t n = n0 + r, m = m0 + c;
        if (n < N && m < M) store_out(p, y, resb, n, m, otile[r * kOutPitch + c]);
    }
}

// ---------------------------------------------------------------------------
// gemm_skinny: N <= 64 tokens (the 48-token action expert), HBM-bound weight
// streaming in two kernels.
//
// gemm_skinny_part: grid = (feature blocks of 128) x (K splits).  The
//   workgroup stages its K slice of the activations (all tokens, bf16) in LDS
//   once; each of its 8 waves then streams 16 weight rows of the slice from
//   HBM with a 4-step-deep branch-free prefetch and feeds MFMA 16x16x32 with
//   activation fragments read from LDS.  Activation bytes per workgroup are
//   48/128 of its weight bytes.  With one K split the epilogue is applied
//   directly; otherwise fp32 partials go to a workspace.
// gemm_skinny_reduce: sums the K-split partials in split order
//   (deterministic) and applies the epilogue.  The kernel boundary orders the
//   partial writes before the reads; no device-scope fences are needed.
// Inside a 128-wide K step the k order is permuted so each lane reads 64
// contiguous bytes of its weight row (a dot product is order-free as long as
// the activation fragment uses the same permutation).
// ---------------------------------------------------------------------------
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyFeat = 16 * kSkinnyWaves;  // features per workgroup
constexpr int kSkinnyDepth = 4;                  // weight prefetch depth (128-wide steps)

template <bool XF32, int NT>
__global__ __launch_bounds__(kSkinnyWaves * 64) void gemm_skinny_part(GemmParams p, float * part, int ks) {
    extern __shared__ __align__(16) uint16_t xs[];  // [16*NT][ks + 8]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int64_t N = p.N, M = p.M, K = p.K;
    const int pitch = ks + 8;
    const int64_t m0 = (int64_t) blockIdx.x * kSkinnyFeat;
    const int64_t kb = (int64_t) blockIdx.y * ks;
    const int64_t ke = min(K, kb + ks);
    const int klen = (int) (ke - kb);

    // Stage x[0..N)[kb..ke) as bf16 (rows past N and columns past ke are zero).
    const int cpr = ks / 8;
    for (int c = tid; c < 16 * NT * cpr; c += kSkinnyWaves * 64) {
        const int r = c / cpr, kc = c % cpr;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (r < N && kc * 8 < klen) v = load_x8<XF32>(p.x, r * p.ldx + kb + kc * 8);
        *(uint4 *) (xs + r * pitch + kc * 8) = v;
    }

    const int64_t mrow = m0 + 16 * wave + r16;
    const uint16_t * wrow = p.w + min(mrow, M - 1) * p.ldw + kb;
    const int nsteps = (klen + 127) / 128;
    uint4 wbuf[kSkinnyDepth][4];
    auto wload = [&](int st, uint4 (&d)[4]) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int k = st * 128 + 32 * g + 8 * c;
            const bool kin = k < klen;
            uint4 v = *(const uint4 *) (wrow + (kin ? k : klen - 8));
            const uint32_t mask = kin ? 0xffffffffu : 0u;
            v.x &= mask;
            v.y &= mask;
            v.z &= mask;
            v.w &= mask;
            d[c] = v;
        }
    };
#pragma unroll
    for (int i = 0; i < kSkinnyDepth; ++i) wload(min(i, nsteps - 1), wbuf[i]);
    __syncthreads();

    f32x4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int st0 = 0; st0 < nsteps; st0 += kSkinnyDepth) {
#pragma unroll
        for (int i = 0; i < kSkinnyDepth; ++i) {
            const int st = st0 + i;
            if (st < nsteps) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int kk = st * 128 + 32 * g + 8 * c;
#pragma unroll
                    for (int t = 0; t < NT; ++t) {
                        const bf16x8_t a = *(const bf16x8_t *) (xs + (16 * t + r16) * pitch + kk);
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8_t, wbuf[i][c]),
                                                                         acc[t], 0, 0, 0);
                    }
                }
            }
            wload(min(st + kSkinnyDepth, nsteps - 1), wbuf[i]);
        }
    }

    // 16x16 fragment: lane holds column (lane & 15) = feature, register r
    // holds row 4*(lane/16) + r = token within the tile.
    if (mrow >= M) return;
    if (gridDim.y == 1) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t n = 16 * t + 4 * g + r;
                if (n < N) store_out(p, p.y, p.res, n, mrow, acc[t][r]);
            }
        return;
    }
    float * pp = part + (int64_t) blockIdx.y * N * M;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t n = 16 * t + 4 * g + r;
            if (n < N) pp[n * M + mrow] = acc[t][r];
        }
}

__global__ __launch_bounds__(256) void gemm_skinny_reduce(GemmParams p, const float * part, int splits) {
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    const int64_t total = p.N * p.M;
    if (i >= total) return;
    float s = part[i];
    for (int sp = 1; sp < splits; ++sp) s += part[(int64_t) sp * total + i];
    store_out(p, p.y, p.res, i / p.M, i % p.M, s);
}

// K split of the skinny path: ~512 workgroups, slices of 256..1024 columns.
static void skinny_plan(int64_t M, int64_t K, int & splits, int & ks) {
    const int64_t nfb = (M + kSkinnyFeat - 1) / kSkinnyFeat;
    int64_t s = (512 + nfb - 1) / nfb;                // aim at ~512 workgroups
    s = std::max<int64_t>(1, std::min<int64_t>(s, K / 256));
    int64_t k = ((K + s - 1) / s + 127) / 128 * 128;  // slice length, multiple of 128
    k = std::min<int64_t>(k, 1024);
    splits = (int) ((K + k - 1) / k);
    ks = (int) k;
}

size_t skinny_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    int splits, ks;
    skinny_plan(M, K, splits, ks);
    return splits > 1 ? (size_t) splits * N * M * sizeof(float) : 0;
}

template <bool XF32>
static hipError_t run_skinny(const GemmParams & p, void * ws, size_t ws_bytes, hipStream_t s) {
    int splits, ks;
    skinny_plan(p.M, p.K, splits, ks);
    if (splits > 1 && (!ws || (size_t) splits * p.N * p.M * sizeof(float) > ws_bytes)) return hipErrorInvalidValue;
    const int nt = (int) ((p.N + 15) / 16);
    const size_t lds = (size_t) 16 * nt * (ks + 8) * sizeof(uint16_t);
    const dim3 grid((unsigned) ((p.M + kSkinnyFeat - 1) / kSkinnyFeat), (unsigned) splits);
    const dim3 block(kSkinnyWaves * 64);
    float * part = (float *) ws;
    switch (nt) {
        case 1: hipLaunchKernelGGL((gemm_skinny_part<XF32, 1>), grid, block, lds, s, p, part, ks); break;
        case 2: hipLaunchKernelGGL((gemm_skinny_part<XF32, 2>), grid, block, lds, s, p, part, ks); break;
        case 3: hipLaunchKernelGGL((gemm_skinny_part<XF32, 3>), grid, block, lds, s, p, part, ks); break;
        default: hipLaunchKernelGGL((gemm_skinny_part<XF32, 4>), grid, block, lds, s, p, part, ks); break;
    }
    if (splits > 1) {
        const int64_t total = p.N * p.M;
        hipLaunchKernelGGL(gemm_skinny_reduce, dim3((unsigned) ((total + 255) / 256)), dim3(256), 0, s, p,
                           (const float *) part, splits);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// gemm_simt: f32 weights (generic MUL_MAT of two f32 tensors, not on the
// native bf16 path).  One thread per output, fp32 FMA over K.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gemm_simt(GemmParams p, int32_t x_type) {
    const int64_t m = (int64_t) blockIdx.x * 256 + threadIdx.x;
    const int64_t n = blockIdx.y;
    const int64_t bz = blockIdx.z, b2 = bz % p.B2, b3 = bz / p.B2;
    if (m >= p.M) return;
    const float * w = (const float *) p.w + (b2 / p.r2) * p.w_bs2 + (b3 / p.r3) * p.w_bs3 + m * p.ldw;
    const int64_t xo = b2 * p.x_bs2 + b3 * p.x_bs3 + n * p.ldx;
    float acc = 0.0f;
    for (int64_t k = 0; k < p.K; ++k) acc = fmaf(w[k], load_as_f32(p.x, x_type, xo + k), acc);
    char * y = (char *) p.y + (b2 * p.y_bs2 + b3 * p.y_bs3) * (p.y_type == WAMX_TYPE_F32 ? 4 : 2);
    store_out(p, y, p.res, n, m, acc);
}

// ---------------------------------------------------------------------------
// Host dispatch
// ---------------------------------------------------------------------------
static bool aligned16(const void * ptr) { return ((uintptr_t) ptr & 15) == 0; }

// Dynamic LDS above 64 KiB has to be allowed per kernel once.
template <typename F>
static void allow_lds(F kernel, size_t bytes) {
    if (bytes > 65536) (void) hipFuncSetAttribute((const void *) kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int) bytes);
}

template <int TR, int TC, bool XF32, bool VEC>
static hipError_t run_tile(const GemmParams & p, int64_t batches, hipStream_t s) {
    const size_t lds = 2 * (size_t) (TR + TC) * kPitch * sizeof(uint16_t);
    static bool once = (allow_lds(gemm_tile<TR, TC, XF32, VEC>, lds), true);
    (void) once;
    dim3 grid((unsigned) ((p.M + TC - 1) / TC), (unsigned) ((p.N + TR - 1) / TR), (unsigned) batches);
    hipLaunchKernelGGL((gemm_tile<TR, TC, XF32, VEC>), grid, dim3(256), lds, s, p);
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmArgs & a, hipStream_t s) {
    GemmParams p{};
    p.w = (const uint16_t *) a.w;
    p.x = a.x;
    p.y = a.y;
    p.bias = (const uint16_t *) a.bias;
    p.res = (const uint16_t *) a.res;
    p.gate = a.gate;
    p.ldw = a.ldw; p.w_bs2 = a.w_bs2; p.w_bs3 = a.w_bs3;
    p.ldx = a.ldx; p.x_bs2 = a.x_bs2; p.x_bs3 = a.x_bs3;
    p.ldy = a.ldy; p.y_bs2 = a.y_bs2; p.y_bs3 = a.y_bs3;
    p.ldres = a.ldres;
    p.M = a.M; p.N = a.N; p.K = a.K;
    p.B2 = a.B2; p.r2 = a.r2; p.r3 = a.r3;
    p.y_type = a.y_type;
    p.epi = a.epi;
    const int64_t batches = a.B2 * a.B3;
    if (a.M <= 0 || a.N <= 0 || batches <= 0) return hipSuccess;
    if (a.K <= 0) return hipErrorInvalidValue;

    if (a.w_type == WAMX_TYPE_F32) {
        dim3 grid((unsigned) ((a.M + 255) / 256), (unsigned) a.N, (unsigned) batches);
        hipLaunchKernelGGL(gemm_simt, grid, dim3(256), 0, s, p, a.x_type);
        return hipGetLastError();
    }
    if (a.w_type != WAMX_TYPE_BF16 || (a.x_type != WAMX_TYPE_BF16 && a.x_type != WAMX_TYPE_F32))
        return hipErrorInvalidValue;
    const bool xf32 = a.x_type == WAMX_TYPE_F32;
    const bool vec = a.K % 8 == 0 && a.ldw % 8 == 0 && a.ldx % 8 == 0 && aligned16(a.w) && aligned16(a.x) &&
                     a.w_bs2 % 8 == 0 && a.w_bs3 % 8 == 0 && a.x_bs2 % 8 == 0 && a.x_bs3 % 8 == 0;

    if (vec && batches == 1 && a.N <= 64) {
        // K slices up to 1024 columns: 64 x 1032 bf16 = 132 KB of LDS.
        constexpr size_t kMaxLds = 160 * 1024;
        static bool once = (allow_lds(gemm_skinny_part<true, 1>, kMaxLds), allow_lds(gemm_skinny_part<false, 1>, kMaxLds),
                            allow_lds(gemm_skinny_part<true, 2>, kMaxLds), allow_lds(gemm_skinny_part<false, 2>, kMaxLds),
                            allow_lds(gemm_skinny_part<true, 3>, kMaxLds), allow_lds(gemm_skinny_part<false, 3>, kMaxLds),
                            allow_lds(gemm_skinny_part<true, 4>, kMaxLds), allow_lds(gemm_skinny_part<false, 4>, kMaxLds),
                            true);
        (void) once;
        return xf32 ? run_skinny<true>(p, a.ws, a.ws_bytes, s) : run_skinny<false>(p, a.ws, a.ws_bytes, s);
    }
    if (vec) return xf32 ? run_tile<128, 128, true, true>(p, batches, s) : run_tile<128, 128, false, true>(p, batches, s);
    return xf32 ? run_tile<128, 128, true, false>(p, batches, s) : run_tile<128, 128, false, false>(p, batches, s);
}

}  // namespace wamx
