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
//                  weight streaming with MFMA 16x16x32, split-K across
//                  workgroups, deterministic in-kernel reduction by the last
//                  workgroup of each feature block.
//  * gemm_simt   — f32 weights (generic MUL_MAT only), plain FMA.
#include "../internal.h"
#include "device.h"

namespace wamx {

struct GemmParams {
    const uint16_t * w;
    const void * x;
    void * y;
    const uint16_t * bias;
    const uint16_t * res;
    const float * gate;
    float * ws;          // split-K partials
    unsigned * counters; // split-K arrival counters (zero between launches)
    int64_t ldw, w_bs2, w_bs3;
    int64_t ldx, x_bs2, x_bs3;
    int64_t ldy, y_bs2, y_bs3;
    int64_t ldres;
    int64_t M, N, K;
    int64_t B2, r2, r3;
    int32_t y_type, epi;
    int32_t splits, kslice;  // skinny: number of K slices and their length
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
// gemm_skinny: N <= 64 tokens.  Grid = (feature blocks of 64) x (K slices).
// The workgroup stages its K slice of x (all tokens, bf16) in LDS once; each
// wave then streams 16 weight rows of the slice straight from HBM into
// registers and feeds MFMA 16x16x32.  The k order inside a 128-wide step is
// permuted so every lane reads 64 contiguous bytes of its weight row (the dot
// product is order-free as long as x uses the same permutation).
// Split-K partials go to ws; the last workgroup to finish a feature block
// sums them in slice order (deterministic) and applies the epilogue.
// ---------------------------------------------------------------------------
constexpr int kSkinnyMB = 64;
constexpr int kSkinnyMaxSlice = 512;

template <bool XF32>
__global__ __launch_bounds__(256) void gemm_skinny(GemmParams p) {
    extern __shared__ __align__(16) uint16_t xs[];  // [64 tokens][kslice + 8]
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pitch = p.kslice + 8;
    const int64_t N = p.N, M = p.M, K = p.K;
    const int ntiles = (int) ((N + 15) / 16);

    // XCD-aware mapping: workgroups are dealt round-robin to the 8 XCDs, so
    // keep all K slices of one feature block on the same XCD (same L2).
    const int64_t nfb = (M + kSkinnyMB - 1) / kSkinnyMB;
    const int64_t lin = blockIdx.x;
    const int64_t xcd = lin & 7, q = lin >> 3;
    const int64_t fb = (q / p.splits) * 8 + xcd;
    const int split = (int) (q % p.splits);
    if (fb >= nfb) return;  // padding workgroups of the XCD-aware grid
    const int64_t m0 = fb * kSkinnyMB;
    const int64_t kb = (int64_t) split * p.kslice;
    const int64_t klen = min((int64_t) p.kslice, K - kb);

    // Stage x[0..N)[kb..kb+klen) as bf16; pad tokens to 16*ntiles and k to a
    // multiple of 128 with zeros.
    const int kpad = (int) ((klen + 127) / 128) * 128;
    const int chunks_per_row = kpad / 8;
    for (int c = tid; c < 16 * ntiles * chunks_per_row; c += 256) {
        const int r = c / chunks_per_row, kc = c % chunks_per_row;
        const int64_t k = kb + kc * 8;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (r < N && kc * 8 < klen) v = load_x8<XF32>(p.x, r * p.ldx + k);
        *(uint4 *) (xs + r * pitch + kc * 8) = v;
    }
    __syncthreads();

    const int64_t mrow = m0 + wave * 16 + (lane & 15);
    const bool row_ok = mrow < M;
    const uint16_t * wrow = p.w + (row_ok ? mrow : 0) * p.ldw + kb;
    const int g = lane >> 4;  // which 32-wide k group of the 128-wide step

    f32x4_t acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int nsteps = kpad / 128;
    uint4 wcur[4], wnext[4];
    auto wload = [&](int st, uint4 * dst) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int kk = st * 128 + 32 * g + 8 * c;
            dst[c] = (row_ok && kk < klen) ? *(const uint4 *) (wrow + kk) : make_uint4(0, 0, 0, 0);
        }
    };
    wload(0, wcur);
    for (int st = 0; st < nsteps; ++st) {
        if (st + 1 < nsteps) wload(st + 1, wnext);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const bf16x8_t bfrag = __builtin_bit_cast(bf16x8_t, wcur[c]);
            const int kk = st * 128 + 32 * g + 8 * c;
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                if (t < ntiles) {
                    const bf16x8_t afrag = *(const bf16x8_t *) (xs + (16 * t + (lane & 15)) * pitch + kk);
                    acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afrag, bfrag, acc[t], 0, 0, 0);
                }
            }
        }
        if (st + 1 < nsteps) {
#pragma unroll
            for (int c = 0; c < 4; ++c) wcur[c] = wnext[c];
        }
    }

    // 16x16 fragment: lane holds column (lane & 15) = feature, register r holds
    // row 4*(lane/16) + r = token within the tile.
    const int64_t m = m0 + wave * 16 + (lane & 15);
    if (p.splits == 1) {
        if (m < M) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int64_t n = 16 * t + 4 * g + r;
                    if (t < ntiles && n < N) store_out(p, p.y, p.res, n, m, acc[t][r]);
                }
        }
        return;
    }

    float * part = p.ws + (int64_t) split * 64 * M;
    if (m < M) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t n = 16 * t + 4 * g + r;
                if (t < ntiles && n < N) part[n * M + m] = acc[t][r];
            }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = atomicAdd(&p.counters[fb], 1u);
        s_last = (prev == (unsigned) (p.splits - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    // Last arrival: reduce the slices in order and run the epilogue.
    for (int e = tid; e < N * kSkinnyMB; e += 256) {
        const int64_t n = e / kSkinnyMB, mm = m0 + e % kSkinnyMB;
        if (mm >= M) continue;
        float s = 0.0f;
        for (int sp = 0; sp < p.splits; ++sp) s += p.ws[((int64_t) sp * 64 + n) * M + mm];
        store_out(p, p.y, p.res, n, mm, s);
    }
    if (tid == 0) atomicExch(&p.counters[fb], 0u);
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
    p.ws = (float *) a.ws;
    p.counters = a.counters;
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

    if (vec && batches == 1 && a.N <= 64 && a.ws && a.counters) {
        // Split K so the grid covers the chip while the partials stay a small
        // fraction of the weight bytes.
        const int64_t nfb = (a.M + kSkinnyMB - 1) / kSkinnyMB;
        int64_t splits = 1;
        const int64_t target_wg = 1024;
        while (nfb * splits < target_wg && (a.K + splits * 2 - 1) / (splits * 2) >= 128) splits *= 2;
        int64_t kslice = (a.K + splits - 1) / splits;
        kslice = (kslice + 127) / 128 * 128;
        while (kslice > kSkinnyMaxSlice) {
            splits *= 2;
            kslice = ((a.K + splits - 1) / splits + 127) / 128 * 128;
        }
        splits = (a.K + kslice - 1) / kslice;
        if (splits * 64 * a.M * 4 <= (int64_t) a.ws_bytes && nfb <= a.max_counters) {
            p.splits = (int32_t) splits;
            p.kslice = (int32_t) kslice;
            const int64_t per_xcd = (nfb + 7) / 8;
            const int64_t grid = per_xcd * splits * 8;
            const size_t lds = (size_t) 64 * (kslice + 8) * sizeof(uint16_t);
            static bool once = (allow_lds(gemm_skinny<true>, (size_t) 64 * (kSkinnyMaxSlice + 8) * 2),
                                allow_lds(gemm_skinny<false>, (size_t) 64 * (kSkinnyMaxSlice + 8) * 2), true);
            (void) once;
            if (xf32) hipLaunchKernelGGL(gemm_skinny<true>, dim3((unsigned) grid), dim3(256), lds, s, p);
            else hipLaunchKernelGGL(gemm_skinny<false>, dim3((unsigned) grid), dim3(256), lds, s, p);
            return hipGetLastError();
        }
    }
    if (vec) return xf32 ? run_tile<128, 128, true, true>(p, batches, s) : run_tile<128, 128, false, true>(p, batches, s);
    return xf32 ? run_tile<128, 128, true, false>(p, batches, s) : run_tile<128, 128, false, false>(p, batches, s);
}

}  // namespace wamx
