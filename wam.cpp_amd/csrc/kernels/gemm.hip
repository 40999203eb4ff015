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
#include "rowops.h"

#include <algorithm>
#include <type_traits>

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
    int32_t vec_out;  // bf16 output written in 16-byte row chunks (see tile_store_lds)
};

// Epilogue for one output element (row n, col m) from the fp32 accumulator.
// Rounding points follow the unfused reference graph: the GEMM writes bf16
// (native-bf16.patch:273-275), the bias ADD is a bf16 + bf16 -> bf16 op
// (weights.cpp:826-828), bias_gelu_bf16 (patch:507-514) and
// gated_residual_bf16 (patch:79-91) read bf16 and round once.
// Kinds: 0 f32 out, 1 bf16 out, 2 bias, 3 bias+GELU, 4 bias+gated residual,
// 5 bias+residual.
enum { kEpiF32 = 0, kEpiBf16, kEpiBias, kEpiBiasGelu, kEpiBiasGated, kEpiBiasResidual };

__host__ __device__ __forceinline__ int epi_kind(const GemmParams & p) {
    switch (p.epi) {
        case WAMX_EPI_NONE: return p.y_type == WAMX_TYPE_F32 ? kEpiF32 : kEpiBf16;
        case WAMX_EPI_BIAS: return kEpiBias;
        case WAMX_EPI_BIAS_GELU: return kEpiBiasGelu;
        case WAMX_EPI_BIAS_GATED: return kEpiBiasGated;
        default: return kEpiBiasResidual;
    }
}

template <int E>
__device__ __forceinline__ void store_out_t(const GemmParams & p, void * yb, const uint16_t * resb, int64_t n,
                                            int64_t m, float acc) {
    const int64_t yi = n * p.ldy + m;
    if constexpr (E == kEpiF32) {
        ((float *) yb)[yi] = acc;
    } else if constexpr (E == kEpiBf16) {
        ((uint16_t *) yb)[yi] = f32_to_bf16(acc);
    } else if constexpr (E == kEpiBias) {
        ((uint16_t *) yb)[yi] = f32_to_bf16(round_bf16(acc) + bf16_to_f32(p.bias[m]));
    } else if constexpr (E == kEpiBiasGelu) {
        ((uint16_t *) yb)[yi] = f32_to_bf16(gelu_tanh(round_bf16(acc) + bf16_to_f32(p.bias[m])));
    } else if constexpr (E == kEpiBiasGated) {
        const float o = round_bf16(round_bf16(acc) + bf16_to_f32(p.bias[m]));
        const float h = bf16_to_f32(resb[n * p.ldres + m]);
        ((uint16_t *) yb)[yi] = f32_to_bf16(fmaf(o, p.gate[m], h));
    } else {
        const float o = round_bf16(round_bf16(acc) + bf16_to_f32(p.bias[m]));
        const float h = bf16_to_f32(resb[n * p.ldres + m]);
        ((uint16_t *) yb)[yi] = f32_to_bf16(h + o);
    }
}

__device__ __forceinline__ void store_out(const GemmParams & p, void * yb, const uint16_t * resb, int64_t n, int64_t m,
                                          float acc) {
    switch (epi_kind(p)) {
        case kEpiF32: store_out_t<kEpiF32>(p, yb, resb, n, m, acc); return;
        case kEpiBf16: store_out_t<kEpiBf16>(p, yb, resb, n, m, acc); return;
        case kEpiBias: store_out_t<kEpiBias>(p, yb, resb, n, m, acc); return;
        case kEpiBiasGelu: store_out_t<kEpiBiasGelu>(p, yb, resb, n, m, acc); return;
        case kEpiBiasGated: store_out_t<kEpiBiasGated>(p, yb, resb, n, m, acc); return;
        default: store_out_t<kEpiBiasResidual>(p, yb, resb, n, m, acc); return;
    }
}

// store_out with the bias, residual and gate values already loaded.
__device__ __forceinline__ void store_pre(const GemmParams & p, void * yb, int64_t n, int64_t m, float acc, float bias,
                                          float res, float gate) {
    const int64_t yi = n * p.ldy + m;
    switch (epi_kind(p)) {
        case kEpiF32: ((float *) yb)[yi] = acc; return;
        case kEpiBf16: ((uint16_t *) yb)[yi] = f32_to_bf16(acc); return;
        case kEpiBias: ((uint16_t *) yb)[yi] = f32_to_bf16(round_bf16(acc) + bias); return;
        case kEpiBiasGelu: ((uint16_t *) yb)[yi] = f32_to_bf16(gelu_tanh(round_bf16(acc) + bias)); return;
        case kEpiBiasGated:
            ((uint16_t *) yb)[yi] = f32_to_bf16(fmaf(round_bf16(round_bf16(acc) + bias), gate, res));
            return;
        default: ((uint16_t *) yb)[yi] = f32_to_bf16(res + round_bf16(round_bf16(acc) + bias)); return;
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
// gemm_tile: BM tokens x BN features per workgroup of WM x WN waves, BK = 64.
// Each wave owns (BM/WM) x (BN/WN) built from 32x32 MFMA fragments; operand
// tiles are double-buffered in LDS with rows padded by 16 bytes, so the
// 128-bit fragment reads of 32 consecutive rows hit distinct banks.  LDS
// read traffic per MAC is (1/wave_rows + 1/wave_cols), which is why the large
// configurations give each wave a 128 x 128 (or 96 x 96) output block held in
// the accumulation registers.
//
// Tile order: workgroups are dispatched round-robin over the 8 XCDs (linear
// id % 8), each with its own L2.  XCD x is given a contiguous range of the
// logical tile order, and that order walks feature tiles inside groups of
// kTileGroup token tiles, so the tiles resident on one XCD at a time share
// their activation and weight panels in that XCD's L2.
// ---------------------------------------------------------------------------
constexpr int kBK = 64;
constexpr int kPitch = kBK + 8;  // elements per LDS row
constexpr int kTileGroup = 4;
constexpr int kXcds = 8;

__device__ __forceinline__ void tile_coords(int pid, int nt_m, int nt_n, int & tm, int & tn) {
    const int T = nt_m * nt_n;
    const int q = T / kXcds, r = T % kXcds;
    const int xcd = pid % kXcds, j = pid / kXcds;
    const int L = (xcd < r ? xcd * (q + 1) : r * (q + 1) + (xcd - r) * q) + j;
    const int per_group = kTileGroup * nt_m;
    const int first_n = (L / per_group) * kTileGroup;
    const int gsize = min(nt_n - first_n, kTileGroup);
    const int in = L % per_group;
    tn = first_n + in % gsize;
    tm = in / gsize;
}

template <int BM, int BN, int WM, int WN>
struct TileCfg {
    static constexpr int kThreads = 64 * WM * WN;
    static constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
    static constexpr int FR = kWaveM / 32, FC = kWaveN / 32;
    static constexpr int CPR = kBK / 8;  // 16-byte chunks per row per K tile
    static constexpr int A_PER = BM * CPR / kThreads, B_PER = BN * CPR / kThreads;
    static constexpr size_t kLds = 2 * (size_t) (BM + BN) * kPitch * sizeof(uint16_t);
    static_assert(FR * 32 * WM == BM && FC * 32 * WN == BN, "wave tile must be whole 32x32 fragments");
    static_assert(A_PER * kThreads == BM * CPR && B_PER * kThreads == BN * CPR, "tile/thread mismatch");
    static_assert(kLds <= 160 * 1024, "LDS budget");
};

// Accumulator fragments -> global, one epilogue kind.  32x32 fragment: lane
// holds feature (lane & 31); register v holds token 8*(v/4) + 4*(lane/32) + v%4.
// The per-feature bias / gate are loaded once per fragment column and the 16
// residual values of a fragment are loaded together before any store, so the
// epilogue waits for memory once per fragment rather than once per element.
template <int E, int FR, int FC>
__device__ __forceinline__ void tile_store(const GemmParams & p, char * __restrict__ y,
                                           const uint16_t * __restrict__ resb, f32x16_t (&acc)[FR][FC], int64_t nb,
                                           int64_t mb, int lane) {
    constexpr bool kBias = E >= kEpiBias, kRes = E >= kEpiBiasGated;
    const uint16_t * __restrict__ bias = p.bias;
    const float * __restrict__ gate = p.gate;
#pragma unroll
    for (int j = 0; j < FC; ++j) {
        const int64_t m = mb + 32 * j + (lane & 31);
        if (m >= p.M) continue;
        const float bv = kBias ? bf16_to_f32(bias[m]) : 0.0f;
        const float gv = E == kEpiBiasGated ? gate[m] : 0.0f;
#pragma unroll
        for (int i = 0; i < FR; ++i) {
            float h[16];
            if constexpr (kRes) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int64_t n = min(nb + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3), p.N - 1);
                    h[v] = bf16_to_f32(resb[n * p.ldres + m]);
                }
            }
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int64_t n = nb + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
                if (n >= p.N) continue;
                const float a = acc[i][j][v];
                const int64_t yi = n * p.ldy + m;
                if constexpr (E == kEpiF32) {
                    ((float *) y)[yi] = a;
                } else if constexpr (E == kEpiBf16) {
                    ((uint16_t *) y)[yi] = f32_to_bf16(a);
                } else if constexpr (E == kEpiBias) {
                    ((uint16_t *) y)[yi] = f32_to_bf16(round_bf16(a) + bv);
                } else if constexpr (E == kEpiBiasGelu) {
                    ((uint16_t *) y)[yi] = f32_to_bf16(gelu_tanh(round_bf16(a) + bv));
                } else if constexpr (E == kEpiBiasGated) {
                    ((uint16_t *) y)[yi] = f32_to_bf16(fmaf(round_bf16(round_bf16(a) + bv), gv, h[v]));
                } else {
                    ((uint16_t *) y)[yi] = f32_to_bf16(h[v] + round_bf16(round_bf16(a) + bv));
                }
            }
        }
    }
}

template <int BM, int BN, int WM, int WN, bool XF32, bool VEC>
__global__ __launch_bounds__(64 * WM * WN) void gemm_tile(GemmParams p, int nt_m, int nt_n) {
    using C = TileCfg<BM, BN, WM, WN>;
    constexpr int NTH = C::kThreads, FR = C::FR, FC = C::FC, CPR = C::CPR;
    constexpr int A_PER = C::A_PER, B_PER = C::B_PER;

    extern __shared__ __align__(16) uint16_t lds[];
    uint16_t * buf0 = lds;
    uint16_t * buf1 = lds + (BM + BN) * kPitch;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave / WN, wc = wave % WN;
    const int64_t bz = blockIdx.z;
    const int64_t b2 = bz % p.B2, b3 = bz / p.B2;
    const uint16_t * w = p.w + (b2 / p.r2) * p.w_bs2 + (b3 / p.r3) * p.w_bs3;
    const char * x = (const char *) p.x + (b2 * p.x_bs2 + b3 * p.x_bs3) * (XF32 ? 4 : 2);
    char * y = (char *) p.y + (b2 * p.y_bs2 + b3 * p.y_bs3) * (p.y_type == WAMX_TYPE_F32 ? 4 : 2);
    int tm, tn;
    tile_coords((int) blockIdx.x, nt_m, nt_n, tm, tn);
    const int64_t n0 = (int64_t) tn * BM, m0 = (int64_t) tm * BN;
    const int64_t N = p.N, M = p.M, K = p.K;

    uint4 ra[A_PER], rb[B_PER];
    float4 raf[XF32 && VEC ? 2 * A_PER : 1];  // raw f32 activations, rounded at LDS store

    auto gload = [&](int64_t k0) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + NTH * i, r = c / CPR, kc = c % CPR;
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
            const int c = tid + NTH * i, r = c / CPR, kc = c % CPR;
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
            const int c = tid + NTH * i, r = c / CPR, kc = c % CPR;
            if constexpr (VEC && XF32) {
                const float4 a = raf[2 * i], b = raf[2 * i + 1];
                ra[i] = make_uint4(pack_bf16x2(a.x, a.y), pack_bf16x2(a.z, a.w), pack_bf16x2(b.x, b.y),
                                   pack_bf16x2(b.z, b.w));
            }
            *(uint4 *) (buf + r * kPitch + kc * 8) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + NTH * i, r = c / CPR, kc = c % CPR;
            *(uint4 *) (buf + (BM + r) * kPitch + kc * 8) = rb[i];
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

    const int arow = wr * C::kWaveM + (lane & 31);
    const int brow = BM + wc * C::kWaveN + (lane & 31);
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

    const uint16_t * resb = p.res ? p.res + (b2 * p.y_bs2 + b3 * p.y_bs3) : nullptr;
    const int64_t nb = n0 + wr * C::kWaveM, mb = m0 + wc * C::kWaveN;
    switch (epi_kind(p)) {
        case kEpiF32: tile_store<kEpiF32>(p, y, resb, acc, nb, mb, lane); break;
        case kEpiBf16: tile_store<kEpiBf16>(p, y, resb, acc, nb, mb, lane); break;
        case kEpiBias: tile_store<kEpiBias>(p, y, resb, acc, nb, mb, lane); break;
        case kEpiBiasGelu: tile_store<kEpiBiasGelu>(p, y, resb, acc, nb, mb, lane); break;
        case kEpiBiasGated: tile_store<kEpiBiasGated>(p, y, resb, acc, nb, mb, lane); break;
        default: tile_store<kEpiBiasResidual>(p, y, resb, acc, nb, mb, lane); break;
    }
}

// ---------------------------------------------------------------------------
// gemm_dma: the bf16 x bf16 MFMA path for large products.  Operand tiles move
// from global memory straight into LDS with global_load_lds_dwordx4 (no VGPR
// staging), through a ring of S stages of BK columns, so S-1 stages are in
// flight while one is multiplied: the L2/HBM latency is covered by the ring,
// not by the registers of the wave.
//
// Each workgroup: BM tokens x BN features, WM x WN waves, 32x32x16 MFMA.
// A stage holds BM activation rows then BN weight rows of BK bf16 each
// (BK/8 chunks of 16 bytes).  One DMA instruction writes 64 consecutive
// chunk slots (lane l -> slot base + l).  Slot p of row r holds chunk
// p ^ swz(r): an XOR swizzle under which the 128-bit fragment reads of 32
// consecutive rows are free of bank conflicts (chosen by measurement on
// gfx950: (r>>2)&3 for 64-byte rows, (r>>1)&7 for 128-byte rows).  Rows past
// N / M are clamped to the last row (their outputs are never stored).  The
// stages are separate LDS objects and the K loop is unrolled by S, so the
// compiler can tell a stage being read from the stages being filled and
// waits only for the stage it needs.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// s_waitcnt immediate: at most n vector-memory operations outstanding, other
// counters untouched (vmcnt in bits [3:0] and [15:14]).
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (((n >> 4) & 3) << 14) | (7 << 4) | (0xF << 8); }

template <int BK>
__host__ __device__ constexpr int dma_swz(int r) {
    return BK == 32 ? (r >> 2) & 3 : (r >> 1) & 7;
}

__device__ __forceinline__ void cta_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Orders a wave's own LDS writes before its later LDS reads (and the reads
// before later writes): LDS executes one wave's instructions in order, so
// only the compiler has to be kept from moving accesses across this point.
__device__ __forceinline__ void wave_lds_fence() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), other counters untouched
    asm volatile("" ::: "memory");
}

// Accumulator fragments -> global through a wave-private LDS region, for bf16
// outputs with M, ldy (and ldres) multiples of 8 and 16-byte aligned rows.
// Per 32-token fragment row the wave writes its GEMM outputs, rounded to bf16
// (the value the unfused MUL_MAT stores), into `region` (32 rows of 32*FC
// features, padded by 8 elements so the rows n and n+4 written by one
// instruction fall in disjoint banks), then reads them back as 16-byte row
// chunks and applies bias / GELU / gated residual on 8 features at a time with
// 16-byte residual loads and stores.  Same rounding points as tile_store.
// MF 16 (16x16 fragments: lane holds feature lane & 15, register v token
// 4*(lane/16) + v): two fragment rows make one 32-token pass.
template <int E, int FR, int FC, int MF = 32, typename AccT = f32x16_t>
__device__ __forceinline__ void tile_store_lds(const GemmParams & p, uint16_t * __restrict__ y,
                                               const uint16_t * __restrict__ resb, AccT (&acc)[FR][FC],
                                               int64_t nb, int64_t mb, int lane, uint16_t * __restrict__ region) {
    constexpr bool kBias = E >= kEpiBias, kRes = E >= kEpiBiasGated;
    constexpr int WN = MF * FC, SP = WN + 8, CPR = WN / 8;
    constexpr int FPP = 32 / MF;                  // fragment rows per 32-token pass
    constexpr int NV = MF * MF / 64;              // accumulator registers per fragment
    constexpr int PER = 32 * CPR / 64;            // 16-byte chunks per lane per pass
    constexpr bool kFixedCol = 64 % CPR == 0;     // each lane keeps one chunk column
    constexpr int G = PER % 4 == 0 ? 4 : PER % 3 == 0 ? 3 : PER;
    static_assert(PER * 64 == 32 * CPR, "fragment row must split evenly over the wave");
    static_assert(FR % FPP == 0, "whole 32-token passes");
    const uint16_t * __restrict__ bias = p.bias;
    const float * __restrict__ gate = p.gate;

    // Per-chunk bias / gate, hoisted when the lane's chunk column is fixed.
    float bfix[8] = {}, gfix[8] = {};
    if constexpr (kFixedCol && kBias) {
        const int64_t m = mb + 8 * (lane % CPR);
        if (m < p.M) {
            unpack8(*(const uint4 *) (bias + m), bfix);
            if constexpr (E == kEpiBiasGated) {
                const float4 g0 = *(const float4 *) (gate + m), g1 = *(const float4 *) (gate + m + 4);
                gfix[0] = g0.x; gfix[1] = g0.y; gfix[2] = g0.z; gfix[3] = g0.w;
                gfix[4] = g1.x; gfix[5] = g1.y; gfix[6] = g1.z; gfix[7] = g1.w;
            }
        }
    }

#pragma unroll
    for (int i = 0; i < FR; i += FPP) {
#pragma unroll
        for (int ii = 0; ii < FPP; ++ii)
#pragma unroll
            for (int j = 0; j < FC; ++j)
#pragma unroll
                for (int v = 0; v < NV; ++v) {
                    const int r = MF == 32 ? 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3) : 16 * ii + 4 * (lane >> 4) + v;
                    region[r * SP + MF * j + (lane & (MF - 1))] = f32_to_bf16(acc[i + ii][j][v]);
                }
        wave_lds_fence();

        // G chunks at a time: their LDS and residual loads are issued together,
        // and the live registers stay small beside the accumulators.
#pragma unroll
        for (int t0 = 0; t0 < PER; t0 += G) {
            uint4 sv[G], hv[G];
#pragma unroll
            for (int u = 0; u < G; ++u) {
                const int c = lane + 64 * (t0 + u), r = c / CPR, cc = c % CPR;
                sv[u] = *(const uint4 *) (region + r * SP + 8 * cc);
                if constexpr (kRes) {
                    const int64_t n = min(nb + MF * i + r, p.N - 1), m = min(mb + 8 * cc, p.M - 8);
                    hv[u] = *(const uint4 *) (resb + n * p.ldres + m);
                }
            }
#pragma unroll
            for (int u = 0; u < G; ++u) {
                const int c = lane + 64 * (t0 + u), r = c / CPR, cc = c % CPR;
                const int64_t n = nb + MF * i + r, m = mb + 8 * cc;
                if (n >= p.N || m >= p.M) continue;
                uint4 out = sv[u];
                if constexpr (kBias) {
                    float s[8], b[8], g[8] = {}, h[8] = {};
                    unpack8(sv[u], s);
                    if constexpr (kFixedCol) {
#pragma unroll
                        for (int e = 0; e < 8; ++e) b[e] = bfix[e], g[e] = gfix[e];
                    } else {
                        unpack8(*(const uint4 *) (bias + m), b);
                        if constexpr (E == kEpiBiasGated) {
                            const float4 g0 = *(const float4 *) (gate + m), g1 = *(const float4 *) (gate + m + 4);
                            g[0] = g0.x; g[1] = g0.y; g[2] = g0.z; g[3] = g0.w;
                            g[4] = g1.x; g[5] = g1.y; g[6] = g1.z; g[7] = g1.w;
                        }
                    }
                    if constexpr (kRes) unpack8(hv[u], h);
                    float o[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        if constexpr (E == kEpiBias) o[e] = s[e] + b[e];
                        else if constexpr (E == kEpiBiasGelu) o[e] = gelu_tanh(s[e] + b[e]);
                        else if constexpr (E == kEpiBiasGated) o[e] = fmaf(round_bf16(s[e] + b[e]), g[e], h[e]);
                        else o[e] = h[e] + round_bf16(s[e] + b[e]);
                    }
                    out = pack8(o);
                }
                *(uint4 *) (y + n * p.ldy + m) = out;
            }
        }
        wave_lds_fence();  // the next fragment row overwrites the region
    }
}

// MF: MFMA fragment edge, 32 (32x32x16) or 16 (16x16x32).  A stage holds the
// BM activation rows and the BN weight rows.  When BM + BN is not a multiple
// of the rows one copy instruction covers (RPI), the last instruction's slots
// past them (padding rows) are not copied: the waves they would fall to skip
// it (gemm_dma_pipe), so the stage needs only the real rows.
template <int BM, int BN, int WM, int WN, int BK, int S, int MF = 32>
struct DmaCfg {
    static constexpr int kThreads = 64 * WM * WN, kWaves = WM * WN;
    static constexpr int kWaveM = BM / WM, kWaveN = BN / WN;
    static constexpr int FR = kWaveM / MF, FC = kWaveN / MF;
    static constexpr int kRows = BM + BN, kChunks = BK / 8;
    static constexpr int RPI = kThreads / kChunks;  // stage rows per copy instruction
    static constexpr int kRowsPad = (kRows + RPI - 1) / RPI * RPI;
    static constexpr int kStageElems = kRows * BK;
    static constexpr int P = kRowsPad / RPI;  // DMA instructions per thread per stage
    static_assert(BK == 32 || BK == 64, "BK");
    static_assert(MF == 32 || MF == 16, "MFMA fragment edge");
    static_assert(S >= 2 && S <= 5, "ring of 2 to 5 stages");
    static_assert(FR * MF * WM == BM && FC * MF * WN == BN, "wave tile must be whole fragments");
    static_assert(P * RPI == kRowsPad && RPI * kChunks == kThreads, "stage/thread mismatch");
    static_assert((size_t) S * kStageElems * 2 <= 160 * 1024, "LDS budget");
};

// Workgroups per CU that a configuration's LDS ring allows (at most 2).
template <int BM, int BN, int WM, int WN, int BK, int S>
constexpr int dma_occupancy() {
    return (size_t) 2 * S * DmaCfg<BM, BN, WM, WN, BK, S>::kStageElems * 2 <= 160 * 1024 ? 2 : 1;
}

template <int BM, int BN, int WM, int WN, int BK, int S, int OCC = 1>
__global__ __launch_bounds__(64 * WM * WN, OCC) void gemm_dma(GemmParams p, int nt_m, int nt_n) {
    using C = DmaCfg<BM, BN, WM, WN, BK, S>;
    constexpr int FR = C::FR, FC = C::FC, P = C::P, E = C::kStageElems, CH = C::kChunks;
    static_assert(C::kRowsPad == C::kRows, "gemm_dma stages hold no padding rows");
    __shared__ __align__(16) uint16_t st0[E];
    __shared__ __align__(16) uint16_t st1[E];
    __shared__ __align__(16) uint16_t st2[S > 2 ? E : 8];
    __shared__ __align__(16) uint16_t st3[S > 3 ? E : 8];
    // Batches along blockIdx.y (run_dma_splitk: K slices, each into its own
    // f32 partial plane): x, w and y advance by their batch strides.
    if (blockIdx.y) {
        const int64_t z = blockIdx.y;
        p.x = (const uint16_t *) p.x + z * p.x_bs2;
        p.w += z * p.w_bs2;
        p.y = (char *) p.y + z * p.y_bs2 * (p.y_type == WAMX_TYPE_F32 ? 4 : 2);
    }

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wr = wave / WN, wc = wave % WN;
    int tm, tn;
    tile_coords((int) blockIdx.x, nt_m, nt_n, tm, tn);
    const int64_t n0 = (int64_t) tn * BM, m0 = (int64_t) tm * BN;
    const int64_t N = p.N, M = p.M;
    const int nk = (int) (p.K / BK);

    // Per-thread DMA sources: P chunk slots per stage, fixed rows and chunks,
    // advanced by BK columns per k tile.
    const char * src[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int slot = (i * C::kWaves + wave) * 64 + lane;
        const int r = slot / CH, c = (slot % CH) ^ dma_swz<BK>(slot / CH);
        if (r < BM) {
            const int64_t n = min(n0 + r, N - 1);
            src[i] = (const char *) ((const uint16_t *) p.x + n * p.ldx + 8 * c);
        } else {
            const int64_t m = min(m0 + (r - BM), M - 1);
            src[i] = (const char *) (p.w + m * p.ldw + 8 * c);
        }
    }
    auto dma = [&](int kt, uint16_t * stage) {
        const int64_t koff = (int64_t) min(kt, nk - 1) * BK * 2;
#pragma unroll
        for (int i = 0; i < P; ++i)
            __builtin_amdgcn_global_load_lds((glb_void_t *) (src[i] + koff),
                                             (lds_void_t *) (stage + (i * C::kWaves + wave) * 64 * 8), 16, 0, 0);
    };

    f32x16_t acc[FR][FC];
#pragma unroll
    for (int i = 0; i < FR; ++i)
#pragma unroll
        for (int j = 0; j < FC; ++j)
#pragma unroll
            for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;

    const int arow = wr * C::kWaveM + (lane & 31);
    const int brow = BM + wc * C::kWaveN + (lane & 31);
    const int sw = dma_swz<BK>(lane & 31);  // rows differ from lane & 31 by multiples of 32
    int koff[BK / 16];
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) koff[s] = ((2 * s + (lane >> 5)) ^ sw) * 8;

    auto mma = [&](const uint16_t * stage) {
#pragma unroll
        for (int s = 0; s < BK / 16; ++s) {
            bf16x8_t a[FR], b[FC];
#pragma unroll
            for (int i = 0; i < FR; ++i) a[i] = *(const bf16x8_t *) (stage + (arow + 32 * i) * BK + koff[s]);
#pragma unroll
            for (int j = 0; j < FC; ++j) b[j] = *(const bf16x8_t *) (stage + (brow + 32 * j) * BK + koff[s]);
#pragma unroll
            for (int i = 0; i < FR; ++i)
#pragma unroll
                for (int j = 0; j < FC; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };
    // Step kt: wait for stage kt (S-2 younger stages may stay in flight),
    // barrier, refill the stage freed by step kt-1 with tile kt+S-1, multiply.
    auto step = [&](int kt, uint16_t * cur, uint16_t * refill) {
        __builtin_amdgcn_s_waitcnt(vmcnt_imm((S - 2) * P));
        cta_barrier();
        dma(kt + S - 1, refill);
        mma(cur);
    };

    dma(0, st0);
    if constexpr (S > 2) dma(1, st1);
    if constexpr (S > 3) dma(2, st2);
    for (int kt = 0; kt < nk; kt += S) {
        if constexpr (S == 2) {
            step(kt, st0, st1);
            if (kt + 1 < nk) step(kt + 1, st1, st0);
        } else if constexpr (S == 3) {
            step(kt, st0, st2);
            if (kt + 1 < nk) step(kt + 1, st1, st0);
            if (kt + 2 < nk) step(kt + 2, st2, st1);
        } else {
            step(kt, st0, st3);
            if (kt + 1 < nk) step(kt + 1, st1, st0);
            if (kt + 2 < nk) step(kt + 2, st2, st1);
            if (kt + 3 < nk) step(kt + 3, st3, st2);
        }
    }
    // Drain the ring's trailing (clamped, unused) refills before the
    // workgroup's LDS can be reused.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

    const int64_t nb = n0 + wr * C::kWaveM, mb = m0 + wc * C::kWaveN;
    if (p.vec_out) {
        // The ring is free once every wave has finished its last multiply and
        // its trailing refills have landed: it becomes the wave-private
        // staging regions of tile_store_lds, WPS regions per stage array.
        constexpr int REG = 32 * (C::kWaveN + 8), WPS = E / REG;
        static_assert(WPS >= 1 && WPS * S >= C::kWaves, "staging regions must fit in the ring");
        __syncthreads();
        const int sa = wave / WPS;
        uint16_t * region = (sa == 0 ? st0 : sa == 1 ? st1 : sa == 2 ? st2 : st3) + (wave % WPS) * REG;
        uint16_t * y = (uint16_t *) p.y;
        switch (epi_kind(p)) {
            case kEpiBias: tile_store_lds<kEpiBias>(p, y, p.res, acc, nb, mb, lane, region); break;
            case kEpiBiasGelu: tile_store_lds<kEpiBiasGelu>(p, y, p.res, acc, nb, mb, lane, region); break;
            case kEpiBiasGated: tile_store_lds<kEpiBiasGated>(p, y, p.res, acc, nb, mb, lane, region); break;
            case kEpiBiasResidual: tile_store_lds<kEpiBiasResidual>(p, y, p.res, acc, nb, mb, lane, region); break;
            default: tile_store_lds<kEpiBf16>(p, y, p.res, acc, nb, mb, lane, region); break;
        }
        return;
    }
    char * y = (char *) p.y;
    switch (epi_kind(p)) {
        case kEpiF32: tile_store<kEpiF32>(p, y, p.res, acc, nb, mb, lane); break;
        case kEpiBf16: tile_store<kEpiBf16>(p, y, p.res, acc, nb, mb, lane); break;
        case kEpiBias: tile_store<kEpiBias>(p, y, p.res, acc, nb, mb, lane); break;
        case kEpiBiasGelu: tile_store<kEpiBiasGelu>(p, y, p.res, acc, nb, mb, lane); break;
        case kEpiBiasGated: tile_store<kEpiBiasGated>(p, y, p.res, acc, nb, mb, lane); break;
        default: tile_store<kEpiBiasResidual>(p, y, p.res, acc, nb, mb, lane); break;
    }
}

// ---------------------------------------------------------------------------
// gemm_dma_pipe: gemm_dma's LDS-DMA ring (BK = 32 or 64, S >= 3 stages) with
// a software-pipelined step.  The compiler's wait insertion cannot tell the
// ring's LDS stages apart and drains every in-flight copy before the first
// fragment read after a barrier; here the fragment reads are explicit
// ds_read_b128 instructions with explicit lgkmcnt waits, so only the wait
// this schedule asks for is taken:
//   step kt: issue the reads of k-step 1 of tile kt; wait for k-step 0's
//   reads; MFMAs of k-step 0; wait for tile kt+1's copies and barrier (every
//   wave is past tile kt-1); refill tile kt-1's stage with tile kt+S-1; wait
//   for k-step 1's reads; issue k-step 0's reads of tile kt+1; MFMAs of
//   k-step 1.  With BK 64 the stage holds four k-steps: k-steps 1-3 are read
//   one ahead of their MFMAs, and the barrier comes before k-step 3's.
// Scheduling barriers keep the MFMA groups on their side of the waits.  Same
// tiles, swizzle, accumulation order and epilogue as gemm_dma: same bits.
//
// SCHED selects how the waves share the step:
//  kSchedSingle: every wave runs the step above.
//  kSchedPingPong (8 waves): waves 0-3 and 4-7 (one of each per SIMD) run the
//    same sequence of K steps, [memory phase: both k-steps' fragment reads of
//    tile kt + this wave's copies of tile kt+S-1; barrier; MFMA phase;
//    barrier], with waves 4-7 one barrier behind.  At every barrier interval
//    one wave of each SIMD reads LDS and issues copies while the other issues
//    MFMAs.  Tile kt+1's copies must have landed by the barrier before either
//    group's memory phase of kt+1.
//  kSchedProducer: WM*WN consumer waves run the step without copies, and as
//    many producer waves (launched after them, a second wave per SIMD) issue
//    every copy, wait for tile kt+1 and meet the consumers at the step's
//    barrier.  The producers' registers are the consumers' allocation, so the
//    consumers must fit in 256.
// ---------------------------------------------------------------------------
enum { kSchedSingle = 0, kSchedPingPong, kSchedProducer };

__device__ __forceinline__ uint32_t lds_addr(const void * ptr) {
    return (uint32_t) (uintptr_t) (const __attribute__((address_space(3))) void *) ptr;
}
template <int OFF>
__device__ __forceinline__ bf16x8_t ds_read128(uint32_t addr) {
    bf16x8_t v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "n"(OFF));
    return v;
}
// At most N LDS operations of this wave outstanding; the fragments are tied
// to the wait so no use of them is scheduled above it.
template <int N, int FR, int FC>
__device__ __forceinline__ void lgkm_wait(bf16x8_t (&a)[FR], bf16x8_t (&b)[FC]) {
    asm volatile("s_waitcnt lgkmcnt(%0)" ::"n"(N));
#pragma unroll
    for (int i = 0; i < FR; ++i) asm volatile("" : "+v"(a[i]));
#pragma unroll
    for (int j = 0; j < FC; ++j) asm volatile("" : "+v"(b[j]));
}

// Fragment reads of one operand: N ds_read_b128 at RS-byte steps from `base`.
template <int RS, int N, int... I>
__device__ __forceinline__ void read_frags(bf16x8_t (&f)[N], uint32_t base, std::integer_sequence<int, I...>) {
    ((f[I] = ds_read128<I * RS>(base)), ...);
}

template <int BM, int BN, int WM, int WN, int S, int SCHED = kSchedSingle, int BK = 32, int MF = 32>
__global__ __launch_bounds__(64 * WM * WN * (SCHED == kSchedProducer ? 2 : 1), 1) void gemm_dma_pipe(
    GemmParams p, int nt_m, int nt_n) {
    constexpr int KS = BK / (512 / MF);  // MFMA k-steps per stage (16 deep for MF 32, 32 deep for MF 16)
    using C = DmaCfg<BM, BN, WM, WN, BK, S, MF>;
    constexpr int FR = C::FR, FC = C::FC, P = C::P, E = C::kStageElems, CH = C::kChunks;
    constexpr bool PP = SCHED == kSchedPingPong, kProd = SCHED == kSchedProducer;
    static_assert(S >= 3, "the mid-step barrier needs three or more stages");
    static_assert(!PP || (WM * WN == 8 && BK == 32), "ping-pong pairs two waves per SIMD, BK 32");
    static_assert(!kProd || WM * WN == 4, "producers take the second wave of each SIMD");
    static_assert(PP || KS >= 2, "the single and producer steps alternate two fragment sets within a stage");
    static_assert(FR + FC <= 15 && FR <= 8 && FC <= 8, "fragment count (lgkmcnt holds 15)");
    __shared__ __align__(16) uint16_t st0[E];
    __shared__ __align__(16) uint16_t st1[E];
    __shared__ __align__(16) uint16_t st2[E];
    __shared__ __align__(16) uint16_t st3[S > 3 ? E : 8];
    __shared__ __align__(16) uint16_t st4[S > 4 ? E : 8];

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Producer waves (kSchedProducer) follow the consumers; `cw` is the wave's
    // index within its role, which fixes its share of each stage's copies.
    const bool producer = kProd && wave >= C::kWaves;
    const int cw = producer ? wave - C::kWaves : wave;
    const int wr = wave / WN, wc = wave % WN;
    int tm, tn;
    tile_coords((int) blockIdx.x, nt_m, nt_n, tm, tn);
    const int64_t n0 = (int64_t) tn * BM, m0 = (int64_t) tm * BN;
    const int64_t N = p.N, M = p.M;
    const int nk = (int) (p.K / BK);
    // Copy sources as 32-bit byte offsets from the activation or weight base
    // (the launcher keeps both operands under 4 GB).  Copy instruction i of a
    // lane covers stage rows RPI i .. RPI (i + 1), all activation rows or all
    // weight rows.
    constexpr int RPI = C::RPI;
    static_assert(BM % RPI == 0, "a copy instruction covers activation rows or weight rows only");
    // A wave whose rows of the last copy instruction are all padding (past
    // BM + BN) skips that copy, and its waits count P - 1 copies per stage.
    constexpr bool kPad = C::kRowsPad != C::kRows;
    static_assert(!kPad || PP, "padded stages run the ping-pong step");
    static_assert(C::kRows % (64 / CH) == 0, "a wave's rows of one copy instruction are all real or all padding");
    const bool skip_last = kPad && ((P - 1) * C::kWaves + cw) * (64 / CH) >= C::kRows;
    uint32_t soff[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
        const int slot = (i * C::kWaves + cw) * 64 + lane;
        const int r = slot / CH, c = (slot % CH) ^ dma_swz<BK>(slot / CH);
        if (i * RPI < BM) soff[i] = (uint32_t) ((min(n0 + r, N - 1) * p.ldx + 8 * c) * 2);
        else soff[i] = (uint32_t) ((min(m0 + min(r - BM, BN - 1), M - 1) * p.ldw + 8 * c) * 2);
    }
    const char * const xb = (const char *) p.x, * const wb = (const char *) p.w;
    uint16_t * const stp[5] = {st0, st1, st2, S > 3 ? st3 : st0, S > 4 ? st4 : st0};
    auto dma = [&](int kt, int stage) {
        const uint32_t koff = (uint32_t) min(kt, nk - 1) * BK * 2;
#pragma unroll
        for (int i = 0; i < P; ++i)
            if (!kPad || i < P - 1 || !skip_last)
                __builtin_amdgcn_global_load_lds((glb_void_t *) ((i * RPI < BM ? xb : wb) + (soff[i] + koff)),
                                                 (lds_void_t *) (stp[stage] + (i * C::kWaves + cw) * 64 * 8), 16, 0,
                                                 0);
    };
    // At most T stages of this wave's copies outstanding.
    auto vm_wait = [&](auto t_c) {
        constexpr int T = decltype(t_c)::value;
        if (kPad && skip_last) __builtin_amdgcn_s_waitcnt(vmcnt_imm(T * (P - 1)));
        else __builtin_amdgcn_s_waitcnt(vmcnt_imm(T * P));
    };
    using W1 = std::integral_constant<int, S - 1>;
    using W2 = std::integral_constant<int, S - 2>;

    if constexpr (kProd) {
        if (producer) {
            // Step kt: tile kt+1 lands before the step's barrier; after it the
            // stage of tile kt-1 (every consumer is past it) takes tile kt+S-1.
            auto pstep = [&](int kt, int cur) {
                __builtin_amdgcn_s_waitcnt(vmcnt_imm((S - 3) * P));
                cta_barrier();
                dma(kt + S - 1, cur == 0 ? S - 1 : cur - 1);
            };
#pragma unroll
            for (int i = 0; i < S - 1; ++i) dma(i, i);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm((S - 2) * P));
            cta_barrier();
            for (int kt = 0; kt < nk; kt += S) {
                pstep(kt, 0);
                if (kt + 1 < nk) pstep(kt + 1, 1);
                if (kt + 2 < nk) pstep(kt + 2, 2);
                if constexpr (S > 3)
                    if (kt + 3 < nk) pstep(kt + 3, 3);
                if constexpr (S > 4)
                    if (kt + 4 < nk) pstep(kt + 4, 4);
            }
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            __syncthreads();  // the consumers' barrier before the epilogue
            return;
        }
    }

    // MF 32: 32x32 fragments (16 registers); MF 16: 16x16 fragments (4).
    using acc_t = std::conditional_t<MF == 32, f32x16_t, f32x4_t>;
    constexpr int NV = MF * MF / 64;
    acc_t acc[FR][FC];
#pragma unroll
    for (int i = 0; i < FR; ++i)
#pragma unroll
        for (int j = 0; j < FC; ++j)
#pragma unroll
            for (int v = 0; v < NV; ++v) acc[i][j][v] = 0.0f;

    // Byte offsets of this lane's A fragments in a stage, per MFMA k-step (lane
    // reads row lane % MF, 16-byte chunk lane / MF of the k-step's 64 / MF
    // chunks); its B fragments sit a wave-uniform distance further (the row
    // swizzle repeats every 16 rows, and the wave tiles start at multiples of 16).
    static_assert(C::kWaveM % 16 == 0 && C::kWaveN % 16 == 0 && BM % 16 == 0, "swizzle period");
    const int arow = wr * C::kWaveM + (lane & (MF - 1));
    const int sw = dma_swz<BK>(lane & (MF - 1));
    const uint32_t bdelta = (uint32_t) ((BM + wc * C::kWaveN - wr * C::kWaveM) * BK * 2);
    uint32_t aoff[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
        aoff[ks] = (uint32_t) (arow * BK + (((64 / MF) * ks + lane / MF) ^ sw) * 8) * 2;
    const uint32_t sbase[5] = {lds_addr(st0), lds_addr(st1), lds_addr(st2), lds_addr(stp[3]), lds_addr(stp[4])};

    constexpr int RS = MF * BK * 2;  // bytes between fragment rows MF apart
    bf16x8_t a0[FR], b0[FC], a1[FR], b1[FC];
    auto read = [&](bf16x8_t (&a)[FR], bf16x8_t (&b)[FC], int stage, int ks) {
        const uint32_t ab = sbase[stage] + aoff[ks], bb = ab + bdelta;
        read_frags<RS>(a, ab, std::make_integer_sequence<int, FR>{});
        read_frags<RS>(b, bb, std::make_integer_sequence<int, FC>{});
    };
    auto mma = [&](bf16x8_t (&a)[FR], bf16x8_t (&b)[FC]) {
#pragma unroll
        for (int i = 0; i < FR; ++i)
#pragma unroll
            for (int j = 0; j < FC; ++j) {
                if constexpr (MF == 32)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
                else
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
            }
    };
    // Step kt: the stage's k-steps alternate between the two fragment sets
    // (the reads of k-step i + 1 in flight while k-step i multiplies); the
    // barrier comes before the last k-step, and the first k-step of tile
    // kt+1 is read behind it.
    auto step = [&](int kt, int cur) {
        const int nxt = cur + 1 == S ? 0 : cur + 1, prv = cur == 0 ? S - 1 : cur - 1;
        read(a1, b1, cur, 1);
        lgkm_wait<FR + FC>(a0, b0);
        mma(a0, b0);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (KS == 4) {
            read(a0, b0, cur, 2);
            lgkm_wait<FR + FC>(a1, b1);
            mma(a1, b1);
            __builtin_amdgcn_sched_barrier(0);
            read(a1, b1, cur, 3);
            lgkm_wait<FR + FC>(a0, b0);
            mma(a0, b0);
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (!kProd) __builtin_amdgcn_s_waitcnt(vmcnt_imm((S - 3) * P));  // tile kt+1 landed
        cta_barrier();
        if constexpr (!kProd) dma(kt + S - 1, prv);
        lgkm_wait<0>(a1, b1);
        if (kt + 1 < nk) read(a0, b0, nxt, 0);
        __builtin_amdgcn_sched_barrier(0);
        mma(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
    };

    // Ping-pong step kt: memory phase (reads of tile kt from stage `cur`,
    // copies of tile kt+S-1 into the stage of tile kt-1), barrier, MFMA
    // phase, barrier.  Before the barrier that follows its memory phase a
    // wave of the first group has issued one tile more than the other waves
    // at that barrier, hence its (S-1)-tile wait.
    const int grp = wave >> 2;
    auto pp_step = [&](int kt, auto cur_c) {
        constexpr int cur = decltype(cur_c)::value, prv = cur == 0 ? S - 1 : cur - 1;
        read(a0, b0, cur, 0);
        if constexpr (KS > 1) read(a1, b1, cur, 1);
        dma(kt + S - 1, prv);
        lgkm_wait<0>(a0, b0);
        if constexpr (KS > 1) lgkm_wait<0>(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        if (grp == 0) vm_wait(W1{});
        else vm_wait(W2{});
        cta_barrier();
        mma(a0, b0);
        if constexpr (KS > 1) mma(a1, b1);
        __builtin_amdgcn_sched_barrier(0);
        vm_wait(W2{});
        cta_barrier();
    };

    if constexpr (!kProd) {
#pragma unroll
        for (int i = 0; i < S - 1; ++i) dma(i, i);
        vm_wait(W2{});
    }
    cta_barrier();
    if constexpr (PP) {
        using I0 = std::integral_constant<int, 0>;
        using I1 = std::integral_constant<int, 1>;
        using I2 = std::integral_constant<int, 2>;
        using I3 = std::integral_constant<int, 3 % S>;
        using I4 = std::integral_constant<int, 4 % S>;
        if (grp == 1) cta_barrier();  // the second group runs one barrier behind
        int kt = 0;
        for (; kt + S <= nk; kt += S) {
            pp_step(kt, I0{});
            pp_step(kt + 1, I1{});
            pp_step(kt + 2, I2{});
            if constexpr (S > 3) pp_step(kt + 3, I3{});
            if constexpr (S > 4) pp_step(kt + 4, I4{});
        }
        if (kt < nk) pp_step(kt, I0{});
        if (kt + 1 < nk) pp_step(kt + 1, I1{});
        if constexpr (S > 3)
            if (kt + 2 < nk) pp_step(kt + 2, I2{});
        if constexpr (S > 4)
            if (kt + 3 < nk) pp_step(kt + 3, I3{});
        if (grp == 0) cta_barrier();  // and the first catches up
    } else {
        read(a0, b0, 0, 0);
        for (int kt = 0; kt < nk; kt += S) {
            step(kt, 0);
            if (kt + 1 < nk) step(kt + 1, 1);
            if (kt + 2 < nk) step(kt + 2, 2);
            if constexpr (S > 3)
                if (kt + 3 < nk) step(kt + 3, 3);
            if constexpr (S > 4)
                if (kt + 4 < nk) step(kt + 4, 4);
        }
    }
    // Drain the ring's trailing (clamped, unused) refills before the LDS is
    // reused by the epilogue.
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));

    const int64_t nb = n0 + wr * C::kWaveM, mb = m0 + wc * C::kWaveN;
    constexpr int REG = 32 * (C::kWaveN + 8), WPS = E / REG;
    static_assert(WPS >= 1 && WPS * S >= C::kWaves, "staging regions must fit in the ring");
    __syncthreads();
    const int sa = wave / WPS;
    uint16_t * region = (sa == 0 ? st0 : sa == 1 ? st1 : sa == 2 ? st2 : sa == 3 ? stp[3] : stp[4]) + (wave % WPS) * REG;
    uint16_t * y = (uint16_t *) p.y;
    switch (epi_kind(p)) {
        case kEpiBias: tile_store_lds<kEpiBias, FR, FC, MF>(p, y, p.res, acc, nb, mb, lane, region); break;
        case kEpiBiasGelu: tile_store_lds<kEpiBiasGelu, FR, FC, MF>(p, y, p.res, acc, nb, mb, lane, region); break;
        case kEpiBiasGated: tile_store_lds<kEpiBiasGated, FR, FC, MF>(p, y, p.res, acc, nb, mb, lane, region); break;
        case kEpiBiasResidual:
            tile_store_lds<kEpiBiasResidual, FR, FC, MF>(p, y, p.res, acc, nb, mb, lane, region);
            break;
        default: tile_store_lds<kEpiBf16, FR, FC, MF>(p, y, p.res, acc, nb, mb, lane, region); break;
    }
}

// ---------------------------------------------------------------------------
// gemm_skinny: N <= 64 tokens (the 48-token action expert), HBM-bound weight
// streaming in two kernels.
//
// gemm_skinny_part: grid = (feature blocks of 128) x (K splits).  The
//   workgroup stages its K slice of the activations (all tokens, bf16) in LDS
//   once, issuing every load of a batch before the first LDS store so the
//   staging costs one memory latency, not one per chunk.  Each of its 8 waves
//   then streams 16 weight rows of the slice from HBM with a 4-step-deep
//   branch-free prefetch, and per 128-column step reads all activation
//   fragments from LDS before feeding MFMA 16x16x32.  Activation bytes per
//   workgroup are 48/128 of its weight bytes.  With one K split the epilogue
//   is applied directly; otherwise fp32 partials go to a workspace.
// gemm_skinny_reduce: sums the K-split partials in split order
//   (deterministic) and applies the epilogue, four outputs per thread with
//   the split loads issued in batches of eight.  The kernel boundary orders
//   the partial writes before the reads; no device-scope fences are needed.
// Inside a 128-wide K step, MFMA chunk c of lane group g covers columns
// 32c + 8g .. +8, so one load instruction reads 64 contiguous bytes of each
// of its 16 weight rows (the activation fragments use the same order).
// ---------------------------------------------------------------------------
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyRows = 32;                            // weight rows per wave (two MFMA groups)
constexpr int kSkinnyFeat = kSkinnyRows * kSkinnyWaves;   // features per workgroup
constexpr int kSkinnyDepth = 2;                            // weight prefetch depth (128-wide steps)
constexpr int kSkinnyMaxKs = 1024;                         // longest K slice (LDS permitting)
constexpr size_t kSkinnyLdsMax = 160 * 1024;

// Stages x[0..N)[kb..kb+klen) as bf16 in LDS rows of ks + 8 elements (rows
// past N and columns past klen are zero).  Addresses are clamped into the
// tensor and the values masked, so every load of a batch is issued before the
// first LDS store.  `prologue` (the weight prefetch) runs after the first
// batch is issued: loads complete in order, so activations queued behind the
// weight stream would wait for it.
template <bool XF32, typename Prologue>
__device__ __forceinline__ void skinny_stage_x(const GemmParams & p, uint16_t * xs, int rows, int ks, int64_t kb,
                                               int klen, Prologue && prologue) {
    const int tid = threadIdx.x, pitch = ks + 8;
    const int cpr = ks / 8, total = rows * cpr;
    constexpr int kStageBatch = 8;
    const int nthr = (int) blockDim.x;
    for (int c0 = 0; c0 < total; c0 += kStageBatch * nthr) {
        uint4 v[kStageBatch];
#pragma unroll
        for (int u = 0; u < kStageBatch; ++u) {
            const int c = min(c0 + u * nthr + tid, total - 1);
            const int r = c / cpr, kc = c % cpr;
            const bool ok = r < p.N && kc * 8 < klen;
            const int64_t idx = (int64_t) min(r, (int) p.N - 1) * p.ldx + kb + min(kc * 8, klen - 8);
            const uint4 x = load_x8<XF32>(p.x, idx);
            v[u] = ok ? x : make_uint4(0, 0, 0, 0);
        }
        if (c0 == 0) prologue();
#pragma unroll
        for (int u = 0; u < kStageBatch; ++u) {
            const int c = c0 + u * nthr + tid;
            if (c < total) *(uint4 *) (xs + (c / cpr) * pitch + (c % cpr) * 8) = v[u];
        }
    }
    __syncthreads();
}

// 16x16 fragments -> fp32 partials of K slice blockIdx.y, or (part ==
// nullptr, a single slice) the epilogue.  Lane holds feature mrow[rg] (column
// lane & 15), register r holds token 16t + 4*(lane/16) + r.
template <int RG, int NT>
__device__ __forceinline__ void skinny_store(const GemmParams & p, float * part, const f32x4_t (&acc)[RG][NT],
                                             const int64_t (&mrow)[RG], const bool (&mok)[RG], int lane) {
    const int64_t N = p.N, M = p.M;
    float * pp = part ? part + (int64_t) blockIdx.y * N * M : nullptr;
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        if (!mok[rg]) continue;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t n = 16 * t + 4 * (lane >> 4) + r;
                if (n >= N) continue;
                if (pp) pp[n * M + mrow[rg]] = acc[rg][t][r];
                else store_out(p, p.y, p.res, n, mrow[rg], acc[rg][t][r]);
            }
    }
}

template <bool XF32, int NT, int DEPTH = kSkinnyDepth>
__global__ __launch_bounds__(kSkinnyWaves * 64) void gemm_skinny_part(GemmParams p, float * part, int ks) {
    constexpr int RG = kSkinnyRows / 16;             // 16-row MFMA groups per wave
    constexpr int LI = kSkinnyRows / 4;              // load instructions per step (4 rows x 256 B each)
    extern __shared__ __align__(16) uint16_t xs[];  // [16*NT][ks + 8], then per-wave weight tiles
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int64_t M = p.M, K = p.K;
    const int pitch = ks + 8;
    const int64_t m0 = (int64_t) blockIdx.x * kSkinnyFeat + (int64_t) wave * kSkinnyRows;
    const int64_t kb = (int64_t) blockIdx.y * ks;
    const int64_t ke = min(K, kb + ks);
    const int klen = (int) (ke - kb);
    // Wave-private weight tile: kSkinnyRows rows x 128 columns, 16-byte chunk j
    // of row r stored at chunk position j ^ (r & 15) (conflict-free row writes
    // and column reads).
    uint16_t * wt = xs + 16 * NT * pitch + wave * (kSkinnyRows * 128);

    // Weight loads, row-coalesced: instruction c of a 128-column step reads
    // rows 4c .. 4c+3 of the wave's rows, 256 contiguous bytes each (16 lanes
    // per row).  Columns past the slice are clamped into it and masked to zero.
    const int lrow = g, lchunk = r16;
    const uint16_t * wbase[LI];
#pragma unroll
    for (int c = 0; c < LI; ++c) wbase[c] = p.w + min(m0 + 4 * c + lrow, M - 1) * p.ldw + kb;
    const int nsteps = (klen + 127) / 128;
    uint4 wbuf[DEPTH][LI];
    // The loads only fill registers; the K-tail mask is applied where the
    // values are consumed (any use of a loaded register right after the load
    // would make the wave wait for it and serialise the prefetch).
    auto wload = [&](int st, uint4 (&d)[LI]) {
        const int k = st * 128 + 8 * lchunk;
        const int kc = k < klen ? k : klen - 8;
#pragma unroll
        for (int c = 0; c < LI; ++c) d[c] = *(const uint4 *) (wbase[c] + kc);
    };
    skinny_stage_x<XF32>(p, xs, 16 * NT, ks, kb, klen, [&]() {
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) wload(min(i, nsteps - 1), wbuf[i]);
    });

    f32x4_t acc[RG][NT];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[rg][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint16_t * xrow = xs + r16 * pitch + 8 * g;
    for (int st0 = 0; st0 < nsteps; st0 += DEPTH) {
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) {
            const int st = st0 + i;
            if (st < nsteps) {
                // registers -> wave tile (row 4c + lrow, chunk lchunk); columns
                // past the slice are zeroed here.
                const uint32_t mask = st * 128 + 8 * lchunk < klen ? 0xffffffffu : 0u;
#pragma unroll
                for (int c = 0; c < LI; ++c) {
                    const int r = 4 * c + lrow;
                    const uint4 v = wbuf[i][c];
                    *(uint4 *) (wt + r * 128 + ((lchunk ^ (r & 15)) << 3)) =
                        make_uint4(v.x & mask, v.y & mask, v.z & mask, v.w & mask);
                }
                // MFMA chunk q: lane holds row r16 of group rg, columns 32q + 8g .. +8
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    bf16x8_t wa[RG], xa[NT];
#pragma unroll
                    for (int rg = 0; rg < RG; ++rg)
                        wa[rg] = *(const bf16x8_t *) (wt + (16 * rg + r16) * 128 + (((4 * q + g) ^ r16) << 3));
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        xa[t] = *(const bf16x8_t *) (xrow + 16 * t * pitch + st * 128 + 32 * q);
#pragma unroll
                    for (int rg = 0; rg < RG; ++rg)
#pragma unroll
                        for (int t = 0; t < NT; ++t)
                            acc[rg][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[t], wa[rg], acc[rg][t], 0, 0, 0);
                }
            }
            // Refilled on every pass (past the end with the last step again, an
            // L2 hit), so every path issues the same loads and the wait before
            // a slot's use counts only the younger slots' loads.
            wload(min(st + DEPTH, nsteps - 1), wbuf[i]);
        }
    }
    int64_t mrow[RG];
    bool mok[RG];
#pragma unroll
    for (int rg = 0; rg < RG; ++rg) {
        mrow[rg] = m0 + 16 * rg + r16;
        mok[rg] = mrow[rg] < M;
    }
    skinny_store<RG, NT>(p, part, acc, mrow, mok, lane);
}

// ---------------------------------------------------------------------------
// MFMA-tiled weights (the tiled buffer type): [M/16][K/32] tiles of 1 KB; in
// tile (gr, q) lane l's 16 bytes are w[16 gr + (l & 15)][32 q + 8 (l >> 4) ..
// +8], which is the B-operand fragment of MFMA 16x16x32 for 16 features and
// 32 k.  One wave load instruction reads one tile (1 KB contiguous) straight
// into MFMA registers; a 16-row group streams along K contiguously.
// ---------------------------------------------------------------------------
__global__ void tile_weights_kernel(const uint16_t * __restrict__ src, uint16_t * __restrict__ dst, int64_t M,
                                    int64_t K, int untile) {
    const int64_t chunk = (int64_t) blockIdx.x * 256 + threadIdx.x;  // 16-byte chunk of the tiled layout
    if (chunk >= M * K / 8) return;
    const int64_t tile = chunk >> 6, kt = K / 32;
    const int l = (int) (chunk & 63);
    const int64_t row = 16 * (tile / kt) + (l & 15), k = 32 * (tile % kt) + 8 * (l >> 4);
    if (untile) *(uint4 *) (dst + row * K + k) = *(const uint4 *) (src + chunk * 8);
    else *(uint4 *) (dst + chunk * 8) = *(const uint4 *) (src + row * K + k);
}

hipError_t launch_tile_weights(const void * src, void * dst, int64_t M, int64_t K, bool untile, hipStream_t s) {
    if (M <= 0 || K <= 0) return hipSuccess;
    if (M % 16 != 0 || K % 32 != 0 || (((uintptr_t) src | (uintptr_t) dst) & 15)) return hipErrorInvalidValue;
    const int64_t chunks = M * K / 8;
    hipLaunchKernelGGL(tile_weights_kernel, dim3((unsigned) ((chunks + 255) / 256)), dim3(256), 0, s,
                       (const uint16_t *) src, (uint16_t *) dst, M, K, untile ? 1 : 0);
    return hipGetLastError();
}

// gemm_skinny_part on tiled weights: each wave of the workgroup owns one
// 16-row group (a workgroup of G waves covers 16 G features, G chosen with the
// K slice so the grid fills the CUs evenly), streams its tiles DEPTH steps
// ahead and feeds them to the MFMAs as loaded, with no LDS on the weight path.
// Within a K slice the accumulation order is that of gemm_skinny_part.
// K % 32 == 0 and M % 16 == 0 (the tiled layout's conditions).
constexpr int kTiledMaxWaves = 16;

template <bool XF32, int NT, int DEPTH = kSkinnyDepth>
__global__ __launch_bounds__(kTiledMaxWaves * 64) void gemm_skinny_tiled(GemmParams p, float * part, int ks) {
    extern __shared__ __align__(16) uint16_t xs[];  // [16*NT][ks + 8]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int64_t M = p.M, K = p.K;
    const int pitch = ks + 8;
    const int64_t ngrp = M / 16, kt = K / 32;
    const int64_t grp = (int64_t) blockIdx.x * (blockDim.x >> 6) + wave;
    const int64_t kb = (int64_t) blockIdx.y * ks;
    const int klen = (int) (min(K, kb + ks) - kb);
    const int nsteps = (klen + 127) / 128, ntiles = klen / 32;
    const uint16_t * wrow = p.w + (min(grp, ngrp - 1) * kt + kb / 32) * 512 + lane * 8;
    uint4 wbuf[DEPTH][4];
    auto wload = [&](int st, uint4 (&d)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) d[q] = *(const uint4 *) (wrow + (int64_t) min(st * 4 + q, ntiles - 1) * 512);
    };
    skinny_stage_x<XF32>(p, xs, 16 * NT, ks, kb, klen, [&]() {
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) wload(min(i, nsteps - 1), wbuf[i]);
    });

    f32x4_t acc[1][NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[0][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    const uint16_t * xrow = xs + r16 * pitch + 8 * g;
    for (int st0 = 0; st0 < nsteps; st0 += DEPTH) {
#pragma unroll
        for (int i = 0; i < DEPTH; ++i) {
            const int st = st0 + i;
            if (st < nsteps) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    if (st * 4 + q >= ntiles) continue;  // K tail: the 32-column chunk is past the slice
                    bf16x8_t xa[NT];
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        xa[t] = *(const bf16x8_t *) (xrow + 16 * t * pitch + st * 128 + 32 * q);
#pragma unroll
                    for (int t = 0; t < NT; ++t)
                        acc[0][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            xa[t], __builtin_bit_cast(bf16x8_t, wbuf[i][q]), acc[0][t], 0, 0, 0);
                }
            }
            wload(min(st + DEPTH, nsteps - 1), wbuf[i]);
        }
    }
    const int64_t mrow[1] = {16 * grp + r16};
    const bool mok[1] = {grp < ngrp};
    skinny_store<1, NT>(p, part, acc, mrow, mok, lane);
}

// LDS bytes of gemm_skinny_part: activation slice + the waves' weight tiles.
static size_t skinny_lds_bytes(int nt, int ks) {
    return (size_t) 16 * nt * (ks + 8) * sizeof(uint16_t) +
           (size_t) kSkinnyWaves * kSkinnyRows * 128 * sizeof(uint16_t);
}

// V outputs per thread (V = 4 needs M % 4 == 0, so the four share a row).
template <int V>
__global__ __launch_bounds__(256) void gemm_skinny_reduce(GemmParams p, const float * __restrict__ part, int splits) {
    typedef __attribute__((__vector_size__(V * sizeof(float)))) float fv_t;
    const int64_t total = p.N * p.M;
    const int64_t i0 = ((int64_t) blockIdx.x * 256 + threadIdx.x) * V;
    if (i0 >= total) return;
    const int64_t n = i0 / p.M, m = i0 % p.M;
    // Epilogue inputs first, so the outputs cost one memory round trip.
    const int ek = epi_kind(p);
    float bias[V] = {}, res[V] = {}, gate[V] = {};
#pragma unroll
    for (int e = 0; e < V; ++e) {
        if (ek >= kEpiBias) bias[e] = bf16_to_f32(p.bias[m + e]);
        if (ek >= kEpiBiasGated) res[e] = bf16_to_f32(p.res[n * p.ldres + m + e]);
        if (ek == kEpiBiasGated) gate[e] = p.gate[m + e];
    }
    fv_t s = *(const fv_t *) (part + i0);
    constexpr int kBatch = 8;
    for (int sp0 = 1; sp0 < splits; sp0 += kBatch) {
        fv_t v[kBatch];
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (sp0 + u < splits) v[u] = *(const fv_t *) (part + (int64_t) (sp0 + u) * total + i0);
#pragma unroll
        for (int u = 0; u < kBatch; ++u)
            if (sp0 + u < splits) s += v[u];
    }
#pragma unroll
    for (int e = 0; e < V; ++e) store_pre(p, p.y, n, m + e, s[e], bias[e], res[e], gate[e]);
}

// ---------------------------------------------------------------------------
// skinny_reduce_row: the split-K reduce of one token row fused with the row op
// that consumes the GEMM output, so a denoise-step projection costs two
// launches (part + this) instead of three.  One workgroup per token (and
// segment); thread c owns 8-column chunk c, which is the chunk layout of the
// standalone row kernels (norm_mod_bf16_vec / qk_norm_rope_vec with one chunk
// per thread), and the row arithmetic is shared with them (rowops.h), so the
// fused and unfused paths give the same bits.  The GEMM output row is written
// as well (16-byte chunks).
//   POST kPostNormAffine / kPostNormModF32 / kPostNormModBf16: LayerNorm of
//     the row (weights, or adaLN modulation in f32 / bf16) into rp.out;
//   POST kPostSegs: up to three segments of rp.width columns, one per
//     workgroup row of the grid, each either RMSNorm + RoPE into a head-major
//     Q/K tensor or a copy into V^T storage.
// ---------------------------------------------------------------------------
enum { kPostNormAffine = 1, kPostNormModF32, kPostNormModBf16, kPostSegs };

// The value store_out_t<E> writes (same rounding points), as f32, for the 8
// outputs m .. m+7 of token row n.
// The epilogue inputs of 8 outputs (bias, residual, gate), loaded ahead of
// the values they combine with.
template <int E>
struct EpiIn {
    float b[8], h[8], g[8];
};
template <int E>
__device__ __forceinline__ void epi_load(const GemmParams & p, int64_t n, int64_t m, EpiIn<E> & in) {
    if constexpr (E != kEpiBf16) unpack8(*(const uint4 *) (p.bias + m), in.b);
    if constexpr (E >= kEpiBiasGated) unpack8(*(const uint4 *) (p.res + n * p.ldres + m), in.h);
    if constexpr (E == kEpiBiasGated) load8_f32(p.gate + m, in.g);
}
template <int E>
__device__ __forceinline__ void epi_apply(const EpiIn<E> & in, const float (&acc)[8], float (&o)[8]) {
    if constexpr (E == kEpiBf16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = round_bf16(acc[e]);
    } else {
        const float(&b)[8] = in.b;
        const float(&h)[8] = in.h;
        const float(&g)[8] = in.g;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float a = round_bf16(acc[e]) + b[e];
            if constexpr (E == kEpiBias) o[e] = round_bf16(a);
            else if constexpr (E == kEpiBiasGelu) o[e] = round_bf16(gelu_tanh(a));
            else if constexpr (E == kEpiBiasGated) o[e] = round_bf16(fmaf(round_bf16(a), g[e], h[e]));
            else o[e] = round_bf16(h[e] + round_bf16(a));
        }
    }
}

// gemm_skinny_wk: few-token product on MFMA-tiled weights with the K split
// over the waves of one workgroup instead of over workgroups, so the output
// (with its epilogue) is written directly: no fp32 partials, no reduce launch.
// For products no row op follows (the action expert's FFN-up + GELU).
//   Workgroup: 8 waves x kWkGroups 16-row groups (64 features); wave w takes
//   k-tiles w, w + 8, w + 16, ... of every group, so at each step the eight
//   waves read eight adjacent 1 KB tiles of a group (25.1 -> 22.1 us on the
//   14336 x 3072 FFN-up against K/32/8 consecutive tiles per wave).  Weight
//   tiles and activation fragments (straight from memory: the 48 x K
//   activations stay in L2) are written as a D-step prefetch; the optimizer
//   folds it into loads a few instructions ahead of their MFMAs, which
//   measured faster than a pinned D-deep schedule of buffer loads.  The
//   waves' accumulators meet in LDS and are summed in wave order
//   (deterministic); one thread per (token, 8 features) applies the epilogue
//   and writes 16 bytes.
constexpr int kWkWaves = 8, kWkGroups = 4, kWkDepth = 4;

template <int NT, int E>
__global__ __launch_bounds__(kWkWaves * 64) void gemm_skinny_wk(GemmParams p) {
    __shared__ __align__(16) float red[kWkWaves][kWkGroups * NT * 4 * 64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 4, r16 = lane & 15;
    const int64_t kt = p.K / 32, grp0 = (int64_t) blockIdx.x * kWkGroups;
    const int ktw = (int) (kt / kWkWaves);
    const int64_t kt0 = wave;
    const uint16_t * wb0 = p.w + (grp0 * kt + kt0) * 512 + lane * 8;
    const uint16_t * x = (const uint16_t *) p.x;
    int64_t xoff[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) xoff[t] = min<int64_t>(16 * t + r16, p.N - 1) * p.ldx + kt0 * 32 + 8 * g;
    uint4 wv[kWkDepth][kWkGroups], xv[kWkDepth][NT];
    auto load = [&](int kk, uint4 (&w)[kWkGroups], uint4 (&xa)[NT]) {
        kk = min(kk, ktw - 1);
#pragma unroll
        for (int rg = 0; rg < kWkGroups; ++rg) w[rg] = *(const uint4 *) (wb0 + ((int64_t) rg * kt + kk * kWkWaves) * 512);
#pragma unroll
        for (int t = 0; t < NT; ++t) xa[t] = *(const uint4 *) (x + xoff[t] + kk * kWkWaves * 32);
    };
#pragma unroll
    for (int i = 0; i < kWkDepth; ++i) load(i, wv[i], xv[i]);
    f32x4_t acc[kWkGroups][NT];
#pragma unroll
    for (int rg = 0; rg < kWkGroups; ++rg)
#pragma unroll
        for (int t = 0; t < NT; ++t) acc[rg][t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int kk0 = 0; kk0 < ktw; kk0 += kWkDepth) {
#pragma unroll
        for (int i = 0; i < kWkDepth; ++i) {
#pragma unroll
            for (int rg = 0; rg < kWkGroups; ++rg)
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    acc[rg][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, xv[i][t]),
                                                                       __builtin_bit_cast(bf16x8_t, wv[i][rg]),
                                                                       acc[rg][t], 0, 0, 0);
            load(kk0 + i + kWkDepth, wv[i], xv[i]);
        }
    }
    // Accumulator lane (g, r16), element v: token 16t + 4g + v, feature
    // 16(grp0 + rg) + r16.  Stored as [rg][t][v][lane] per wave.
    float * my = red[wave];
#pragma unroll
    for (int rg = 0; rg < kWkGroups; ++rg)
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int v = 0; v < 4; ++v) my[((rg * NT + t) * 4 + v) * 64 + lane] = acc[rg][t][v];
    __syncthreads();
    if (tid >= kWkGroups * NT * 4 * 4 * 2) return;
    const int half = tid & 1, gg = (tid >> 1) & 3, v = (tid >> 3) & 3, t = (tid >> 5) % NT, rg = (tid >> 5) / NT;
    const int64_t n = 16 * t + 4 * gg + v, m = 16 * (grp0 + rg) + 8 * half;
    if (n >= p.N) return;
    EpiIn<E> in;
    epi_load<E>(p, n, m, in);
    const int base = ((rg * NT + t) * 4 + v) * 64 + 16 * gg + 8 * half;
    float sum[8];
#pragma unroll
    for (int w = 0; w < kWkWaves; ++w) {
        const float4 a = *(const float4 *) (red[w] + base), b = *(const float4 *) (red[w] + base + 4);
        const float r[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) sum[e] = w == 0 ? r[e] : sum[e] + r[e];
    }
    float o[8];
    epi_apply<E>(in, sum, o);
    *(uint4 *) ((uint16_t *) p.y + n * p.ldy + m) = pack8(o);
}

// Device copy of the row op (RowPost with the RoPE scales precomputed).
struct RowSegDev {
    int32_t kind, rope_mode;
    int64_t col, dst_tokens, tok0, vt_ld, vt_hs, chunk_tokens, chunk_stride;
    int32_t vt_tok;  // V^T segment: tokens per workgroup (1, or kVtTok when its stores can be 16-byte runs)
    const uint16_t * w;
    uint16_t * dst;
    const int32_t *pos0, *pos1, *pos2;
    float eps, l2ts128, l2ts44, l2ts42;
};
struct RowPostDev {
    const void * scale;
    const void * shift;
    int64_t ss, ldo;
    uint16_t * out;
    float eps;
    int32_t width, head_dim;
    RowSegDev seg[3];
};

// A V^T segment with vt_tok == kVtTok runs kVtTok tokens x (width / kVtTok)
// columns per workgroup instead of one token row: each thread reduces the
// same (token, 8-column chunk) as in the one-row form, the values meet in
// LDS, and each thread then stores one column's kVtTok consecutive tokens
// as one 16-byte run of V^T, where the one-row form stores 8 scattered
// 2-byte values per thread.
constexpr int kVtTok = 8;

template <int E, int POST>
__global__ __launch_bounds__(512) void skinny_reduce_row(GemmParams p, const float * __restrict__ part, int splits,
                                                         RowPostDev rp) {
    __shared__ float red[16];
    const RowSegDev & sg = rp.seg[POST == kPostSegs ? blockIdx.y : 0];
    const bool vt_block = POST == kPostSegs && sg.kind == kRowSegVt && sg.vt_tok == kVtTok;  // workgroup-uniform
    const int cpb = (int) blockDim.x / kVtTok;  // chunks per column block of a V^T block
    const int64_t n = vt_block ? (int64_t) (blockIdx.x / kVtTok) * kVtTok + threadIdx.x / cpb : (int64_t) blockIdx.x;
    const int c = vt_block ? (int) (blockIdx.x % kVtTok) * cpb + (int) threadIdx.x % cpb : (int) threadIdx.x;
    const int64_t NM = p.N * p.M;
    const int64_t m = (POST == kPostSegs ? sg.col : 0) + 8 * c;
    const float * src = part + n * p.M + m;
    // The row op's and the epilogue's inputs are requested first, then every
    // split (in batches of kB), so the row costs one memory round trip; the
    // sums run in split order, as in gemm_skinny_reduce.
    EpiIn<E> ein;
    epi_load<E>(p, n, m, ein);
    constexpr bool kNorm = POST != kPostSegs;
    constexpr bool kAffine = POST == kPostNormAffine, kSsBf16 = POST != kPostNormModF32;
    float a[8], b[8];
    uint4 wv = make_uint4(0, 0, 0, 0);
    RopeTok rt{};
    if constexpr (kNorm) {
        const int64_t so = n * rp.ss + 8 * c;
        if constexpr (kSsBf16) {
            unpack8(*(const uint4 *) ((const uint16_t *) rp.scale + so), a);
            unpack8(*(const uint4 *) ((const uint16_t *) rp.shift + so), b);
        } else {
            load8_f32((const float *) rp.scale + so, a);
            load8_f32((const float *) rp.shift + so, b);
        }
    }
    // Chunk of row n and its token within the chunk (segment stores).
    const int64_t cb = POST == kPostSegs ? n / sg.chunk_tokens : 0, tl = n - cb * (POST == kPostSegs ? sg.chunk_tokens : 0);
    if constexpr (!kNorm) {
        if (sg.kind == kRowSegQk) {
            wv = *(const uint4 *) (sg.w + 8 * c);
            rt = rope_tok(sg.rope_mode, sg.pos0, sg.pos1, sg.pos2, tl, sg.l2ts128, sg.l2ts44, sg.l2ts42);
        }
    }
    constexpr int kB = 20;
    float acc[8];
    for (int sp0 = 0; sp0 < splits; sp0 += kB) {
        float t[kB][8];
#pragma unroll
        for (int u = 0; u < kB; ++u)
            if (sp0 + u < splits) load8_f32(src + (int64_t) (sp0 + u) * NM, t[u]);
#pragma unroll
        for (int u = 0; u < kB; ++u)
            if (sp0 + u < splits)
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[e] = sp0 + u == 0 ? t[u][e] : acc[e] + t[u][e];
    }
    float v[1][8];
    epi_apply<E>(ein, acc, v[0]);
    *(uint4 *) ((uint16_t *) p.y + n * p.ldy + m) = pack8(v[0]);

    if constexpr (kNorm) {
        float mean, inv_std;
        row_mean_istd<1>(v, (int) blockDim.x, (int) p.M, rp.eps, red, mean, inv_std);
        *(uint4 *) (rp.out + n * rp.ldo + 8 * c) = norm_chunk<kAffine>(v[0], mean, inv_std, a, b);
    } else {
        const int hd = rp.head_dim, e0 = 8 * c, h = e0 / hd, dd0 = e0 % hd;
        if (sg.kind == kRowSegQk) {
            const float inv_rms = row_inv_rms<1>(v, rp.width, sg.eps, red);
            *(uint4 *) (sg.dst + cb * sg.chunk_stride + ((int64_t) h * sg.dst_tokens + sg.tok0 + tl) * hd + dd0) =
                qk_chunk(v[0], inv_rms, wv, dd0, rt);
        } else if (vt_block) {
            // v holds bf16 values (the epilogue rounds), so the packing below
            // stores the bits the one-row form stores.
            __shared__ __align__(16) uint16_t vtile[kVtTok * 512];
            const int row = (int) threadIdx.x / cpb, k = (int) threadIdx.x % cpb, bw = (int) blockDim.x;
            *(uint4 *) (vtile + row * bw + 8 * k) = pack8(v[0]);
            __syncthreads();
            const int f = (int) (blockIdx.x % kVtTok) * bw + (int) threadIdx.x;  // column of the segment
            const int64_t n0 = (int64_t) (blockIdx.x / kVtTok) * kVtTok;
            const int64_t cb0 = n0 / sg.chunk_tokens, tl0 = n0 - cb0 * sg.chunk_tokens;
            uint32_t w[kVtTok / 2];
#pragma unroll
            for (int j = 0; j < kVtTok / 2; ++j)
                w[j] = (uint32_t) vtile[(2 * j) * bw + threadIdx.x] | ((uint32_t) vtile[(2 * j + 1) * bw + threadIdx.x] << 16);
            *(uint4 *) (sg.dst + cb0 * sg.chunk_stride + (int64_t) (f / hd) * sg.vt_hs + (int64_t) (f % hd) * sg.vt_ld +
                        sg.tok0 + tl0) = make_uint4(w[0], w[1], w[2], w[3]);
        } else {
            uint16_t * d = sg.dst + cb * sg.chunk_stride + (int64_t) h * sg.vt_hs + sg.tok0 + tl;
#pragma unroll
            for (int e = 0; e < 8; ++e) d[(int64_t) (dd0 + e) * sg.vt_ld] = f32_to_bf16(v[0][e]);
        }
    }
}

// K split of the skinny path, from a small cost model (microseconds): the
// slowest CU streams ceil(workgroups / 256) slices of kSkinnyFeat x ks
// weights at its 1/256 share of 8 TB/s, plus a ramp per workgroup (one
// workgroup per CU is resident: 8 waves of ~155 VGPRs); a split adds the fp32
// partials (written and read once) and the reduce launch.  Measured on the
// 48-token shapes this picks the fastest slice of the sweep for each.
static void skinny_plan(int64_t M, int64_t N, int64_t K, int & splits, int & ks) {
    const int64_t nfb = (M + kSkinnyFeat - 1) / kSkinnyFeat;
    const int64_t nt = (N + 15) / 16;
    double best = 1e30;
    splits = (int) ((K + 127) / 128);
    ks = 128;
    for (int k = 128; k <= kSkinnyMaxKs; k += 128) {
        const int64_t s = (K + k - 1) / k;
        if (s > 1 && (int64_t) k * (s - 1) >= K) continue;
        const size_t lds = skinny_lds_bytes((int) nt, k);
        if (lds > kSkinnyLdsMax) break;
        const int64_t wgs = nfb * s;
        const int64_t per_cu = (wgs + 255) / 256;
        double t = per_cu * ((double) kSkinnyFeat * std::min<int64_t>(k, K) * 2 / 31.25e3 + 1.5);
        if (s > 1) t += (double) s * N * M * 4 * 2 / 8e6 + 3.0;
        if (t < best) {
            best = t;
            splits = (int) s;
            ks = k;
        }
        if (k >= K) break;
    }
}

size_t skinny_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    int splits, ks;
    skinny_plan(M, N, K, splits, ks);
    return splits > 1 ? (size_t) splits * N * M * sizeof(float) : 0;
}

static int64_t tiles_of(const GemmParams & p, int bm, int bn);
static int dma_splitk_plan(const GemmParams & p, size_t ws_bytes);

// The K split launch_gemm takes for a plain product with row-major weights:
// the skinny plan up to 64 tokens, else the K-sliced 128 x 128 GEMM that
// dispatch_dma runs for bf16 activations on grids too small for the 256 /
// 192 tiles (whose slice count depends on the workspace size).
size_t linear_split_bytes(int64_t M, int64_t N, int64_t K, int32_t x_type, size_t ws_bytes) {
    if (M <= 0 || N <= 0 || K <= 0) return 0;
    if (N <= 64) return skinny_workspace_bytes(M, N, K);
    GemmParams p{};
    p.M = M;
    p.N = N;
    p.K = K;
    if (x_type != WAMX_TYPE_BF16 || K % 64 != 0 || tiles_of(p, 256, 256) >= 256 || tiles_of(p, 192, 192) >= 192)
        return 0;
    const int splits = dma_splitk_plan(p, ws_bytes);
    return splits > 1 ? (size_t) splits * N * M * sizeof(float) : 0;
}

// gemm_skinny_part over `splits` K slices of ks columns; part == nullptr
// (single slice only) applies the epilogue in the part kernel.
// Workgroup shape of the tiled kernel: G waves (16 G features) by a K slice
// of ks columns.  Measured on the action expert's projections (48 and 1
// tokens, part + reduce, weights streamed from HBM) over G = 4..12 and ks =
// 256..1536:
//   * one workgroup per CU (grid <= 256) of many waves beats two or more
//     smaller ones per CU, and a grid that leaves CUs idle or uneven costs
//     less than a longer slice;
//   * a wave's time grows with its slice (16 ks bf16 per step), the reduce's
//     with the partials (splits x M);
// so the plan takes the smallest G that fits the grid in `rounds` x 256
// workgroups for each slice, scores ks + 64 splits M / 3072, and widens the
// grid (rounds) only when no G <= 12 fits.  Chosen: 3072 x 3072 G6/384,
// QKV 9216 x 3072 G9/768, FFN-up 14336 x 3072 G11/1024, FFN-down
// 3072 x 14336 G12/896 (each within 0.1-0.7 us of the sweep's best).
// A one-token product (the state token) runs beside the visual tokens'
// kernels on the second stream; its rounds are of 64 workgroups, so it
// takes a quarter of the CUs and delays fewer of the other stream's
// one-round kernels (whole action chunk 83.40 against 83.60 ms at rounds of
// 256; 32 and 16 were slower than 64).
static void skinny_tiled_plan(int64_t M, int64_t N, int64_t K, int & splits, int & ks, int & waves) {
    const int64_t cap = N == 1 ? 64 : 256;
    const int64_t ngrp = M / 16;
    const int nt = (int) ((N + 15) / 16);
    const int64_t kwhole = (K + 127) / 128 * 128;  // one slice over all of K
    splits = (int) ((K + 383) / 384);
    ks = 384;
    waves = kSkinnyWaves;
    // Slices of 384..1536 columns, or all of a shorter K in one.  One always
    // fits the LDS (a 16 x 64-token activation slice of 384 columns is 49 KB),
    // and with G = 4 every grid fits some number of rounds, so the search
    // ends; the bound on rounds is a guard.
    for (int64_t rounds = 1; rounds <= (int64_t) 1 << 30; rounds *= 2) {
        double best = 1e30;
        for (int64_t c = 128; c <= 1536; c += 128) {
            const int64_t s = (K + c - 1) / c;
            if (s == 1 ? c != kwhole : c < 384) continue;
            if ((size_t) 16 * nt * (c + 8) * sizeof(uint16_t) > kSkinnyLdsMax) continue;
            int G = (int) std::min<int64_t>(4, std::max<int64_t>(1, ngrp));
            while (G <= 12 && (ngrp + G - 1) / G * s > cap * rounds) ++G;
            if (G > 12) continue;
            const double score = (double) c + 64.0 * (double) s * (double) M / 3072.0;
            if (score < best) {
                best = score;
                splits = (int) s;
                ks = (int) c;
                waves = G;
            }
        }
        if (best < 1e30) return;
    }
}

static void skinny_plan_for(const GemmParams & p, bool tiled, int & splits, int & ks, int & waves) {
    waves = kSkinnyWaves;
    if (tiled) skinny_tiled_plan(p.M, p.N, p.K, splits, ks, waves);
    else skinny_plan(p.M, p.N, p.K, splits, ks);
}

// gemm_skinny_part (or gemm_skinny_tiled) over `splits` K slices of ks
// columns; part == nullptr (single slice only) applies the epilogue in the
// part kernel.
static void launch_skinny_part(const GemmParams & p, bool xf32, bool tiled, float * part, int splits, int ks,
                               int waves, hipStream_t s) {
    const int nt = (int) ((p.N + 15) / 16);
    const dim3 block(kSkinnyWaves * 64);
    if (tiled) {
        const size_t lds = (size_t) 16 * nt * (ks + 8) * sizeof(uint16_t);
        const dim3 grid((unsigned) ((p.M / 16 + waves - 1) / waves), (unsigned) splits), tblock((unsigned) (64 * waves));
#define WAMX_TILED(XF, NT) hipLaunchKernelGGL((gemm_skinny_tiled<XF, NT>), grid, tblock, lds, s, p, part, ks)
        switch (nt) {
            case 1: if (xf32) WAMX_TILED(true, 1); else WAMX_TILED(false, 1); break;
            case 2: if (xf32) WAMX_TILED(true, 2); else WAMX_TILED(false, 2); break;
            case 3: if (xf32) WAMX_TILED(true, 3); else WAMX_TILED(false, 3); break;
            default: if (xf32) WAMX_TILED(true, 4); else WAMX_TILED(false, 4); break;
        }
#undef WAMX_TILED
        return;
    }
    const size_t lds = skinny_lds_bytes(nt, ks);
    const dim3 grid((unsigned) ((p.M + kSkinnyFeat - 1) / kSkinnyFeat), (unsigned) splits);
#define WAMX_SKINNY(XF, NT) hipLaunchKernelGGL((gemm_skinny_part<XF, NT>), grid, block, lds, s, p, part, ks)
    switch (nt) {
        case 1: if (xf32) WAMX_SKINNY(true, 1); else WAMX_SKINNY(false, 1); break;
        case 2: if (xf32) WAMX_SKINNY(true, 2); else WAMX_SKINNY(false, 2); break;
        case 3: if (xf32) WAMX_SKINNY(true, 3); else WAMX_SKINNY(false, 3); break;
        default: if (xf32) WAMX_SKINNY(true, 4); else WAMX_SKINNY(false, 4); break;
    }
#undef WAMX_SKINNY
}

// WAMX_DISABLE_SKINNY_WK=1 keeps the split-K path for these products (read at
// every launch, so one process can compare the two).
static bool skinny_wk_enabled() {
    const char * e = getenv("WAMX_DISABLE_SKINNY_WK");
    return !(e && e[0] && e[0] != '0');
}

// Whether gemm_skinny_wk takes the product: tiled weights, bf16 activations
// and output with the vector epilogue, 64-feature groups filling most of the
// CUs, and whole k-tile steps per wave.
static bool skinny_wk_ok(const GemmParams & p, bool xf32, bool tiled) {
    const int64_t kt = p.K / 32;
    return tiled && !xf32 && p.vec_out && epi_kind(p) != kEpiF32 && p.N <= 64 && p.M % (16 * kWkGroups) == 0 &&
           p.M / (16 * kWkGroups) >= 192 && p.K % 32 == 0 && kt % kWkWaves == 0 && (kt / kWkWaves) % kWkDepth == 0;
}

template <int NT>
static void launch_skinny_wk(const GemmParams & p, hipStream_t s) {
    const dim3 grid((unsigned) (p.M / (16 * kWkGroups))), block(kWkWaves * 64);
    switch (epi_kind(p)) {
        case kEpiBias: hipLaunchKernelGGL((gemm_skinny_wk<NT, kEpiBias>), grid, block, 0, s, p); break;
        case kEpiBiasGelu: hipLaunchKernelGGL((gemm_skinny_wk<NT, kEpiBiasGelu>), grid, block, 0, s, p); break;
        case kEpiBiasGated: hipLaunchKernelGGL((gemm_skinny_wk<NT, kEpiBiasGated>), grid, block, 0, s, p); break;
        case kEpiBiasResidual: hipLaunchKernelGGL((gemm_skinny_wk<NT, kEpiBiasResidual>), grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL((gemm_skinny_wk<NT, kEpiBf16>), grid, block, 0, s, p); break;
    }
}

static hipError_t run_skinny(const GemmParams & p, bool xf32, bool tiled, void * ws, size_t ws_bytes, hipStream_t s) {
    if (skinny_wk_ok(p, xf32, tiled) && skinny_wk_enabled()) {
        switch ((p.N + 15) / 16) {
            case 1: launch_skinny_wk<1>(p, s); break;
            case 2: launch_skinny_wk<2>(p, s); break;
            case 3: launch_skinny_wk<3>(p, s); break;
            default: launch_skinny_wk<4>(p, s); break;
        }
        return hipGetLastError();
    }
    int splits, ks, waves;
    skinny_plan_for(p, tiled, splits, ks, waves);
    if (splits > 1 && (!ws || (size_t) splits * p.N * p.M * sizeof(float) > ws_bytes || ((uintptr_t) ws & 15)))
        return hipErrorInvalidValue;
    float * part = splits > 1 ? (float *) ws : nullptr;
    launch_skinny_part(p, xf32, tiled, part, splits, ks, waves, s);
    if (splits > 1) {
        const int64_t total = p.N * p.M;
        if (p.M % 4 == 0)
            hipLaunchKernelGGL(gemm_skinny_reduce<4>, dim3((unsigned) ((total / 4 + 255) / 256)), dim3(256), 0, s, p,
                               (const float *) part, splits);
        else
            hipLaunchKernelGGL(gemm_skinny_reduce<1>, dim3((unsigned) ((total + 255) / 256)), dim3(256), 0, s, p,
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

template <int BM, int BN, int WM, int WN, bool XF32, bool VEC>
static hipError_t run_tile(const GemmParams & p, int64_t batches, hipStream_t s) {
    using C = TileCfg<BM, BN, WM, WN>;
    static bool once = (allow_lds(gemm_tile<BM, BN, WM, WN, XF32, VEC>, C::kLds), true);
    (void) once;
    const int nt_m = (int) ((p.M + BN - 1) / BN), nt_n = (int) ((p.N + BM - 1) / BM);
    dim3 grid((unsigned) (nt_m * nt_n), 1, (unsigned) batches);
    hipLaunchKernelGGL((gemm_tile<BM, BN, WM, WN, XF32, VEC>), grid, dim3(C::kThreads), C::kLds, s, p, nt_m, nt_n);
    return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int BK, int S>
static hipError_t run_dma(const GemmParams & p, hipStream_t s) {
    constexpr int occ = dma_occupancy<BM, BN, WM, WN, BK, S>();
    const int nt_m = (int) ((p.M + BN - 1) / BN), nt_n = (int) ((p.N + BM - 1) / BM);
    hipLaunchKernelGGL((gemm_dma<BM, BN, WM, WN, BK, S, occ>), dim3((unsigned) (nt_m * nt_n)), dim3(64 * WM * WN), 0, s,
                       p, nt_m, nt_n);
    return hipGetLastError();
}
// The pipelined kernel addresses its copies by 32-bit offsets and stores bf16
// rows in 16-byte chunks.
static bool pipe_ok(const GemmParams & p) {
    return p.vec_out && (uint64_t) p.N * p.ldx * 2 < (1ull << 32) && (uint64_t) p.M * p.ldw * 2 < (1ull << 32);
}
template <int BM, int BN, int WM, int WN, int S, int SCHED, int BKP, int MF = 32>
static hipError_t launch_dma_pipe(const GemmParams & p, hipStream_t s) {
    const int nt_m = (int) ((p.M + BN - 1) / BN), nt_n = (int) ((p.N + BM - 1) / BM);
    const int threads = 64 * WM * WN * (SCHED == kSchedProducer ? 2 : 1);
    hipLaunchKernelGGL((gemm_dma_pipe<BM, BN, WM, WN, S, SCHED, BKP, MF>), dim3((unsigned) (nt_m * nt_n)),
                       dim3(threads), 0, s, p, nt_m, nt_n);
    return hipGetLastError();
}
// The pipelined form (K steps of BKP) where pipe_ok, else gemm_dma.
template <int BM, int BN, int WM, int WN, int S, int BKF, int SF, int SCHED = kSchedSingle, int BKP = 32>
static hipError_t run_dma_pipe(const GemmParams & p, hipStream_t s) {
    if (!pipe_ok(p)) return run_dma<BM, BN, WM, WN, BKF, SF>(p, s);
    return launch_dma_pipe<BM, BN, WM, WN, S, SCHED, BKP>(p, s);
}

static int64_t tiles_of(const GemmParams & p, int bm, int bn) { return ((p.N + bm - 1) / bm) * ((p.M + bn - 1) / bn); }

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

// Split-K for the 128 x 128 tiles (two workgroups per CU) when the tiles
// alone fill few of the CUs' slots: 384 tokens (eight 48-token chunks) x 3072
// features makes 72 tiles for 512 slots.  Returns the number of K slices (1:
// no split): the divisor s of K/64 that fills the slots best, if that beats
// the unsplit grid by a fifth of the slots, with at least 4 k-steps per slice
// and the s f32 partial planes within the workspace.  A grid that already
// fills half the slots is not split: the partial planes and their reduce cost
// more than the fill gains (384 x 14336 x 3072 with bias + GELU: 63 us
// unsplit against 71 us in 3 slices; 3072 x 3072 at 14% fill: 26 us in 6
// slices against 52 us unsplit).
static int dma_splitk_plan(const GemmParams & p, size_t ws_bytes) {
    const int64_t tiles = tiles_of(p, 128, 128), slots = 2 * (int64_t) device_cus(), kb = p.K / 64;
    if (slots <= 0 || 2 * tiles >= slots || p.K % 64 != 0) return 1;
    auto fill = [&](int64_t sp) {
        const int64_t w = tiles * sp;
        return (double) w / (double) (slots * ((w + slots - 1) / slots));
    };
    int best = 1;
    double best_fill = fill(1);
    for (int sp = 2; sp <= 16; ++sp) {
        if (kb % sp != 0 || kb / sp < 4 || (size_t) sp * p.N * p.M * sizeof(float) > ws_bytes) continue;
        const double f = fill(sp);
        if (f > best_fill + 0.2 * (best == 1) && f > best_fill) {
            best = sp;
            best_fill = f;
        }
    }
    return best;
}

// K split over blockIdx.y of gemm_dma<128, 128>: slice z multiplies K columns
// [z*K/s, (z+1)*K/s) into f32 partial plane z of ws, then gemm_skinny_reduce
// sums the planes in slice order (deterministic) and applies the epilogue.
static void launch_dma_splitk_parts(const GemmParams & p, int splits, void * ws, hipStream_t s) {
    GemmParams q = p;
    const int64_t ks = p.K / splits;
    q.K = ks;
    q.x_bs2 = ks;
    q.w_bs2 = ks;
    q.y = ws;
    q.y_type = WAMX_TYPE_F32;
    q.ldy = p.M;
    q.y_bs2 = p.N * p.M;
    q.epi = WAMX_EPI_NONE;
    q.vec_out = 0;
    const int nt_m = (int) ((p.M + 127) / 128), nt_n = (int) ((p.N + 127) / 128);
    constexpr int occ = dma_occupancy<128, 128, 2, 2, 64, 2>();
    hipLaunchKernelGGL((gemm_dma<128, 128, 2, 2, 64, 2, occ>), dim3((unsigned) (nt_m * nt_n), (unsigned) splits),
                       dim3(256), 0, s, q, nt_m, nt_n);
}
static hipError_t run_dma_splitk(const GemmParams & p, int splits, void * ws, hipStream_t s) {
    launch_dma_splitk_parts(p, splits, ws, s);
    const int64_t total = p.N * p.M;
    if (p.M % 4 == 0)
        hipLaunchKernelGGL(gemm_skinny_reduce<4>, dim3((unsigned) ((total / 4 + 255) / 256)), dim3(256), 0, s, p,
                           (const float *) ws, splits);
    else
        hipLaunchKernelGGL(gemm_skinny_reduce<1>, dim3((unsigned) ((total + 255) / 256)), dim3(256), 0, s, p,
                           (const float *) ws, splits);
    return hipGetLastError();
}

// Tile shape of the bf16 x bf16 DMA path, chosen so the grid fills the 256 CUs
// (measured on the 3072-token products of the prefix pass):
//  * 256 x 256, 8 waves: when it gives at least one tile per CU, ping-pong
//    with BK 32 and 4 stages (6-9% faster than the single-group schedule);
//    256 x 224 with 16x16 fragments instead where its whole rounds finish
//    sooner (prefer_tile224: FFN-up 14336 x 3072 in 768 tiles, 3 rounds,
//    against 672; QKV 9216 x 3072 in 504 against 432), same bits;
//  * 192 x 192, 4 waves: 3072 x 3072 products, which it cuts into exactly 256
//    tiles (256 x 256 leaves 112 CUs idle), pipelined with BK 64 and 3
//    stages, copies issued by 4 producer waves (2-4% faster on O and
//    FFN-down than without them);
//  (f32 or unaligned outputs take gemm_dma with BK 32 / 64 and 3 stages);
//  * 128 x 128, BK 64, 2 stages, 4 waves, two workgroups per CU: small grids
//    (512-token prompt projections).
// Returns false when the shape does not meet the path's preconditions.
static bool tile224_enabled() {
    static const bool on = [] {
        const char * e = getenv("WAMX_DISABLE_TILE224");
        return !(e && e[0] && e[0] != '0');
    }();
    return on;
}

// Whether 256 x 224 tiles (16x16 fragments) finish the grid sooner than 256 x
// 256 ones: a 224-wide tile is 7/8 of the work, so it wins when its rounds of
// one tile per CU, weighted by that, come to fewer than the 256-wide rounds.
static bool prefer_tile224(const GemmParams & p) {
    const int64_t cus = device_cus();
    if (cus <= 0 || !tile224_enabled()) return false;
    const int64_t r256 = (tiles_of(p, 256, 256) + cus - 1) / cus, r224 = (tiles_of(p, 256, 224) + cus - 1) / cus;
    return 7 * r224 < 8 * r256;
}

static bool dispatch_dma(const GemmParams & p, void * ws, size_t ws_bytes, hipStream_t s, hipError_t & err) {
    if (p.K % 32 != 0) return false;
    if (tiles_of(p, 256, 256) >= 256) {
        // 256 x 224: FFN-up (14336 features x 3072 tokens) takes 768 tiles,
        // three whole rounds of 256 CUs, where 256 x 256 leaves 672 (2.6).
        if (pipe_ok(p) && prefer_tile224(p))
            err = launch_dma_pipe<256, 224, 4, 2, 4, kSchedPingPong, 32, 16>(p, s);
        else
            err = run_dma_pipe<256, 256, 4, 2, 4, 32, 3, kSchedPingPong>(p, s);
        return true;
    }
    if (p.K % 64 != 0) return false;
    if (tiles_of(p, 192, 192) >= 192) {
        // K steps of 64 in a 3-stage ring (144 KB): half the barriers and
        // waits per K of the 4-stage BK 32 ring, same bits.  3072^2 55.6
        // against 64.0 us, FFN-down (K 14336) 234 against 280.
        err = run_dma_pipe<192, 192, 2, 2, 3, 64, 3, kSchedProducer, 64>(p, s);
        return true;
    }
    const int splits = ws && ((uintptr_t) ws & 15) == 0 ? dma_splitk_plan(p, ws_bytes) : 1;
    err = splits > 1 ? run_dma_splitk(p, splits, ws, s) : run_dma<128, 128, 2, 2, 64, 2>(p, s);
    return true;
}

static GemmParams make_params(const GemmArgs & a) {
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
    p.vec_out = epi_kind(p) != kEpiF32 && a.M % 8 == 0 && a.ldy % 8 == 0 && aligned16(a.y) && aligned16(a.bias) &&
                aligned16(a.gate) && aligned16(a.res) && (a.res == nullptr || a.ldres % 8 == 0);
    return p;
}

static bool vec_operands(const GemmArgs & a) {
    return a.K % 8 == 0 && a.ldw % 8 == 0 && a.ldx % 8 == 0 && aligned16(a.w) && aligned16(a.x) && a.w_bs2 % 8 == 0 &&
           a.w_bs3 % 8 == 0 && a.x_bs2 % 8 == 0 && a.x_bs3 % 8 == 0;
}

static void allow_skinny_lds() {
    // The activation slice and the weight tiles may use all 160 KB of LDS.
    constexpr size_t kMaxLds = kSkinnyLdsMax;
    static bool once = (allow_lds(gemm_skinny_part<true, 1>, kMaxLds), allow_lds(gemm_skinny_part<false, 1>, kMaxLds),
                        allow_lds(gemm_skinny_part<true, 2>, kMaxLds), allow_lds(gemm_skinny_part<false, 2>, kMaxLds),
                        allow_lds(gemm_skinny_part<true, 3>, kMaxLds), allow_lds(gemm_skinny_part<false, 3>, kMaxLds),
                        allow_lds(gemm_skinny_part<true, 4>, kMaxLds), allow_lds(gemm_skinny_part<false, 4>, kMaxLds),
                        allow_lds(gemm_skinny_tiled<true, 1>, kMaxLds), allow_lds(gemm_skinny_tiled<false, 1>, kMaxLds),
                        allow_lds(gemm_skinny_tiled<true, 2>, kMaxLds), allow_lds(gemm_skinny_tiled<false, 2>, kMaxLds),
                        allow_lds(gemm_skinny_tiled<true, 3>, kMaxLds), allow_lds(gemm_skinny_tiled<false, 3>, kMaxLds),
                        allow_lds(gemm_skinny_tiled<true, 4>, kMaxLds), allow_lds(gemm_skinny_tiled<false, 4>, kMaxLds),
                        true);
    (void) once;
}

// RoPE section scales as launch_qk_norm_rope computes them (host log2f).
static void rope_scales(int64_t head_dim, float base, float & l128, float & l44, float & l42) {
    l128 = -2.0f / (float) head_dim * log2f(base);
    l44 = -2.0f / 44.0f * log2f(base);
    l42 = -2.0f / 42.0f * log2f(base);
}

hipError_t launch_gemm_rowpost(const GemmArgs & a, const RowPost & post, hipStream_t s) {
    const GemmParams p = make_params(a);
    const int E = epi_kind(p);
    if (a.w_type != WAMX_TYPE_BF16 || (a.x_type != WAMX_TYPE_BF16 && a.x_type != WAMX_TYPE_F32) ||
        a.y_type != WAMX_TYPE_BF16 || a.B2 * a.B3 != 1 || a.N <= 0 || a.M <= 0 || a.K <= 0 || !vec_operands(a) ||
        !p.vec_out || E == kEpiF32 || !a.ws || !aligned16(a.ws))
        return hipErrorNotSupported;
    if (a.w_tiled && (p.M % 16 != 0 || p.K % 32 != 0)) return hipErrorNotSupported;
    // More than 64 tokens: only the products that dispatch_dma runs as the
    // K-sliced 128 x 128 GEMM (its partial planes are the reduce's layout).
    const bool dma = a.N > 64;
    int splits = 1, ks = 0, waves = 0;
    if (dma) {
        if (a.w_tiled || a.x_type != WAMX_TYPE_BF16 || p.K % 64 != 0 || tiles_of(p, 256, 256) >= 256 ||
            tiles_of(p, 192, 192) >= 192)
            return hipErrorNotSupported;
        splits = dma_splitk_plan(p, a.ws_bytes);
        if (splits <= 1) return hipErrorNotSupported;
    } else {
        skinny_plan_for(p, a.w_tiled, splits, ks, waves);
    }
    if ((size_t) splits * p.N * p.M * sizeof(float) > a.ws_bytes) return hipErrorNotSupported;

    // The row op: one thread per 8-column chunk, the whole row (or segment)
    // in one workgroup whose size is a multiple of the wave.
    RowPostDev d{};
    int post_kind, nseg = 1;
    int64_t nchunk;
    if (post.kind == kRowPostNorm) {
        const int es = (post.affine || post.ss_type == WAMX_TYPE_BF16) ? 2 : 4;
        if (!post.out || post.ldo % 8 != 0 || !aligned16(post.out) || !aligned16(post.scale) || !aligned16(post.shift) ||
            (post.ss * es) % 16 != 0)
            return hipErrorNotSupported;
        post_kind = post.affine ? kPostNormAffine : post.ss_type == WAMX_TYPE_BF16 ? kPostNormModBf16 : kPostNormModF32;
        nchunk = p.M / 8;
        d.scale = post.scale;
        d.shift = post.shift;
        d.ss = post.ss;
        d.out = (uint16_t *) post.out;
        d.ldo = post.ldo;
        d.eps = post.eps;
    } else if (post.kind == kRowPostSegs) {
        if (post.nseg < 1 || post.nseg > 3 || post.head_dim <= 0 || post.head_dim % 8 != 0 || post.width <= 0 ||
            post.width % post.head_dim != 0)
            return hipErrorNotSupported;
        if (E != kEpiBf16 && E != kEpiBias) return hipErrorNotSupported;
        post_kind = kPostSegs;
        nseg = post.nseg;
        nchunk = post.width / 8;
        d.width = (int32_t) post.width;
        d.head_dim = (int32_t) post.head_dim;
        for (int i = 0; i < nseg; ++i) {
            const RowSeg & g = post.seg[i];
            RowSegDev & o = d.seg[i];
            if (g.col < 0 || g.col % 8 != 0 || g.col + post.width > p.M || !g.dst) return hipErrorNotSupported;
            if (g.kind == kRowSegQk) {
                if (!aligned16(g.w) || !aligned16(g.dst) || !g.w || (g.rope_mode != 2 && !g.pos0) ||
                    (g.rope_mode == 1 && (!g.pos1 || !g.pos2)))
                    return hipErrorNotSupported;
            } else if (g.kind != kRowSegVt) {
                return hipErrorNotSupported;
            }
            o.kind = g.kind;
            o.rope_mode = g.rope_mode;
            o.col = g.col;
            o.dst_tokens = g.dst_tokens;
            o.tok0 = g.tok0;
            o.vt_ld = g.vt_ld;
            o.vt_hs = g.vt_hs;
            o.w = (const uint16_t *) g.w;
            o.dst = (uint16_t *) g.dst;
            o.pos0 = g.pos0;
            o.pos1 = g.pos1;
            o.pos2 = g.pos2;
            o.eps = g.eps;
            o.chunk_tokens = g.chunk_tokens > 0 ? g.chunk_tokens : p.N;
            o.chunk_stride = g.chunk_tokens > 0 ? g.chunk_stride : 0;
            if (p.N % o.chunk_tokens != 0) return hipErrorNotSupported;
            // V^T in blocks of kVtTok tokens: more than 64 tokens (eight
            // 48-token chunks: decode 111.0 -> 109.8 ms; at 48 tokens the
            // blocks' LDS pass cost the chunk 0.25 ms), whole blocks per
            // chunk, 16-byte aligned runs, and a row of chunks that splits
            // into kVtTok column blocks (a row is a multiple of 64 chunks).
            o.vt_tok = g.kind == kRowSegVt && p.N > 64 && o.chunk_tokens % kVtTok == 0 && g.tok0 % kVtTok == 0 &&
                               g.vt_ld % 8 == 0 && g.vt_hs % 8 == 0 && o.chunk_stride % 8 == 0 && aligned16(g.dst) &&
                               (post.width / 8) % kVtTok == 0 && post.width / 8 <= 512
                           ? kVtTok
                           : 1;
            rope_scales(post.head_dim, g.freq_base, o.l2ts128, o.l2ts44, o.l2ts42);
        }
    } else {
        return hipErrorNotSupported;
    }
    if (nchunk <= 0 || nchunk > 512 || nchunk % 64 != 0) return hipErrorNotSupported;

    const float * part = (const float *) a.ws;
    if (dma) {
        launch_dma_splitk_parts(p, splits, a.ws, s);
    } else {
        allow_skinny_lds();
        launch_skinny_part(p, a.x_type == WAMX_TYPE_F32, a.w_tiled, (float *) a.ws, splits, ks, waves, s);
    }
    const dim3 grid((unsigned) p.N, (unsigned) nseg), block((unsigned) nchunk);
#define WAMX_ROW(EK, PK) hipLaunchKernelGGL((skinny_reduce_row<EK, PK>), grid, block, 0, s, p, part, splits, d)
#define WAMX_ROW_NORM(EK)                                                   \
    switch (post_kind) {                                                    \
        case kPostNormAffine: WAMX_ROW(EK, kPostNormAffine); break;         \
        case kPostNormModBf16: WAMX_ROW(EK, kPostNormModBf16); break;       \
        default: WAMX_ROW(EK, kPostNormModF32); break;                      \
    }
    if (post_kind == kPostSegs) {
        if (E == kEpiBf16) WAMX_ROW(kEpiBf16, kPostSegs);
        else WAMX_ROW(kEpiBias, kPostSegs);
    } else {
        switch (E) {
            case kEpiBf16: WAMX_ROW_NORM(kEpiBf16) break;
            case kEpiBias: WAMX_ROW_NORM(kEpiBias) break;
            case kEpiBiasGelu: WAMX_ROW_NORM(kEpiBiasGelu) break;
            case kEpiBiasGated: WAMX_ROW_NORM(kEpiBiasGated) break;
            default: WAMX_ROW_NORM(kEpiBiasResidual) break;
        }
    }
#undef WAMX_ROW_NORM
#undef WAMX_ROW
    return hipGetLastError();
}

// f32 activations rounded to bf16 rows [rows][K] (round to nearest even, the
// rounding the f32-activation kernels apply on load), 8 values per thread.
__global__ void round_rows_bf16_kernel(const float * __restrict__ x, int64_t ldx, uint16_t * __restrict__ y,
                                       int64_t K, int64_t rows) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x, cpr = K / 8;
    if (i >= rows * cpr) return;
    const int64_t r = i / cpr, c = i - r * cpr;
    const float4 a = *(const float4 *) (x + r * ldx + 8 * c), b = *(const float4 *) (x + r * ldx + 8 * c + 4);
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    *(uint4 *) (y + r * K + 8 * c) = pack8(v);
}

hipError_t launch_gemm(const GemmArgs & a, hipStream_t s) {
    const GemmParams p = make_params(a);
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
    const bool vec = vec_operands(a);

    // Tiled weights exist for the few-token products only.
    if (a.w_tiled && (!vec || batches != 1 || a.N > 64 || a.M % 16 != 0 || a.K % 32 != 0))
        return hipErrorNotSupported;
    if (vec && batches == 1 && a.N <= 64) {
        allow_skinny_lds();
        return run_skinny(p, xf32, a.w_tiled, a.ws, a.ws_bytes, s);
    }
    if (vec && !xf32 && batches == 1) {
        hipError_t err = hipSuccess;
        if (dispatch_dma(p, a.ws, a.ws_bytes, s, err)) return err;
    }
    // f32 activations on more than 64 tokens (the 512-token text embedder):
    // one rounding pass into the workspace, then the bf16 DMA GEMM on the
    // rounded copy, whose split-K partials (if any) take the workspace's rest.
    // 12.9 GFLOP at 512 x 3072 x 4096: 88 us on the f32-activation tile
    // kernel.
    if (vec && xf32 && batches == 1 && a.K % 32 == 0 && a.ws && aligned16(a.ws)) {
        const size_t xb = ((size_t) a.N * (size_t) a.K * 2 + 255) / 256 * 256;
        if (xb < a.ws_bytes) {
            uint16_t * xr = (uint16_t *) a.ws;
            const int64_t chunks = a.N * (a.K / 8);
            hipLaunchKernelGGL(round_rows_bf16_kernel, dim3((unsigned) ((chunks + 255) / 256)), dim3(256), 0, s,
                               (const float *) a.x, a.ldx, xr, a.K, a.N);
            GemmParams q = p;
            q.x = xr;
            q.ldx = a.K;
            hipError_t err = hipSuccess;
            if (dispatch_dma(q, (char *) a.ws + xb, a.ws_bytes - xb, s, err)) return err;
            return run_tile<128, 128, 2, 2, false, true>(q, 1, s);
        }
    }
    if (vec) return xf32 ? run_tile<128, 128, 2, 2, true, true>(p, batches, s) : run_tile<128, 128, 2, 2, false, true>(p, batches, s);
    return xf32 ? run_tile<128, 128, 2, 2, true, false>(p, batches, s) : run_tile<128, 128, 2, 2, false, false>(p, batches, s);
}

}  // namespace wamx
