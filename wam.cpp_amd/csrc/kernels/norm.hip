// Row-wise bandwidth kernels of the fused elementwise path:
//   * LayerNorm + adaLN modulation, bf16 io (norm_bf16_fused<.,false>,
//     native-bf16.patch:368-409) and the affine bf16 LayerNorm
//     (norm_bf16_fused<.,true>, used by layer_norm, weights.cpp:919-930);
//   * RMSNorm bf16 -> f32 over the full row (rms_norm_bf16_f32, patch:411-430);
//   * the F32 profile's fused norm + modulation (norm_modulation_f32,
//     p7-fusions.patch:19-51) and plain f32 NORM / RMS_NORM;
//   * gated residuals (bf16: patch:79-91, f32: p7-fusions.patch:122-134) and
//     bias + GELU-tanh (patch:507-514).
//
// One 256-thread workgroup per row.  A row is read once from HBM into
// registers (up to kMaxCache elements per thread), reduced across the block,
// normalised and written once: bytes = row in + row out.
#include "../internal.h"
#include "device.h"
#include "rowops.h"

#include <algorithm>

namespace wamx {

constexpr int kNormThreads = 256;
constexpr int kMaxCache = 32;  // elements per thread held in registers (rows up to 8192)

// Two-pass mean/centred-variance norm of a bf16 row; affine selects n*w+b
// with bf16 w/b, otherwise n*(1+scale)+shift with f32 or bf16 scale/shift.
template <bool AFFINE, bool SS_BF16>
__global__ __launch_bounds__(kNormThreads) void norm_mod_bf16_kernel(const uint16_t * __restrict__ x, int64_t ldx,
                                                                      const void * __restrict__ scale,
                                                                      const void * __restrict__ shift, int64_t ss,
                                                                      uint16_t * __restrict__ y, int64_t ldy, int cols,
                                                                      float eps) {
    __shared__ float red[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const uint16_t * xr = x + row * ldx;
    float v[kMaxCache];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxCache; ++i) {
        const int c = threadIdx.x + i * kNormThreads;
        v[i] = c < cols ? bf16_to_f32(xr[c]) : 0.0f;
        sum += v[i];
    }
    for (int c = threadIdx.x + kMaxCache * kNormThreads; c < cols; c += kNormThreads) sum += bf16_to_f32(xr[c]);
    const float mean = block_sum(sum, red) / (float) cols;
    float var = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxCache; ++i) {
        const int c = threadIdx.x + i * kNormThreads;
        if (c < cols) {
            const float d = v[i] - mean;
            var = fmaf(d, d, var);
        }
    }
    for (int c = threadIdx.x + kMaxCache * kNormThreads; c < cols; c += kNormThreads) {
        const float d = bf16_to_f32(xr[c]) - mean;
        var = fmaf(d, d, var);
    }
    var = block_sum(var, red) / (float) cols;
    const float inv_std = rsqrtf(var + eps);
    uint16_t * yr = y + row * ldy;
    const int64_t so = row * ss;
    auto emit = [&](int c, float xv) {
        const float n = (xv - mean) * inv_std;
        float a, b;
        if (SS_BF16) {
            a = bf16_to_f32(((const uint16_t *) scale)[so + c]);
            b = bf16_to_f32(((const uint16_t *) shift)[so + c]);
        } else {
            a = ((const float *) scale)[so + c];
            b = ((const float *) shift)[so + c];
        }
        yr[c] = f32_to_bf16(AFFINE ? fmaf(n, a, b) : fmaf(n, 1.0f + a, b));
    };
#pragma unroll
    for (int i = 0; i < kMaxCache; ++i) {
        const int c = threadIdx.x + i * kNormThreads;
        if (c < cols) emit(c, v[i]);
    }
    for (int c = threadIdx.x + kMaxCache * kNormThreads; c < cols; c += kNormThreads) emit(c, bf16_to_f32(xr[c]));
}

__global__ __launch_bounds__(kNormThreads) void rms_norm_bf16_f32_kernel(const uint16_t * __restrict__ x, int64_t ldx,
                                                                          const uint16_t * __restrict__ w,
                                                                          float * __restrict__ y, int64_t ldy, int cols,
                                                                          float eps) {
    __shared__ float red[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const uint16_t * xr = x + row * ldx;
    float v[kMaxCache];
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxCache; ++i) {
        const int c = threadIdx.x + i * kNormThreads;
        v[i] = c < cols ? bf16_to_f32(xr[c]) : 0.0f;
        sum = fmaf(v[i], v[i], sum);
    }
    for (int c = threadIdx.x + kMaxCache * kNormThreads; c < cols; c += kNormThreads) {
        const float t = bf16_to_f32(xr[c]);
        sum = fmaf(t, t, sum);
    }
    const float inv_rms = rsqrtf(block_sum(sum, red) / (float) cols + eps);
    float * yr = y + row * ldy;
#pragma unroll
    for (int i = 0; i < kMaxCache; ++i) {
        const int c = threadIdx.x + i * kNormThreads;
        if (c < cols) yr[c] = v[i] * inv_rms * bf16_to_f32(w[c]);
    }
    for (int c = threadIdx.x + kMaxCache * kNormThreads; c < cols; c += kNormThreads)
        yr[c] = bf16_to_f32(xr[c]) * inv_rms * bf16_to_f32(w[c]);
}

// p7-fusions.patch:19-51: one-pass E[x], E[x^2]; out = (n + n*scale) + shift,
// each product and sum rounded separately (no contraction).
#pragma clang fp contract(off)
__global__ __launch_bounds__(kNormThreads) void norm_mod_f32_kernel(const float * __restrict__ x, int64_t ldx,
                                                                     const float * __restrict__ scale,
                                                                     const float * __restrict__ shift, int64_t ss,
                                                                     float * __restrict__ y, int cols, float eps) {
    __shared__ float red[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const float * xr = x + row * ldx;
    float s1 = 0.0f, s2 = 0.0f;
    for (int c = threadIdx.x; c < cols; c += kNormThreads) {
        const float xi = xr[c];
        s1 += xi;
        s2 += xi * xi;
    }
    s1 = block_sum(s1, red);
    s2 = block_sum(s2, red);
    const float mean = s1 / (float) cols;
    const float var = s2 / (float) cols - mean * mean;
    const float inv_std = rsqrtf(var + eps);
    const float * sc = scale + row * ss;
    const float * sh = shift + row * ss;
    float * yr = y + row * (int64_t) cols;
    for (int c = threadIdx.x; c < cols; c += kNormThreads) {
        const float n = (xr[c] - mean) * inv_std;
        const float scaled = n * sc[c];
        yr[c] = (n + scaled) + sh[c];
    }
}

// ggml NORM / RMS_NORM on f32 rows (stock ggml ops of the F32 profile).
__global__ __launch_bounds__(kNormThreads) void norm_f32_kernel(const float * __restrict__ x, int64_t ldx,
                                                                 float * __restrict__ y, int64_t ldy, int cols,
                                                                 float eps, int rms) {
    __shared__ float red[kNormThreads / 64];
    const int64_t row = blockIdx.x;
    const float * xr = x + row * ldx;
    float mean = 0.0f;
    if (!rms) {
        float s = 0.0f;
        for (int c = threadIdx.x; c < cols; c += kNormThreads) s += xr[c];
        mean = block_sum(s, red) / (float) cols;
    }
    float s2 = 0.0f;
    for (int c = threadIdx.x; c < cols; c += kNormThreads) {
        const float d = xr[c] - mean;
        s2 += d * d;
    }
    const float inv = rsqrtf(block_sum(s2, red) / (float) cols + eps);
    float * yr = y + row * ldy;
    for (int c = threadIdx.x; c < cols; c += kNormThreads) yr[c] = (xr[c] - mean) * inv;
}

__global__ void gated_residual_f32_kernel(const float * __restrict__ r, int64_t ldr, const float * __restrict__ b,
                                          int64_t ldb, const float * __restrict__ g, int64_t gs, float * __restrict__ y,
                                          int cols) {
    const int64_t row = blockIdx.y;
    const int col = blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= cols) return;
    const float scaled = b[row * ldb + col] * g[row * gs + col];
    y[row * (int64_t) cols + col] = r[row * ldr + col] + scaled;
}
#pragma clang fp contract(on)

template <bool GATE_BF16>
__global__ void gated_residual_bf16_kernel(const uint16_t * __restrict__ h, int64_t ldh, const uint16_t * __restrict__ b,
                                           int64_t ldb, const void * __restrict__ g, int64_t gs,
                                           uint16_t * __restrict__ y, int cols) {
    const int64_t row = blockIdx.y;
    const int col = blockIdx.x * blockDim.x + threadIdx.x;
    if (col >= cols) return;
    const float gv = GATE_BF16 ? bf16_to_f32(((const uint16_t *) g)[row * gs + col]) : ((const float *) g)[row * gs + col];
    const float v = fmaf(bf16_to_f32(b[row * ldb + col]), gv, bf16_to_f32(h[row * ldh + col]));
    y[row * (int64_t) cols + col] = f32_to_bf16(v);
}

__global__ void bias_gelu_bf16_kernel(const uint16_t * __restrict__ x, const uint16_t * __restrict__ bias,
                                      uint16_t * __restrict__ y, int64_t n, int64_t width) {
    const int64_t i = (int64_t) blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float v = bf16_to_f32(x[i]) + bf16_to_f32(bias[i % width]);
    y[i] = f32_to_bf16(gelu_tanh(v));
}

// ---------------------------------------------------------------------------
// Vectorised form of norm_mod_bf16_kernel for 16-byte aligned rows with
// cols % 8 == 0: thread i of the row owns CPT chunks of 8 elements, and the
// row, scale and shift chunks are all loaded before the first reduction, so a
// row costs one memory round trip.  The block is sized to the row (up to
// 1024 threads), which spreads a short batch of rows over more waves.
template <bool AFFINE, bool SS_BF16, int CPT>
__global__ __launch_bounds__(1024) void norm_mod_bf16_vec(const uint16_t * __restrict__ x, int64_t ldx,
                                                           const void * __restrict__ scale,
                                                           const void * __restrict__ shift, int64_t ss,
                                                           uint16_t * __restrict__ y, int64_t ldy, int cols, float eps) {
    __shared__ float red[16];
    const int64_t row = blockIdx.x;
    const int nchunk = cols >> 3;
    const int64_t so = row * ss;
    uint4 xv[CPT], ha[CPT], hb[CPT];
    float4 fa[CPT][2], fb[CPT][2];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = min((int) threadIdx.x + i * (int) blockDim.x, nchunk - 1);
        xv[i] = *(const uint4 *) (x + row * ldx + 8 * c);
        if constexpr (SS_BF16) {
            ha[i] = *(const uint4 *) ((const uint16_t *) scale + so + 8 * c);
            hb[i] = *(const uint4 *) ((const uint16_t *) shift + so + 8 * c);
        } else {
            fa[i][0] = *(const float4 *) ((const float *) scale + so + 8 * c);
            fa[i][1] = *(const float4 *) ((const float *) scale + so + 8 * c + 4);
            fb[i][0] = *(const float4 *) ((const float *) shift + so + 8 * c);
            fb[i][1] = *(const float4 *) ((const float *) shift + so + 8 * c + 4);
        }
    }
    float v[CPT][8];
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        unpack8(xv[i], v[i]);
        if ((int) threadIdx.x + i * (int) blockDim.x >= nchunk)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[i][e] = 0.0f;
    }
    float mean, inv_std;
    row_mean_istd<CPT>(v, nchunk, cols, eps, red, mean, inv_std);
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
        const int c = (int) threadIdx.x + i * (int) blockDim.x;
        if (c >= nchunk) continue;
        float a[8], b[8];
        if constexpr (SS_BF16) {
            unpack8(ha[i], a);
            unpack8(hb[i], b);
        } else {
            const float af[8] = {fa[i][0].x, fa[i][0].y, fa[i][0].z, fa[i][0].w, fa[i][1].x, fa[i][1].y, fa[i][1].z, fa[i][1].w};
            const float bf[8] = {fb[i][0].x, fb[i][0].y, fb[i][0].z, fb[i][0].w, fb[i][1].x, fb[i][1].y, fb[i][1].z, fb[i][1].w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                a[e] = af[e];
                b[e] = bf[e];
            }
        }
        *(uint4 *) (y + row * ldy + 8 * c) = norm_chunk<AFFINE>(v[i], mean, inv_std, a, b);
    }
}

template <bool AFFINE, bool SS_BF16>
static hipError_t run_norm_mod_vec(const void * x, int64_t ldx, const void * scale, const void * shift, int64_t ss,
                                   void * y, int64_t ldy, int64_t rows, int64_t cols, float eps, hipStream_t s) {
    const int64_t nchunk = cols / 8;
    const int cpt = nchunk <= 1024 ? 1 : nchunk <= 2048 ? 2 : 4;
    const int threads = (int) std::min<int64_t>(1024, ((nchunk + cpt - 1) / cpt + 63) / 64 * 64);
    const dim3 grid((unsigned) rows), block((unsigned) threads);
    const uint16_t * xp = (const uint16_t *) x;
    uint16_t * yp = (uint16_t *) y;
    if (cpt == 1)
        hipLaunchKernelGGL((norm_mod_bf16_vec<AFFINE, SS_BF16, 1>), grid, block, 0, s, xp, ldx, scale, shift, ss, yp, ldy,
                           (int) cols, eps);
    else if (cpt == 2)
        hipLaunchKernelGGL((norm_mod_bf16_vec<AFFINE, SS_BF16, 2>), grid, block, 0, s, xp, ldx, scale, shift, ss, yp, ldy,
                           (int) cols, eps);
    else
        hipLaunchKernelGGL((norm_mod_bf16_vec<AFFINE, SS_BF16, 4>), grid, block, 0, s, xp, ldx, scale, shift, ss, yp, ldy,
                           (int) cols, eps);
    return hipGetLastError();
}

static bool aligned16(const void * p) { return ((uintptr_t) p & 15) == 0; }

hipError_t launch_norm_mod_bf16(const void * x, int64_t ldx, const void * scale, const void * shift, int32_t ss_type,
                                int64_t ss, void * y, int64_t ldy, int64_t rows, int64_t cols, float eps, bool affine,
                                hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    const bool sb = ss_type == WAMX_TYPE_BF16;
    const int ss_es = (affine || sb) ? 2 : 4;
    const bool vec = cols % 8 == 0 && cols / 8 <= 4096 && ldx % 8 == 0 && ldy % 8 == 0 && (ss * ss_es) % 16 == 0 &&
                     aligned16(x) && aligned16(y) && aligned16(scale) && aligned16(shift);
    if (vec) {
        if (affine) return run_norm_mod_vec<true, true>(x, ldx, scale, shift, ss, y, ldy, rows, cols, eps, s);
        if (sb) return run_norm_mod_vec<false, true>(x, ldx, scale, shift, ss, y, ldy, rows, cols, eps, s);
        return run_norm_mod_vec<false, false>(x, ldx, scale, shift, ss, y, ldy, rows, cols, eps, s);
    }
    const dim3 grid((unsigned) rows), block(kNormThreads);
    if (affine) {
        hipLaunchKernelGGL((norm_mod_bf16_kernel<true, true>), grid, block, 0, s, (const uint16_t *) x, ldx, scale, shift,
                           ss, (uint16_t *) y, ldy, (int) cols, eps);
    } else if (sb) {
        hipLaunchKernelGGL((norm_mod_bf16_kernel<false, true>), grid, block, 0, s, (const uint16_t *) x, ldx, scale,
                           shift, ss, (uint16_t *) y, ldy, (int) cols, eps);
    } else {
        hipLaunchKernelGGL((norm_mod_bf16_kernel<false, false>), grid, block, 0, s, (const uint16_t *) x, ldx, scale,
                           shift, ss, (uint16_t *) y, ldy, (int) cols, eps);
    }
    return hipGetLastError();
}

hipError_t launch_rms_norm_bf16_f32(const void * x, int64_t ldx, const void * w, float * y, int64_t ldy, int64_t rows,
                                    int64_t cols, float eps, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(rms_norm_bf16_f32_kernel, dim3((unsigned) rows), dim3(kNormThreads), 0, s, (const uint16_t *) x,
                       ldx, (const uint16_t *) w, y, ldy, (int) cols, eps);
    return hipGetLastError();
}

hipError_t launch_norm_mod_f32(const float * x, int64_t ldx, const float * scale, const float * shift, int64_t ss,
                               float * y, int64_t rows, int64_t cols, float eps, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(norm_mod_f32_kernel, dim3((unsigned) rows), dim3(kNormThreads), 0, s, x, ldx, scale, shift, ss, y,
                       (int) cols, eps);
    return hipGetLastError();
}

hipError_t launch_norm_f32(const float * x, int64_t ldx, float * y, int64_t ldy, int64_t rows, int64_t cols, float eps,
                           bool rms, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(norm_f32_kernel, dim3((unsigned) rows), dim3(kNormThreads), 0, s, x, ldx, y, ldy, (int) cols, eps,
                       rms ? 1 : 0);
    return hipGetLastError();
}

hipError_t launch_gated_residual_bf16(const void * h, int64_t ldh, const void * b, int64_t ldb, const void * g,
                                      int32_t g_type, int64_t gs, void * y, int64_t rows, int64_t cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const dim3 grid((unsigned) ((cols + 255) / 256), (unsigned) rows);
    if (g_type == WAMX_TYPE_BF16)
        hipLaunchKernelGGL(gated_residual_bf16_kernel<true>, grid, dim3(256), 0, s, (const uint16_t *) h, ldh,
                           (const uint16_t *) b, ldb, g, gs, (uint16_t *) y, (int) cols);
    else
        hipLaunchKernelGGL(gated_residual_bf16_kernel<false>, grid, dim3(256), 0, s, (const uint16_t *) h, ldh,
                           (const uint16_t *) b, ldb, g, gs, (uint16_t *) y, (int) cols);
    return hipGetLastError();
}

hipError_t launch_gated_residual_f32(const float * r, int64_t ldr, const float * b, int64_t ldb, const float * g,
                                     int64_t gs, float * y, int64_t rows, int64_t cols, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const dim3 grid((unsigned) ((cols + 255) / 256), (unsigned) rows);
    hipLaunchKernelGGL(gated_residual_f32_kernel, grid, dim3(256), 0, s, r, ldr, b, ldb, g, gs, y, (int) cols);
    return hipGetLastError();
}

hipError_t launch_bias_gelu_bf16(const void * x, const void * bias, void * y, int64_t n, int64_t width, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(bias_gelu_bf16_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, s, (const uint16_t *) x,
                       (const uint16_t *) bias, (uint16_t *) y, n, width);
    return hipGetLastError();
}

}  // namespace wamx
