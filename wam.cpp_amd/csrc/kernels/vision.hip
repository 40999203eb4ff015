// The vision front-end of the GWP-0.5 request: the three camera views
// composed into one canvas and patchified for the VAE encoder, and the VAE's
// BF16 convolutions.
//
//  * preprocess_views_kernel (the role of wam.cpp's preprocess_kernel,
//    src/models/gwp05/kernels/cuda_preprocess.cu:45-137, and of the CPU
//    compose_and_patchify, src/models/gwp05/engine/vae.cpp:1-133): canvas
//    out_w x out_h, top half the high camera, bottom-left / bottom-right the
//    two wrist cameras; each view is resized to cover its region (scale =
//    max of the two axis ratios, sizes rounded half away from zero) and
//    centre-cropped, with a triangle (bilinear, antialiased when shrinking:
//    support max(1, 1/scale)) filter whose taps are clamped to the image and
//    normalised to sum 1, applied along x, then along y.  The canvas is
//    written 2x2 pixel-unshuffled as f32 [12][out_h/2][out_w/2], channel
//    4c + 2dx + dy, mapped to [-1, 1] (v * 2 - 1); u8 pixels are v / 255.
//    One thread per output value.
//  * conv2d: ggml_conv_2d_direct on bf16 (the patch's cuDNN implicit GEMM,
//    native-bf16.patch:174-218) as a GEMM on MFMA over an im2col of the
//    input taken a row range at a time (so the column matrix never exceeds a
//    workspace half): y[b][oc][p] = sum_k col[p][k] w[oc][k], k = ic*KH*KW +
//    ky*KW + kx, f32 accumulation, one rounding to the output type.
#include <algorithm>

#include "../internal.h"
#include "device.h"

namespace wamx {

struct ViewDev {
    const void * data;
    int32_t format, w, h;       // format 0: u8 RGB, 1: f32 RGB in [0, 1]
    int32_t dw, dh, x0, y0;     // destination region of the canvas
};
struct Views {
    ViewDev v[3];
};

__device__ __forceinline__ float pixel(const ViewDev & v, int x, int y, int c) {
    const size_t i = ((size_t) y * v.w + x) * 3 + c;
    return v.format == 0 ? (float) ((const uint8_t *) v.data)[i] * (1.0f / 255.0f) : ((const float *) v.data)[i];
}

// Taps of output position `o` along one axis: the source range [first,
// last], the filter centre and support.
struct Axis {
    int first, last;
    float center, support;
};
__device__ __forceinline__ Axis axis_of(int o, int src, int resized, int dst) {
    const int crop = (resized - dst) / 2;
    const float scale = (float) resized / (float) src;
    Axis a;
    a.support = fmaxf(1.0f, 1.0f / scale);
    a.center = ((float) (o + crop) + 0.5f) / scale - 0.5f;
    a.first = (int) ceilf(a.center - a.support);
    a.last = (int) floorf(a.center + a.support);
    return a;
}
__device__ __forceinline__ float tap(const Axis & a, int s) {
    return fmaxf(0.0f, 1.0f - fabsf((float) s - a.center) / a.support);
}

__global__ __launch_bounds__(256) void preprocess_views_kernel(Views views, int out_w, int out_h, float * out) {
    const int pw = out_w / 2, ph = out_h / 2;
    const int64_t n = (int64_t) 12 * pw * ph;
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const int x = (int) (i % pw), y = (int) ((i / pw) % ph), ch = (int) (i / ((int64_t) pw * ph));
    const int c = ch / 4, dx = (ch % 4) / 2, dy = ch % 2;
    const int cx = 2 * x + dx, cy = 2 * y + dy;
    const int vi = cy < out_h / 2 ? 0 : (cx < out_w / 2 ? 1 : 2);
    const ViewDev & v = views.v[vi];
    const int lx = cx - v.x0, ly = cy - v.y0;
    const float s = fmaxf((float) v.dw / (float) v.w, (float) v.dh / (float) v.h);
    const int rw = (int) roundf((float) v.w * s), rh = (int) roundf((float) v.h * s);
    const Axis ax = axis_of(lx, v.w, rw, v.dw), ay = axis_of(ly, v.h, rh, v.dh);
    float tx = 0.0f, ty = 0.0f;
    for (int sx = ax.first; sx <= ax.last; ++sx) tx += tap(ax, sx);
    for (int sy = ay.first; sy <= ay.last; ++sy) ty += tap(ay, sy);
    float acc = 0.0f;
    for (int sy = ay.first; sy <= ay.last; ++sy) {
        const int yy = min(max(sy, 0), v.h - 1);
        float row = 0.0f;
        for (int sx = ax.first; sx <= ax.last; ++sx)
            row += pixel(v, min(max(sx, 0), v.w - 1), yy, c) * (tap(ax, sx) / tx);
        acc += row * (tap(ay, sy) / ty);
    }
    out[i] = acc * 2.0f - 1.0f;
}

// Rows [p0, p0 + rows) of the column matrix of batch image `b`: col[r][k],
// zero where the tap falls in the padding.  Source bf16 or f32, column bf16
// (or f32 for an f32 convolution).
struct ConvDev {
    const void * x;
    void * col;
    int32_t x_type, col_type;
    int64_t IW, IH, IC, KW, KH, OW, OH;
    int32_t s0, s1, p0, p1, d0, d1;
};
__global__ __launch_bounds__(256) void conv_col_kernel(ConvDev c, int64_t b, int64_t p_begin, int64_t rows) {
    const int64_t K = c.IC * c.KH * c.KW;
    const int64_t i = (int64_t) blockIdx.x * 256 + threadIdx.x;
    if (i >= rows * K) return;
    const int64_t r = i / K, k = i % K, p = p_begin + r;
    const int64_t oy = p / c.OW, ox = p % c.OW;
    const int64_t ic = k / (c.KH * c.KW), ky = (k / c.KW) % c.KH, kx = k % c.KW;
    const int64_t iy = oy * c.s1 - c.p1 + ky * c.d1, ix = ox * c.s0 - c.p0 + kx * c.d0;
    const bool in = iy >= 0 && iy < c.IH && ix >= 0 && ix < c.IW;
    const int64_t si = ((b * c.IC + ic) * c.IH + (in ? iy : 0)) * c.IW + (in ? ix : 0);
    if (c.col_type == WAMX_TYPE_BF16) {
        uint16_t v = 0;
        if (in) v = c.x_type == WAMX_TYPE_BF16 ? ((const uint16_t *) c.x)[si] : f32_to_bf16(((const float *) c.x)[si]);
        ((uint16_t *) c.col)[i] = v;
    } else {
        ((float *) c.col)[i] = in ? ((const float *) c.x)[si] : 0.0f;
    }
}

hipError_t launch_conv2d(const TensorRef & kernel, const TensorRef & input, const TensorRef & dst, const int32_t * pp,
                         void * ws, size_t ws_bytes, hipStream_t s) {
    const bool bf = kernel.type == WAMX_TYPE_BF16;
    if ((bf && (input.type != WAMX_TYPE_BF16 || dst.type != WAMX_TYPE_BF16)) ||
        (!bf && (kernel.type != WAMX_TYPE_F32 || input.type != WAMX_TYPE_F32 || dst.type != WAMX_TYPE_F32)))
        return hipErrorInvalidValue;
    ConvDev c{};
    c.x = input.data;
    c.x_type = input.type;
    c.col_type = bf ? WAMX_TYPE_BF16 : WAMX_TYPE_F32;
    c.IW = input.ne[0];
    c.IH = input.ne[1];
    c.IC = input.ne[2];
    c.KW = kernel.ne[0];
    c.KH = kernel.ne[1];
    c.OW = dst.ne[0];
    c.OH = dst.ne[1];
    c.s0 = pp[0];
    c.s1 = pp[1];
    c.p0 = pp[2];
    c.p1 = pp[3];
    c.d0 = pp[4];
    c.d1 = pp[5];
    const int64_t K = c.IC * c.KH * c.KW, P = c.OW * c.OH, OC = kernel.ne[3], B = input.ne[3];
    const size_t es = bf ? 2 : 4;
    // Upper workspace half: the column chunk; lower half: the GEMM's split-K partials.
    const size_t half = ws_bytes / 2 / 256 * 256;
    int64_t cap = (int64_t) (half / (K * es));
    if (cap >= 64) cap = cap / 64 * 64;
    const int64_t chunk = std::min<int64_t>(P, cap);
    if (!ws || chunk < 1) return hipErrorInvalidValue;
    c.col = (char *) ws + half;
    for (int64_t b = 0; b < B; ++b)
        for (int64_t p = 0; p < P; p += chunk) {
            const int64_t rows = std::min(chunk, P - p);
            hipLaunchKernelGGL(conv_col_kernel, dim3((unsigned) ((rows * K + 255) / 256)), dim3(256), 0, s, c, b, p,
                               rows);
            GemmArgs g;
            g.w = c.col;
            g.w_type = c.col_type;
            g.ldw = K;
            g.x = kernel.data;
            g.x_type = kernel.type;
            g.ldx = K;
            g.y = (char *) dst.data + (size_t) ((b * OC) * P + p) * es;
            g.y_type = dst.type;
            g.ldy = P;
            g.M = rows;
            g.N = OC;
            g.K = K;
            g.ws = ws;
            g.ws_bytes = half;
            const hipError_t e = launch_gemm(g, s);
            if (e != hipSuccess) return e;
        }
    return hipGetLastError();
}

}  // namespace wamx

using namespace wamx;

struct wamx_preprocessor {
    wamx_backend_t be = nullptr;
    void * buf[3] = {};
    size_t cap[3] = {};
};

extern "C" {

wamx_preprocessor_t wamx_preprocessor_create(wamx_backend_t be) {
    clear_error();
    if (!be) {
        set_error("wamx_preprocessor_create: null backend");
        return nullptr;
    }
    auto * p = new (std::nothrow) wamx_preprocessor();
    if (p) p->be = be;
    return p;
}

void wamx_preprocessor_free(wamx_preprocessor_t p) {
    if (!p) return;
    for (void * b : p->buf)
        if (b) (void) hipFree(b);
    delete p;
}

wamx_status wamx_preprocess_views(wamx_preprocessor_t p, const wamx_image_view * views, int32_t n_views, int32_t out_w,
                                  int32_t out_h, float * out_device) {
    WAMX_REQUIRE(p && views && out_device, "wamx_preprocess_views: null argument");
    WAMX_REQUIRE(n_views == 3, "wamx_preprocess_views: exactly three camera views are required (got %d)", n_views);
    WAMX_REQUIRE(out_w > 0 && out_h > 0, "wamx_preprocess_views: invalid canvas %dx%d", out_w, out_h);
    hipStream_t s = (hipStream_t) wamx_backend_stream(p->be);
    Views v{};
    for (int i = 0; i < 3; ++i) {
        const wamx_image_view & im = views[i];
        WAMX_REQUIRE(im.data && im.w > 0 && im.h > 0 && (im.format == 0 || im.format == 1),
                     "wamx_preprocess_views: invalid image %d", i);
    }
    for (int i = 0; i < 3; ++i) {
        const wamx_image_view & im = views[i];
        const size_t bytes = (size_t) im.w * im.h * 3 * (im.format == 0 ? 1 : 4);
        if (bytes > p->cap[i]) {
            if (p->buf[i]) WAMX_HIP_TRY(hipFree(p->buf[i]));
            p->buf[i] = nullptr;
            p->cap[i] = 0;
            WAMX_HIP_TRY(hipMalloc(&p->buf[i], bytes));
            p->cap[i] = bytes;
        }
        WAMX_HIP_TRY(hipMemcpyAsync(p->buf[i], im.data, bytes, hipMemcpyHostToDevice, s));
        v.v[i].data = p->buf[i];
        v.v[i].format = im.format;
        v.v[i].w = im.w;
        v.v[i].h = im.h;
    }
    const int top = out_h / 2, left = out_w / 2;
    v.v[0].dw = out_w, v.v[0].dh = top, v.v[0].x0 = 0, v.v[0].y0 = 0;
    v.v[1].dw = left, v.v[1].dh = out_h - top, v.v[1].x0 = 0, v.v[1].y0 = top;
    v.v[2].dw = out_w - left, v.v[2].dh = out_h - top, v.v[2].x0 = left, v.v[2].y0 = top;
    const int64_t n = (int64_t) 12 * (out_w / 2) * (out_h / 2);
    if (n > 0)
        hipLaunchKernelGGL(preprocess_views_kernel, dim3((unsigned) ((n + 255) / 256)), dim3(256), 0, s, v, out_w, out_h,
                       out_device);
    WAMX_HIP_TRY(hipGetLastError());
    WAMX_HIP_TRY(hipStreamSynchronize(s));
    return WAMX_STATUS_SUCCESS;
}

}  // extern "C"
