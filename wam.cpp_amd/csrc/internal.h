// Internal declarations of libwamx: kernel launchers and backend internals.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace wamx {

const char * last_error_cstr();

// Validators of the ops a constructor checks (null when well formed, else the
// reason); supports_op runs them on every node, whoever built it.
const char * check_linear(const wamx_tensor * t);
const char * check_qk_norm_rope(const wamx_tensor * t);
const char * check_joint_attn(const wamx_tensor * t);
const char * check_modulation(const wamx_tensor * t);
const char * check_euler_step(const wamx_tensor * t);
const char * check_mlp_small(const wamx_tensor * t);
const char * check_im2col(const wamx_tensor * t);
const char * check_conv_2d(const wamx_tensor * t);

// ---------------------------------------------------------------------------
// GEMM: y[b][n][m] = sum_k w[b/r][m][k] * x[b][n][k]  (the ggml MUL_MAT layout:
// both operands K-contiguous, "NT").  w is bf16 (or f32 for the SIMT path),
// x is bf16 or f32 (rounded to bf16 on load when w is bf16).
// ---------------------------------------------------------------------------
struct GemmArgs {
    const void * w = nullptr;
    int32_t w_type = WAMX_TYPE_BF16;
    int64_t ldw = 0, w_bs2 = 0, w_bs3 = 0;   // element strides
    const void * x = nullptr;
    int32_t x_type = WAMX_TYPE_BF16;
    int64_t ldx = 0, x_bs2 = 0, x_bs3 = 0;
    void * y = nullptr;
    int32_t y_type = WAMX_TYPE_F32;
    int64_t ldy = 0, y_bs2 = 0, y_bs3 = 0;
    int64_t M = 0, N = 0, K = 0;
    int64_t B2 = 1, B3 = 1;                  // batches of y / x
    int64_t r2 = 1, r3 = 1;                  // broadcast ratio: w batch = b / r
    int32_t epi = WAMX_EPI_NONE;             // wamx_linear_epilogue
    const void * bias = nullptr;             // bf16 [M]
    const void * res = nullptr;              // bf16 [N][ldres]
    int64_t ldres = 0;
    const float * gate = nullptr;            // f32 [M]
    void * ws = nullptr;                     // K-split partials of the skinny path
    size_t ws_bytes = 0;
    bool w_tiled = false;                    // w in the MFMA-tiled layout (launch_tile_weights)
};

hipError_t launch_gemm(const GemmArgs & a, hipStream_t s);
// Row-major bf16 [M][K] <-> the MFMA-tiled weight layout of the tiled buffer
// type ([M/16][K/32] tiles of 1 KB; M % 16 == 0, K % 32 == 0).
hipError_t launch_tile_weights(const void * src, void * dst, int64_t M, int64_t K, bool untile, hipStream_t s);
// Whether t is a weight stored in the tiled layout (placed in a tiled buffer).
bool tensor_is_tiled(const wamx_tensor * t);
// Writes the row-major device array src into t, tiling it when t is tiled.
hipError_t tensor_set_from_device(wamx_tensor * t, const void * src, hipStream_t s);
// Workspace the skinny path needs for an M x N x K product (0 when unsplit).
size_t skinny_workspace_bytes(int64_t M, int64_t N, int64_t K);
// Workspace of a backend: K-split GEMM and key-split attention partials.
constexpr size_t kBackendWorkspaceBytes = 64ull << 20;
// Bytes of fp32 K-split partials that launch_gemm writes to its workspace
// for a plain bf16-weight product (row-major, contiguous, one batch) of N
// tokens, given ws_bytes of workspace; 0 when the product takes no K split.
size_t linear_split_bytes(int64_t M, int64_t N, int64_t K, int32_t x_type, size_t ws_bytes);

// Row ops that consume a skinny GEMM's output, applied by its split-K reduce
// in the same launch (one workgroup per token row).  The GEMM output itself
// is still written.
enum { kRowSegQk = 0, kRowSegVt = 1 };
struct RowSeg {
    int32_t kind = kRowSegQk;
    int64_t col = 0;                 // first GEMM output column of the segment
    // kRowSegQk: RMSNorm over the segment * w (bf16), RoPE, bf16 into
    // dst[h][tok0 + t][dd] with dst_tokens rows per head (launch_qk_norm_rope).
    const void * w = nullptr;
    int64_t dst_tokens = 0, tok0 = 0;
    int32_t rope_mode = 2;
    const int32_t * pos0 = nullptr;
    const int32_t * pos1 = nullptr;
    const int32_t * pos2 = nullptr;
    float eps = 0.0f, freq_base = 10000.0f;
    // kRowSegVt: bf16 copy into dst[h * vt_hs + dd * vt_ld + t] (V^T storage).
    int64_t vt_ld = 0, vt_hs = 0;
    void * dst = nullptr;
    // Rows of the product in chunks of chunk_tokens (0: one chunk): row n is
    // token t = n % chunk_tokens of chunk n / chunk_tokens, whose destination
    // starts chunk_stride elements after the previous chunk's (the RoPE
    // position is t's).
    int64_t chunk_tokens = 0, chunk_stride = 0;
};
enum { kRowPostNorm = 1, kRowPostSegs = 2 };
struct RowPost {
    int32_t kind = 0;
    // kRowPostNorm: LayerNorm of the whole row into out (launch_norm_mod_bf16
    // arguments: scale/shift of ss_type with row stride ss, affine).
    const void * scale = nullptr;
    const void * shift = nullptr;
    int32_t ss_type = WAMX_TYPE_F32;
    bool affine = false;
    int64_t ss = 0;
    void * out = nullptr;
    int64_t ldo = 0;
    float eps = 0.0f;
    // kRowPostSegs: up to three segments of `width` columns, heads x head_dim.
    int32_t nseg = 0;
    int64_t width = 0, head_dim = 0;
    RowSeg seg[3];
};
// The split-K GEMM whose reduce applies `post`: the skinny part kernel for up
// to 64 tokens, the K-sliced 128 x 128 DMA GEMM for more tokens on grids
// that it splits (the batched denoise step).  Returns hipErrorNotSupported,
// launching nothing, when the product or the row op does not fit that path.
hipError_t launch_gemm_rowpost(const GemmArgs & a, const RowPost & post, hipStream_t s);

// ---------------------------------------------------------------------------
// Row-wise norms (bf16 / f32), bias+GELU, gated residuals.
// ---------------------------------------------------------------------------
hipError_t launch_norm_mod_bf16(const void * x, int64_t ldx, const void * scale, const void * shift, int32_t ss_type,
                                int64_t ss, void * y, int64_t ldy, int64_t rows, int64_t cols, float eps, bool affine,
                                hipStream_t s);
hipError_t launch_rms_norm_bf16_f32(const void * x, int64_t ldx, const void * w, float * y, int64_t ldy, int64_t rows,
                                    int64_t cols, float eps, hipStream_t s);
hipError_t launch_norm_mod_f32(const float * x, int64_t ldx, const float * scale, const float * shift, int64_t ss,
                               float * y, int64_t rows, int64_t cols, float eps, hipStream_t s);
hipError_t launch_norm_f32(const float * x, int64_t ldx, float * y, int64_t ldy, int64_t rows, int64_t cols, float eps,
                           bool rms, hipStream_t s);
hipError_t launch_gated_residual_bf16(const void * h, int64_t ldh, const void * b, int64_t ldb, const void * g,
                                      int32_t g_type, int64_t gs, void * y, int64_t rows, int64_t cols, hipStream_t s);
hipError_t launch_gated_residual_f32(const float * r, int64_t ldr, const float * b, int64_t ldb, const float * g,
                                     int64_t gs, float * y, int64_t rows, int64_t cols, hipStream_t s);
hipError_t launch_bias_gelu_bf16(const void * x, const void * bias, void * y, int64_t n, int64_t width, hipStream_t s);

// ---------------------------------------------------------------------------
// Generic strided tensor kernels (ggml glue ops).  A TensorRef describes a
// 4-D strided view: data + ne[] + byte strides nb[] + type.
// ---------------------------------------------------------------------------
struct TensorRef {
    void * data;
    int32_t type;
    int64_t ne[4];
    int64_t nb[4];
};
TensorRef ref_of(const wamx_tensor * t);

// dst[i] = convert(src[i]) elementwise over dst's shape; src broadcast by modulo.
hipError_t launch_copy(const TensorRef & src, const TensorRef & dst, hipStream_t s);
// dst = a (op) b with b broadcast (ggml bin_bcast).  op: 0 add, 1 mul, 2 repeat b.
hipError_t launch_binary(int op, const TensorRef & a, const TensorRef & b, const TensorRef & dst, hipStream_t s);
// dst = unary(a) for op = WAMX_UNARY_GELU / _GELU_ERF / _SILU, or
// a * scale + bias for op = kUnaryScale (ggml_scale).
constexpr int kUnaryScale = -1;
hipError_t launch_unary(int op, const TensorRef & a, const TensorRef & dst, float scale, float bias, hipStream_t s);
hipError_t launch_concat(const TensorRef & a, const TensorRef & b, const TensorRef & dst, int dim, hipStream_t s);
hipError_t launch_get_rows(const TensorRef & a, const int32_t * rows, const TensorRef & dst, hipStream_t s);
// SOFT_MAX_EXT: y = softmax(x * scale + mask) over ne0; mask (data may be null)
// F32 or F16, row i1 of plane (i2 % ne2, i3 % ne3).
hipError_t launch_softmax_f32(const TensorRef & x, const TensorRef & mask, const TensorRef & y, float scale,
                              hipStream_t s);
hipError_t launch_rope_f32(const TensorRef & x, const int32_t * pos, const TensorRef & y, int n_dims, float freq_base,
                           hipStream_t s);
hipError_t launch_im2col(const TensorRef & src, const TensorRef & dst, int KW, int KH, int s0, int s1, int p0, int p1,
                         int d0, int d1, hipStream_t s);
// ggml_conv_2d_direct (kernel [KW,KH,IC,OC], input [IW,IH,IC,N], dst
// [OW,OH,OC,N]; pp = {s0, s1, p0, p1, d0, d1}): im2col row chunks in the
// upper half of ws, the GEMM's partials in the lower half.
hipError_t launch_conv2d(const TensorRef & kernel, const TensorRef & input, const TensorRef & dst, const int32_t * pp,
                         void * ws, size_t ws_bytes, hipStream_t s);
hipError_t launch_modulation(const void * mod, int32_t mod_type, const void * tables, int32_t tab_type, float * out,
                             int64_t per_layer, int64_t layers, hipStream_t s, int64_t steps = 1);
// atomicMin of the index of every Inf / NaN of p[0, n) into *first (n < 2^32).
hipError_t launch_nonfinite_scan(const float * p, int64_t n, uint32_t * first, hipStream_t s);
// bf16 out[i] = bf16(f32(a[i]) + f32(v[i]) * dt[0]), product and sum rounded apart.
hipError_t launch_euler_step(const void * a, const void * v, const float * dt, void * out, int64_t n, hipStream_t s);
// Two small linear layers (wamx_mlp_small): x bf16 [N][K0], w1 [M1][K0],
// w2 [M2][M1], biases bf16, y bf16 [N][M2]; flags WAMX_MLP_GELU_*.
hipError_t launch_mlp_small(const void * x, const void * w1, const void * b1, const void * w2, const void * b2, void * y,
                            int64_t N, int64_t K0, int64_t M1, int64_t M2, int32_t flags, hipStream_t s);

// ---------------------------------------------------------------------------
// Fused attention-side kernels.
// ---------------------------------------------------------------------------
// Rows of x are chunk_tokens-token chunks (0: one chunk): token tl of chunk b
// takes position pos[tl] and goes to dst + b * chunk_stride (elements).
// Chunk b's rows start at x + b * x_cs (-1: right after chunk b - 1's) and
// use the norm weight w + b * w_cs (0: one weight for every chunk).
hipError_t launch_qk_norm_rope(const void * x, int64_t ldx, const void * w, void * dst, int64_t heads, int64_t head_dim,
                               int64_t tokens, int64_t dst_tokens, int64_t tok0, int rope_mode, const int32_t * pos0,
                               const int32_t * pos1, const int32_t * pos2, float eps, float freq_base, hipStream_t s,
                               int64_t chunk_tokens = 0, int64_t chunk_stride = 0, int64_t lo_off = 0,
                               const float * tab = nullptr, int64_t x_cs = -1, int64_t w_cs = 0);
// (cos, sin) of every rope pair of `tokens` tokens (rope mode 0 or 1
// positions) into out [tokens][head_dim]: the table of rope mode 3.
hipError_t launch_rope_table(int rope_mode, const int32_t * pos0, const int32_t * pos1, const int32_t * pos2,
                             int64_t tokens, int64_t head_dim, float freq_base, float * out, hipStream_t s);

struct AttnArgs {
    const void * q = nullptr;      // bf16 [batch][H][Tq][dh]
    const void * k_a = nullptr;    // bf16 [H][na][dh]
    const void * vt_a = nullptr;   // bf16 [H][dh][vt_ld_a]
    int64_t na = 0, vt_ld_a = 0;
    const void * k_b = nullptr;    // bf16 [H][nb][dh] or null
    const void * vt_b = nullptr;   // bf16 [H][dh][vt_ld_b]
    int64_t nb = 0, vt_ld_b = 0;
    int64_t na_split = 0;          // reference key order: a[0,na_split), b, a[na_split,na)
    void * out = nullptr;          // bf16 [Tq][H*dh]
    int64_t heads = 0, head_dim = 0, tq = 0;
    // Independent chunks: heads = batch x hb; chunk b's sources and queries
    // are heads [b * hb, (b + 1) * hb) of the arrays above (each array
    // contiguous across chunks) and its output rows [b * tq, (b + 1) * tq)
    // of out [batch][tq][hb * head_dim].  0: one chunk (hb = heads).
    int64_t hb = 0;
    float scale = 1.0f;
    void * ws = nullptr;           // fp32 partials of the key-split path
    size_t ws_bytes = 0;
    // f32-accurate scores: q and k_a are the bf16 roundings of f32 Q and K
    // and q_lo / k_lo the rest (same layouts); S = K Q^T + K Q_lo^T +
    // K_lo Q^T.  One key source, one chunk.
    const void * q_lo = nullptr;
    const void * k_lo = nullptr;
};
hipError_t launch_joint_attn(const AttnArgs & a, hipStream_t s);

// Synthetic N(mean, std) fill: splitmix64(seed ^ index) -> Box-Muller.
hipError_t launch_fill_normal(void * dst, int32_t type, int64_t n, uint64_t seed, float mean, float std, hipStream_t s);
hipError_t launch_fill_f32(float * dst, int64_t n, float v, hipStream_t s);

}  // namespace wamx
