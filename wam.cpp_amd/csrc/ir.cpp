// Tensor / graph IR of libwamx: contexts own tensor metadata, constructors
// record op + sources the way ggml's graph constructors do (ggml b9866, whose
// constructors the engine calls in src/models/gwp05/engine/*.cpp), and graphs
// are topologically ordered node lists.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>

#include <atomic>
#include <memory>
#include <unordered_set>
#include <vector>

#include "common.h"
#include "internal.h"

namespace wamx {

static thread_local std::string g_last_error;

void set_error(const std::string & msg) { g_last_error = msg; }
void set_errorf(const char * fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
}
void clear_error() { g_last_error.clear(); }
const char * last_error_cstr() { return g_last_error.c_str(); }

}  // namespace wamx

using namespace wamx;

struct wamx_context {
    std::vector<std::unique_ptr<wamx_tensor>> tensors;
    std::vector<std::unique_ptr<wamx_cgraph>> graphs;
    size_t max_tensors = 0;
    int32_t lane = 0;  // lane of the tensors created from now on
};

struct wamx_cgraph {
    std::vector<wamx_tensor *> nodes;
    std::vector<wamx_tensor *> leafs;
    std::unordered_set<const wamx_tensor *> visited;
    size_t max_nodes = 0;
    uint64_t uid = 0;
};

static std::atomic<uint64_t> g_next_graph_uid{1};

static wamx_tensor * new_tensor_impl(wamx_context * ctx, int32_t type, int n_dims, const int64_t * ne) {
    if (!ctx) {
        set_error("wamx_new_tensor: null context");
        return nullptr;
    }
    if (ctx->tensors.size() >= ctx->max_tensors) {
        set_errorf("wamx_new_tensor: context full (%zu tensors)", ctx->max_tensors);
        return nullptr;
    }
    if (wamx_type_size(type) == 0) {
        set_errorf("wamx_new_tensor: unsupported type %d", type);
        return nullptr;
    }
    auto t = std::make_unique<wamx_tensor>();
    memset(t.get(), 0, sizeof(wamx_tensor));
    t->type = type;
    for (int i = 0; i < WAMX_MAX_DIMS; ++i) t->ne[i] = i < n_dims ? ne[i] : 1;
    t->nb[0] = wamx_type_size(type);
    for (int i = 1; i < WAMX_MAX_DIMS; ++i) t->nb[i] = t->nb[i - 1] * (size_t)t->ne[i - 1];
    t->op = WAMX_OP_NONE;
    t->lane = ctx->lane;
    wamx_tensor * raw = t.get();
    ctx->tensors.push_back(std::move(t));
    return raw;
}

// A tensor that aliases `a` (same buffer memory) with its own shape/strides.
static wamx_tensor * view_impl(wamx_context * ctx, wamx_tensor * a, int n_dims, const int64_t * ne, size_t offset) {
    if (!a) return nullptr;
    wamx_tensor * t = new_tensor_impl(ctx, a->type, n_dims, ne);
    if (!t) return nullptr;
    t->view_src = a->view_src ? a->view_src : a;
    t->view_offs = a->view_offs + offset;
    t->buffer = a->buffer;
    if (a->data) t->data = (char *) a->data + offset;
    t->op = WAMX_OP_VIEW;
    t->src[0] = a;
    return t;
}

static bool is_bf16(const wamx_tensor * t) { return t && t->type == WAMX_TYPE_BF16; }
static bool is_f32(const wamx_tensor * t) { return t && t->type == WAMX_TYPE_F32; }

static wamx_tensor * fail(const char * what) {
    set_errorf("%s: invalid arguments", what);
    return nullptr;
}

static void set_param_f32(wamx_tensor * t, int i, float v) { memcpy(&t->op_params[i], &v, 4); }

namespace wamx {

// Node validators shared by the constructors and supports_op: a graph
// mirrored from ggml (wamx_graph_from_ggml) or built by hand reaches
// graph_compute without going through the constructors.  Each returns null
// when the node is well formed, else the reason.
static bool contig(const wamx_tensor * t) { return t && wamx_is_contiguous(t); }

const char * check_linear(const wamx_tensor * t) {
    const wamx_tensor *w = t->src[0], *x = t->src[1], *bias = t->src[2], *res = t->src[3], *gate = t->src[4];
    const int32_t epi = t->op_params[0];
    if (!is_bf16(w) || !x || (x->type != WAMX_TYPE_BF16 && x->type != WAMX_TYPE_F32)) return "types";
    if (w->ne[0] != x->ne[0] || w->ne[2] != 1 || w->ne[3] != 1 || x->ne[2] != 1 || x->ne[3] != 1) return "shapes";
    if (w->nb[0] != 2 || x->nb[0] != wamx_type_size(x->type)) return "rows must be contiguous";
    const int64_t M = w->ne[1], N = x->ne[1];
    if (epi < WAMX_EPI_NONE || epi > WAMX_EPI_BIAS_RESIDUAL) return "epilogue";
    if (epi != WAMX_EPI_NONE && (!is_bf16(bias) || bias->ne[0] != M || bias->nb[0] != 2)) return "bias";
    if (epi == WAMX_EPI_BIAS_GATED || epi == WAMX_EPI_BIAS_RESIDUAL) {
        if (!is_bf16(res) || res->ne[0] != M || res->ne[1] != N || res->nb[0] != 2) return "residual";
    }
    if (epi == WAMX_EPI_BIAS_GATED && (!is_f32(gate) || gate->ne[0] != M || gate->nb[0] != 4)) return "gate";
    if (!is_bf16(t) || t->ne[0] != M || t->ne[1] != N || !contig(t)) return "output";
    return nullptr;
}

const char * check_qk_norm_rope(const wamx_tensor * t) {
    const wamx_tensor *x = t->src[0], *weight = t->src[1], *dst = t->src[2];
    if (!is_bf16(x) || !is_bf16(weight) || !is_bf16(dst) || !is_bf16(t)) return "types";
    // dst [dh, tokens, H, C]: C chunks of T tokens.  x is [d, C*T] (the
    // chunks' rows one after another) or [d, T, C] (chunk c's rows x->nb[2]
    // bytes apart, e.g. column ranges of a packed projection); weight is one
    // norm weight [d] or one per chunk [d, C].  Hi/lo form (op_params[4] = 1):
    // dst [dh, tokens, H, 2C] holds for chunk c the bf16 rounding of the f32
    // result in plane 2c and the rest in plane 2c + 1.
    const bool hilo = t->op_params[4] != 0;
    const int64_t dh = dst->ne[0], H = dst->ne[2];
    if (hilo && (dst->ne[3] % 2 != 0 || dst->ne[3] < 2)) return "hi/lo destination needs two planes per chunk";
    const int64_t C = hilo ? dst->ne[3] / 2 : dst->ne[3];
    const bool layered = x->ne[2] > 1;
    if (C < 1 || x->ne[3] != 1 || (layered ? x->ne[2] != C : x->ne[1] % C != 0))
        return "rows must split into the destination's chunks";
    const int64_t T = layered ? x->ne[1] : x->ne[1] / C;
    if (x->ne[0] != dh * H || weight->ne[0] != x->ne[0] || x->nb[0] != 2 || weight->nb[0] != 2 || (dh & 1))
        return "shapes";
    if (weight->ne[2] != 1 || weight->ne[3] != 1 || (weight->ne[1] != 1 && weight->ne[1] != C))
        return "norm weight: one row, or one per chunk";
    // Destination chunks are contiguous [dh, tokens, H] blocks, 16-byte
    // aligned apart (any distance); hi/lo planes are contiguous throughout.
    if (dst->nb[0] != 2 || dst->nb[1] != (size_t) dh * 2 || dst->nb[2] != dst->nb[1] * (size_t) dst->ne[1] ||
        (C > 1 && (dst->nb[3] < dst->nb[2] * (size_t) H || dst->nb[3] % 16 != 0)) || (hilo && !contig(dst)))
        return "destination layout";
    if ((layered || weight->ne[1] > 1) &&
        (x->nb[1] % 16 != 0 || x->nb[2] % 16 != 0 || (weight->ne[1] > 1 && weight->nb[1] % 16 != 0)))
        return "per-chunk rows and weights need 16-byte strides";
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] != dst->ne[i] || t->nb[i] != dst->nb[i]) return "result must be the destination";
    const int64_t tok0 = t->op_params[0];
    const int rope_mode = t->op_params[1];
    if (tok0 < 0 || tok0 + T > dst->ne[1]) return "token range";
    if (rope_mode < 0 || rope_mode > 3) return "rope mode";
    auto pos_ok = [T](const wamx_tensor * p) { return p && p->type == WAMX_TYPE_I32 && p->ne[0] == T && p->nb[0] == 4; };
    // Rope mode 3: a table of (cos, sin) per pair, f32 [head_dim, T].
    if (rope_mode == 3 && (!t->src[3] || !is_f32(t->src[3]) || t->src[3]->ne[0] != dh || t->src[3]->ne[1] != T ||
                           !contig(t->src[3]) || dh % 8 != 0))
        return "rope table";
    if (rope_mode == 0 && !pos_ok(t->src[3])) return "positions";
    if (rope_mode == 1 && (dh != 128 || !pos_ok(t->src[3]) || !pos_ok(t->src[4]) || !pos_ok(t->src[5])))
        return "3-D rope needs head_dim 128 and three position streams";
    return nullptr;
}

const char * check_joint_attn(const wamx_tensor * t) {
    const wamx_tensor *q = t->src[0], *k_a = t->src[1], *v_a = t->src[2], *k_b = t->src[3], *v_b = t->src[4];
    if (!is_bf16(q) || !is_bf16(k_a) || !is_bf16(v_a)) return "types";
    if (t->op_params[2]) {
        // f32-accurate scores from hi/lo planes: q [dh, Tq, H, 2], k [dh, nk, H, 2],
        // V^T [nk, dh, H] with rows of a multiple of 8 keys; one key source.
        const int64_t dh = q->ne[0], Tq = q->ne[1], H = q->ne[2], nk = k_a->ne[1];
        if (dh != 128) return "head_dim must be 128";
        if (q->ne[3] != 2 || k_a->ne[3] != 2 || k_a->ne[0] != dh || k_a->ne[2] != H || !contig(q) || !contig(k_a))
            return "hi/lo q and k: two contiguous planes";
        if (k_b || v_b || t->op_params[0] != 0) return "hi/lo scores take one key source";
        if (nk < 8) return "hi/lo scores need at least 8 keys";
        if (v_a->ne[0] != nk || v_a->ne[1] != dh || v_a->ne[2] != H || v_a->ne[3] != 1 || v_a->nb[0] != 2 ||
            v_a->nb[1] % 16 != 0 || v_a->nb[1] < (size_t) nk * 2 || v_a->nb[2] != v_a->nb[1] * (size_t) dh)
            return "V^T layout";
        if (!is_bf16(t) || t->ne[0] != dh * H || t->ne[1] != Tq || t->ne[2] != 1 || t->ne[3] != 1 || !contig(t))
            return "output";
        return nullptr;
    }
    // dim 3 is the chunk: B independent key sets and query sets.
    const int64_t dh = q->ne[0], Tq = q->ne[1], H = q->ne[2], B = q->ne[3];
    const int64_t na = k_a->ne[1];
    if (dh != 128) return "head_dim must be 128";
    if (k_a->ne[0] != dh || k_a->ne[2] != H || k_a->ne[3] != B || v_a->ne[0] != na || v_a->ne[1] != dh ||
        v_a->ne[2] != H || v_a->ne[3] != B)
        return "kv_a shapes";
    if ((k_b == nullptr) != (v_b == nullptr)) return "kv_b pair";
    if (k_b) {
        const int64_t nb = k_b->ne[1];
        if (!is_bf16(k_b) || !is_bf16(v_b) || k_b->ne[0] != dh || k_b->ne[2] != H || k_b->ne[3] != B ||
            v_b->ne[0] != nb || v_b->ne[1] != dh || v_b->ne[2] != H || v_b->ne[3] != B)
            return "kv_b shapes";
    }
    if (na + (k_b ? k_b->ne[1] : 0) <= 0) return "no keys (softmax over an empty key set)";
    const int64_t na_split = t->op_params[0];
    if (na_split < 0 || na_split > na) return "split";
    for (const wamx_tensor * s : {q, k_a, k_b})
        if (s && !contig(s)) return "q and k must be contiguous";
    // V^T rows may be padded: 8-byte aligned row stride covering ne[0] keys;
    // heads and chunks follow each other.
    for (const wamx_tensor * s : {v_a, v_b})
        if (s && (s->nb[0] != 2 || s->nb[1] % 8 != 0 || s->nb[1] < (size_t) s->ne[0] * 2 ||
                  s->nb[2] != s->nb[1] * (size_t) s->ne[1] || s->nb[3] != s->nb[2] * (size_t) s->ne[2]))
            return "V^T layout";
    if (!is_bf16(t) || t->ne[0] != dh * H || t->ne[1] != Tq || t->ne[2] != B || t->ne[3] != 1 || !contig(t))
        return "output";
    return nullptr;
}

const char * check_modulation(const wamx_tensor * t) {
    const wamx_tensor *mod = t->src[0], *tables = t->src[1];
    if (!mod || !tables || !contig(mod) || !contig(tables)) return "contiguous operands";
    if ((mod->type != WAMX_TYPE_BF16 && mod->type != WAMX_TYPE_F32) ||
        (tables->type != WAMX_TYPE_BF16 && tables->type != WAMX_TYPE_F32))
        return "types";
    // mod holds S columns of ne0 * ne1 values (S timesteps): one output
    // [ne0, ne1, L] per column.
    const int64_t per = tables->ne[0] * tables->ne[1];
    if (per <= 0 || wamx_nelements(mod) % per != 0) return "sizes";
    const int64_t S = wamx_nelements(mod) / per;
    if (!is_f32(t) || !contig(t) || wamx_nelements(t) != wamx_nelements(tables) * S || t->ne[3] != S) return "output";
    return nullptr;
}

const char * check_euler_step(const wamx_tensor * t) {
    const wamx_tensor *a = t->src[0], *v = t->src[1], *dt = t->src[2];
    if (!is_bf16(a) || !is_bf16(v) || !is_f32(dt) || !is_bf16(t)) return "types (bf16 action and velocity, f32 dt)";
    if (!wamx_are_same_shape(a, v) || !wamx_are_same_shape(a, t) || !contig(a) || !contig(v) || !contig(t))
        return "action, velocity and output: one contiguous shape";
    if (wamx_nelements(dt) != 1) return "dt is one value";
    return nullptr;
}

const char * check_mlp_small(const wamx_tensor * t) {
    const wamx_tensor *x = t->src[0], *w1 = t->src[1], *b1 = t->src[2], *w2 = t->src[3], *b2 = t->src[4];
    if (!is_bf16(x) || !is_bf16(w1) || !is_bf16(b1) || !is_bf16(w2) || !is_bf16(b2) || !is_bf16(t)) return "types";
    const int64_t K0 = x->ne[0], N = x->ne[1], M1 = w1->ne[1], M2 = w2->ne[1];
    if (w1->ne[0] != K0 || w2->ne[0] != M1 || b1->ne[0] != M1 || b2->ne[0] != M2) return "shapes";
    if (K0 < 1 || M1 < 1 || M2 < 1 || K0 > 128 || M1 > 128 || M2 > 128) return "widths must be 1..128";
    if (x->ne[2] != 1 || x->ne[3] != 1 || w1->ne[2] != 1 || w2->ne[2] != 1 || !contig(x) || !contig(w1) ||
        !contig(w2) || !contig(b1) || !contig(b2))
        return "contiguous 2-D operands";
    if (t->ne[0] != M2 || t->ne[1] != N || t->ne[2] != 1 || t->ne[3] != 1 || !contig(t)) return "output";
    if (t->op_params[0] & ~7) return "flags";
    return nullptr;
}

// ggml_im2col, 2-D only: op_params {s0, s1, p0, p1, d0, d1, is_2D}, kernel
// shape from src[0]->ne, f32 input src[1].
const char * check_im2col(const wamx_tensor * t) {
    const wamx_tensor *kernel = t->src[0], *input = t->src[1];
    const int32_t * p = t->op_params;
    if (!kernel || !is_f32(input) || (t->type != WAMX_TYPE_F32 && t->type != WAMX_TYPE_BF16)) return "types";
    if (p[6] != 1) return "only the 2-D form";
    if (p[0] < 1 || p[1] < 1 || p[4] < 1 || p[5] < 1 || p[2] < 0 || p[3] < 0) return "stride/padding/dilation";
    const int64_t KW = kernel->ne[0], KH = kernel->ne[1], IC = input->ne[2];
    if (kernel->ne[2] != IC) return "channels";
    const int64_t OW = (input->ne[0] + 2 * p[2] - p[4] * (KW - 1) - 1) / p[0] + 1;
    const int64_t OH = (input->ne[1] + 2 * p[3] - p[5] * (KH - 1) - 1) / p[1] + 1;
    if (OW <= 0 || OH <= 0 || t->ne[0] != IC * KH * KW || t->ne[1] != OW || t->ne[2] != OH || t->ne[3] != input->ne[3])
        return "output shape";
    return nullptr;
}

// ggml_conv_2d_direct: kernel [KW,KH,IC,OC], input [IW,IH,IC,N] of one type
// (bf16 or f32, contiguous), dst [OW,OH,OC,N] of that type, op_params
// {s0, s1, p0, p1, d0, d1}.
const char * check_conv_2d(const wamx_tensor * t) {
    const wamx_tensor *kernel = t->src[0], *input = t->src[1];
    const int32_t * p = t->op_params;
    if (!kernel || !input) return "operands";
    if (!((kernel->type == WAMX_TYPE_BF16 && input->type == WAMX_TYPE_BF16) ||
          (kernel->type == WAMX_TYPE_F32 && input->type == WAMX_TYPE_F32)) ||
        t->type != input->type)
        return "types (bf16 or f32 throughout)";
    if (!wamx_is_contiguous(kernel) || !wamx_is_contiguous(input) || !wamx_is_contiguous(t)) return "layout";
    if (p[0] < 1 || p[1] < 1 || p[4] < 1 || p[5] < 1 || p[2] < 0 || p[3] < 0) return "stride/padding/dilation";
    const int64_t KW = kernel->ne[0], KH = kernel->ne[1];
    if (kernel->ne[2] != input->ne[2]) return "channels";
    const int64_t OW = (input->ne[0] + 2 * p[2] - p[4] * (KW - 1) - 1) / p[0] + 1;
    const int64_t OH = (input->ne[1] + 2 * p[3] - p[5] * (KH - 1) - 1) / p[1] + 1;
    if (OW <= 0 || OH <= 0 || t->ne[0] != OW || t->ne[1] != OH || t->ne[2] != kernel->ne[3] ||
        t->ne[3] != input->ne[3])
        return "output shape";
    return nullptr;
}

}  // namespace wamx

// Builds node `t` of an op validated by `check`; on failure the (unlinked)
// tensor stays in the context and NULL is returned with the reason.
static wamx_tensor * checked(wamx_tensor * t, const char * (*check)(const wamx_tensor *), const char * what) {
    if (!t) return nullptr;
    const char * why = check(t);
    if (why) {
        set_errorf("%s: %s", what, why);
        return nullptr;
    }
    return t;
}

extern "C" {

const char * wamx_last_error(void) { return last_error_cstr(); }

wamx_context * wamx_init(size_t max_tensors) {
    auto * ctx = new (std::nothrow) wamx_context();
    if (!ctx) return nullptr;
    ctx->max_tensors = max_tensors ? max_tensors : 4096;
    ctx->tensors.reserve(std::min<size_t>(ctx->max_tensors, 1u << 16));
    return ctx;
}

void wamx_free(wamx_context * ctx) { delete ctx; }

size_t wamx_type_size(int32_t type) {
    switch (type) {
        case WAMX_TYPE_F32: return 4;
        case WAMX_TYPE_F16: return 2;
        case WAMX_TYPE_BF16: return 2;
        case WAMX_TYPE_I32: return 4;
        default: return 0;
    }
}

const char * wamx_type_name(int32_t type) {
    switch (type) {
        case WAMX_TYPE_F32: return "f32";
        case WAMX_TYPE_F16: return "f16";
        case WAMX_TYPE_BF16: return "bf16";
        case WAMX_TYPE_I32: return "i32";
        default: return "unknown";
    }
}

const char * wamx_op_name(int32_t op) {
    static const char * names[WAMX_OP_COUNT] = {
        "NONE", "DUP", "ADD", "MUL", "SCALE", "CPY", "CONT", "RESHAPE", "VIEW", "PERMUTE",
        "TRANSPOSE", "CONCAT", "REPEAT", "NORM", "RMS_NORM", "MUL_MAT", "SOFT_MAX", "ROPE",
        "UNARY", "GET_ROWS", "IM2COL", "CONV_2D", "LINEAR", "QK_NORM_ROPE", "JOINT_ATTN", "MODULATION",
        "EULER_STEP", "MLP_SMALL",
    };
    return (op >= 0 && op < WAMX_OP_COUNT) ? names[op] : "?";
}

int64_t wamx_nelements(const wamx_tensor * t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
int64_t wamx_nrows(const wamx_tensor * t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

size_t wamx_nbytes(const wamx_tensor * t) {
    // Span of memory touched: 1 element + sum of (ne-1)*nb over dims.
    if (wamx_nelements(t) == 0) return 0;
    size_t n = wamx_type_size(t->type);
    for (int i = 0; i < WAMX_MAX_DIMS; ++i) n += (size_t)(t->ne[i] - 1) * t->nb[i];
    return n;
}

bool wamx_is_contiguous(const wamx_tensor * t) {
    size_t expect = wamx_type_size(t->type);
    for (int i = 0; i < WAMX_MAX_DIMS; ++i) {
        if (t->ne[i] != 1 && t->nb[i] != expect) return false;
        expect *= (size_t)t->ne[i];
    }
    return true;
}

bool wamx_are_same_shape(const wamx_tensor * a, const wamx_tensor * b) {
    for (int i = 0; i < WAMX_MAX_DIMS; ++i)
        if (a->ne[i] != b->ne[i]) return false;
    return true;
}

void wamx_set_name(wamx_tensor * t, const char * name) {
    if (!t) return;
    snprintf(t->name, sizeof t->name, "%s", name ? name : "");
}
void wamx_set_input(wamx_tensor * t) { if (t) t->flags |= WAMX_TENSOR_FLAG_INPUT; }
void wamx_set_output(wamx_tensor * t) { if (t) t->flags |= WAMX_TENSOR_FLAG_OUTPUT; }

void wamx_set_lane(wamx_context * ctx, int lane) {
    if (ctx) ctx->lane = lane ? 1 : 0;
}

wamx_tensor * wamx_new_tensor(wamx_context * ctx, int32_t type, int n_dims, const int64_t * ne) {
    if (n_dims < 1 || n_dims > WAMX_MAX_DIMS) return fail("wamx_new_tensor");
    return new_tensor_impl(ctx, type, n_dims, ne);
}
wamx_tensor * wamx_new_tensor_1d(wamx_context * ctx, int32_t type, int64_t ne0) {
    int64_t ne[1] = {ne0};
    return new_tensor_impl(ctx, type, 1, ne);
}
wamx_tensor * wamx_new_tensor_2d(wamx_context * ctx, int32_t type, int64_t ne0, int64_t ne1) {
    int64_t ne[2] = {ne0, ne1};
    return new_tensor_impl(ctx, type, 2, ne);
}
wamx_tensor * wamx_new_tensor_3d(wamx_context * ctx, int32_t type, int64_t ne0, int64_t ne1, int64_t ne2) {
    int64_t ne[3] = {ne0, ne1, ne2};
    return new_tensor_impl(ctx, type, 3, ne);
}
wamx_tensor * wamx_new_tensor_4d(wamx_context * ctx, int32_t type, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return new_tensor_impl(ctx, type, 4, ne);
}

// ---------------------------------------------------------------------------
// Views
// ---------------------------------------------------------------------------
wamx_tensor * wamx_view_1d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, size_t offset) {
    int64_t ne[1] = {ne0};
    return view_impl(ctx, a, 1, ne, offset);
}
wamx_tensor * wamx_view_2d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, size_t nb1, size_t offset) {
    int64_t ne[2] = {ne0, ne1};
    wamx_tensor * t = view_impl(ctx, a, 2, ne, offset);
    if (!t) return nullptr;
    t->nb[1] = nb1;
    t->nb[2] = nb1 * (size_t)ne1;
    t->nb[3] = t->nb[2];
    return t;
}
wamx_tensor * wamx_view_3d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, size_t nb1,
                           size_t nb2, size_t offset) {
    int64_t ne[3] = {ne0, ne1, ne2};
    wamx_tensor * t = view_impl(ctx, a, 3, ne, offset);
    if (!t) return nullptr;
    t->nb[1] = nb1;
    t->nb[2] = nb2;
    t->nb[3] = nb2 * (size_t)ne2;
    return t;
}
wamx_tensor * wamx_view_4d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3,
                           size_t nb1, size_t nb2, size_t nb3, size_t offset) {
    int64_t ne[4] = {ne0, ne1, ne2, ne3};
    wamx_tensor * t = view_impl(ctx, a, 4, ne, offset);
    if (!t) return nullptr;
    t->nb[1] = nb1;
    t->nb[2] = nb2;
    t->nb[3] = nb3;
    return t;
}

static wamx_tensor * reshape_impl(wamx_context * ctx, wamx_tensor * a, int n, const int64_t * ne) {
    if (!a || !wamx_is_contiguous(a)) return fail("wamx_reshape (source must be contiguous)");
    int64_t total = 1;
    for (int i = 0; i < n; ++i) total *= ne[i];
    if (total != wamx_nelements(a)) return fail("wamx_reshape (element count)");
    wamx_tensor * t = view_impl(ctx, a, n, ne, 0);
    if (t) t->op = WAMX_OP_RESHAPE;
    return t;
}
wamx_tensor * wamx_reshape_2d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1) {
    int64_t ne[2] = {ne0, ne1};
    return reshape_impl(ctx, a, 2, ne);
}
wamx_tensor * wamx_reshape_3d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2) {
    int64_t ne[3] = {ne0, ne1, ne2};
    return reshape_impl(ctx, a, 3, ne);
}
wamx_tensor * wamx_reshape_4d(wamx_context * ctx, wamx_tensor * a, int64_t ne0, int64_t ne1, int64_t ne2, int64_t ne3) {
    int64_t ne[4] = {ne0, ne1, ne2, ne3};
    return reshape_impl(ctx, a, 4, ne);
}

// Source dim i moves to position axis_i (ggml_permute convention).
wamx_tensor * wamx_permute(wamx_context * ctx, wamx_tensor * a, int axis0, int axis1, int axis2, int axis3) {
    const int ax[4] = {axis0, axis1, axis2, axis3};
    bool seen[4] = {false, false, false, false};
    for (int i = 0; i < 4; ++i) {
        if (ax[i] < 0 || ax[i] > 3 || seen[ax[i]]) return fail("wamx_permute");
        seen[ax[i]] = true;
    }
    wamx_tensor * t = view_impl(ctx, a, 4, a->ne, 0);
    if (!t) return nullptr;
    for (int i = 0; i < 4; ++i) {
        t->ne[ax[i]] = a->ne[i];
        t->nb[ax[i]] = a->nb[i];
    }
    t->op = WAMX_OP_PERMUTE;
    for (int i = 0; i < 4; ++i) t->op_params[i] = ax[i];
    return t;
}

wamx_tensor * wamx_transpose(wamx_context * ctx, wamx_tensor * a) {
    wamx_tensor * t = wamx_permute(ctx, a, 1, 0, 2, 3);
    if (t) t->op = WAMX_OP_TRANSPOSE;
    return t;
}

// ---------------------------------------------------------------------------
// Compute ops
// ---------------------------------------------------------------------------
static wamx_tensor * unary_result(wamx_context * ctx, wamx_tensor * a, int32_t op) {
    if (!a) return fail(wamx_op_name(op));
    wamx_tensor * t = new_tensor_impl(ctx, a->type, 4, a->ne);
    if (!t) return nullptr;
    t->op = op;
    t->src[0] = a;
    return t;
}

wamx_tensor * wamx_dup(wamx_context * ctx, wamx_tensor * a) { return unary_result(ctx, a, WAMX_OP_DUP); }
wamx_tensor * wamx_cont(wamx_context * ctx, wamx_tensor * a) { return unary_result(ctx, a, WAMX_OP_CONT); }

wamx_tensor * wamx_cast(wamx_context * ctx, wamx_tensor * a, int32_t type) {
    if (!a) return fail("wamx_cast");
    wamx_tensor * t = new_tensor_impl(ctx, type, 4, a->ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_CPY;
    t->src[0] = a;
    return t;
}

// Copy a into the memory of b (ggml_cpy): the result is a view of b.
wamx_tensor * wamx_cpy(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b) {
    if (!a || !b || wamx_nelements(a) != wamx_nelements(b)) return fail("wamx_cpy");
    wamx_tensor * t = view_impl(ctx, b, 4, b->ne, 0);
    if (!t) return nullptr;
    memcpy(t->nb, b->nb, sizeof t->nb);
    t->op = WAMX_OP_CPY;
    t->src[0] = a;
    t->src[1] = b;
    return t;
}

wamx_tensor * wamx_concat(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b, int dim) {
    if (!a || !b || a->type != b->type || dim < 0 || dim > 3) return fail("wamx_concat");
    for (int i = 0; i < 4; ++i)
        if (i != dim && a->ne[i] != b->ne[i]) return fail("wamx_concat (shape)");
    int64_t ne[4] = {a->ne[0], a->ne[1], a->ne[2], a->ne[3]};
    ne[dim] += b->ne[dim];
    wamx_tensor * t = new_tensor_impl(ctx, a->type, 4, ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_CONCAT;
    t->op_params[0] = dim;
    t->src[0] = a;
    t->src[1] = b;
    return t;
}

static bool can_repeat(const wamx_tensor * small, const wamx_tensor * big) {
    for (int i = 0; i < 4; ++i)
        if (small->ne[i] == 0 || big->ne[i] % small->ne[i] != 0) return false;
    return true;
}

wamx_tensor * wamx_repeat(wamx_context * ctx, wamx_tensor * a, wamx_tensor * shape) {
    if (!a || !shape || !can_repeat(a, shape)) return fail("wamx_repeat");
    wamx_tensor * t = new_tensor_impl(ctx, a->type, 4, shape->ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_REPEAT;
    t->src[0] = a;
    return t;
}

static wamx_tensor * binary_impl(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b, int32_t op) {
    if (!a || !b || !can_repeat(b, a)) return fail(wamx_op_name(op));
    wamx_tensor * t = new_tensor_impl(ctx, a->type, 4, a->ne);
    if (!t) return nullptr;
    t->op = op;
    t->src[0] = a;
    t->src[1] = b;
    return t;
}
wamx_tensor * wamx_add(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b) { return binary_impl(ctx, a, b, WAMX_OP_ADD); }
wamx_tensor * wamx_mul(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b) { return binary_impl(ctx, a, b, WAMX_OP_MUL); }

wamx_tensor * wamx_scale(wamx_context * ctx, wamx_tensor * a, float s) {
    wamx_tensor * t = unary_result(ctx, a, WAMX_OP_SCALE);
    if (t) {
        set_param_f32(t, 0, s);
        set_param_f32(t, 1, 0.0f);
    }
    return t;
}

static wamx_tensor * unary_op(wamx_context * ctx, wamx_tensor * a, int32_t which) {
    wamx_tensor * t = unary_result(ctx, a, WAMX_OP_UNARY);
    if (t) t->op_params[0] = which;
    return t;
}
wamx_tensor * wamx_gelu(wamx_context * ctx, wamx_tensor * a) { return unary_op(ctx, a, WAMX_UNARY_GELU); }
wamx_tensor * wamx_gelu_erf(wamx_context * ctx, wamx_tensor * a) { return unary_op(ctx, a, WAMX_UNARY_GELU_ERF); }
wamx_tensor * wamx_silu(wamx_context * ctx, wamx_tensor * a) { return unary_op(ctx, a, WAMX_UNARY_SILU); }

wamx_tensor * wamx_norm(wamx_context * ctx, wamx_tensor * a, float eps) {
    if (!is_f32(a)) return fail("wamx_norm (f32 input)");
    wamx_tensor * t = unary_result(ctx, a, WAMX_OP_NORM);
    if (t) set_param_f32(t, 0, eps);
    return t;
}
wamx_tensor * wamx_rms_norm(wamx_context * ctx, wamx_tensor * a, float eps) {
    if (!is_f32(a)) return fail("wamx_rms_norm (f32 input)");
    wamx_tensor * t = unary_result(ctx, a, WAMX_OP_RMS_NORM);
    if (t) set_param_f32(t, 0, eps);
    return t;
}

// ggml_mul_mat_out_type (native-bf16.patch:566-592): ne = {a.ne1, b.ne1, b.ne2, b.ne3}.
wamx_tensor * wamx_mul_mat_out_type(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b, int32_t type) {
    if (!a || !b) return fail("wamx_mul_mat");
    const bool can = a->ne[0] == b->ne[0] && b->ne[2] % a->ne[2] == 0 && b->ne[3] % a->ne[3] == 0;
    if (!can) return fail("wamx_mul_mat (shapes)");
    if (a->nb[0] > a->nb[1]) return fail("wamx_mul_mat (transposed a)");
    if (type != WAMX_TYPE_F32 && type != WAMX_TYPE_BF16) return fail("wamx_mul_mat (output type)");
    int64_t ne[4] = {a->ne[1], b->ne[1], b->ne[2], b->ne[3]};
    wamx_tensor * t = new_tensor_impl(ctx, type, 4, ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_MUL_MAT;
    t->src[0] = a;
    t->src[1] = b;
    return t;
}
wamx_tensor * wamx_mul_mat(wamx_context * ctx, wamx_tensor * a, wamx_tensor * b) {
    return wamx_mul_mat_out_type(ctx, a, b, WAMX_TYPE_F32);
}
void wamx_mul_mat_set_prec(wamx_tensor * a, int32_t prec) {
    if (a) a->op_params[0] = prec;
}

// ggml_soft_max_ext: mask rows i1, broadcast over dims 2 and 3 by modulo.
wamx_tensor * wamx_soft_max_ext(wamx_context * ctx, wamx_tensor * a, wamx_tensor * mask, float scale, float max_bias) {
    if (!is_f32(a) || max_bias != 0.0f) return fail("wamx_soft_max_ext (f32, no ALiBi)");
    if (mask && ((mask->type != WAMX_TYPE_F32 && mask->type != WAMX_TYPE_F16) || mask->ne[0] != a->ne[0] ||
                 mask->ne[1] < a->ne[1] || a->ne[2] % mask->ne[2] != 0 || a->ne[3] % mask->ne[3] != 0))
        return fail("wamx_soft_max_ext (mask: f32/f16, ne0 = a.ne0, ne1 >= a.ne1, broadcast over dims 2, 3)");
    wamx_tensor * t = unary_result(ctx, a, WAMX_OP_SOFT_MAX);
    if (!t) return nullptr;
    t->src[1] = mask;
    set_param_f32(t, 0, scale);
    set_param_f32(t, 1, max_bias);
    return t;
}

// ggml_rope_ext op_params layout: [n_past, n_dims, mode, n_ctx, n_ctx_orig,
// freq_base, freq_scale, ext_factor, attn_factor, beta_fast, beta_slow].
wamx_tensor * wamx_rope_ext(wamx_context * ctx, wamx_tensor * a, wamx_tensor * positions, wamx_tensor * freq_factors,
                            int n_dims, int mode, int n_ctx_orig, float freq_base, float freq_scale,
                            float ext_factor, float attn_factor, float beta_fast, float beta_slow) {
    if (!a || !positions || positions->type != WAMX_TYPE_I32 || positions->ne[0] != a->ne[2])
        return fail("wamx_rope_ext");
    if (freq_factors || mode != 0 || (n_dims & 1) || n_dims > a->ne[0])
        return fail("wamx_rope_ext (only NORMAL mode without freq factors)");
    if (!is_f32(a)) return fail("wamx_rope_ext (f32 input)");
    int64_t ne[4] = {a->ne[0], a->ne[1], a->ne[2], a->ne[3]};
    wamx_tensor * t = new_tensor_impl(ctx, a->type, 4, ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_ROPE;
    t->src[0] = a;
    t->src[1] = positions;
    t->op_params[0] = 0;
    t->op_params[1] = n_dims;
    t->op_params[2] = mode;
    t->op_params[3] = 0;
    t->op_params[4] = n_ctx_orig;
    set_param_f32(t, 5, freq_base);
    set_param_f32(t, 6, freq_scale);
    set_param_f32(t, 7, ext_factor);
    set_param_f32(t, 8, attn_factor);
    set_param_f32(t, 9, beta_fast);
    set_param_f32(t, 10, beta_slow);
    return t;
}

wamx_tensor * wamx_get_rows(wamx_context * ctx, wamx_tensor * a, wamx_tensor * rows) {
    if (!a || !rows || rows->type != WAMX_TYPE_I32) return fail("wamx_get_rows");
    int64_t ne[4] = {a->ne[0], rows->ne[0], rows->ne[1], rows->ne[2]};
    wamx_tensor * t = new_tensor_impl(ctx, WAMX_TYPE_F32, 4, ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_GET_ROWS;
    t->src[0] = a;
    t->src[1] = rows;
    return t;
}

wamx_tensor * wamx_im2col(wamx_context * ctx, wamx_tensor * kernel, wamx_tensor * input, int s0, int s1, int p0,
                          int p1, int d0, int d1, int32_t dst_type) {
    if (!kernel || !input || s0 < 1 || s1 < 1 || d0 < 1 || d1 < 1) return fail("wamx_im2col");
    const int64_t KW = kernel->ne[0], KH = kernel->ne[1], IC = input->ne[2];
    const int64_t OW = (input->ne[0] + 2 * p0 - d0 * (KW - 1) - 1) / s0 + 1;
    const int64_t OH = (input->ne[1] + 2 * p1 - d1 * (KH - 1) - 1) / s1 + 1;
    if (OW <= 0 || OH <= 0) return fail("wamx_im2col (output size)");
    int64_t ne[4] = {IC * KH * KW, OW, OH, input->ne[3]};
    wamx_tensor * t = new_tensor_impl(ctx, dst_type, 4, ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_IM2COL;
    // ggml's layout: {s0, s1, p0, p1, d0, d1, is_2D}; the kernel size is
    // src[0]->ne[0..1] (ggml_im2col keeps the kernel tensor as src[0]).
    const int32_t params[7] = {s0, s1, p0, p1, d0, d1, 1};
    memcpy(t->op_params, params, sizeof params);
    t->src[0] = kernel;
    t->src[1] = input;
    return checked(t, check_im2col, "wamx_im2col");
}

wamx_tensor * wamx_conv_2d_direct(wamx_context * ctx, wamx_tensor * kernel, wamx_tensor * input, int s0, int s1, int p0,
                                  int p1, int d0, int d1) {
    if (!kernel || !input || s0 < 1 || s1 < 1 || d0 < 1 || d1 < 1) return fail("wamx_conv_2d_direct");
    const int64_t KW = kernel->ne[0], KH = kernel->ne[1];
    const int64_t OW = (input->ne[0] + 2 * p0 - d0 * (KW - 1) - 1) / s0 + 1;
    const int64_t OH = (input->ne[1] + 2 * p1 - d1 * (KH - 1) - 1) / s1 + 1;
    if (OW <= 0 || OH <= 0) return fail("wamx_conv_2d_direct (output size)");
    int64_t ne[4] = {OW, OH, kernel->ne[3], input->ne[3]};
    wamx_tensor * t = new_tensor_impl(ctx, input->type, 4, ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_CONV_2D;
    const int32_t params[6] = {s0, s1, p0, p1, d0, d1};  // ggml's layout
    memcpy(t->op_params, params, sizeof params);
    t->src[0] = kernel;
    t->src[1] = input;
    return checked(t, check_conv_2d, "wamx_conv_2d_direct");
}

// --- native-bf16.patch:594-678 ---------------------------------------------
wamx_tensor * wamx_gated_residual_bf16(wamx_context * ctx, wamx_tensor * hidden, wamx_tensor * branch, wamx_tensor * gate) {
    if (!is_bf16(hidden) || !is_bf16(branch) || !gate || (gate->type != WAMX_TYPE_F32 && gate->type != WAMX_TYPE_BF16))
        return fail("wamx_gated_residual_bf16 (types)");
    if (!wamx_are_same_shape(hidden, branch) ||
        !(wamx_are_same_shape(hidden, gate) || (hidden->ne[0] == gate->ne[0] && gate->ne[1] == 1)))
        return fail("wamx_gated_residual_bf16 (shapes)");
    wamx_tensor * t = new_tensor_impl(ctx, hidden->type, 4, hidden->ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_ADD;
    t->src[0] = hidden;
    t->src[1] = branch;
    t->src[2] = gate;
    return t;
}

wamx_tensor * wamx_bias_gelu_bf16(wamx_context * ctx, wamx_tensor * input, wamx_tensor * bias) {
    if (!is_bf16(input) || !is_bf16(bias) || bias->ne[0] != input->ne[0]) return fail("wamx_bias_gelu_bf16");
    wamx_tensor * t = new_tensor_impl(ctx, input->type, 4, input->ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_UNARY;
    t->op_params[0] = WAMX_UNARY_GELU;
    t->src[0] = input;
    t->src[1] = bias;
    return t;
}

wamx_tensor * wamx_norm_modulation_bf16(wamx_context * ctx, wamx_tensor * input, wamx_tensor * scale,
                                        wamx_tensor * shift, float eps) {
    if (!is_bf16(input) || !scale || !shift || scale->type != shift->type ||
        (scale->type != WAMX_TYPE_F32 && scale->type != WAMX_TYPE_BF16))
        return fail("wamx_norm_modulation_bf16 (types)");
    if (scale->ne[0] != input->ne[0] || shift->ne[0] != input->ne[0]) return fail("wamx_norm_modulation_bf16 (shapes)");
    wamx_tensor * t = new_tensor_impl(ctx, input->type, 4, input->ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_NORM;
    set_param_f32(t, 0, eps);
    t->src[0] = input;
    t->src[1] = scale;
    t->src[2] = shift;
    return t;
}

wamx_tensor * wamx_layer_norm_bf16(wamx_context * ctx, wamx_tensor * input, wamx_tensor * weight, wamx_tensor * bias,
                                   float eps) {
    if (!is_bf16(input) || !is_bf16(weight) || !is_bf16(bias)) return fail("wamx_layer_norm_bf16 (types)");
    if (weight->ne[0] != input->ne[0] || bias->ne[0] != input->ne[0]) return fail("wamx_layer_norm_bf16 (shapes)");
    wamx_tensor * t = new_tensor_impl(ctx, input->type, 4, input->ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_NORM;
    set_param_f32(t, 0, eps);
    t->src[0] = input;
    t->src[1] = weight;
    t->src[2] = bias;
    return t;
}

wamx_tensor * wamx_rms_norm_bf16_f32(wamx_context * ctx, wamx_tensor * input, wamx_tensor * weight, float eps) {
    if (!is_bf16(input) || !is_bf16(weight) || weight->ne[0] != input->ne[0]) return fail("wamx_rms_norm_bf16_f32");
    wamx_tensor * t = new_tensor_impl(ctx, WAMX_TYPE_F32, 4, input->ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_RMS_NORM;
    set_param_f32(t, 0, eps);
    t->src[0] = input;
    t->src[1] = weight;
    return t;
}

// --- fused ops of this backend -------------------------------------------
wamx_tensor * wamx_linear(wamx_context * ctx, wamx_tensor * w, wamx_tensor * x, wamx_tensor * bias, int32_t epilogue,
                          wamx_tensor * residual, wamx_tensor * gate) {
    if (!w || !x) return fail("wamx_linear");
    wamx_tensor * t = wamx_new_tensor_2d(ctx, WAMX_TYPE_BF16, w->ne[1], x->ne[1]);
    if (!t) return nullptr;
    t->op = WAMX_OP_LINEAR;
    t->op_params[0] = epilogue;
    t->src[0] = w;
    t->src[1] = x;
    t->src[2] = epilogue != WAMX_EPI_NONE ? bias : nullptr;
    t->src[3] = (epilogue == WAMX_EPI_BIAS_GATED || epilogue == WAMX_EPI_BIAS_RESIDUAL) ? residual : nullptr;
    t->src[4] = epilogue == WAMX_EPI_BIAS_GATED ? gate : nullptr;
    return checked(t, check_linear, "wamx_linear");
}

wamx_tensor * wamx_qk_norm_rope(wamx_context * ctx, wamx_tensor * x, wamx_tensor * weight, wamx_tensor * dst,
                                int64_t tok0, int rope_mode, wamx_tensor * pos0, wamx_tensor * pos1, wamx_tensor * pos2,
                                float eps, float freq_base) {
    if (!x || !weight || !dst) return fail("wamx_qk_norm_rope");
    wamx_tensor * t = view_impl(ctx, dst, 4, dst->ne, 0);
    if (!t) return nullptr;
    memcpy(t->nb, dst->nb, sizeof t->nb);
    t->op = WAMX_OP_QK_NORM_ROPE;
    t->op_params[0] = (int32_t) tok0;
    t->op_params[1] = rope_mode;
    set_param_f32(t, 2, eps);
    set_param_f32(t, 3, freq_base);
    t->src[0] = x;
    t->src[1] = weight;
    t->src[2] = dst;
    t->src[3] = rope_mode <= 1 || rope_mode == 3 ? pos0 : nullptr;
    t->src[4] = rope_mode == 1 ? pos1 : nullptr;
    t->src[5] = rope_mode == 1 ? pos2 : nullptr;
    if (tok0 != (int64_t) t->op_params[0]) return fail("wamx_qk_norm_rope (token offset)");
    return checked(t, check_qk_norm_rope, "wamx_qk_norm_rope");
}

wamx_tensor * wamx_qk_norm_rope_hilo(wamx_context * ctx, wamx_tensor * x, wamx_tensor * weight, wamx_tensor * dst,
                                     int64_t tok0, int rope_mode, wamx_tensor * pos0, wamx_tensor * pos1,
                                     wamx_tensor * pos2, float eps, float freq_base) {
    if (!x || !weight || !dst) return fail("wamx_qk_norm_rope_hilo");
    wamx_tensor * t = view_impl(ctx, dst, 4, dst->ne, 0);
    if (!t) return nullptr;
    memcpy(t->nb, dst->nb, sizeof t->nb);
    t->op = WAMX_OP_QK_NORM_ROPE;
    t->op_params[0] = (int32_t) tok0;
    t->op_params[1] = rope_mode;
    set_param_f32(t, 2, eps);
    set_param_f32(t, 3, freq_base);
    t->op_params[4] = 1;
    t->src[0] = x;
    t->src[1] = weight;
    t->src[2] = dst;
    t->src[3] = rope_mode <= 1 || rope_mode == 3 ? pos0 : nullptr;
    t->src[4] = rope_mode == 1 ? pos1 : nullptr;
    t->src[5] = rope_mode == 1 ? pos2 : nullptr;
    if (tok0 != (int64_t) t->op_params[0]) return fail("wamx_qk_norm_rope_hilo (token offset)");
    return checked(t, check_qk_norm_rope, "wamx_qk_norm_rope_hilo");
}

wamx_tensor * wamx_joint_attn_hilo(wamx_context * ctx, wamx_tensor * q, wamx_tensor * k, wamx_tensor * v,
                                   float scale) {
    if (!q || !k || !v) return fail("wamx_joint_attn_hilo");
    wamx_tensor * t = wamx_new_tensor_3d(ctx, WAMX_TYPE_BF16, q->ne[0] * q->ne[2], q->ne[1], 1);
    if (!t) return nullptr;
    t->op = WAMX_OP_JOINT_ATTN;
    t->op_params[0] = 0;
    set_param_f32(t, 1, scale);
    t->op_params[2] = 1;
    t->src[0] = q;
    t->src[1] = k;
    t->src[2] = v;
    return checked(t, check_joint_attn, "wamx_joint_attn_hilo");
}

wamx_tensor * wamx_joint_attn(wamx_context * ctx, wamx_tensor * q, wamx_tensor * k_a, wamx_tensor * v_a,
                              wamx_tensor * k_b, wamx_tensor * v_b, int64_t na_split, float scale) {
    if (!q || !k_a || !v_a) return fail("wamx_joint_attn");
    wamx_tensor * t = wamx_new_tensor_3d(ctx, WAMX_TYPE_BF16, q->ne[0] * q->ne[2], q->ne[1], q->ne[3]);
    if (!t) return nullptr;
    t->op = WAMX_OP_JOINT_ATTN;
    t->op_params[0] = (int32_t) na_split;
    set_param_f32(t, 1, scale);
    t->src[0] = q;
    t->src[1] = k_a;
    t->src[2] = v_a;
    t->src[3] = k_b;
    t->src[4] = v_b;
    if (na_split != (int64_t) t->op_params[0]) return fail("wamx_joint_attn (split)");
    return checked(t, check_joint_attn, "wamx_joint_attn");
}

wamx_tensor * wamx_modulation(wamx_context * ctx, wamx_tensor * mod, wamx_tensor * tables) {
    if (!mod || !tables) return fail("wamx_modulation");
    const int64_t per = tables->ne[0] * tables->ne[1];
    if (per <= 0 || wamx_nelements(mod) % per != 0) return fail("wamx_modulation (sizes)");
    wamx_tensor * t = wamx_new_tensor_4d(ctx, WAMX_TYPE_F32, tables->ne[0], tables->ne[1], tables->ne[2] * tables->ne[3],
                                         wamx_nelements(mod) / per);
    if (!t) return nullptr;
    t->op = WAMX_OP_MODULATION;
    t->src[0] = mod;
    t->src[1] = tables;
    return checked(t, check_modulation, "wamx_modulation");
}

wamx_tensor * wamx_euler_step(wamx_context * ctx, wamx_tensor * action, wamx_tensor * velocity, wamx_tensor * dt) {
    if (!action || !velocity || !dt) return fail("wamx_euler_step");
    wamx_tensor * t = new_tensor_impl(ctx, WAMX_TYPE_BF16, 4, action->ne);
    if (!t) return nullptr;
    t->op = WAMX_OP_EULER_STEP;
    t->src[0] = action;
    t->src[1] = velocity;
    t->src[2] = dt;
    return checked(t, check_euler_step, "wamx_euler_step");
}

wamx_tensor * wamx_mlp_small(wamx_context * ctx, wamx_tensor * x, wamx_tensor * w1, wamx_tensor * b1, wamx_tensor * w2,
                             wamx_tensor * b2, int32_t flags) {
    if (!x || !w1 || !b1 || !w2 || !b2) return fail("wamx_mlp_small");
    wamx_tensor * t = wamx_new_tensor_2d(ctx, WAMX_TYPE_BF16, w2->ne[1], x->ne[1]);
    if (!t) return nullptr;
    t->op = WAMX_OP_MLP_SMALL;
    t->op_params[0] = flags;
    t->src[0] = x;
    t->src[1] = w1;
    t->src[2] = b1;
    t->src[3] = w2;
    t->src[4] = b2;
    return checked(t, check_mlp_small, "wamx_mlp_small");
}

// ---------------------------------------------------------------------------
// Graphs
// ---------------------------------------------------------------------------
wamx_cgraph * wamx_new_graph(wamx_context * ctx, size_t max_nodes) {
    if (!ctx) return nullptr;
    auto g = std::make_unique<wamx_cgraph>();
    g->max_nodes = max_nodes ? max_nodes : 2048;
    g->nodes.reserve(g->max_nodes);
    wamx_cgraph * raw = g.get();
    ctx->graphs.push_back(std::move(g));
    return raw;
}

static bool visit(wamx_cgraph * g, wamx_tensor * t) {
    // Iterative post-order DFS: sources before the tensor that reads them.
    std::vector<std::pair<wamx_tensor *, int>> stack;
    if (g->visited.count(t)) return true;
    stack.push_back({t, 0});
    g->visited.insert(t);
    while (!stack.empty()) {
        auto & top = stack.back();
        wamx_tensor * cur = top.first;
        bool pushed = false;
        while (top.second < WAMX_MAX_SRC) {
            wamx_tensor * s = cur->src[top.second++];
            if (s && !g->visited.count(s)) {
                g->visited.insert(s);
                stack.push_back({s, 0});
                pushed = true;
                break;
            }
        }
        if (pushed) continue;
        if (cur->op == WAMX_OP_NONE) {
            g->leafs.push_back(cur);
        } else {
            if (g->nodes.size() >= g->max_nodes) {
                set_errorf("graph full (%zu nodes)", g->max_nodes);
                return false;
            }
            g->nodes.push_back(cur);
        }
        stack.pop_back();
    }
    return true;
}

void wamx_build_forward_expand(wamx_cgraph * g, wamx_tensor * t) {
    if (g && t) visit(g, t);
}
int wamx_graph_n_nodes(const wamx_cgraph * g) { return g ? (int) g->nodes.size() : 0; }
wamx_tensor * wamx_graph_node(wamx_cgraph * g, int i) {
    if (!g) return nullptr;
    const int n = (int) g->nodes.size();
    if (i < 0) i += n;
    return (i >= 0 && i < n) ? g->nodes[i] : nullptr;
}
void wamx_graph_assign_uid(wamx_cgraph * g) {
    if (g && g->uid == 0) g->uid = g_next_graph_uid.fetch_add(1);
}
uint64_t wamx_graph_uid(const wamx_cgraph * g) { return g ? g->uid : 0; }

// ---------------------------------------------------------------------------
// ggml op correspondence by the names ggml_op_name() returns (b9866 numeric
// values are not available to verify, so nothing here depends on them).
// ---------------------------------------------------------------------------
static const struct {
    const char * ggml;
    int32_t wamx;
} k_ggml_ops[] = {
    {"NONE", WAMX_OP_NONE},         {"DUP", WAMX_OP_DUP},
    {"ADD", WAMX_OP_ADD},           {"MUL", WAMX_OP_MUL},
    {"SCALE", WAMX_OP_SCALE},       {"CPY", WAMX_OP_CPY},
    {"CONT", WAMX_OP_CONT},         {"RESHAPE", WAMX_OP_RESHAPE},
    {"VIEW", WAMX_OP_VIEW},         {"PERMUTE", WAMX_OP_PERMUTE},
    {"TRANSPOSE", WAMX_OP_TRANSPOSE}, {"CONCAT", WAMX_OP_CONCAT},
    {"REPEAT", WAMX_OP_REPEAT},     {"NORM", WAMX_OP_NORM},
    {"RMS_NORM", WAMX_OP_RMS_NORM}, {"MUL_MAT", WAMX_OP_MUL_MAT},
    {"SOFT_MAX", WAMX_OP_SOFT_MAX}, {"ROPE", WAMX_OP_ROPE},
    {"UNARY", WAMX_OP_UNARY},       {"GET_ROWS", WAMX_OP_GET_ROWS},
    {"IM2COL", WAMX_OP_IM2COL},
    {"CONV_2D", WAMX_OP_CONV_2D},
};

// ggml_backend_alloc_ctx_tensors: one buffer for every unallocated,
// non-view tensor of the context; views then alias their sources.
wamx_buffer_t wamx_backend_alloc_ctx_tensors(wamx_context * ctx, wamx_backend_t be) {
    if (!ctx || !be) return nullptr;
    return wamx_backend_alloc_ctx_tensors_from_buft(ctx, wamx_backend_get_default_buffer_type(be));
}

// ggml_backend_alloc_ctx_tensors_from_buft; every placed tensor goes through
// the buffer's init_tensor (which marks weights of a tiled buffer).
wamx_buffer_t wamx_backend_alloc_ctx_tensors_from_buft(wamx_context * ctx, wamx_buffer_type_t buft) {
    if (!ctx || !buft) return nullptr;
    const size_t align = wamx_buft_get_alignment(buft);
    size_t total = 0;
    for (auto & t : ctx->tensors)
        if (!t->data && !t->view_src) total += (wamx_nbytes(t.get()) + align - 1) / align * align;
    if (total == 0) total = align;
    wamx_buffer_t buf = wamx_buft_alloc_buffer(buft, total);
    if (!buf) return nullptr;
    char * base = (char *) wamx_buffer_get_base(buf);
    size_t off = 0;
    const wamx_buffer_i * bi = wamx_buffer_iface();
    for (auto & t : ctx->tensors) {
        if (t->data || t->view_src) continue;
        t->data = base + off;
        t->buffer = buf;
        bi->init_tensor(buf, t.get());
        off += (wamx_nbytes(t.get()) + align - 1) / align * align;
    }
    for (auto & t : ctx->tensors) {
        if (t->view_src && t->view_src->data && !t->data) {
            t->data = (char *) t->view_src->data + t->view_offs;
            t->buffer = t->view_src->buffer;
        }
    }
    return buf;
}

// ---------------------------------------------------------------------------
// Graph import from ggml descriptors (wamx_ggml_tensor).  Everything is
// matched by name, so no ggml enum value is assumed.
// ---------------------------------------------------------------------------
static int32_t ggml_type_by_name(const char * name) {
    if (!name) return -1;
    static const struct {
        const char * n;
        int32_t t;
    } types[] = {{"f32", WAMX_TYPE_F32}, {"f16", WAMX_TYPE_F16}, {"bf16", WAMX_TYPE_BF16}, {"i32", WAMX_TYPE_I32}};
    for (const auto & e : types)
        if (!strcmp(name, e.n)) return e.t;
    return -1;
}

static int32_t ggml_op_by_name(const char * name) {
    if (!name) return -1;
    for (const auto & e : k_ggml_ops)
        if (!strcmp(name, e.ggml)) return e.wamx;
    return -1;
}

// ggml_unary_op_name() strings of the unary ops this backend runs.
static int32_t ggml_unary_by_name(const char * name) {
    if (!name) return -1;
    if (!strcmp(name, "GELU")) return WAMX_UNARY_GELU;
    if (!strcmp(name, "GELU_ERF")) return WAMX_UNARY_GELU_ERF;
    if (!strcmp(name, "SILU")) return WAMX_UNARY_SILU;
    return -1;
}

wamx_cgraph * wamx_graph_from_ggml(wamx_context * ctx, const wamx_ggml_tensor * d, int n_tensors,
                                   const int32_t * graph_nodes, int n_graph_nodes) {
    if (!ctx || !d || n_tensors <= 0 || !graph_nodes || n_graph_nodes < 0) {
        set_error("wamx_graph_from_ggml: bad arguments");
        return nullptr;
    }
    std::vector<wamx_tensor *> t((size_t) n_tensors, nullptr);
    for (int i = 0; i < n_tensors; ++i) {
        const wamx_ggml_tensor & g = d[i];
        const int32_t type = ggml_type_by_name(g.type);
        const int32_t op = ggml_op_by_name(g.op);
        const char * nm = g.name ? g.name : "";
        if (type < 0) {
            set_errorf("wamx_graph_from_ggml: tensor %d '%s': unsupported type '%s'", i, nm, g.type ? g.type : "(null)");
            return nullptr;
        }
        if (op < 0) {
            set_errorf("wamx_graph_from_ggml: tensor %d '%s': unsupported op '%s'", i, nm, g.op ? g.op : "(null)");
            return nullptr;
        }
        wamx_tensor * w = new_tensor_impl(ctx, type, 4, g.ne);
        if (!w) return nullptr;
        memcpy(w->nb, g.nb, sizeof w->nb);
        w->op = op;
        memcpy(w->op_params, g.op_params, sizeof w->op_params);
        w->flags = g.flags;
        w->data = g.data;
        w->view_offs = g.view_offs;
        wamx_set_name(w, nm);
        if (op == WAMX_OP_UNARY) {
            const int32_t u = ggml_unary_by_name(g.unary_op);
            if (u < 0) {
                set_errorf("wamx_graph_from_ggml: tensor %d '%s': unsupported unary op '%s'", i, nm,
                           g.unary_op ? g.unary_op : "(null)");
                return nullptr;
            }
            w->op_params[0] = u;
        }
        t[(size_t) i] = w;
    }
    auto idx_ok = [n_tensors](int32_t k) { return k >= -1 && k < n_tensors; };
    for (int i = 0; i < n_tensors; ++i) {
        const wamx_ggml_tensor & g = d[i];
        if (!idx_ok(g.view_src)) {
            set_errorf("wamx_graph_from_ggml: tensor %d: view source index %d out of range", i, g.view_src);
            return nullptr;
        }
        t[(size_t) i]->view_src = g.view_src >= 0 ? t[(size_t) g.view_src] : nullptr;
        for (int k = 0; k < WAMX_MAX_SRC; ++k) {
            if (!idx_ok(g.src[k])) {
                set_errorf("wamx_graph_from_ggml: tensor %d: source %d index %d out of range", i, k, g.src[k]);
                return nullptr;
            }
            t[(size_t) i]->src[k] = g.src[k] >= 0 ? t[(size_t) g.src[k]] : nullptr;
        }
    }
    // A view's root is the root of its source chain, as in ggml.
    for (int i = 0; i < n_tensors; ++i) {
        wamx_tensor * w = t[(size_t) i];
        int hops = 0;
        while (w->view_src && w->view_src->view_src && hops++ < n_tensors) w->view_src = w->view_src->view_src;
        if (w->view_src) w->buffer = w->view_src->buffer;
    }
    wamx_cgraph * graph = wamx_new_graph(ctx, (size_t) n_tensors + 16);
    if (!graph) return nullptr;
    for (int i = 0; i < n_graph_nodes; ++i) {
        const int32_t k = graph_nodes[i];
        if (k < 0 || k >= n_tensors) {
            set_errorf("wamx_graph_from_ggml: graph node %d index %d out of range", i, k);
            return nullptr;
        }
        if (!visit(graph, t[(size_t) k])) return nullptr;
    }
    return graph;
}

int wamx_ggml_op_count(void) { return (int) (sizeof k_ggml_ops / sizeof k_ggml_ops[0]); }
const char * wamx_ggml_op_name(int i) { return (i >= 0 && i < wamx_ggml_op_count()) ? k_ggml_ops[i].ggml : nullptr; }
int32_t wamx_ggml_op_to_wamx(int i) { return (i >= 0 && i < wamx_ggml_op_count()) ? k_ggml_ops[i].wamx : -1; }

}  // extern "C"
