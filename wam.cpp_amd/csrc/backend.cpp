// The HIP backend of libwamx: device registry, buffer types and buffers,
// graph allocation, graph_compute dispatch with HIP-graph capture/replay, and
// the single-op entry points.  Restates the ggml backend plugin interface of
// llama.cpp b9866 (ggml-backend-impl.h: ggml_backend_i, ggml_backend_device_i,
// ggml_backend_buffer_type_i, ggml_backend_buffer_i, ggml_backend_reg_i) that
// wam.cpp's engine drives (weights.cpp:582-625, mot.cpp:526-594,
// cache.cpp:113-130).
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <map>
#include <memory>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "internal.h"

using namespace wamx;

static constexpr size_t kAlign = 256;
static constexpr size_t kWorkspaceBytes = kBackendWorkspaceBytes;

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

struct wamx_device {
    int index = 0;
    char name[32] = {0};
    char desc[256] = {0};
};

struct wamx_buffer_type {
    wamx_device * dev = nullptr;
    char name[32] = {0};
    bool tiled = false;  // weights placed here are stored MFMA-tiled (see tensor_is_tiled)
};

struct wamx_buffer {
    wamx_buffer_type * buft = nullptr;
    void * base = nullptr;
    size_t size = 0;
};

struct GraphCacheEntry {
    uint64_t signature = 0;
    int n_nodes = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

struct wamx_backend {
    wamx_device * dev = nullptr;
    hipStream_t stream = nullptr;
    void * workspace = nullptr;  // K-split partials, reused by consecutive GEMMs on the stream
    // Lane 1 of two-lane graphs: its own stream and partials workspace, made
    // on first use.  cs / cws are the stream and workspace of the node being
    // launched (lane 0's outside a two-lane graph).
    hipStream_t stream2 = nullptr;
    void * workspace2 = nullptr;
    hipStream_t cs = nullptr;
    void * cws = nullptr;
    std::vector<hipEvent_t> events;  // cross-lane ordering, reused from graph to graph
    bool use_graphs = true;
    bool fuse_rows = true;       // split-K reduce + consuming row op in one launch
    bool fuse_norm_mod_f32 = true;       // F32 NORM -> MUL -> ADD -> ADD as one launch
    bool fuse_gated_residual_f32 = true; // F32 MUL -> ADD as one launch
    std::unordered_map<uint64_t, GraphCacheEntry> graphs;
};

struct wamx_backend_reg {
    std::vector<wamx_device> devices;
    std::vector<wamx_buffer_type> bufts;
    std::vector<wamx_buffer_type> tiled_bufts;
};

// ---------------------------------------------------------------------------
// Registry
// ---------------------------------------------------------------------------
static struct wamx_backend_reg * registry() {
    static struct wamx_backend_reg * reg = [] {
        auto * r = new struct wamx_backend_reg();
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
        r->devices.resize(n);
        r->bufts.resize(n);
        r->tiled_bufts.resize(n);
        for (int i = 0; i < n; ++i) {
            r->devices[i].index = i;
            snprintf(r->devices[i].name, sizeof r->devices[i].name, "ROCm%d", i);
            hipDeviceProp_t prop;
            if (hipGetDeviceProperties(&prop, i) == hipSuccess)
                snprintf(r->devices[i].desc, sizeof r->devices[i].desc, "%s (%s, %d CUs)", prop.name, prop.gcnArchName,
                         prop.multiProcessorCount);
            r->bufts[i].dev = &r->devices[i];
            snprintf(r->bufts[i].name, sizeof r->bufts[i].name, "ROCm%d", i);
            r->tiled_bufts[i].dev = &r->devices[i];
            r->tiled_bufts[i].tiled = true;
            snprintf(r->tiled_bufts[i].name, sizeof r->tiled_bufts[i].name, "ROCm%d_Tiled", i);
        }
        return r;
    }();
    return reg;
}

// ---------------------------------------------------------------------------
// Buffer type / buffer interface
// ---------------------------------------------------------------------------
static const char * buft_get_name(wamx_buffer_type_t buft) { return buft->name; }
static size_t buft_get_alignment(wamx_buffer_type_t) { return kAlign; }
static size_t buft_get_max_size(wamx_buffer_type_t) { return SIZE_MAX; }
static size_t buft_get_alloc_size(wamx_buffer_type_t, const wamx_tensor * t) { return align_up(wamx_nbytes(t), kAlign); }
static bool buft_is_host(wamx_buffer_type_t) { return false; }

static wamx_buffer_t buft_alloc_buffer(wamx_buffer_type_t buft, size_t size) {
    if (!buft) return nullptr;
    hipSetDevice(buft->dev->index);
    auto * b = new (std::nothrow) wamx_buffer();
    if (!b) return nullptr;
    b->buft = buft;
    b->size = align_up(std::max<size_t>(size, 1), kAlign);
    if (hipMalloc(&b->base, b->size) != hipSuccess) {
        set_errorf("hipMalloc(%zu) failed", b->size);
        delete b;
        return nullptr;
    }
    return b;
}

// ---------------------------------------------------------------------------
// Tiled weights.  A 2-D bf16 tensor [K][M] (ggml ne = {K, M}) with M % 16 == 0
// and K % 32 == 0 placed in a tiled buffer is stored in the MFMA-tiled layout
// of launch_tile_weights and marked by t->extra; set/get/copy convert from and
// to the row-major ggml layout, so callers always see row-major data.  The
// skinny GEMM reads such weights with one 1 KB load per MFMA fragment.  This
// plays the part of ggml's repacking "extra" buffer types (the CPU backend's
// weight repack), for the few-token projections.
// ---------------------------------------------------------------------------
static int k_tiled_tag;

static bool tileable(const wamx_tensor * t) {
    return t->type == WAMX_TYPE_BF16 && !t->view_src && t->ne[2] == 1 && t->ne[3] == 1 && t->ne[1] % 16 == 0 &&
           t->ne[0] % 32 == 0 && t->nb[0] == 2 && t->nb[1] == (size_t) t->ne[0] * 2;
}

namespace wamx {
bool tensor_is_tiled(const wamx_tensor * t) { return t && t->extra == &k_tiled_tag; }

hipError_t tensor_set_from_device(wamx_tensor * t, const void * src, hipStream_t s) {
    if (!tensor_is_tiled(t)) return hipMemcpyAsync(t->data, src, wamx_nbytes(t), hipMemcpyDeviceToDevice, s);
    return launch_tile_weights(src, t->data, t->ne[1], t->ne[0], false, s);
}
}  // namespace wamx

// Whole-tensor conversions through a temporary device buffer.
static hipError_t tiled_set(wamx_tensor * t, const void * host) {
    void * tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, wamx_nbytes(t));
    if (e != hipSuccess) return e;
    e = hipMemcpy(tmp, host, wamx_nbytes(t), hipMemcpyHostToDevice);
    if (e == hipSuccess) e = launch_tile_weights(tmp, t->data, t->ne[1], t->ne[0], false, nullptr);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    hipFree(tmp);
    return e;
}
static hipError_t tiled_get(const wamx_tensor * t, void * host, size_t off, size_t size) {
    void * tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, wamx_nbytes(t));
    if (e != hipSuccess) return e;
    e = launch_tile_weights(t->data, tmp, t->ne[1], t->ne[0], true, nullptr);
    if (e == hipSuccess) e = hipMemcpy(host, (const char *) tmp + off, size, hipMemcpyDeviceToHost);
    hipFree(tmp);
    return e;
}
static hipError_t tensor_copy_impl(const wamx_tensor * src, wamx_tensor * dst) {
    const bool ts = tensor_is_tiled(src), td = tensor_is_tiled(dst);
    if (ts == td) return hipMemcpy(dst->data, src->data, wamx_nbytes(src), hipMemcpyDeviceToDevice);
    const wamx_tensor * t = ts ? src : dst;  // the tiled side fixes M and K
    hipError_t e = launch_tile_weights(src->data, dst->data, t->ne[1], t->ne[0], ts, nullptr);
    return e == hipSuccess ? hipDeviceSynchronize() : e;
}

static void buffer_free(wamx_buffer_t b) {
    if (!b) return;
    if (b->base) hipFree(b->base);
    delete b;
}
static void * buffer_get_base(wamx_buffer_t b) { return b ? b->base : nullptr; }
static wamx_status buffer_init_tensor(wamx_buffer_t b, wamx_tensor * t) {
    if (t->view_src && t->view_src->data) t->data = (char *) t->view_src->data + t->view_offs;
    if (b && b->buft && b->buft->tiled && tileable(t)) t->extra = &k_tiled_tag;
    return WAMX_STATUS_SUCCESS;
}
static void buffer_memset_tensor(wamx_buffer_t, wamx_tensor * t, uint8_t v, size_t off, size_t size) {
    hipMemset((char *) t->data + off, v, size);
}
static void buffer_set_tensor(wamx_buffer_t, wamx_tensor * t, const void * data, size_t off, size_t size) {
    if (tensor_is_tiled(t) && off == 0 && size == wamx_nbytes(t)) tiled_set(t, data);
    else if (!tensor_is_tiled(t)) hipMemcpy((char *) t->data + off, data, size, hipMemcpyHostToDevice);
}
static void buffer_get_tensor(wamx_buffer_t, const wamx_tensor * t, void * data, size_t off, size_t size) {
    if (tensor_is_tiled(t)) tiled_get(t, data, off, size);
    else hipMemcpy(data, (const char *) t->data + off, size, hipMemcpyDeviceToHost);
}
static bool buffer_cpy_tensor(wamx_buffer_t, const wamx_tensor * src, wamx_tensor * dst) {
    if (!src->data || !dst->data || wamx_nbytes(src) != wamx_nbytes(dst)) return false;
    if ((tensor_is_tiled(src) || tensor_is_tiled(dst)) && !wamx_are_same_shape(src, dst)) return false;
    return tensor_copy_impl(src, dst) == hipSuccess;
}
static void buffer_clear(wamx_buffer_t b, uint8_t v) {
    if (b && b->base) hipMemset(b->base, v, b->size);
}
static void buffer_reset(wamx_buffer_t) {}

static const wamx_buffer_type_i k_buft_iface = {
    buft_get_name, buft_alloc_buffer, buft_get_alignment, buft_get_max_size, buft_get_alloc_size, buft_is_host,
};
static const wamx_buffer_i k_buffer_iface = {
    buffer_free,       buffer_get_base,   buffer_init_tensor, buffer_memset_tensor, buffer_set_tensor,
    buffer_get_tensor, buffer_cpy_tensor, buffer_clear,       buffer_reset,
};

// ---------------------------------------------------------------------------
// Op dispatch
// ---------------------------------------------------------------------------
static int64_t es(const wamx_tensor * t) { return (int64_t) wamx_type_size(t->type); }

static bool rows_contig(const wamx_tensor * t) { return t->nb[0] == (size_t) es(t); }

static hipError_t run_mul_mat(wamx_backend * be, const wamx_tensor * node) {
    const wamx_tensor * a = node->src[0];
    const wamx_tensor * b = node->src[1];
    GemmArgs g;
    g.w = a->data;
    g.w_type = a->type;
    g.ldw = (int64_t) a->nb[1] / es(a);
    g.w_bs2 = (int64_t) a->nb[2] / es(a);
    g.w_bs3 = (int64_t) a->nb[3] / es(a);
    g.x = b->data;
    g.x_type = b->type;
    g.ldx = (int64_t) b->nb[1] / es(b);
    g.x_bs2 = (int64_t) b->nb[2] / es(b);
    g.x_bs3 = (int64_t) b->nb[3] / es(b);
    g.y = node->data;
    g.y_type = node->type;
    g.ldy = (int64_t) node->nb[1] / es(node);
    g.y_bs2 = (int64_t) node->nb[2] / es(node);
    g.y_bs3 = (int64_t) node->nb[3] / es(node);
    g.M = a->ne[1];
    g.N = b->ne[1];
    g.K = a->ne[0];
    g.B2 = b->ne[2];
    g.B3 = b->ne[3];
    g.r2 = b->ne[2] / a->ne[2];
    g.r3 = b->ne[3] / a->ne[3];
    g.ws = be->cws;
    g.ws_bytes = kWorkspaceBytes;
    g.w_tiled = tensor_is_tiled(a);
    return launch_gemm(g, be->cs);
}

static GemmArgs linear_args(wamx_backend * be, const wamx_tensor * node) {
    const wamx_tensor * w = node->src[0];
    const wamx_tensor * x = node->src[1];
    GemmArgs g;
    g.w = w->data;
    g.w_type = WAMX_TYPE_BF16;
    g.ldw = (int64_t) w->nb[1] / 2;
    g.x = x->data;
    g.x_type = x->type;
    g.ldx = (int64_t) x->nb[1] / es(x);
    g.y = node->data;
    g.y_type = WAMX_TYPE_BF16;
    g.ldy = (int64_t) node->nb[1] / 2;
    g.M = w->ne[1];
    g.N = x->ne[1];
    g.K = w->ne[0];
    g.epi = node->op_params[0];
    g.bias = node->src[2] ? node->src[2]->data : nullptr;
    g.res = node->src[3] ? node->src[3]->data : nullptr;
    g.ldres = node->src[3] ? (int64_t) node->src[3]->nb[1] / 2 : 0;
    g.gate = node->src[4] ? (const float *) node->src[4]->data : nullptr;
    g.ws = be->cws;
    g.ws_bytes = kWorkspaceBytes;
    g.w_tiled = tensor_is_tiled(w);
    return g;
}

static hipError_t run_linear(wamx_backend * be, const wamx_tensor * node) {
    return launch_gemm(linear_args(be, node), be->cs);
}

static float param_f32(const wamx_tensor * t, int i) {
    float v;
    memcpy(&v, &t->op_params[i], 4);
    return v;
}

// ---------------------------------------------------------------------------
// Row fusion: a LINEAR on a few tokens (the split-K skinny path) followed
// directly by the row ops that consume its output runs as the GEMM's part
// kernel plus one reduce that applies those row ops (launch_gemm_rowpost):
//   * LINEAR -> NORM of its output (LayerNorm / adaLN modulation), the
//     residual-stream pattern h = lin(..., h); n = norm(h) of mot.cpp:130-145,
//     284-346;
//   * LINEAR -> up to three of QK_NORM_ROPE of a column range and the V^T
//     copy (CPY of a permuted column range), the QKV split of mot.cpp:245-265,
//     395-401.
// The matched nodes are computed by the fused launch and skipped; anything
// the fused path does not take runs node by node as before.
// ---------------------------------------------------------------------------
static bool is_noop(const wamx_tensor * t) {
    switch (t->op) {
        case WAMX_OP_NONE:
        case WAMX_OP_VIEW:
        case WAMX_OP_RESHAPE:
        case WAMX_OP_PERMUTE:
        case WAMX_OP_TRANSPOSE:
            return true;
        default:
            return false;
    }
}

// Next node after i that launches work; in a two-lane graph (`lanes`) only
// nodes of node i's lane count, so a LINEAR fuses with its own lane's row ops.
static int next_compute(wamx_cgraph * g, int i, int n, bool lanes) {
    const int lane = wamx_graph_node(g, i)->lane;
    for (int j = i + 1; j < n; ++j) {
        const wamx_tensor * t = wamx_graph_node(g, j);
        if (!is_noop(t) && (!lanes || t->lane == lane)) return j;
    }
    return n;
}

// Column offset of x inside the rows of `base` (x is base, or a view taking a
// column range of each of its rows).
static bool column_view(const wamx_tensor * x, const wamx_tensor * base, int64_t & col) {
    if (x == base) {
        col = 0;
        return true;
    }
    if (x->op != WAMX_OP_VIEW || x->view_src != base || x->type != base->type || x->nb[0] != base->nb[0] ||
        x->nb[1] != base->nb[1] || x->ne[1] != base->ne[1] || x->ne[2] != 1 || x->ne[3] != 1)
        return false;
    if (x->view_offs % base->nb[0] != 0 || x->view_offs + x->ne[0] * x->nb[0] > base->nb[1]) return false;
    col = (int64_t) (x->view_offs / base->nb[0]);
    return true;
}

// Matches the row ops after LINEAR node i; returns the index of the last node
// they cover (> i), or -1.
static int match_row_post(wamx_cgraph * g, int i, int n, RowPost & post, bool lanes) {
    const wamx_tensor * lin = wamx_graph_node(g, i);
    // Up to 64 tokens (the skinny path) or a few chunks of them (the batched
    // denoise step's K-sliced products); launch_gemm_rowpost refuses the rest.
    if (lin->type != WAMX_TYPE_BF16 || lin->ne[1] > 512 || lin->ne[2] != 1 || lin->ne[3] != 1 || lin->view_src)
        return -1;
    int j = next_compute(g, i, n, lanes);
    if (j >= n) return -1;
    const wamx_tensor * t = wamx_graph_node(g, j);
    if (t->op == WAMX_OP_NORM) {
        const wamx_tensor * sc = t->src[1];
        const wamx_tensor * sh = t->src[2];
        if (t->src[0] != lin || !sc || !sh || t->type != WAMX_TYPE_BF16 || !wamx_are_same_shape(t, lin) ||
            t->nb[0] != 2)
            return -1;
        post.kind = kRowPostNorm;
        post.scale = sc->data;
        post.shift = sh->data;
        post.ss_type = sc->type;
        post.affine = sc->type == WAMX_TYPE_BF16;  // as compute_node: bf16 weights are the affine LayerNorm
        post.ss = sc->ne[1] == 1 ? 0 : (int64_t) (sc->nb[1] / wamx_type_size(sc->type));
        post.out = t->data;
        post.ldo = (int64_t) t->nb[1] / 2;
        post.eps = param_f32(t, 0);
        return j;
    }
    post.kind = kRowPostSegs;
    post.nseg = 0;
    int last = -1;
    const int64_t T = lin->ne[1];
    while (j < n && post.nseg < 3) {
        t = wamx_graph_node(g, j);
        RowSeg seg;
        int64_t width, head_dim;
        if (t->op == WAMX_OP_QK_NORM_ROPE) {
            const wamx_tensor * x = t->src[0];
            if (!column_view(x, lin, seg.col) || !t->src[1] || t->type != WAMX_TYPE_BF16 || t->op_params[4] ||
                t->op_params[1] == 3 || x->ne[2] > 1 || t->src[1]->ne[1] > 1)
                break;
            head_dim = t->ne[0];
            width = x->ne[0];
            if (width != head_dim * t->ne[2] || x->ne[1] % t->ne[3] != 0) break;
            seg.chunk_tokens = t->ne[3] > 1 ? x->ne[1] / t->ne[3] : 0;  // rows of chunk b at dst + b * nb[3]
            seg.chunk_stride = (int64_t) t->nb[3] / 2;
            seg.kind = kRowSegQk;
            seg.w = t->src[1]->data;
            seg.dst = t->data;
            seg.dst_tokens = t->ne[1];
            seg.tok0 = t->op_params[0];
            seg.rope_mode = t->op_params[1];
            seg.pos0 = t->src[3] ? (const int32_t *) t->src[3]->data : nullptr;
            seg.pos1 = t->src[4] ? (const int32_t *) t->src[4]->data : nullptr;
            seg.pos2 = t->src[5] ? (const int32_t *) t->src[5]->data : nullptr;
            seg.eps = param_f32(t, 2);
            seg.freq_base = param_f32(t, 3);
        } else if (t->op == WAMX_OP_CPY) {
            // V^T store: CPY(permute(view(lin) as [dh, H, T], 1, 2, 0), dst [T, dh, H]).
            const wamx_tensor * p = t->src[0];
            const wamx_tensor * v = p ? p->src[0] : nullptr;
            if (!p || p->op != WAMX_OP_PERMUTE || !v || v->op != WAMX_OP_VIEW || v->view_src != lin ||
                t->type != WAMX_TYPE_BF16 || p->type != WAMX_TYPE_BF16)
                break;
            head_dim = p->ne[1];
            width = head_dim * p->ne[2];
            // Chunks (ne[3] > 1): consecutive row ranges of the product.
            if (p->ne[0] * p->ne[3] != T || (p->ne[3] > 1 && p->nb[3] != (size_t) p->ne[0] * lin->nb[1]) ||
                p->nb[0] != lin->nb[1] || p->nb[1] != 2 || p->nb[2] != (size_t) head_dim * 2 ||
                !wamx_are_same_shape(t, p) || t->nb[0] != 2)
                break;
            seg.chunk_tokens = p->ne[3] > 1 ? p->ne[0] : 0;
            seg.chunk_stride = (int64_t) t->nb[3] / 2;
            if (v->view_offs % 2 != 0 || v->view_offs + (size_t) width * 2 > lin->nb[1]) break;
            seg.kind = kRowSegVt;
            seg.col = (int64_t) (v->view_offs / 2);
            seg.dst = t->data;
            seg.vt_ld = (int64_t) t->nb[1] / 2;
            seg.vt_hs = (int64_t) t->nb[2] / 2;
        } else {
            break;
        }
        if (post.nseg > 0 && (width != post.width || head_dim != post.head_dim)) break;
        post.width = width;
        post.head_dim = head_dim;
        post.seg[post.nseg++] = seg;
        last = j;
        j = next_compute(g, j, n, lanes);
    }
    // The fused reduce writes the product's output only in its segments'
    // columns, so the segments must tile every column: a row op of the
    // product that does not follow here (another lane's node, or any node
    // between them) reads its columns from that output.
    if (post.nseg == 0 || post.nseg * post.width != lin->ne[0]) return -1;
    bool covered[3] = {false, false, false};
    for (int k = 0; k < post.nseg; ++k) {
        const int64_t c = post.seg[k].col;
        if (c % post.width != 0 || c / post.width >= post.nseg || covered[c / post.width]) return -1;
        covered[c / post.width] = true;
    }
    return last;
}

// ---------------------------------------------------------------------------
// The reference's F32-profile fusions (p7-fusions.patch:173-245), matched in
// the graph the way ggml-cuda's evaluator matches them:
//   NORM -> VIEW(scale) -> MUL -> ADD -> VIEW(shift) -> ADD, the modulated
//     norm of mot.cpp:154-158 (norm + norm * scale + shift), with every
//     intermediate used once, becomes norm_modulation_f32;
//   MUL(branch, gate view) -> ADD(residual), the gated residual of
//     mot.cpp:161-164, becomes gated_residual_f32.
// Both kernels round each operation separately (no FMA), as the reference's.
// ---------------------------------------------------------------------------
struct F32Fusion {
    int kind = 0;  // 1 norm-modulation, 2 gated residual
    const wamx_tensor *x = nullptr, *scale = nullptr, *shift = nullptr, *branch = nullptr, *gate = nullptr;
    wamx_tensor * out = nullptr;
    float eps = 0.0f;
};

static int uses_of(wamx_cgraph * g, int n, const wamx_tensor * t) {
    int u = 0;
    for (int j = 0; j < n; ++j) {
        const wamx_tensor * m = wamx_graph_node(g, j);
        for (int k = 0; k < WAMX_MAX_SRC; ++k) u += m->src[k] == t;
    }
    return u;
}

static bool row_broadcast_or_same(const wamx_tensor * a, const wamx_tensor * v) {
    return wamx_are_same_shape(a, v) || (a->ne[0] == v->ne[0] && v->ne[1] == 1 && v->ne[2] == 1 && v->ne[3] == 1);
}

// Returns the last node the fusion starting at node i covers (> i), or -1.
static int match_f32_fusion(const wamx_backend * be, wamx_cgraph * g, int i, int n, F32Fusion & f) {
    wamx_tensor * node = wamx_graph_node(g, i);
    auto same_lane = [&](int a, int b) {
        for (int j = a; j <= b; ++j)
            if (wamx_graph_node(g, j)->lane != node->lane) return false;
        return true;
    };
    auto f32 = [](const wamx_tensor * t) { return t && t->type == WAMX_TYPE_F32; };
    if (be->fuse_norm_mod_f32 && node->op == WAMX_OP_NORM && !node->src[1] && i + 5 < n) {
        wamx_tensor *sc = wamx_graph_node(g, i + 1), *mul = wamx_graph_node(g, i + 2), *as = wamx_graph_node(g, i + 3);
        wamx_tensor *sh = wamx_graph_node(g, i + 4), *ash = wamx_graph_node(g, i + 5);
        auto has = [](const wamx_tensor * t, const wamx_tensor * a, const wamx_tensor * b) {
            return (t->src[0] == a && t->src[1] == b) || (t->src[0] == b && t->src[1] == a);
        };
        const bool ok = sc->op == WAMX_OP_VIEW && mul->op == WAMX_OP_MUL && as->op == WAMX_OP_ADD && !as->src[2] &&
                        sh->op == WAMX_OP_VIEW && ash->op == WAMX_OP_ADD && !ash->src[2] && has(mul, node, sc) &&
                        has(as, node, mul) && has(ash, as, sh) && uses_of(g, n, node) == 2 && uses_of(g, n, sc) == 1 &&
                        uses_of(g, n, mul) == 1 && uses_of(g, n, as) == 1 && uses_of(g, n, sh) == 1 &&
                        !(as->flags & WAMX_TENSOR_FLAG_OUTPUT) && !(mul->flags & WAMX_TENSOR_FLAG_OUTPUT) &&
                        !(node->flags & WAMX_TENSOR_FLAG_OUTPUT) && f32(node) && f32(node->src[0]) && f32(sc) &&
                        f32(sh) && f32(ash) && row_broadcast_or_same(node, sc) && row_broadcast_or_same(node, sh) &&
                        wamx_are_same_shape(node, ash) && node->ne[2] == 1 && node->ne[3] == 1 &&
                        node->src[0]->nb[0] == 4 && sc->nb[0] == 4 && sh->nb[0] == 4 && wamx_is_contiguous(ash) &&
                        (sc->ne[1] == 1 ? sh->ne[1] == 1 : sc->nb[1] == sh->nb[1]) && same_lane(i, i + 5);
        if (ok) {
            f.kind = 1;
            f.x = node->src[0];
            f.scale = sc;
            f.shift = sh;
            f.out = ash;
            memcpy(&f.eps, &node->op_params[0], 4);
            return i + 5;
        }
    }
    if (be->fuse_gated_residual_f32 && node->op == WAMX_OP_MUL && i + 1 < n) {
        wamx_tensor * add = wamx_graph_node(g, i + 1);
        const wamx_tensor *a = node->src[0], *b = node->src[1];
        if (add->op != WAMX_OP_ADD || add->src[2] || !(add->src[0] == node || add->src[1] == node) ||
            uses_of(g, n, node) != 1 || (node->flags & WAMX_TENSOR_FLAG_OUTPUT) || !a || !b)
            return -1;
        const wamx_tensor * residual = add->src[0] == node ? add->src[1] : add->src[0];
        auto gate_like = [](const wamx_tensor * x, const wamx_tensor * other) {
            return x->op == WAMX_OP_VIEW && (!wamx_is_contiguous(x) || (x->ne[1] == 1 && other->ne[1] > 1));
        };
        const bool a_gate = gate_like(a, b), b_gate = gate_like(b, a);
        const wamx_tensor * gate = a_gate ? a : b;
        const wamx_tensor * branch = a_gate ? b : a;
        const bool ok = a_gate != b_gate && f32(node) && f32(branch) && f32(gate) && f32(residual) && f32(add) &&
                        branch->ne[2] == 1 && branch->ne[3] == 1 && wamx_are_same_shape(node, branch) &&
                        row_broadcast_or_same(branch, gate) && wamx_are_same_shape(node, residual) &&
                        wamx_are_same_shape(node, add) && branch->nb[0] == 4 && gate->nb[0] == 4 &&
                        residual->nb[0] == 4 && wamx_is_contiguous(add) && same_lane(i, i + 1);
        if (ok) {
            f.kind = 2;
            f.x = residual;
            f.branch = branch;
            f.gate = gate;
            f.out = add;
            return i + 1;
        }
    }
    return -1;
}

static hipError_t run_f32_fusion(wamx_backend * be, const F32Fusion & f) {
    const int64_t rows = wamx_nrows(f.out), cols = f.out->ne[0];
    if (f.kind == 1)
        return launch_norm_mod_f32((const float *) f.x->data, (int64_t) f.x->nb[1] / 4, (const float *) f.scale->data,
                                   (const float *) f.shift->data, f.scale->ne[1] == 1 ? 0 : (int64_t) f.scale->nb[1] / 4,
                                   (float *) f.out->data, rows, cols, f.eps, be->cs);
    return launch_gated_residual_f32((const float *) f.x->data, (int64_t) f.x->nb[1] / 4,
                                     (const float *) f.branch->data, (int64_t) f.branch->nb[1] / 4,
                                     (const float *) f.gate->data, f.gate->ne[1] == 1 ? 0 : (int64_t) f.gate->nb[1] / 4,
                                     (float *) f.out->data, rows, cols, be->cs);
}

static hipError_t run_joint_attn(wamx_backend * be, const wamx_tensor * node) {
    const wamx_tensor * q = node->src[0];
    AttnArgs a;
    a.q = q->data;
    a.k_a = node->src[1]->data;
    a.vt_a = node->src[2]->data;
    a.na = node->src[1]->ne[1];
    a.vt_ld_a = (int64_t) node->src[2]->nb[1] / 2;
    if (node->src[3]) {
        a.k_b = node->src[3]->data;
        a.vt_b = node->src[4]->data;
        a.nb = node->src[3]->ne[1];
        a.vt_ld_b = (int64_t) node->src[4]->nb[1] / 2;
    }
    a.na_split = node->op_params[0];
    a.out = node->data;
    a.heads = q->ne[2] * q->ne[3];   // chunk b's heads follow chunk b - 1's
    a.hb = q->ne[2];
    a.head_dim = q->ne[0];
    a.tq = q->ne[1];
    a.scale = param_f32(node, 1);
    a.ws = be->cws;
    a.ws_bytes = kWorkspaceBytes;
    if (node->op_params[2]) {  // hi/lo planes: plane 1 of q and k
        a.heads = a.hb = q->ne[2];
        a.q_lo = (const char *) q->data + q->nb[3];
        a.k_lo = (const char *) node->src[1]->data + node->src[1]->nb[3];
    }
    return launch_joint_attn(a, be->cs);
}

static hipError_t compute_node(wamx_backend * be, wamx_tensor * node) {
    hipStream_t s = be->cs;
    wamx_tensor * s0 = node->src[0];
    wamx_tensor * s1 = node->src[1];
    switch (node->op) {
        case WAMX_OP_NONE:
        case WAMX_OP_VIEW:
        case WAMX_OP_RESHAPE:
        case WAMX_OP_PERMUTE:
        case WAMX_OP_TRANSPOSE:
            return hipSuccess;
        case WAMX_OP_DUP:
        case WAMX_OP_CONT:
        case WAMX_OP_CPY:
            return launch_copy(ref_of(s0), ref_of(node), s);
        case WAMX_OP_ADD:
            if (node->src[2]) {
                const wamx_tensor * g = node->src[2];
                return launch_gated_residual_bf16(s0->data, (int64_t) s0->nb[1] / 2, s1->data, (int64_t) s1->nb[1] / 2,
                                                  g->data, g->type, g->ne[1] == 1 ? 0 : (int64_t) g->nb[1] / es(g),
                                                  node->data, wamx_nrows(s0), s0->ne[0], s);
            }
            return launch_binary(0, ref_of(s0), ref_of(s1), ref_of(node), s);
        case WAMX_OP_MUL:
            return launch_binary(1, ref_of(s0), ref_of(s1), ref_of(node), s);
        case WAMX_OP_REPEAT:
            return launch_binary(2, ref_of(node), ref_of(s0), ref_of(node), s);
        case WAMX_OP_SCALE:
            return launch_unary(kUnaryScale, ref_of(s0), ref_of(node), param_f32(node, 0), param_f32(node, 1), s);
        case WAMX_OP_CONCAT:
            return launch_concat(ref_of(s0), ref_of(s1), ref_of(node), node->op_params[0], s);
        case WAMX_OP_NORM: {
            const float eps = param_f32(node, 0);
            if (node->src[1]) {
                const wamx_tensor * sc = node->src[1];
                const wamx_tensor * sh = node->src[2];
                const bool affine = sc->type == WAMX_TYPE_BF16;  // native-bf16.patch:393-400
                const int64_t ss = sc->ne[1] == 1 ? 0 : (int64_t) sc->nb[1] / es(sc);
                (void) sh;
                return launch_norm_mod_bf16(s0->data, (int64_t) s0->nb[1] / 2, sc->data, sh->data, sc->type, ss,
                                            node->data, (int64_t) node->nb[1] / 2, wamx_nrows(s0), s0->ne[0], eps,
                                            affine, s);
            }
            return launch_norm_f32((const float *) s0->data, (int64_t) s0->nb[1] / 4, (float *) node->data,
                                   (int64_t) node->nb[1] / 4, wamx_nrows(s0), s0->ne[0], eps, false, s);
        }
        case WAMX_OP_RMS_NORM: {
            const float eps = param_f32(node, 0);
            if (node->src[1])
                return launch_rms_norm_bf16_f32(s0->data, (int64_t) s0->nb[1] / 2, node->src[1]->data,
                                                (float *) node->data, (int64_t) node->nb[1] / 4, wamx_nrows(s0),
                                                s0->ne[0], eps, s);
            return launch_norm_f32((const float *) s0->data, (int64_t) s0->nb[1] / 4, (float *) node->data,
                                   (int64_t) node->nb[1] / 4, wamx_nrows(s0), s0->ne[0], eps, true, s);
        }
        case WAMX_OP_MUL_MAT:
            return run_mul_mat(be, node);
        case WAMX_OP_SOFT_MAX: {
            TensorRef mask{};
            if (s1) mask = ref_of(s1);
            return launch_softmax_f32(ref_of(s0), mask, ref_of(node), param_f32(node, 0), s);
        }
        case WAMX_OP_ROPE:
            return launch_rope_f32(ref_of(s0), (const int32_t *) s1->data, ref_of(node), node->op_params[1],
                                   param_f32(node, 5), s);
        case WAMX_OP_UNARY:
            if (node->src[1])
                return launch_bias_gelu_bf16(s0->data, s1->data, node->data, wamx_nelements(s0), s1->ne[0], s);
            return launch_unary(node->op_params[0], ref_of(s0), ref_of(node), 1.0f, 0.0f, s);
        case WAMX_OP_GET_ROWS:
            return launch_get_rows(ref_of(s0), (const int32_t *) s1->data, ref_of(node), s);
        case WAMX_OP_IM2COL: {
            // ggml_im2col: kernel size from the kernel tensor, op_params {s0, s1, p0, p1, d0, d1, is_2D}.
            const int32_t * pp = node->op_params;
            return launch_im2col(ref_of(s1), ref_of(node), (int) s0->ne[0], (int) s0->ne[1], pp[0], pp[1], pp[2], pp[3],
                                 pp[4], pp[5], s);
        }
        case WAMX_OP_CONV_2D:
            return launch_conv2d(ref_of(s0), ref_of(s1), ref_of(node), node->op_params, be->cws, kWorkspaceBytes, s);
        case WAMX_OP_LINEAR:
            return run_linear(be, node);
        case WAMX_OP_QK_NORM_ROPE: {
            const wamx_tensor * x = node->src[0];
            const wamx_tensor * w = node->src[1];
            const bool hilo = node->op_params[4] != 0;  // plane 2c + 1 takes chunk c's lo parts
            const bool table = node->op_params[1] == 3;  // src[3]: the (cos, sin) table
            const int64_t C = hilo ? node->ne[3] / 2 : node->ne[3];
            const bool layered = x->ne[2] > 1;           // chunk c's rows at x + c * nb[2]
            const int64_t T = layered ? x->ne[1] : x->ne[1] / C;
            const int64_t plane = (int64_t) node->nb[3] / 2;
            return launch_qk_norm_rope(x->data, (int64_t) x->nb[1] / 2, w->data, node->data, node->ne[2],
                                       node->ne[0], T * C, node->ne[1], node->op_params[0], node->op_params[1],
                                       node->src[3] && !table ? (const int32_t *) node->src[3]->data : nullptr,
                                       node->src[4] ? (const int32_t *) node->src[4]->data : nullptr,
                                       node->src[5] ? (const int32_t *) node->src[5]->data : nullptr,
                                       param_f32(node, 2), param_f32(node, 3), s, T, hilo ? 2 * plane : plane,
                                       hilo ? plane : 0, table ? (const float *) node->src[3]->data : nullptr,
                                       layered ? (int64_t) x->nb[2] / 2 : -1, w->ne[1] > 1 ? (int64_t) w->nb[1] / 2 : 0);
        }
        case WAMX_OP_JOINT_ATTN:
            return run_joint_attn(be, node);
        case WAMX_OP_MODULATION:
            return launch_modulation(s0->data, s0->type, s1->data, s1->type, (float *) node->data,
                                     s1->ne[0] * s1->ne[1], s1->ne[2] * s1->ne[3], s, node->ne[3]);
        case WAMX_OP_EULER_STEP:
            return launch_euler_step(s0->data, s1->data, (const float *) node->src[2]->data, node->data,
                                     wamx_nelements(node), s);
        case WAMX_OP_MLP_SMALL:
            return launch_mlp_small(s0->data, s1->data, node->src[2]->data, node->src[3]->data, node->src[4]->data,
                                    node->data, s0->ne[1], s0->ne[0], s1->ne[1], node->src[3]->ne[1],
                                    node->op_params[0], s);
        default:
            return hipErrorNotSupported;
    }
}

// A tiled weight multiplies only the few-token activations of the skinny path.
static bool tiled_product_ok(const wamx_tensor * x) {
    return (x->type == WAMX_TYPE_BF16 || x->type == WAMX_TYPE_F32) && x->ne[1] <= 64 && x->ne[2] == 1 && x->ne[3] == 1 &&
           rows_contig(x);
}

// Whether b broadcasts onto a by modulo in every dim (ggml_can_repeat).
static bool can_repeat(const wamx_tensor * b, const wamx_tensor * a) {
    for (int i = 0; i < 4; ++i)
        if (b->ne[i] <= 0 || a->ne[i] % b->ne[i] != 0) return false;
    return true;
}

// Whether the backend can run node t as it stands.  Every shape and layout
// assumption of the launch path is checked here, because a node may come
// from a graph mirrored from ggml (wamx_graph_from_ggml) rather than from the
// constructors of wamx.h.
static bool supports(const wamx_tensor * t) {
    auto ok_type = [](const wamx_tensor * x) {
        return x && (x->type == WAMX_TYPE_F32 || x->type == WAMX_TYPE_BF16 || x->type == WAMX_TYPE_F16 ||
                     x->type == WAMX_TYPE_I32);
    };
    auto float_type = [](const wamx_tensor * x) {
        return x && (x->type == WAMX_TYPE_F32 || x->type == WAMX_TYPE_BF16 || x->type == WAMX_TYPE_F16);
    };
    const wamx_tensor * s0 = t->src[0];
    const wamx_tensor * s1 = t->src[1];
    const bool view_op = t->op == WAMX_OP_NONE || t->op == WAMX_OP_VIEW || t->op == WAMX_OP_RESHAPE ||
                         t->op == WAMX_OP_PERMUTE || t->op == WAMX_OP_TRANSPOSE;
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] < 0) return false;
    // A tiled weight is read only whole, as the weight of MUL_MAT / LINEAR:
    // any other reader, or a reader of a view of it, would see the tiled order.
    for (int i = 0; i < WAMX_MAX_SRC && !view_op; ++i) {
        const wamx_tensor * x = t->src[i];
        if (!x) continue;
        if (x->view_src && tensor_is_tiled(x->view_src)) return false;
        if (tensor_is_tiled(x) && !(i == 0 && (t->op == WAMX_OP_MUL_MAT || t->op == WAMX_OP_LINEAR))) return false;
    }
    switch (t->op) {
        case WAMX_OP_NONE:
        case WAMX_OP_VIEW:
        case WAMX_OP_RESHAPE:
        case WAMX_OP_PERMUTE:
        case WAMX_OP_TRANSPOSE:
            return true;
        case WAMX_OP_DUP:
        case WAMX_OP_CONT:
        case WAMX_OP_CPY:
            return ok_type(s0) && ok_type(t) && wamx_nelements(s0) == wamx_nelements(t);
        case WAMX_OP_ADD:
            if (t->src[2]) {  // gated residual bf16 (native-bf16.patch:594-612)
                const wamx_tensor * g = t->src[2];
                return s0 && s1 && s0->type == WAMX_TYPE_BF16 && s1->type == WAMX_TYPE_BF16 && t->type == WAMX_TYPE_BF16 &&
                       (g->type == WAMX_TYPE_F32 || g->type == WAMX_TYPE_BF16) && wamx_are_same_shape(s0, s1) &&
                       wamx_are_same_shape(s0, t) && g->ne[0] == s0->ne[0] &&
                       (g->ne[1] == 1 || g->ne[1] == s0->ne[1]) && g->ne[2] == 1 && g->ne[3] == 1 && rows_contig(s0) &&
                       rows_contig(s1) && rows_contig(g) && s0->ne[2] == 1 && s0->ne[3] == 1 && wamx_is_contiguous(t);
            }
            [[fallthrough]];
        case WAMX_OP_MUL:
            return float_type(s0) && float_type(s1) && float_type(t) && can_repeat(s1, s0) && wamx_are_same_shape(s0, t);
        case WAMX_OP_REPEAT:
            return ok_type(s0) && ok_type(t) && s0->type == t->type && can_repeat(s0, t);
        case WAMX_OP_SCALE:
            return float_type(s0) && float_type(t) && wamx_are_same_shape(s0, t);
        case WAMX_OP_CONCAT: {
            const int dim = t->op_params[0];
            if (!ok_type(s0) || !s1 || s0->type != s1->type || s0->type != t->type || dim < 0 || dim > 3) return false;
            for (int i = 0; i < 4; ++i)
                if (i != dim ? (s0->ne[i] != s1->ne[i] || s0->ne[i] != t->ne[i]) : t->ne[i] != s0->ne[i] + s1->ne[i])
                    return false;
            return true;
        }
        case WAMX_OP_GET_ROWS:
            return ok_type(s0) && s1 && s1->type == WAMX_TYPE_I32 && rows_contig(s1) && t->ne[0] == s0->ne[0] &&
                   t->ne[1] == s1->ne[0] && t->ne[2] == s1->ne[1] && float_type(t);
        case WAMX_OP_NORM:
            if (t->src[1]) {  // norm_modulation_bf16 / layer_norm_bf16 (native-bf16.patch:630-663)
                const wamx_tensor *sc = t->src[1], *sh = t->src[2];
                return sh && s0->type == WAMX_TYPE_BF16 && t->type == WAMX_TYPE_BF16 && sc->type == sh->type &&
                       (sc->type == WAMX_TYPE_F32 || sc->type == WAMX_TYPE_BF16) && sc->ne[0] == s0->ne[0] &&
                       sh->ne[0] == s0->ne[0] && wamx_are_same_shape(s0, t) && rows_contig(s0) && rows_contig(t) &&
                       rows_contig(sc) && rows_contig(sh) && s0->ne[2] == 1 && s0->ne[3] == 1 && t->nb[1] % 2 == 0 &&
                       sc->ne[1] == sh->ne[1] && (sc->ne[1] == 1 || sc->ne[1] == s0->ne[1]) &&
                       (sc->ne[1] == 1 || sc->nb[1] / es(sc) == sh->nb[1] / es(sh));
            }
            return s0->type == WAMX_TYPE_F32 && t->type == WAMX_TYPE_F32 && rows_contig(s0) && rows_contig(t) &&
                   wamx_are_same_shape(s0, t);
        case WAMX_OP_RMS_NORM:
            if (t->src[1])  // rms_norm_bf16_f32 (native-bf16.patch:665-678)
                return s0->type == WAMX_TYPE_BF16 && s1->type == WAMX_TYPE_BF16 && s1->ne[0] == s0->ne[0] &&
                       rows_contig(s1) && t->type == WAMX_TYPE_F32 && rows_contig(s0) && rows_contig(t) &&
                       wamx_are_same_shape(s0, t);
            return s0->type == WAMX_TYPE_F32 && t->type == WAMX_TYPE_F32 && rows_contig(s0) && rows_contig(t) &&
                   wamx_are_same_shape(s0, t);
        case WAMX_OP_MUL_MAT: {
            if (!s0 || !s1 || s0->ne[0] != s1->ne[0] || s0->ne[2] <= 0 || s0->ne[3] <= 0 ||
                s1->ne[2] % s0->ne[2] != 0 || s1->ne[3] % s0->ne[3] != 0 || t->ne[0] != s0->ne[1] ||
                t->ne[1] != s1->ne[1] || t->ne[2] != s1->ne[2] || t->ne[3] != s1->ne[3] ||
                (t->type != WAMX_TYPE_F32 && t->type != WAMX_TYPE_BF16))
                return false;
            if (tensor_is_tiled(s0)) return tiled_product_ok(s1) && wamx_is_contiguous(t);
            return (s0->type == WAMX_TYPE_BF16 || s0->type == WAMX_TYPE_F32) &&
                   (s1->type == WAMX_TYPE_BF16 || s1->type == WAMX_TYPE_F32) && rows_contig(s0) && rows_contig(s1) &&
                   wamx_is_contiguous(t);
        }
        case WAMX_OP_SOFT_MAX: {
            if (!s0 || s0->type != WAMX_TYPE_F32 || t->type != WAMX_TYPE_F32 || !wamx_are_same_shape(s0, t) ||
                param_f32(t, 1) != 0.0f || t->src[2])
                return false;
            if (s1 && ((s1->type != WAMX_TYPE_F32 && s1->type != WAMX_TYPE_F16) || s1->ne[0] != s0->ne[0] ||
                       s1->ne[1] < s0->ne[1] || s1->ne[2] <= 0 || s1->ne[3] <= 0 || s0->ne[2] % s1->ne[2] != 0 ||
                       s0->ne[3] % s1->ne[3] != 0))
                return false;
            return true;
        }
        case WAMX_OP_ROPE: {
            // NORMAL mode, no frequency factors, no YaRN: ggml_rope_ext with
            // freq_scale 1, ext_factor 0, attn_factor 1 (mot.cpp:175-202).
            const int n_dims = t->op_params[1];
            return s0 && s0->type == WAMX_TYPE_F32 && t->type == WAMX_TYPE_F32 && wamx_are_same_shape(s0, t) && s1 &&
                   s1->type == WAMX_TYPE_I32 && s1->ne[0] == s0->ne[2] && rows_contig(s1) && !t->src[2] &&
                   t->op_params[2] == 0 && n_dims > 0 && !(n_dims & 1) && n_dims <= s0->ne[0] &&
                   param_f32(t, 6) == 1.0f && param_f32(t, 7) == 0.0f && param_f32(t, 8) == 1.0f;
        }
        case WAMX_OP_UNARY:
            if (t->src[1])  // bias + GELU-tanh bf16 (native-bf16.patch:614-628)
                return t->op_params[0] == WAMX_UNARY_GELU && s0->type == WAMX_TYPE_BF16 && wamx_is_contiguous(s0) &&
                       s1->type == WAMX_TYPE_BF16 && s1->ne[0] == s0->ne[0] && rows_contig(s1) &&
                       t->type == WAMX_TYPE_BF16 && wamx_is_contiguous(t) && wamx_are_same_shape(s0, t);
            return float_type(s0) && float_type(t) && wamx_are_same_shape(s0, t) &&
                   (t->op_params[0] == WAMX_UNARY_GELU || t->op_params[0] == WAMX_UNARY_GELU_ERF ||
                    t->op_params[0] == WAMX_UNARY_SILU);
        case WAMX_OP_LINEAR:
            if (check_linear(t)) return false;
            return !tensor_is_tiled(s0) || tiled_product_ok(s1);
        case WAMX_OP_IM2COL:
            return check_im2col(t) == nullptr;
        case WAMX_OP_CONV_2D:
            return check_conv_2d(t) == nullptr;
        case WAMX_OP_QK_NORM_ROPE:
            return check_qk_norm_rope(t) == nullptr;
        case WAMX_OP_JOINT_ATTN:
            return check_joint_attn(t) == nullptr;
        case WAMX_OP_MODULATION:
            return check_modulation(t) == nullptr;
        case WAMX_OP_EULER_STEP:
            return check_euler_step(t) == nullptr;
        case WAMX_OP_MLP_SMALL:
            return check_mlp_small(t) == nullptr;
        default:
            return false;
    }
}

// Signature of a graph: op, shapes and addresses of every node and source.
// A captured HIP graph is replayed only when the signature is unchanged.
static uint64_t graph_signature(wamx_cgraph * g) {
    uint64_t h = 1469598103934665603ull;
    auto mix = [&h](uint64_t v) {
        h ^= v;
        h *= 1099511628211ull;
    };
    const int n = wamx_graph_n_nodes(g);
    for (int i = 0; i < n; ++i) {
        const wamx_tensor * t = wamx_graph_node(g, i);
        mix((uint64_t) t->op);
        mix((uint64_t) (uintptr_t) t->data);
        for (int d = 0; d < 4; ++d) mix((uint64_t) t->ne[d] ^ ((uint64_t) t->nb[d] << 20));
        for (int k = 0; k < 16; ++k) mix((uint64_t) (uint32_t) t->op_params[k]);
        for (int k = 0; k < WAMX_MAX_SRC; ++k)
            if (t->src[k]) mix((uint64_t) (uintptr_t) t->src[k]->data);
    }
    return h;
}

static const wamx_tensor * root_of_c(const wamx_tensor * t) { return t->view_src ? t->view_src : t; }

// Cross-lane order of a two-lane graph.  Memory is tracked per root tensor
// (views resolve to their root): a node of lane A follows the latest node of
// lane B that wrote a root it reads (RAW), wrote or read a root it writes
// (WAW, WAR).  Within a lane the stream keeps node order, so waiting for the
// latest such node of the other lane covers every earlier one.  wait_for[i] is
// that node (-1: none); signal[j] marks the nodes whose completion is waited
// for.  Returns false when every node is on lane 0.
static bool plan_lanes(wamx_cgraph * g, std::vector<int> & wait_for, std::vector<char> & signal) {
    const int n = wamx_graph_n_nodes(g);
    wait_for.assign(n, -1);
    signal.assign(n, 0);
    bool two = false;
    for (int i = 0; i < n && !two; ++i) two = wamx_graph_node(g, i)->lane != 0;
    if (!two) return false;
    struct Use {
        int write[2] = {-1, -1};
        int read[2] = {-1, -1};
    };
    std::unordered_map<const wamx_tensor *, Use> use;
    for (int i = 0; i < n; ++i) {
        const wamx_tensor * node = wamx_graph_node(g, i);
        if (is_noop(node)) continue;
        const int a = node->lane ? 1 : 0, b = 1 - a;
        const wamx_tensor * w = root_of_c(node);
        int dep = -1;
        Use & uw = use[w];
        dep = std::max({dep, uw.write[b], uw.read[b]});
        for (int k = 0; k < WAMX_MAX_SRC; ++k) {
            if (!node->src[k]) continue;
            const wamx_tensor * r = root_of_c(node->src[k]);
            if (r != w) dep = std::max(dep, use[r].write[b]);
        }
        for (int k = 0; k < WAMX_MAX_SRC; ++k) {
            if (!node->src[k]) continue;
            const wamx_tensor * r = root_of_c(node->src[k]);
            if (r != w) use[r].read[a] = i;
        }
        use[w].write[a] = i;
        if (dep >= 0) wait_for[i] = dep;
    }
    // A lane that has waited for node j of the other lane need not wait for
    // an earlier node of it: that lane's stream completes its nodes in order,
    // so j's event covers them (a fused launch goes out at its first member's
    // place, before the later members' own places).  Each wait costs the
    // stream several microseconds even when its event has long completed.
    int waited[2] = {-1, -1};
    for (int i = 0; i < n; ++i) {
        if (wait_for[i] < 0) continue;
        const int a = wamx_graph_node(g, i)->lane ? 1 : 0;
        if (wait_for[i] <= waited[a]) {
            wait_for[i] = -1;
        } else {
            waited[a] = wait_for[i];
            signal[wait_for[i]] = 1;
        }
    }
    return true;
}

static hipError_t ensure_lane1(wamx_backend * be, size_t nevents) {
    if (!be->stream2 && hipStreamCreate(&be->stream2) != hipSuccess) return hipErrorOutOfMemory;
    if (!be->workspace2 && hipMalloc(&be->workspace2, kWorkspaceBytes) != hipSuccess) return hipErrorOutOfMemory;
    while (be->events.size() < nevents) {
        hipEvent_t e = nullptr;
        if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return hipErrorOutOfMemory;
        be->events.push_back(e);
    }
    return hipSuccess;
}

// Launches every node.  In a two-lane graph lane-1 nodes go to the second
// stream, each node first waits for the other lane's node it must follow
// (plan_lanes), and nodes the other lane waits for record an event (events 0
// and 1 fork and join the lanes, signalling nodes use 2, 3, ... in node order).
// A LINEAR fused with its row ops takes its members' waits and records their
// events.
static wamx_status run_nodes(wamx_backend * be, wamx_cgraph * g) {
    const int n = wamx_graph_n_nodes(g);
    std::vector<int> wait_for;
    std::vector<char> signal;
    const bool two = plan_lanes(g, wait_for, signal);
    std::vector<int> slot(n, -1);
    int nsig = 0;
    if (two)
        for (int i = 0; i < n; ++i)
            if (signal[i]) slot[i] = 2 + nsig++;
    if (two) {
        const hipError_t e = ensure_lane1(be, (size_t) nsig + 2);
        if (e != hipSuccess) {
            set_error("graph_compute: second lane stream, workspace or events unavailable");
            return WAMX_STATUS_ALLOC_FAILED;
        }
        // Fork: lane 1 starts after everything queued on lane 0 so far.
        hipEventRecord(be->events[0], be->stream);
        hipStreamWaitEvent(be->stream2, be->events[0], 0);
    }
    std::vector<char> done(n, 0);
    wamx_status status = WAMX_STATUS_SUCCESS;
    for (int i = 0; i < n && status == WAMX_STATUS_SUCCESS; ++i) {
        if (done[i]) continue;
        wamx_tensor * node = wamx_graph_node(g, i);
        for (int k = 0; k < WAMX_MAX_SRC; ++k) {
            const wamx_tensor * s = node->src[k];
            if (s && !s->data && wamx_nelements(s) > 0) {
                set_errorf("graph_compute: node %d (%s '%s') source %d '%s' has no data", i, wamx_op_name(node->op),
                           node->name, k, s->name);
                status = WAMX_STATUS_FAILED;
                break;
            }
        }
        if (status != WAMX_STATUS_SUCCESS) break;
        if (!node->data && wamx_nelements(node) > 0) {
            set_errorf("graph_compute: node %d (%s '%s') is not allocated", i, wamx_op_name(node->op), node->name);
            status = WAMX_STATUS_ALLOC_FAILED;
            break;
        }
        const int lane = two && node->lane ? 1 : 0;
        be->cs = lane ? be->stream2 : be->stream;
        be->cws = lane ? be->workspace2 : be->workspace;
        // Members of this launch: the node, or the LINEAR and its fused row ops.
        int members[8] = {i};
        int nm = 1;
        bool fused = false;
        if (node->op == WAMX_OP_LINEAR && be->fuse_rows) {
            RowPost post;
            const int last = match_row_post(g, i, n, post, two);
            if (last > i) {
                for (int j = i + 1; j <= last && nm < 8; ++j) {
                    const wamx_tensor * t = wamx_graph_node(g, j);
                    if (!is_noop(t) && (!two || (t->lane ? 1 : 0) == lane)) members[nm++] = j;
                }
                int dep = -1;
                for (int m = 0; m < nm; ++m) dep = std::max(dep, two ? wait_for[members[m]] : -1);
                // A member that must follow an other-lane node launched after
                // this LINEAR cannot run in this launch: run them one by one.
                hipError_t ferr = hipErrorNotSupported;
                if (dep <= i) {
                    if (dep >= 0) hipStreamWaitEvent(be->cs, be->events[slot[dep]], 0);
                    ferr = launch_gemm_rowpost(linear_args(be, node), post, be->cs);
                }
                if (ferr == hipSuccess) {
                    fused = true;
                    for (int m = 0; m < nm; ++m) done[members[m]] = 1;
                } else if (ferr != hipErrorNotSupported) {
                    set_errorf("graph_compute: node %d (%s '%s') with its row ops failed: %s", i,
                               wamx_op_name(node->op), node->name, hipGetErrorString(ferr));
                    status = WAMX_STATUS_FAILED;
                    break;
                } else {
                    nm = 1;
                }
            }
        }
        if (!fused && (node->op == WAMX_OP_NORM || node->op == WAMX_OP_MUL)) {
            F32Fusion f;
            const int last = match_f32_fusion(be, g, i, n, f);
            int dep = -1;
            for (int j = i; j <= last; ++j) dep = std::max(dep, two ? wait_for[j] : -1);
            if (last > i && dep < i) {
                if (dep >= 0) hipStreamWaitEvent(be->cs, be->events[slot[dep]], 0);
                const hipError_t err = run_f32_fusion(be, f);
                if (err != hipSuccess) {
                    set_errorf("graph_compute: node %d (%s '%s') fused with its F32 chain failed: %s", i,
                               wamx_op_name(node->op), node->name, hipGetErrorString(err));
                    status = WAMX_STATUS_FAILED;
                    break;
                }
                nm = 0;
                for (int j = i; j <= last && nm < 8; ++j) {
                    done[j] = 1;
                    members[nm++] = j;
                }
                fused = true;
            }
        }
        if (!fused) {
            if (two && wait_for[i] >= 0) hipStreamWaitEvent(be->cs, be->events[slot[wait_for[i]]], 0);
            const hipError_t err = compute_node(be, node);
            if (err != hipSuccess) {
                set_errorf("graph_compute: node %d (%s '%s') failed: %s", i, wamx_op_name(node->op), node->name,
                           hipGetErrorString(err));
                status = WAMX_STATUS_FAILED;
                break;
            }
            done[i] = 1;
        }
        if (two)
            for (int m = 0; m < nm; ++m)
                if (signal[members[m]]) hipEventRecord(be->events[slot[members[m]]], be->cs);
    }
    if (two) {
        // Join: lane 0 ends after lane 1's last launch.
        hipEventRecord(be->events[1], be->stream2);
        hipStreamWaitEvent(be->stream, be->events[1], 0);
    }
    be->cs = be->stream;
    be->cws = be->workspace;
    return status;
}

static void release_graph(GraphCacheEntry & e) {
    if (e.exec) hipGraphExecDestroy(e.exec);
    if (e.graph) hipGraphDestroy(e.graph);
    e.exec = nullptr;
    e.graph = nullptr;
}

static wamx_status graph_compute_impl(wamx_backend * be, wamx_cgraph * g) {
    if (!be || !g) {
        set_error("graph_compute: null argument");
        return WAMX_STATUS_FAILED;
    }
    hipSetDevice(be->dev->index);
    const int n = wamx_graph_n_nodes(g);
    for (int i = 0; i < n; ++i) {
        const wamx_tensor * node = wamx_graph_node(g, i);
        if (!supports(node)) {
            set_errorf("graph_compute: unsupported op %s at node %d ('%s')", wamx_op_name(node->op), i, node->name);
            return WAMX_STATUS_FAILED;
        }
    }
    const uint64_t uid = wamx_graph_uid(g);
    if (!be->use_graphs || uid == 0) return run_nodes(be, g);

    const uint64_t sig = graph_signature(g);
    GraphCacheEntry & e = be->graphs[uid];
    if (!e.exec || e.signature != sig || e.n_nodes != n) {
        release_graph(e);
        if (hipStreamBeginCapture(be->stream, hipStreamCaptureModeRelaxed) != hipSuccess) {
            (void) hipGetLastError();
            return run_nodes(be, g);
        }
        const wamx_status st = run_nodes(be, g);
        hipGraph_t graph = nullptr;
        const hipError_t end = hipStreamEndCapture(be->stream, &graph);
        if (st != WAMX_STATUS_SUCCESS) {
            if (graph) hipGraphDestroy(graph);
            return st;
        }
        if (end != hipSuccess || !graph) {
            set_errorf("graph_compute: stream capture failed: %s", hipGetErrorString(end));
            return WAMX_STATUS_FAILED;
        }
        hipGraphExec_t exec = nullptr;
        if (hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0) != hipSuccess) {
            hipGraphDestroy(graph);
            set_error("graph_compute: hipGraphInstantiate failed");
            return WAMX_STATUS_FAILED;
        }
        e.graph = graph;
        e.exec = exec;
        e.signature = sig;
        e.n_nodes = n;
    }
    const hipError_t err = hipGraphLaunch(e.exec, be->stream);
    if (err != hipSuccess) {
        set_errorf("graph_compute: hipGraphLaunch failed: %s", hipGetErrorString(err));
        return WAMX_STATUS_FAILED;
    }
    return WAMX_STATUS_SUCCESS;
}

// ---------------------------------------------------------------------------
// Backend / device / registry interfaces
// ---------------------------------------------------------------------------
static const char * be_get_name(wamx_backend_t be) { return be ? be->dev->name : ""; }
static void be_free(wamx_backend_t be);
static void be_set_tensor_async(wamx_backend_t be, wamx_tensor * t, const void * data, size_t off, size_t size) {
    hipMemcpyAsync((char *) t->data + off, data, size, hipMemcpyHostToDevice, be->stream);
}
static void be_get_tensor_async(wamx_backend_t be, const wamx_tensor * t, void * data, size_t off, size_t size) {
    hipMemcpyAsync(data, (const char *) t->data + off, size, hipMemcpyDeviceToHost, be->stream);
}
static bool be_cpy_tensor_async(wamx_backend_t src, wamx_backend_t, const wamx_tensor * a, wamx_tensor * b) {
    if (!a->data || !b->data || wamx_nbytes(a) != wamx_nbytes(b)) return false;
    return hipMemcpyAsync(b->data, a->data, wamx_nbytes(a), hipMemcpyDeviceToDevice, src->stream) == hipSuccess;
}
static void be_synchronize(wamx_backend_t be) {
    if (be) hipStreamSynchronize(be->stream);
}
static wamx_status be_graph_compute(wamx_backend_t be, wamx_cgraph * g) { return graph_compute_impl(be, g); }

static const wamx_backend_i k_backend_iface = {
    be_get_name, be_free, be_set_tensor_async, be_get_tensor_async, be_cpy_tensor_async, be_synchronize, be_graph_compute,
};

static const char * dev_get_name(wamx_device_t d) { return d->name; }
static const char * dev_get_description(wamx_device_t d) { return d->desc; }
static void dev_get_memory(wamx_device_t d, size_t * free_b, size_t * total_b) {
    hipSetDevice(d->index);
    if (hipMemGetInfo(free_b, total_b) != hipSuccess) *free_b = *total_b = 0;
}
static wamx_backend_t dev_init_backend(wamx_device_t d, const char *) { return wamx_backend_init(d->index); }
static wamx_buffer_type_t dev_get_buffer_type(wamx_device_t d) { return wamx_backend_buffer_type(d->index); }
static bool dev_supports_op(wamx_device_t, const wamx_tensor * op) { return op && supports(op); }
static bool dev_supports_buft(wamx_device_t d, wamx_buffer_type_t buft) { return buft && buft->dev == d; }
static bool dev_offload_op(wamx_device_t, const wamx_tensor *) { return true; }

static const wamx_device_i k_device_iface = {
    dev_get_name, dev_get_description, dev_get_memory, dev_init_backend,
    dev_get_buffer_type, dev_supports_op, dev_supports_buft, dev_offload_op,
};

static const char * reg_get_name(wamx_backend_reg_t) { return "ROCm"; }
static size_t reg_get_device_count(wamx_backend_reg_t r) { return r->devices.size(); }
static wamx_device_t reg_get_device(wamx_backend_reg_t r, size_t i) { return i < r->devices.size() ? &r->devices[i] : nullptr; }
static void * reg_get_proc_address(wamx_backend_reg_t, const char * name);

static const wamx_backend_reg_i k_reg_iface = {reg_get_name, reg_get_device_count, reg_get_device, reg_get_proc_address};

// ---------------------------------------------------------------------------
// Graph allocator
// ---------------------------------------------------------------------------
struct wamx_gallocr {
    wamx_backend * be = nullptr;
    wamx_buffer * buffer = nullptr;
};

struct FreeList {
    std::map<size_t, size_t> blocks;  // offset -> size
    size_t high = 0;
    size_t alloc(size_t size) {
        auto best = blocks.end();
        for (auto it = blocks.begin(); it != blocks.end(); ++it)
            if (it->second >= size && (best == blocks.end() || it->second < best->second)) best = it;
        if (best != blocks.end()) {
            const size_t off = best->first, bsz = best->second;
            blocks.erase(best);
            if (bsz > size) blocks[off + size] = bsz - size;
            return off;
        }
        // Grow: merge with a trailing free block if there is one.
        if (!blocks.empty()) {
            auto last = std::prev(blocks.end());
            if (last->first + last->second == high) {
                const size_t off = last->first;
                blocks.erase(last);
                high = off + size;
                return off;
            }
        }
        const size_t off = high;
        high += size;
        return off;
    }
    void release(size_t off, size_t size) {
        auto it = blocks.emplace(off, size).first;
        auto nx = std::next(it);
        if (nx != blocks.end() && it->first + it->second == nx->first) {
            it->second += nx->second;
            blocks.erase(nx);
        }
        if (it != blocks.begin()) {
            auto pv = std::prev(it);
            if (pv->first + pv->second == it->first) {
                pv->second += it->second;
                blocks.erase(it);
            }
        }
    }
};

static wamx_tensor * root_of(wamx_tensor * t) { return t->view_src ? t->view_src : t; }

// Memory plan in node order: a root tensor is placed at its first use and its
// block recycled after its last use.  In a two-lane graph each lane has its own
// arena, and a tensor is placed in the arena of the lane that touches it first
// (a lane's nodes run in order on its stream, so reuse inside a lane is safe;
// memory the other lane freed may still be in use there).  Tensors touched by
// nodes of both lanes are never recycled, since the other lane may still be
// reading them when a later node of the first lane would take their memory.
static bool gallocr_alloc(wamx_gallocr * ga, wamx_cgraph * g) {
    const int n = wamx_graph_n_nodes(g);
    std::vector<wamx_tensor *> order;  // tensors that need memory, in first-use order
    std::unordered_map<wamx_tensor *, int> last_use;
    std::unordered_map<wamx_tensor *, int> first_def;
    std::unordered_map<wamx_tensor *, int> lanes;       // bit l: touched by a lane-l node
    std::unordered_map<wamx_tensor *, int> first_lane;  // lane of the first node touching it
    const int kForever = 1 << 30;
    auto needs = [](wamx_tensor * t) { return t && !t->data && !t->view_src && wamx_nelements(t) > 0; };
    auto touch = [&](wamx_tensor * t, int i, int lane) {
        wamx_tensor * r = root_of(t);
        if (!needs(r)) return;
        if (!first_def.count(r)) {
            first_def[r] = i;
            first_lane[r] = lane;
            order.push_back(r);
        }
        lanes[r] |= 1 << lane;
        int & lu = last_use[r];
        lu = std::max(lu, i);
        // Graph inputs and outputs stay put; unallocated leaves without the
        // input flag are scratch (written in place by a later node) and are
        // recycled after their last reader like any intermediate.
        if (r->flags & (WAMX_TENSOR_FLAG_OUTPUT | WAMX_TENSOR_FLAG_INPUT)) lu = kForever;
        if (t->flags & WAMX_TENSOR_FLAG_OUTPUT) lu = kForever;
    };
    for (int i = 0; i < n; ++i) {
        wamx_tensor * node = wamx_graph_node(g, i);
        const int lane = node->lane ? 1 : 0;
        for (int k = 0; k < WAMX_MAX_SRC; ++k)
            if (node->src[k]) touch(node->src[k], i, lane);
        touch(node, i, lane);
    }
    for (auto * t : order)
        if (lanes[t] == 3) last_use[t] = kForever;
    // A LINEAR that run_nodes fuses with the row ops after it (match_row_post)
    // runs them in one launch at its own position: the reduce reads the
    // LINEAR's and the members' sources while it writes the members' outputs.
    // Those sources therefore stay live through the last member, so no member
    // output can take their memory.
    // The F32 fusions read their chain's first inputs while writing its last
    // output: those inputs stay live through the last member too.
    for (int i = 0; i < n; ++i) {
        F32Fusion f;
        const int last = match_f32_fusion(ga->be, g, i, n, f);
        if (last <= i) continue;
        for (int j = i; j <= last; ++j) {
            wamx_tensor * m = wamx_graph_node(g, j);
            for (int k = 0; k < WAMX_MAX_SRC; ++k) {
                wamx_tensor * r = m->src[k] ? root_of(m->src[k]) : nullptr;
                if (r && last_use.count(r)) last_use[r] = std::max(last_use[r], last);
            }
        }
    }
    if (ga->be->fuse_rows) {
        bool two = false;
        for (int i = 0; i < n && !two; ++i) two = wamx_graph_node(g, i)->lane != 0;
        for (int i = 0; i < n; ++i) {
            wamx_tensor * node = wamx_graph_node(g, i);
            if (node->op != WAMX_OP_LINEAR) continue;
            RowPost post;
            const int last = match_row_post(g, i, n, post, two);
            if (last <= i) continue;
            for (int j = i; j <= last; ++j) {
                wamx_tensor * m = wamx_graph_node(g, j);
                if (j > i && (is_noop(m) || (two && m->lane != node->lane))) continue;
                for (int k = 0; k < WAMX_MAX_SRC; ++k) {
                    wamx_tensor * r = m->src[k] ? root_of(m->src[k]) : nullptr;
                    if (r && last_use.count(r)) last_use[r] = std::max(last_use[r], last);
                }
            }
        }
    }
    // Leaf inputs and tensors first touched as sources are live from the start.
    FreeList fl[2];
    auto arena = [&](wamx_tensor * t) { return first_lane[t]; };
    std::unordered_map<wamx_tensor *, size_t> offset;
    std::vector<std::vector<wamx_tensor *>> frees(n);
    for (auto * t : order)
        if (last_use[t] < n) frees[last_use[t]].push_back(t);
    auto size_of = [](wamx_tensor * t) { return align_up(wamx_nbytes(t), kAlign); };
    auto place = [&](wamx_tensor * t) { offset[t] = fl[arena(t)].alloc(size_of(t)); };
    for (auto * t : order)
        if (first_def[t] == 0 || (t->flags & WAMX_TENSOR_FLAG_INPUT)) place(t);
    for (int i = 0; i < n; ++i) {
        wamx_tensor * node = wamx_graph_node(g, i);
        for (int k = 0; k < WAMX_MAX_SRC; ++k) {
            wamx_tensor * r = node->src[k] ? root_of(node->src[k]) : nullptr;
            if (r && needs(r) && !offset.count(r)) place(r);
        }
        wamx_tensor * r = root_of(node);
        if (needs(r) && !offset.count(r)) place(r);
        for (auto * t : frees[i]) fl[arena(t)].release(offset[t], size_of(t));
    }
    // Lane 1's arena follows lane 0's.
    const size_t base1 = align_up(fl[0].high, kAlign);
    for (auto & kv : offset)
        if (arena(kv.first) == 1) kv.second += base1;
    const size_t high = base1 + fl[1].high;
    const size_t total = std::max<size_t>(high, kAlign);
    if (!ga->buffer || ga->buffer->size < total) {
        if (ga->buffer) buffer_free(ga->buffer);
        ga->buffer = buft_alloc_buffer(wamx_backend_get_default_buffer_type(ga->be), total);
        if (!ga->buffer) return false;
    }
    for (auto & kv : offset) {
        kv.first->data = (char *) ga->buffer->base + kv.second;
        kv.first->buffer = ga->buffer;
    }
    // Views (and their views) alias their allocated roots.
    for (int i = 0; i < n; ++i) {
        wamx_tensor * node = wamx_graph_node(g, i);
        for (int k = -1; k < WAMX_MAX_SRC; ++k) {
            wamx_tensor * t = k < 0 ? node : node->src[k];
            if (t && t->view_src && t->view_src->data) {
                t->data = (char *) t->view_src->data + t->view_offs;
                t->buffer = t->view_src->buffer;
            }
        }
    }
    return true;
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

wamx_backend_reg_t wamx_backend_reg(void) { return registry(); }
const wamx_backend_reg_i * wamx_backend_reg_iface(void) { return &k_reg_iface; }
const wamx_device_i * wamx_device_iface(void) { return &k_device_iface; }
const wamx_backend_i * wamx_backend_iface(void) { return &k_backend_iface; }
const wamx_buffer_type_i * wamx_buffer_type_iface(void) { return &k_buft_iface; }
const wamx_buffer_i * wamx_buffer_iface(void) { return &k_buffer_iface; }

int wamx_get_device_count(void) { return (int) registry()->devices.size(); }

wamx_backend_t wamx_backend_init(int device) {
    clear_error();
    struct wamx_backend_reg * reg = registry();
    if (device < 0 || device >= (int) reg->devices.size()) {
        set_errorf("wamx_backend_init: device %d not present (%zu devices)", device, reg->devices.size());
        return nullptr;
    }
    if (hipSetDevice(device) != hipSuccess) {
        set_errorf("wamx_backend_init: hipSetDevice(%d) failed", device);
        return nullptr;
    }
    auto * be = new (std::nothrow) wamx_backend();
    if (!be) return nullptr;
    be->dev = &reg->devices[device];
    const char * env = getenv("WAMX_DISABLE_HIP_GRAPHS");
    be->use_graphs = !(env && env[0] && env[0] != '0');
    env = getenv("WAMX_DISABLE_ROW_FUSION");
    be->fuse_rows = !(env && env[0] && env[0] != '0');
    // The reference's switches for its F32 fusions (p7-fusions.patch:173-174, :216-217).
    env = getenv("WAMX_DISABLE_NORM_MODULATION_FUSION");
    be->fuse_norm_mod_f32 = !(env && env[0] && env[0] != '0');
    env = getenv("WAMX_DISABLE_GATED_RESIDUAL_FUSION");
    be->fuse_gated_residual_f32 = !(env && env[0] && env[0] != '0');
    // A blocking stream, so synchronous tensor_set/get on the null stream are
    // ordered with the graph work (default priority).
    if (hipStreamCreate(&be->stream) != hipSuccess || hipMalloc(&be->workspace, kWorkspaceBytes) != hipSuccess) {
        set_error("wamx_backend_init: stream or workspace allocation failed");
        be_free(be);
        return nullptr;
    }
    be->cs = be->stream;
    be->cws = be->workspace;
    return be;
}

static void be_free(wamx_backend_t be) {
    if (!be) return;
    hipSetDevice(be->dev->index);
    if (be->stream) hipStreamSynchronize(be->stream);
    if (be->stream2) hipStreamSynchronize(be->stream2);
    for (auto & kv : be->graphs) release_graph(kv.second);
    for (hipEvent_t e : be->events) hipEventDestroy(e);
    if (be->workspace2) hipFree(be->workspace2);
    if (be->stream2) hipStreamDestroy(be->stream2);
    if (be->workspace) hipFree(be->workspace);
    if (be->stream) hipStreamDestroy(be->stream);
    delete be;
}

void wamx_backend_free(wamx_backend_t be) { be_free(be); }
const char * wamx_backend_name(wamx_backend_t be) { return be_get_name(be); }
void * wamx_backend_stream(wamx_backend_t be) { return be ? (void *) be->stream : nullptr; }

wamx_buffer_type_t wamx_backend_buffer_type(int device) {
    struct wamx_backend_reg * reg = registry();
    if (device < 0 || device >= (int) reg->bufts.size()) return nullptr;
    return &reg->bufts[device];
}
wamx_buffer_type_t wamx_backend_get_default_buffer_type(wamx_backend_t be) {
    return be ? wamx_backend_buffer_type(be->dev->index) : nullptr;
}
wamx_buffer_type_t wamx_backend_tiled_buffer_type(int device) {
    struct wamx_backend_reg * reg = registry();
    if (device < 0 || device >= (int) reg->tiled_bufts.size()) return nullptr;
    return &reg->tiled_bufts[device];
}

wamx_buffer_t wamx_buft_alloc_buffer(wamx_buffer_type_t buft, size_t size) { return buft_alloc_buffer(buft, size); }
size_t wamx_buft_get_alignment(wamx_buffer_type_t buft) { return buft_get_alignment(buft); }
size_t wamx_buft_get_alloc_size(wamx_buffer_type_t buft, const wamx_tensor * t) { return buft_get_alloc_size(buft, t); }
wamx_buffer_t wamx_backend_alloc_buffer(wamx_backend_t be, size_t size) {
    return buft_alloc_buffer(wamx_backend_get_default_buffer_type(be), size);
}
void wamx_buffer_free(wamx_buffer_t buf) { buffer_free(buf); }
void * wamx_buffer_get_base(wamx_buffer_t buf) { return buffer_get_base(buf); }
size_t wamx_buffer_get_size(wamx_buffer_t buf) { return buf ? buf->size : 0; }

wamx_status wamx_tensor_alloc(wamx_buffer_t buf, wamx_tensor * t, void * addr) {
    WAMX_REQUIRE(buf && t && addr, "wamx_tensor_alloc: null argument");
    const char * base = (const char *) buf->base;
    WAMX_REQUIRE((const char *) addr >= base && (const char *) addr + wamx_nbytes(t) <= base + buf->size,
                 "wamx_tensor_alloc: tensor does not fit in the buffer");
    t->data = addr;
    t->buffer = buf;
    return WAMX_STATUS_SUCCESS;
}

wamx_status wamx_backend_tensor_set(wamx_tensor * t, const void * data, size_t offset, size_t size) {
    WAMX_REQUIRE(t && t->data, "tensor_set: tensor not allocated");
    WAMX_REQUIRE(offset + size <= wamx_nbytes(t), "tensor_set: out of range");
    if (tensor_is_tiled(t)) {
        WAMX_REQUIRE(offset == 0 && size == wamx_nbytes(t), "tensor_set: a tiled weight is set whole");
        WAMX_HIP_TRY(tiled_set(t, data));
        return WAMX_STATUS_SUCCESS;
    }
    WAMX_HIP_TRY(hipMemcpy((char *) t->data + offset, data, size, hipMemcpyHostToDevice));
    return WAMX_STATUS_SUCCESS;
}
wamx_status wamx_backend_tensor_get(const wamx_tensor * t, void * data, size_t offset, size_t size) {
    WAMX_REQUIRE(t && t->data, "tensor_get: tensor not allocated");
    WAMX_REQUIRE(offset + size <= wamx_nbytes(t), "tensor_get: out of range");
    if (tensor_is_tiled(t)) {
        WAMX_HIP_TRY(tiled_get(t, data, offset, size));
        return WAMX_STATUS_SUCCESS;
    }
    WAMX_HIP_TRY(hipMemcpy(data, (const char *) t->data + offset, size, hipMemcpyDeviceToHost));
    return WAMX_STATUS_SUCCESS;
}
wamx_status wamx_backend_tensor_copy(const wamx_tensor * src, wamx_tensor * dst) {
    WAMX_REQUIRE(src && dst && src->data && dst->data, "tensor_copy: unallocated tensor");
    WAMX_REQUIRE(wamx_nbytes(src) == wamx_nbytes(dst), "tensor_copy: size mismatch");
    WAMX_REQUIRE((!tensor_is_tiled(src) && !tensor_is_tiled(dst)) || wamx_are_same_shape(src, dst),
                 "tensor_copy: a tiled weight copies to or from a tensor of its shape");
    WAMX_HIP_TRY(tensor_copy_impl(src, dst));
    return WAMX_STATUS_SUCCESS;
}
wamx_status wamx_backend_tensor_memset(wamx_tensor * t, uint8_t value, size_t offset, size_t size) {
    WAMX_REQUIRE(t && t->data && offset + size <= wamx_nbytes(t), "tensor_memset: bad range");
    // A byte fill is layout-independent only over the whole tiled tensor.
    WAMX_REQUIRE(!tensor_is_tiled(t) || (offset == 0 && size == wamx_nbytes(t)),
                 "tensor_memset: a tiled weight is filled whole");
    WAMX_HIP_TRY(hipMemset((char *) t->data + offset, value, size));
    return WAMX_STATUS_SUCCESS;
}
void wamx_backend_synchronize(wamx_backend_t be) { be_synchronize(be); }

wamx_gallocr_t wamx_gallocr_new(wamx_backend_t be) {
    if (!be) return nullptr;
    auto * ga = new (std::nothrow) wamx_gallocr();
    if (ga) ga->be = be;
    return ga;
}
bool wamx_gallocr_alloc_graph(wamx_gallocr_t ga, wamx_cgraph * g) { return ga && g && gallocr_alloc(ga, g); }
size_t wamx_gallocr_get_buffer_size(wamx_gallocr_t ga) { return ga && ga->buffer ? ga->buffer->size : 0; }
void wamx_gallocr_free(wamx_gallocr_t ga) {
    if (!ga) return;
    buffer_free(ga->buffer);
    delete ga;
}

wamx_status wamx_backend_graph_compute(wamx_backend_t be, wamx_cgraph * g) {
    clear_error();
    return graph_compute_impl(be, g);
}
bool wamx_backend_supports_op(wamx_backend_t, const wamx_tensor * op) { return op && supports(op); }

// --- single-op entry points ---------------------------------------------
#define WAMX_LAUNCH(expr)                                                                  \
    do {                                                                                   \
        const hipError_t e__ = (expr);                                                     \
        if (e__ != hipSuccess) {                                                           \
            set_errorf("%s: launch failed: %s", __func__, hipGetErrorString(e__));         \
            return WAMX_STATUS_FAILED;                                                     \
        }                                                                                  \
        return WAMX_STATUS_SUCCESS;                                                        \
    } while (0)

wamx_status wamx_op_mul_mat(wamx_backend_t be, const void * w, int64_t ldw, const void * x, int32_t x_type, int64_t ldx,
                            void * y, int32_t y_type, int64_t ldy, int64_t M, int64_t N, int64_t K) {
    WAMX_REQUIRE(be && w && x && y, "wamx_op_mul_mat: null argument");
    WAMX_REQUIRE(x_type == WAMX_TYPE_F32 || x_type == WAMX_TYPE_BF16, "wamx_op_mul_mat: x type");
    WAMX_REQUIRE(y_type == WAMX_TYPE_F32 || y_type == WAMX_TYPE_BF16, "wamx_op_mul_mat: y type");
    WAMX_REQUIRE(M > 0 && N > 0 && K > 0 && ldw >= K && ldx >= K && ldy >= M, "wamx_op_mul_mat: sizes");
    GemmArgs g;
    g.w = w;
    g.ldw = ldw;
    g.x = x;
    g.x_type = x_type;
    g.ldx = ldx;
    g.y = y;
    g.y_type = y_type;
    g.ldy = ldy;
    g.M = M;
    g.N = N;
    g.K = K;
    g.ws = be->workspace;
    g.ws_bytes = kWorkspaceBytes;
    WAMX_LAUNCH(launch_gemm(g, be->stream));
}

static wamx_status op_linear(wamx_backend_t be, const void * w, bool w_tiled, const void * x, int32_t x_type,
                             const void * bias, int32_t epilogue, const void * residual, const float * gate, void * y,
                             int64_t M, int64_t N, int64_t K) {
    WAMX_REQUIRE(be && w && x && y && M > 0 && N > 0 && K > 0, "wamx_op_linear: bad arguments");
    WAMX_REQUIRE(epilogue >= WAMX_EPI_NONE && epilogue <= WAMX_EPI_BIAS_RESIDUAL, "wamx_op_linear: epilogue");
    WAMX_REQUIRE(epilogue == WAMX_EPI_NONE || bias, "wamx_op_linear: bias required");
    WAMX_REQUIRE((epilogue != WAMX_EPI_BIAS_GATED && epilogue != WAMX_EPI_BIAS_RESIDUAL) || residual,
                 "wamx_op_linear: residual required");
    WAMX_REQUIRE(epilogue != WAMX_EPI_BIAS_GATED || gate, "wamx_op_linear: gate required");
    GemmArgs g;
    g.w = w;
    g.ldw = K;
    g.x = x;
    g.x_type = x_type;
    g.ldx = K;
    g.y = y;
    g.y_type = WAMX_TYPE_BF16;
    g.ldy = M;
    g.M = M;
    g.N = N;
    g.K = K;
    g.epi = epilogue;
    g.bias = bias;
    g.res = residual;
    g.ldres = M;
    g.gate = gate;
    g.w_tiled = w_tiled;
    g.ws = be->workspace;
    g.ws_bytes = kWorkspaceBytes;
    WAMX_LAUNCH(launch_gemm(g, be->stream));
}

wamx_status wamx_op_linear(wamx_backend_t be, const void * w, const void * x, int32_t x_type, const void * bias,
                           int32_t epilogue, const void * residual, const float * gate, void * y, int64_t M, int64_t N,
                           int64_t K) {
    return op_linear(be, w, false, x, x_type, bias, epilogue, residual, gate, y, M, N, K);
}

wamx_status wamx_op_linear_tiled(wamx_backend_t be, const void * w, const void * x, int32_t x_type, const void * bias,
                                 int32_t epilogue, const void * residual, const float * gate, void * y, int64_t M,
                                 int64_t N, int64_t K) {
    WAMX_REQUIRE(M % 16 == 0 && K % 32 == 0 && N <= 64, "wamx_op_linear_tiled: needs M %% 16 == 0, K %% 32 == 0, N <= 64");
    return op_linear(be, w, true, x, x_type, bias, epilogue, residual, gate, y, M, N, K);
}

wamx_status wamx_op_norm_modulation_bf16(wamx_backend_t be, const void * x, int64_t ldx, const float * scale,
                                         const float * shift, int64_t ss, void * y, int64_t rows, int64_t cols,
                                         float eps) {
    WAMX_REQUIRE(be && x && scale && shift && y && cols > 0, "wamx_op_norm_modulation_bf16: bad arguments");
    WAMX_LAUNCH(launch_norm_mod_bf16(x, ldx, scale, shift, WAMX_TYPE_F32, ss, y, cols, rows, cols, eps, false,
                                     be->stream));
}

wamx_status wamx_op_layer_norm_bf16(wamx_backend_t be, const void * x, int64_t ldx, const void * w, const void * b,
                                    void * y, int64_t rows, int64_t cols, float eps) {
    WAMX_REQUIRE(be && x && w && b && y && cols > 0, "wamx_op_layer_norm_bf16: bad arguments");
    WAMX_LAUNCH(launch_norm_mod_bf16(x, ldx, w, b, WAMX_TYPE_BF16, 0, y, cols, rows, cols, eps, true, be->stream));
}

wamx_status wamx_op_rms_norm_bf16_f32(wamx_backend_t be, const void * x, int64_t ldx, const void * w, float * y,
                                      int64_t rows, int64_t cols, float eps) {
    WAMX_REQUIRE(be && x && w && y && cols > 0, "wamx_op_rms_norm_bf16_f32: bad arguments");
    WAMX_LAUNCH(launch_rms_norm_bf16_f32(x, ldx, w, y, cols, rows, cols, eps, be->stream));
}

wamx_status wamx_op_norm_modulation_f32(wamx_backend_t be, const float * x, int64_t ldx, const float * scale,
                                        const float * shift, int64_t ss, float * y, int64_t rows, int64_t cols,
                                        float eps) {
    WAMX_REQUIRE(be && x && scale && shift && y && cols > 0, "wamx_op_norm_modulation_f32: bad arguments");
    WAMX_LAUNCH(launch_norm_mod_f32(x, ldx, scale, shift, ss, y, rows, cols, eps, be->stream));
}

wamx_status wamx_op_gated_residual_bf16(wamx_backend_t be, const void * h, const void * b, const void * g,
                                        int32_t gate_type, int64_t gs, void * y, int64_t rows, int64_t cols) {
    WAMX_REQUIRE(be && h && b && g && y, "wamx_op_gated_residual_bf16: bad arguments");
    WAMX_REQUIRE(gate_type == WAMX_TYPE_F32 || gate_type == WAMX_TYPE_BF16, "wamx_op_gated_residual_bf16: gate type");
    WAMX_LAUNCH(launch_gated_residual_bf16(h, cols, b, cols, g, gate_type, gs, y, rows, cols, be->stream));
}

wamx_status wamx_op_gated_residual_f32(wamx_backend_t be, const float * r, const float * b, const float * g, int64_t gs,
                                       float * y, int64_t rows, int64_t cols) {
    WAMX_REQUIRE(be && r && b && g && y, "wamx_op_gated_residual_f32: bad arguments");
    WAMX_LAUNCH(launch_gated_residual_f32(r, cols, b, cols, g, gs, y, rows, cols, be->stream));
}

wamx_status wamx_op_bias_gelu_bf16(wamx_backend_t be, const void * x, const void * bias, void * y, int64_t n,
                                   int64_t width) {
    WAMX_REQUIRE(be && x && bias && y && width > 0, "wamx_op_bias_gelu_bf16: bad arguments");
    WAMX_LAUNCH(launch_bias_gelu_bf16(x, bias, y, n, width, be->stream));
}

wamx_status wamx_op_rope_f32(wamx_backend_t be, const float * x, const int32_t * pos, float * y, int64_t head_dim,
                             int64_t heads, int64_t tokens, int n_dims, float freq_base) {
    WAMX_REQUIRE(be && x && pos && y && n_dims > 0 && n_dims <= head_dim && !(n_dims & 1), "wamx_op_rope_f32: bad args");
    TensorRef rx{(void *) x, WAMX_TYPE_F32, {head_dim, heads, tokens, 1},
                 {4, 4 * head_dim, 4 * head_dim * heads, 4 * head_dim * heads * tokens}};
    TensorRef ry = rx;
    ry.data = y;
    WAMX_LAUNCH(launch_rope_f32(rx, pos, ry, n_dims, freq_base, be->stream));
}

wamx_status wamx_op_qk_norm_rope(wamx_backend_t be, const void * x, int64_t ldx, const void * w, void * dst,
                                 int64_t heads, int64_t head_dim, int64_t tokens, int64_t dst_tokens, int64_t tok0,
                                 int rope_mode, const int32_t * pos0, const int32_t * pos1, const int32_t * pos2,
                                 float eps, float freq_base) {
    WAMX_REQUIRE(be && x && w && dst, "wamx_op_qk_norm_rope: null argument");
    WAMX_REQUIRE(rope_mode >= 0 && rope_mode <= 2, "wamx_op_qk_norm_rope: rope mode");
    WAMX_REQUIRE(rope_mode == 2 || pos0, "wamx_op_qk_norm_rope: positions required");
    WAMX_REQUIRE(rope_mode != 1 || (pos1 && pos2 && head_dim == 128), "wamx_op_qk_norm_rope: 3-D positions");
    WAMX_REQUIRE(tok0 >= 0 && tok0 + tokens <= dst_tokens, "wamx_op_qk_norm_rope: token range");
    WAMX_LAUNCH(launch_qk_norm_rope(x, ldx, w, dst, heads, head_dim, tokens, dst_tokens, tok0, rope_mode, pos0, pos1,
                                    pos2, eps, freq_base, be->stream));
}

wamx_status wamx_op_rope_table(wamx_backend_t be, int rope_mode, const int32_t * pos0, const int32_t * pos1,
                               const int32_t * pos2, int64_t tokens, int64_t head_dim, float freq_base, float * out) {
    WAMX_REQUIRE(be && out, "wamx_op_rope_table: null argument");
    WAMX_LAUNCH(launch_rope_table(rope_mode, pos0, pos1, pos2, tokens, head_dim, freq_base, out, be->stream));
}

wamx_status wamx_op_qk_norm_rope_table(wamx_backend_t be, const void * x, int64_t ldx, const void * w, void * dst,
                                       int64_t heads, int64_t head_dim, int64_t tokens, int64_t dst_tokens,
                                       int64_t tok0, const float * table, float eps) {
    WAMX_REQUIRE(be && x && w && dst && table, "wamx_op_qk_norm_rope_table: null argument");
    WAMX_REQUIRE(tok0 >= 0 && tok0 + tokens <= dst_tokens, "wamx_op_qk_norm_rope_table: token range");
    WAMX_LAUNCH(launch_qk_norm_rope(x, ldx, w, dst, heads, head_dim, tokens, dst_tokens, tok0, 3, nullptr, nullptr,
                                    nullptr, eps, 10000.0f, be->stream, 0, 0, 0, table));
}

wamx_status wamx_op_qk_norm_rope_hilo(wamx_backend_t be, const void * x, int64_t ldx, const void * w, void * dst_hi,
                                      void * dst_lo, int64_t heads, int64_t head_dim, int64_t tokens, int64_t dst_tokens,
                                      int64_t tok0, int rope_mode, const int32_t * pos0, const int32_t * pos1,
                                      const int32_t * pos2, float eps, float freq_base) {
    WAMX_REQUIRE(be && x && w && dst_hi && dst_lo, "wamx_op_qk_norm_rope_hilo: null argument");
    WAMX_REQUIRE(rope_mode >= 0 && rope_mode <= 2, "wamx_op_qk_norm_rope_hilo: rope mode");
    WAMX_REQUIRE(rope_mode == 2 || pos0, "wamx_op_qk_norm_rope_hilo: positions required");
    WAMX_REQUIRE(rope_mode != 1 || (pos1 && pos2 && head_dim == 128), "wamx_op_qk_norm_rope_hilo: 3-D positions");
    WAMX_REQUIRE(tok0 >= 0 && tok0 + tokens <= dst_tokens, "wamx_op_qk_norm_rope_hilo: token range");
    const ptrdiff_t off = (const char *) dst_lo - (const char *) dst_hi;
    WAMX_REQUIRE(off != 0 && off % 16 == 0, "wamx_op_qk_norm_rope_hilo: the lo plane must be 16-byte aligned to the hi plane");
    WAMX_LAUNCH(launch_qk_norm_rope(x, ldx, w, dst_hi, heads, head_dim, tokens, dst_tokens, tok0, rope_mode, pos0, pos1,
                                    pos2, eps, freq_base, be->stream, 0, 0, (int64_t) (off / 2)));
}

wamx_status wamx_op_joint_attn_hilo(wamx_backend_t be, const void * q, const void * q_lo, const void * k,
                                    const void * k_lo, const void * vt, int64_t nk, int64_t vt_ld, void * out,
                                    int64_t heads, int64_t head_dim, int64_t tq, float scale) {
    WAMX_REQUIRE(be && q && q_lo && k && k_lo && vt && out, "wamx_op_joint_attn_hilo: null argument");
    WAMX_REQUIRE(head_dim == 128, "wamx_op_joint_attn_hilo: head_dim must be 128");
    WAMX_REQUIRE(nk >= 8 && vt_ld >= nk && vt_ld % 8 == 0 && heads > 0 && tq >= 0,
                 "wamx_op_joint_attn_hilo: at least 8 keys, V^T rows a multiple of 8 keys");
    AttnArgs a;
    a.q = q;
    a.q_lo = q_lo;
    a.k_a = k;
    a.k_lo = k_lo;
    a.vt_a = vt;
    a.na = nk;
    a.vt_ld_a = vt_ld;
    a.out = out;
    a.heads = heads;
    a.head_dim = head_dim;
    a.tq = tq;
    a.scale = scale;
    a.ws = be->workspace;
    a.ws_bytes = kWorkspaceBytes;
    WAMX_LAUNCH(launch_joint_attn(a, be->stream));
}

wamx_status wamx_op_joint_attn(wamx_backend_t be, const void * q, const void * k_a, const void * vt_a, int64_t na,
                               const void * k_b, const void * vt_b, int64_t nb, int64_t na_split, void * out,
                               int64_t heads, int64_t head_dim, int64_t tq, float scale) {
    WAMX_REQUIRE(be && q && k_a && vt_a && out, "wamx_op_joint_attn: null argument");
    WAMX_REQUIRE(head_dim == 128, "wamx_op_joint_attn: head_dim must be 128");
    WAMX_REQUIRE(na % 4 == 0 && (!k_b || nb % 4 == 0),
                 "wamx_op_joint_attn: key counts must be multiples of 4 (pad V^T rows)");
    WAMX_REQUIRE(na >= 0 && nb >= 0 && heads > 0 && tq >= 0 && na_split >= 0 && na_split <= na,
                 "wamx_op_joint_attn: negative size or split outside the first source");
    WAMX_REQUIRE(na + (k_b ? nb : 0) > 0, "wamx_op_joint_attn: no keys (softmax over an empty key set)");
    AttnArgs a;
    a.q = q;
    a.k_a = k_a;
    a.vt_a = vt_a;
    a.na = na;
    a.vt_ld_a = na;
    a.k_b = k_b;
    a.vt_b = vt_b;
    a.nb = k_b ? nb : 0;
    a.vt_ld_b = a.nb;
    a.na_split = na_split;
    a.out = out;
    a.heads = heads;
    a.head_dim = head_dim;
    a.tq = tq;
    a.scale = scale;
    a.ws = be->workspace;
    a.ws_bytes = kWorkspaceBytes;
    WAMX_LAUNCH(launch_joint_attn(a, be->stream));
}

wamx_status wamx_op_soft_max_f32(wamx_backend_t be, const float * x, float * y, int64_t rows, int64_t cols, float scale) {
    WAMX_REQUIRE(be && x && y && cols > 0, "wamx_op_soft_max_f32: bad arguments");
    TensorRef rx{(void *) x, WAMX_TYPE_F32, {cols, rows, 1, 1}, {4, 4 * cols, 4 * cols * rows, 4 * cols * rows}};
    TensorRef ry = rx;
    ry.data = y;
    const TensorRef no_mask{};
    WAMX_LAUNCH(launch_softmax_f32(rx, no_mask, ry, scale, be->stream));
}

wamx_status wamx_fill_normal(wamx_backend_t be, void * dst, int32_t type, int64_t n, uint64_t seed, float mean,
                             float stdv) {
    WAMX_REQUIRE(be && dst, "wamx_fill_normal: null argument");
    WAMX_LAUNCH(launch_fill_normal(dst, type, n, seed, mean, stdv, be->stream));
}

void * wamx_device_malloc(wamx_backend_t be, size_t size) {
    if (!be) return nullptr;
    hipSetDevice(be->dev->index);
    void * p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(size, 1)) != hipSuccess) {
        set_errorf("hipMalloc(%zu) failed", size);
        return nullptr;
    }
    return p;
}
void wamx_device_free(wamx_backend_t, void * p) {
    if (p) hipFree(p);
}
wamx_status wamx_memcpy_h2d(wamx_backend_t be, void * dst, const void * src, size_t size) {
    WAMX_REQUIRE(be, "null backend");
    WAMX_HIP_TRY(hipMemcpy(dst, src, size, hipMemcpyHostToDevice));
    return WAMX_STATUS_SUCCESS;
}
wamx_status wamx_memcpy_d2h(wamx_backend_t be, void * dst, const void * src, size_t size) {
    WAMX_REQUIRE(be, "null backend");
    WAMX_HIP_TRY(hipStreamSynchronize(be->stream));
    WAMX_HIP_TRY(hipMemcpy(dst, src, size, hipMemcpyDeviceToHost));
    return WAMX_STATUS_SUCCESS;
}

struct wamx_timer {
    wamx_backend * be;
    hipEvent_t a, b;
};
wamx_timer_t wamx_timer_new(wamx_backend_t be) {
    if (!be) return nullptr;
    auto * t = new wamx_timer{be, nullptr, nullptr};
    hipEventCreate(&t->a);
    hipEventCreate(&t->b);
    return t;
}
void wamx_timer_start(wamx_timer_t t) {
    if (t) hipEventRecord(t->a, t->be->stream);
}
float wamx_timer_stop_ms(wamx_timer_t t) {
    if (!t) return -1.0f;
    hipEventRecord(t->b, t->be->stream);
    hipEventSynchronize(t->b);
    float ms = -1.0f;
    hipEventElapsedTime(&ms, t->a, t->b);
    return ms;
}
void wamx_timer_free(wamx_timer_t t) {
    if (!t) return;
    hipEventDestroy(t->a);
    hipEventDestroy(t->b);
    delete t;
}

}  // extern "C"

static void * reg_get_proc_address(wamx_backend_reg_t, const char * name) {
    if (!name) return nullptr;
    if (!strcmp(name, "wamx_backend_graph_compute")) return (void *) &wamx_backend_graph_compute;
    if (!strcmp(name, "wamx_backend_supports_op")) return (void *) &wamx_backend_supports_op;
    if (!strcmp(name, "wamx_backend_init")) return (void *) &wamx_backend_init;
    return nullptr;
}
