// Synthetic GWP-0.5-shaped Mixture-of-Transformers driver.
//
// Builds the three graphs wam.cpp submits per request in its BF16 latency
// profile and runs them through this backend's graph_compute:
//   1. prompt projection: action text embedder + per-layer cross-attention
//      K/V of the prompt (src/models/gwp05/engine/cache.cpp:53-137),
//   2. prefix pass: state token through the action expert and the visual
//      tokens through the visual expert, joint self-attention, per-layer K/V
//      written to the resident prefix cache (cache.cpp:139-485),
//   3. unrolled denoise: num_steps flow-matching steps of the action expert
//      attending [state, action, reference] keys and the cached prompt K/V
//      (mot.cpp:358-594).
// Op order and bf16 rounding points follow those files; the fused ops of this
// backend (LINEAR, QK_NORM_ROPE, JOINT_ATTN, MODULATION) replace the unfused
// ggml subgraphs with the same rounding points.
#include <math.h>
#include <stdio.h>

#include <algorithm>
#include <map>
#include <memory>
#include <string>
#include <thread>
#include <vector>

#include "common.h"
#include "internal.h"

using namespace wamx;

namespace {

struct Mlp3 {  // action/state encoder and action decoder (mot.cpp:16-55)
    wamx_tensor *in_w, *in_b, *mid_w, *mid_b, *out_w, *out_b;
};

struct Cond {  // condition embedder (mot.cpp:63-99)
    wamx_tensor *t1_w, *t1_b, *t2_w, *t2_b, *tp_w, *tp_b, *x1_w, *x1_b, *x2_w, *x2_b;
};

struct ExpertLayer {  // one expert of one MoT block
    wamx_tensor *qkv_w, *qkv_b, *norm_q, *norm_k, *o_w, *o_b;
    wamx_tensor *n2_w, *n2_b;
    wamx_tensor *cq_w, *cq_b, *ck_w, *ck_b, *cv_w, *cv_b, *cnq, *cnk, *co_w, *co_b;
    wamx_tensor *up_w, *up_b, *dn_w, *dn_b;
};

uint64_t fnv1a(const std::string & s) {
    uint64_t h = 1469598103934665603ull;
    for (unsigned char c : s) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

}  // namespace

struct wamx_gwp_model {
    wamx_backend_t be = nullptr;
    wamx_gwp_config cfg{};
    int64_t P = 0, Ppad = 0, nimg = 0, NLpad = 0, Tpad = 0;
    int64_t B = 1;  // independent chunks (cfg.batch)

    wamx_context * wctx = nullptr;
    wamx_buffer_t wbuf = nullptr;
    // The action expert's few-token projections, in the tiled buffer type.
    wamx_context * tctx = nullptr;
    wamx_buffer_t tbuf = nullptr;
    std::vector<std::pair<std::string, wamx_tensor *>> weights;
    std::map<std::string, wamx_tensor *> by_name;

    wamx_tensor *patch_w = nullptr, *patch_b = nullptr, *action_sst = nullptr;
    wamx_tensor *a_tables = nullptr, *v_tables = nullptr;  // [d, 6, L] bf16
    // Cross-attention K/V projections of every layer, per expert (0 action,
    // 1 visual): weight [w, 2·L·d] and bias [2·L·d]; layer l's to_k rows start
    // at 2l·d and its to_v rows at (2l+1)·d.  The per-layer weights are views.
    wamx_tensor *kv_w[2] = {nullptr, nullptr}, *kv_b[2] = {nullptr, nullptr};
    // Each expert's attn2.norm_k weights of every layer, packed [d, L] (the
    // per-layer weights are views with their reference names), so the prompt
    // keys of every layer are normalised by one launch.
    wamx_tensor * cnk_all[2] = {nullptr, nullptr};
    Mlp3 state_enc{}, action_enc{}, action_dec{};
    Cond acond{}, vcond{};
    std::vector<ExpertLayer> act, vis;

    // Resident storage (prefix / prompt caches) and inputs; the last dim of
    // each is the chunk.
    wamx_context * sctx = nullptr;
    wamx_buffer_t sbuf = nullptr;
    wamx_tensor * action_prompt = nullptr;        // [da, NL, B]
    std::vector<wamx_tensor *> pk, pv_raw, pv;    // prefix K [dh,P,H,B]; V^T [Ppad,dh,H,B] and its [P,dh,H,B] view
    std::vector<wamx_tensor *> lk, lv_raw, lv;    // prompt K [dh,NL,H,B]; V^T
    // The layers' prompt caches in one allocation each, layer-major
    // ([dh, NL, H, L*B] and [NLpad, dh, H, L*B]); lk[l] and lv_raw[l] are
    // views of them, so the prompt graph fills every layer in one launch.
    wamx_tensor *lk_all = nullptr, *lv_raw_all = nullptr;
    wamx_tensor *in_state = nullptr, *in_latent = nullptr, *in_prompt = nullptr, *in_action = nullptr;
    wamx_tensor *in_apos = nullptr, *in_spos = nullptr, *in_vt = nullptr, *in_vh = nullptr, *in_vw = nullptr;
    wamx_tensor *in_freq0 = nullptr, *in_freqs = nullptr, *in_dts = nullptr;
    // (cos, sin) of the 3-D rope of every visual token [dh, nimg] (rope mode
    // 3): the positions are the grid's, fixed, so the prefix's Q and K of
    // every layer rotate from this table.
    wamx_tensor * vis_rope = nullptr;

    // Graphs: a prompt and a prefix graph per chunk, then the denoise graph
    // of all chunks (graphs[2B]).
    std::vector<wamx_context *> gctx;
    std::vector<wamx_cgraph *> graph;
    std::vector<wamx_gallocr_t> galloc;
    wamx_tensor * action_out = nullptr;
    // The action decoder's output of every denoise step, bf16 [A, B*T] (the
    // velocity the scheduler step adds, kept as graph outputs so the
    // allocator never reuses their memory).
    std::vector<wamx_tensor *> velocity;
    wamx_timer_t timer = nullptr;
    // Projected-prompt reuse across requests (cache.cpp:53-137): with a
    // nonzero capacity, the prompt whose K/V the prompt caches hold is kept on
    // the host; a request whose prompt has the same bytes skips the upload and
    // the prompt graphs.  prompt_stale: the uploaded prompt is not projected.
    size_t prompt_cache_capacity = 0;
    std::vector<float> prompt_sig;
    bool prompt_stale = true;
    uint64_t prompt_hits = 0, prompt_misses = 0;
    // Device staging of the f32 latent and prompt of set_inputs: uploaded
    // there, scanned for Inf / NaN on the GPU (first bad index of each in
    // `flags`), and copied into the input tensors only when both are finite.
    void * stage = nullptr;
    uint32_t * flags = nullptr;

    int n_graphs() const { return (int) (2 * B + 1); }
    int prompt_graph(int64_t b) const { return (int) b; }
    int prefix_graph(int64_t b) const { return (int) (B + b); }
    int denoise_graph() const { return (int) (2 * B); }

    ~wamx_gwp_model() {
        if (stage) wamx_device_free(be, stage);
        for (size_t i = 0; i < graph.size(); ++i) {
            wamx_gallocr_free(galloc[i]);
            wamx_free(gctx[i]);
        }
        wamx_timer_free(timer);
        wamx_buffer_free(sbuf);
        wamx_free(sctx);
        wamx_buffer_free(wbuf);
        wamx_free(wctx);
        wamx_buffer_free(tbuf);
        wamx_free(tctx);
    }

    wamx_tensor * add_weight(const std::string & name, int64_t ne0, int64_t ne1 = 1, int64_t ne2 = 1, int64_t ne3 = 1,
                             bool tiled = false) {
        wamx_tensor * t = wamx_new_tensor_4d(tiled ? tctx : wctx, WAMX_TYPE_BF16, ne0, ne1, ne2, ne3);
        if (!t) return nullptr;
        wamx_set_name(t, name.c_str());
        weights.push_back({name, t});
        by_name[name] = t;
        return t;
    }
    // Linear layer [out][in]: ggml ne = {in, out}; `tiled` places the weight
    // in the tiled buffer (products of at most 64 tokens only).
    void add_linear(const std::string & prefix, int64_t in, int64_t out, wamx_tensor ** w, wamx_tensor ** b,
                    bool tiled = false) {
        *w = add_weight(prefix + ".weight", in, out, 1, 1, tiled);
        *b = add_weight(prefix + ".bias", out);
    }
    // A linear layer whose weight rows [row0, row0+out) and bias entries live
    // inside the packed tensors `pw` [in, R] and `pb` [R].
    // A 1-D weight of n elements at element offset off of the packed tensor `pk`.
    wamx_tensor * add_weight_view(const std::string & name, wamx_tensor * pk, int64_t off, int64_t n) {
        wamx_tensor * t = wamx_view_1d(wctx, pk, n, (size_t) off * pk->nb[0]);
        if (t) wamx_set_name(t, name.c_str());
        weights.push_back({name, t});
        by_name[name] = t;
        return t;
    }
    void add_linear_view(const std::string & prefix, wamx_tensor * pw, wamx_tensor * pb, int64_t row0, int64_t out,
                         wamx_tensor ** w, wamx_tensor ** b) {
        *w = wamx_view_2d(wctx, pw, pw->ne[0], out, pw->nb[1], (size_t) row0 * pw->nb[1]);
        *b = wamx_view_1d(wctx, pb, out, (size_t) row0 * pb->nb[0]);
        for (auto & [name, t] : {std::pair<std::string, wamx_tensor *>{prefix + ".weight", *w}, {prefix + ".bias", *b}}) {
            if (t) wamx_set_name(t, name.c_str());
            weights.push_back({name, t});
            by_name[name] = t;
        }
    }
};

// ---------------------------------------------------------------------------
// Graph-building helpers (ctx-local)
// ---------------------------------------------------------------------------
namespace {

struct Builder {
    wamx_gwp_model * m;
    wamx_context * ctx;
    const wamx_gwp_config & c;
    float scale;

    Builder(wamx_gwp_model * model, wamx_context * context)
        : m(model), ctx(context), c(model->cfg), scale(1.0f / sqrtf((float) model->cfg.head_dim)) {}

    wamx_tensor * lin(wamx_tensor * w, wamx_tensor * b, wamx_tensor * x, int epi = WAMX_EPI_BIAS,
                      wamx_tensor * res = nullptr, wamx_tensor * gate = nullptr) {
        return wamx_linear(ctx, w, x, b, epi, res, gate);
    }

    // action_encoder / action_decoder (mot.cpp:16-55): linear + GELU_ERF x2 + linear.
    // The two layers that are at most 128 wide on both sides run as one
    // MLP_SMALL node: in + mid of the encoder (action_dim -> hidden ->
    // hidden), mid + out of the decoder (hidden -> hidden -> action_dim).
    wamx_tensor * mlp3(const Mlp3 & p, wamx_tensor * x) {
        auto small = [](const wamx_tensor * w) { return w->ne[0] <= 128 && w->ne[1] <= 128; };
        if (x->type == WAMX_TYPE_BF16 && small(p.in_w) && small(p.mid_w)) {
            wamx_tensor * h = wamx_mlp_small(ctx, x, p.in_w, p.in_b, p.mid_w, p.mid_b,
                                             WAMX_MLP_GELU_MID | WAMX_MLP_GELU_OUT);
            return lin(p.out_w, p.out_b, h);
        }
        if (small(p.mid_w) && small(p.out_w)) {
            wamx_tensor * h = lin(p.in_w, p.in_b, x);
            return wamx_mlp_small(ctx, h, p.mid_w, p.mid_b, p.out_w, p.out_b, WAMX_MLP_GELU_IN | WAMX_MLP_GELU_MID);
        }
        wamx_tensor * h = wamx_gelu_erf(ctx, lin(p.in_w, p.in_b, x));
        h = wamx_gelu_erf(ctx, lin(p.mid_w, p.mid_b, h));
        return lin(p.out_w, p.out_b, h);
    }

    // build_condition time branch (mot.cpp:69-82): temb and the 6-way modulation.
    void condition(const Cond & p, wamx_tensor * freq, wamx_tensor ** temb, wamx_tensor ** mod) {
        wamx_tensor * t = lin(p.t1_w, p.t1_b, freq);
        t = lin(p.t2_w, p.t2_b, wamx_silu(ctx, t));
        *temb = t;
        *mod = lin(p.tp_w, p.tp_b, wamx_silu(ctx, t));
    }

    // build_condition text branch (mot.cpp:84-92): linear + GELU + linear.
    wamx_tensor * text(const Cond & p, wamx_tensor * prompt) {
        wamx_tensor * h = wamx_gelu(ctx, lin(p.x1_w, p.x1_b, prompt));
        return lin(p.x2_w, p.x2_b, h);
    }

    // The attention output [d, T, B] as the [d, B*T] rows the projections read.
    wamx_tensor * rows(wamx_tensor * att) {
        return att->ne[2] == 1 ? att : wamx_reshape_2d(ctx, att, att->ne[0], att->ne[1] * att->ne[2]);
    }

    // View (layer l, part i, step s) of a modulation tensor [width, 6, L, S] (f32).
    wamx_tensor * part(wamx_tensor * mods, int64_t width, int l, int i, int s = 0) {
        const int64_t L = mods->ne[2];
        return wamx_view_1d(ctx, mods, width, (size_t) (((int64_t) s * L + l) * 6 + i) * width * sizeof(float));
    }

    // Column view [ne0 = cols, ne1 = rows] of a packed projection output.
    wamx_tensor * cols(wamx_tensor * x, int64_t ncols, int64_t off_elems) {
        return wamx_view_2d(ctx, x, ncols, x->ne[1], x->nb[1], (size_t) off_elems * 2);
    }

    // V part of a packed [3d, tokens] projection, transposed into a V^T view
    // [tokens, dh, H] of `dst` (ggml_cont(ggml_permute(v, 1, 2, 0, 3)),
    // mot.cpp:397-401, written in place as cache.cpp:316-339 stores it).
    // With chunks (dst_view [T, dh, H, B]) the rows of qkv are B chunks of T
    // tokens.
    wamx_tensor * store_v(wamx_tensor * qkv, int64_t v_off, wamx_tensor * dst_view) {
        const int64_t dh = c.head_dim, H = c.n_heads, B = dst_view->ne[3], T = qkv->ne[1] / B;
        wamx_tensor * v = B == 1 ? wamx_view_3d(ctx, qkv, dh, H, T, (size_t) dh * 2, qkv->nb[1], (size_t) v_off * 2)
                                 : wamx_view_4d(ctx, qkv, dh, H, T, B, (size_t) dh * 2, qkv->nb[1],
                                                qkv->nb[1] * (size_t) T, (size_t) v_off * 2);
        wamx_tensor * vp = wamx_permute(ctx, v, 1, 2, 0, 3);
        return wamx_cpy(ctx, vp, dst_view);
    }

    // Layer l's K (half 0) or V (half 1) columns of a packed projection of
    // every layer [2·L·d, T], as [d, T, L]: layer l's at columns (2l + half)·d.
    // (The first `layers` layers.)
    wamx_tensor * layer_cols(wamx_tensor * kv, int half, int64_t layers) {
        const int64_t d = (int64_t) c.n_heads * c.head_dim;
        return wamx_view_3d(ctx, kv, d, kv->ne[1], layers, kv->nb[1], (size_t) (2 * d) * kv->nb[0],
                            (size_t) (half * d) * kv->nb[0]);
    }
    // The first dst->ne[3] layers' V^T [T, dh, H, layers] from a packed
    // projection of every layer [2·L·d, T] into `dst` (one transposing copy).
    wamx_tensor * store_v_layers(wamx_tensor * kv, wamx_tensor * dst) {
        const int64_t dh = c.head_dim, H = c.n_heads, d = dh * H, T = kv->ne[1];
        wamx_tensor * v = wamx_view_4d(ctx, kv, dh, H, T, dst->ne[3], (size_t) dh * kv->nb[0], kv->nb[1],
                                       (size_t) (2 * d) * kv->nb[0], (size_t) d * kv->nb[0]);
        return wamx_cpy(ctx, wamx_permute(ctx, v, 1, 2, 0, 3), dst);
    }

    // V^T view of `raw` [ld, dh, H(, B)] covering key columns [k0, k0+n).
    wamx_tensor * vt_view(wamx_tensor * raw, int64_t k0, int64_t n) {
        if (raw->ne[3] == 1)
            return wamx_view_3d(ctx, raw, n, raw->ne[1], raw->ne[2], raw->nb[1], raw->nb[2], (size_t) k0 * 2);
        return wamx_view_4d(ctx, raw, n, raw->ne[1], raw->ne[2], raw->ne[3], raw->nb[1], raw->nb[2], raw->nb[3],
                            (size_t) k0 * 2);
    }

    // Chunk b of a storage tensor whose last dim (dim 3) is the chunk.
    wamx_tensor * chunk(wamx_tensor * t, int64_t b) {
        return wamx_view_3d(ctx, t, t->ne[0], t->ne[1], t->ne[2], t->nb[1], t->nb[2], t->nb[3] * (size_t) b);
    }

    // expert_cross_ffn with cached prompt K/V (mot.cpp:284-347, cached branch).
    wamx_tensor * cross_ffn_cached(const ExpertLayer & e, wamx_tensor * h, wamx_tensor * pk, wamx_tensor * pv,
                                   wamx_tensor * cshift, wamx_tensor * cscale, wamx_tensor * cgate) {
        const int64_t B = pk->ne[3], T = h->ne[1] / B;  // rows: B chunks of T tokens
        wamx_tensor * n = wamx_layer_norm_bf16(ctx, h, e.n2_w, e.n2_b, c.eps);
        wamx_tensor * q = lin(e.cq_w, e.cq_b, n);
        wamx_tensor * Q = wamx_new_tensor_4d(ctx, WAMX_TYPE_BF16, c.head_dim, T, c.n_heads, B);
        Q = wamx_qk_norm_rope(ctx, q, e.cnq, Q, 0, 2, nullptr, nullptr, nullptr, c.eps, 10000.0f);
        wamx_tensor * att = rows(wamx_joint_attn(ctx, Q, pk, pv, nullptr, nullptr, 0, scale));
        h = lin(e.co_w, e.co_b, att, WAMX_EPI_BIAS_RESIDUAL, h);
        return ffn(e, h, cshift, cscale, cgate);
    }

    // expert_cross_ffn against uncached text (build_attention, text_encoder.cpp:26-73).
    // RMSNorm keeps Q and K in f32 there and the scores are f32 x f32
    // (rms_norm_bf16_f32, then MUL_MAT at GGML_PREC_F32): Q and K are held as
    // bf16 hi/lo planes and the scores formed f32-accurate from them.  K (the
    // layer's text keys, hi/lo [dh, NL, H, 2]) and V (their V^T [NL, dh, H])
    // come from text_kv, which makes them for every layer at once.
    wamx_tensor * cross_ffn_uncached(const ExpertLayer & e, wamx_tensor * h, wamx_tensor * K, wamx_tensor * V,
                                     wamx_tensor * cshift, wamx_tensor * cscale, wamx_tensor * cgate) {
        const int64_t T = h->ne[1];
        wamx_tensor * n = wamx_layer_norm_bf16(ctx, h, e.n2_w, e.n2_b, c.eps);
        wamx_tensor * q = lin(e.cq_w, e.cq_b, n);
        wamx_tensor * Q = wamx_new_tensor_4d(ctx, WAMX_TYPE_BF16, c.head_dim, T, c.n_heads, 2);
        Q = wamx_qk_norm_rope_hilo(ctx, q, e.cnq, Q, 0, 2, nullptr, nullptr, nullptr, c.eps, 10000.0f);
        wamx_tensor * att = wamx_joint_attn_hilo(ctx, Q, K, V, scale);
        h = lin(e.co_w, e.co_b, att, WAMX_EPI_BIAS_RESIDUAL, h);
        return ffn(e, h, cshift, cscale, cgate);
    }

    // FFN half (mot.cpp:339-346): modulated norm, up + bias + GELU-tanh, down +
    // bias + gated residual.
    wamx_tensor * ffn(const ExpertLayer & e, wamx_tensor * h, wamx_tensor * cshift, wamx_tensor * cscale,
                      wamx_tensor * cgate) {
        wamx_tensor * n = wamx_norm_modulation_bf16(ctx, h, cscale, cshift, c.eps);
        wamx_tensor * u = lin(e.up_w, e.up_b, n, WAMX_EPI_BIAS_GELU);
        return lin(e.dn_w, e.dn_b, u, WAMX_EPI_BIAS_GATED, h, cgate);
    }
};

// Make `t` depend on `dep` without reading it (views ignore src[1]).
wamx_tensor * after(wamx_tensor * t, wamx_tensor * dep) {
    if (t && dep && t->op == WAMX_OP_VIEW && !t->src[1]) t->src[1] = dep;
    return t;
}

}  // namespace

// ---------------------------------------------------------------------------
// Model construction
// ---------------------------------------------------------------------------
static bool create_weights(wamx_gwp_model * m) {
    const wamx_gwp_config & c = m->cfg;
    const int64_t d = (int64_t) c.n_heads * c.head_dim, da = c.action_hidden, E = c.enc_hidden, A = c.action_dim;
    const int64_t L = c.n_layers;
    m->wctx = wamx_init(64 * L + 256);
    m->tctx = wamx_init(8 * L + 16);
    if (!m->wctx || !m->tctx) return false;
    m->patch_w = m->add_weight("gwp.patch_embedding.weight", 2, 2, c.z_dim, d);
    m->patch_b = m->add_weight("gwp.patch_embedding.bias", d);
    // The action encoder's out_proj (hidden -> da) and the decoder's in_proj
    // (da -> hidden) run on the denoise tokens only: tiled when those are few.
    const bool few = m->B * c.action_chunk <= 64;
    auto mlp = [&](const std::string & p, int64_t in, int64_t out, Mlp3 & r, bool t_in, bool t_out) {
        m->add_linear(p + ".in_proj", in, E, &r.in_w, &r.in_b, t_in && E % 16 == 0 && in % 32 == 0);
        m->add_linear(p + ".mid_proj", E, E, &r.mid_w, &r.mid_b);
        m->add_linear(p + ".out_proj", E, out, &r.out_w, &r.out_b, t_out && out % 16 == 0 && E % 32 == 0);
    };
    mlp("gwp.state_encoder", A, da, m->state_enc, false, false);
    mlp("gwp.action_encoder", A, da, m->action_enc, false, few);
    mlp("gwp.action_decoder", da, A, m->action_dec, few, false);
    auto cond = [&](const std::string & p, int64_t w, Cond & r) {
        m->add_linear(p + ".time_embedder.linear_1", 256, w, &r.t1_w, &r.t1_b);
        m->add_linear(p + ".time_embedder.linear_2", w, w, &r.t2_w, &r.t2_b);
        m->add_linear(p + ".time_proj", w, 6 * w, &r.tp_w, &r.tp_b);
        m->add_linear(p + ".text_embedder.linear_1", c.t5_hidden, w, &r.x1_w, &r.x1_b);
        m->add_linear(p + ".text_embedder.linear_2", w, w, &r.x2_w, &r.x2_b);
    };
    cond("gwp.action_condition_embedder", da, m->acond);
    cond("gwp.condition_embedder", d, m->vcond);
    m->action_sst = m->add_weight("gwp.action_scale_shift_table", da, 2);
    // Per-layer scale_shift_table [6][width] of each expert, packed [width, 6, L].
    m->a_tables = m->add_weight("gwp.blocks.action_expert.scale_shift_table", da, 6, L);
    m->v_tables = m->add_weight("gwp.blocks.visual_expert.scale_shift_table", d, 6, L);
    // The action expert's projections run on 48 denoise tokens (and the 1
    // state token of the prefix) and use the tiled layout; its cross-attention
    // K/V projections run on the 512 prompt tokens and stay row-major.  With
    // several chunks the denoise projections see batch x 48 tokens, past the
    // few-token path the tiled layout serves, and every weight is row-major.
    // The prompt-token K/V projections of all layers are packed per expert, so
    // the prompt's K and V for every layer come out of one GEMM (one launch of
    // 2·L·d features instead of 2·L launches of d).
    for (int x = 0; x < 2; ++x) {
        m->kv_w[x] = wamx_new_tensor_2d(m->wctx, WAMX_TYPE_BF16, x == 0 ? da : d, 2 * L * d);
        m->kv_b[x] = wamx_new_tensor_1d(m->wctx, WAMX_TYPE_BF16, 2 * L * d);
        m->cnk_all[x] = wamx_new_tensor_2d(m->wctx, WAMX_TYPE_BF16, d, L);
        if (!m->kv_w[x] || !m->kv_b[x] || !m->cnk_all[x]) return false;
    }
    // x: 0 action expert, 1 visual expert (the packed K/V weight); t: tiled.
    auto expert = [&](const std::string & p, int64_t w, int64_t ffn, ExpertLayer & e, int x, bool t, int64_t l) {
        m->add_linear(p + ".attn1.to_qkv", w, 3 * d, &e.qkv_w, &e.qkv_b, t);
        e.norm_q = m->add_weight(p + ".attn1.norm_q.weight", d);
        e.norm_k = m->add_weight(p + ".attn1.norm_k.weight", d);
        m->add_linear(p + ".attn1.to_out.0", d, w, &e.o_w, &e.o_b, t);
        e.n2_w = m->add_weight(p + ".norm2.weight", w);
        e.n2_b = m->add_weight(p + ".norm2.bias", w);
        m->add_linear(p + ".attn2.to_q", w, d, &e.cq_w, &e.cq_b, t);
        m->add_linear_view(p + ".attn2.to_k", m->kv_w[x], m->kv_b[x], 2 * l * d, d, &e.ck_w, &e.ck_b);
        m->add_linear_view(p + ".attn2.to_v", m->kv_w[x], m->kv_b[x], (2 * l + 1) * d, d, &e.cv_w, &e.cv_b);
        e.cnq = m->add_weight(p + ".attn2.norm_q.weight", d);
        e.cnk = m->add_weight_view(p + ".attn2.norm_k.weight", m->cnk_all[x], l * d, d);
        m->add_linear(p + ".attn2.to_out.0", d, w, &e.co_w, &e.co_b, t);
        m->add_linear(p + ".ffn.net.0.proj", w, ffn, &e.up_w, &e.up_b, t);
        m->add_linear(p + ".ffn.net.2", ffn, w, &e.dn_w, &e.dn_b, t);
    };
    m->act.resize(L);
    m->vis.resize(L);
    for (int64_t l = 0; l < L; ++l) {
        const std::string b = "gwp.blocks." + std::to_string(l);
        expert(b + ".action_expert", da, c.action_ffn_dim, m->act[l], 0, m->B * c.action_chunk <= 64, l);
        expert(b + ".visual_expert", d, c.ffn_dim, m->vis[l], 1, false, l);
    }
    for (auto & kv : m->weights)
        if (!kv.second) return false;
    m->wbuf = wamx_backend_alloc_ctx_tensors(m->wctx, m->be);
    // The tiled buffer type of the backend's device.
    wamx_buffer_type_t tb = nullptr;
    for (int i = 0; i < wamx_get_device_count(); ++i)
        if (wamx_backend_buffer_type(i) == wamx_backend_get_default_buffer_type(m->be)) tb = wamx_backend_tiled_buffer_type(i);
    m->tbuf = tb ? wamx_backend_alloc_ctx_tensors_from_buft(m->tctx, tb) : nullptr;
    return m->wbuf != nullptr && m->tbuf != nullptr;
}

static bool create_storage(wamx_gwp_model * m) {
    const wamx_gwp_config & c = m->cfg;
    const int64_t dh = c.head_dim, H = c.n_heads, L = c.n_layers, B = m->B;
    m->sctx = wamx_init(16 * L + 64);
    if (!m->sctx) return false;
    wamx_context * s = m->sctx;
    m->action_prompt = wamx_new_tensor_3d(s, WAMX_TYPE_BF16, c.action_hidden, c.n_lang, B);
    for (int64_t l = 0; l < L; ++l) {
        m->pk.push_back(wamx_new_tensor_4d(s, WAMX_TYPE_BF16, dh, m->P, H, B));
        m->pv_raw.push_back(wamx_new_tensor_4d(s, WAMX_TYPE_BF16, m->Ppad, dh, H, B));
    }
    m->lk_all = wamx_new_tensor_4d(s, WAMX_TYPE_BF16, dh, c.n_lang, H, L * B);
    m->lv_raw_all = wamx_new_tensor_4d(s, WAMX_TYPE_BF16, m->NLpad, dh, H, L * B);
    if (!m->lk_all || !m->lv_raw_all) return false;
    m->in_state = wamx_new_tensor_2d(s, WAMX_TYPE_F32, c.action_dim, B);
    m->in_latent = wamx_new_tensor_4d(s, WAMX_TYPE_F32, 2 * c.grid_w, 2 * c.grid_h, c.z_dim, B);
    m->in_prompt = wamx_new_tensor_3d(s, WAMX_TYPE_F32, c.t5_hidden, c.n_lang, B);
    m->in_action = wamx_new_tensor_2d(s, WAMX_TYPE_BF16, c.action_dim, c.action_chunk * B);
    m->in_apos = wamx_new_tensor_1d(s, WAMX_TYPE_I32, c.action_chunk);
    m->in_spos = wamx_new_tensor_1d(s, WAMX_TYPE_I32, 1);
    m->in_vt = wamx_new_tensor_1d(s, WAMX_TYPE_I32, m->nimg);
    m->in_vh = wamx_new_tensor_1d(s, WAMX_TYPE_I32, m->nimg);
    m->in_vw = wamx_new_tensor_1d(s, WAMX_TYPE_I32, m->nimg);
    m->in_freq0 = wamx_new_tensor_2d(s, WAMX_TYPE_F32, 256, 1);
    m->in_freqs = wamx_new_tensor_2d(s, WAMX_TYPE_F32, 256, c.num_steps);
    m->in_dts = wamx_new_tensor_1d(s, WAMX_TYPE_F32, c.num_steps);
    m->vis_rope = wamx_new_tensor_2d(s, WAMX_TYPE_F32, dh, m->nimg);
    m->sbuf = wamx_backend_alloc_ctx_tensors(s, m->be);
    if (!m->sbuf) return false;
    // Layer l's prompt caches: chunks l*B .. l*B + B-1 of the joint ones.
    for (int64_t l = 0; l < L; ++l)
        for (wamx_tensor * a : {m->lk_all, m->lv_raw_all})
            (a == m->lk_all ? m->lk : m->lv_raw)
                .push_back(wamx_view_4d(s, a, a->ne[0], a->ne[1], a->ne[2], B, a->nb[1], a->nb[2], a->nb[3],
                                        a->nb[3] * (size_t) (l * B)));
    // Views of the padded V^T storage covering the real key columns.
    for (int64_t l = 0; l < L; ++l) {
        wamx_tensor * r = m->pv_raw[l];
        m->pv.push_back(wamx_view_4d(s, r, m->P, dh, H, B, r->nb[1], r->nb[2], r->nb[3], 0));
        wamx_tensor * q = m->lv_raw[l];
        m->lv.push_back(wamx_view_4d(s, q, c.n_lang, dh, H, B, q->nb[1], q->nb[2], q->nb[3], 0));
    }
    // Zero the storage once so padded V^T columns hold finite values.
    for (auto * t : m->pv_raw) wamx_backend_tensor_memset(t, 0, 0, wamx_nbytes(t));
    wamx_backend_tensor_memset(m->lv_raw_all, 0, 0, wamx_nbytes(m->lv_raw_all));
    // Constant inputs: positions (semantics.cpp:210-257), schedule and
    // timestep embeddings (scheduler.cpp:26-55, text_encoder.cpp:1-12).
    std::vector<int32_t> apos(c.action_chunk), vt(m->nimg, 0), vh(m->nimg), vw(m->nimg);
    for (int i = 0; i < c.action_chunk; ++i) apos[i] = i + 1;
    for (int64_t y = 0; y < c.grid_h; ++y)
        for (int64_t x = 0; x < c.grid_w; ++x) {
            vh[y * c.grid_w + x] = (int32_t) y;
            vw[y * c.grid_w + x] = (int32_t) x;
        }
    const int32_t spos = 0;
    wamx_backend_tensor_set(m->in_apos, apos.data(), 0, apos.size() * 4);
    wamx_backend_tensor_set(m->in_spos, &spos, 0, 4);
    wamx_backend_tensor_set(m->in_vt, vt.data(), 0, vt.size() * 4);
    wamx_backend_tensor_set(m->in_vh, vh.data(), 0, vh.size() * 4);
    wamx_backend_tensor_set(m->in_vw, vw.data(), 0, vw.size() * 4);
    {
        hipStream_t st = (hipStream_t) wamx_backend_stream(m->be);
        if (launch_rope_table(1, (const int32_t *) m->in_vt->data, (const int32_t *) m->in_vh->data,
                              (const int32_t *) m->in_vw->data, m->nimg, dh, 10000.0f, (float *) m->vis_rope->data,
                              st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            set_error("wamx_gwp_create: rope table failed");
            return false;
        }
    }
    auto embed = [](float t, float * out) {
        for (int i = 0; i < 128; ++i) {
            const float f = expf(-logf(10000.0f) * (float) i / 128.0f);
            out[i] = cosf(t * f);
            out[i + 128] = sinf(t * f);
        }
    };
    std::vector<float> f0(256);
    embed(0.0f, f0.data());
    wamx_backend_tensor_set(m->in_freq0, f0.data(), 0, 256 * 4);
    // Flow-match Euler schedule, f32 endpoint then f64 linspace + shift.
    const int S = c.num_steps;
    std::vector<float> sig(S + 1), ts(S), freqs(256 * (size_t) S), dts(S);
    const float train = 1.0f / 1000.0f;
    const float smin = c.shift * train / (1.0f + (c.shift - 1.0f) * train);
    const double tmin = (double) smin * 1000.0;
    for (int i = 0; i < S; ++i) {
        const double t = S == 1 ? 1000.0 : 1000.0 + (tmin - 1000.0) * i / (S - 1);
        const double g = t / 1000.0;
        sig[i] = (float) ((double) c.shift * g / (1.0 + ((double) c.shift - 1.0) * g));
        ts[i] = sig[i] * 1000.0f;
    }
    sig[S] = 0.0f;
    for (int i = 0; i < S; ++i) {
        embed(ts[i], &freqs[256 * (size_t) i]);
        dts[i] = sig[i + 1] - sig[i];
    }
    wamx_backend_tensor_set(m->in_freqs, freqs.data(), 0, freqs.size() * 4);
    wamx_backend_tensor_set(m->in_dts, dts.data(), 0, dts.size() * 4);
    return true;
}

// Graph 1: prompt projection of chunk b (cache.cpp:53-137, build_cross_kv
// mot.cpp:101-128).
static bool build_prompt_graph(wamx_gwp_model * m, int64_t cb) {
    const wamx_gwp_config & c = m->cfg;
    const int gi = m->prompt_graph(cb);
    wamx_context * ctx = m->gctx[gi] = wamx_init(64 * c.n_layers + 256);
    Builder b(m, ctx);
    wamx_cgraph * g = m->graph[gi] = wamx_new_graph(ctx, 64 * c.n_layers + 256);
    wamx_tensor * prompt = wamx_view_2d(ctx, m->in_prompt, c.t5_hidden, c.n_lang, m->in_prompt->nb[1],
                                        m->in_prompt->nb[2] * (size_t) cb);
    wamx_tensor * txt = b.text(m->acond, prompt);
    wamx_tensor * ap = wamx_view_2d(ctx, m->action_prompt, c.action_hidden, c.n_lang, m->action_prompt->nb[1],
                                    m->action_prompt->nb[2] * (size_t) cb);
    wamx_build_forward_expand(g, wamx_cpy(ctx, txt, ap));
    wamx_tensor * kv = b.lin(m->kv_w[0], m->kv_b[0], txt);  // every layer's prompt K/V [2·L·d, NL]
    // Every layer's K (RMSNorm by the layer's own norm_k, no rope) and V^T
    // cache of this chunk, one launch each: the layers are the chunks of the
    // joint caches, chunk l*B + cb.
    wamx_tensor * lk = wamx_view_4d(ctx, m->lk_all, c.head_dim, c.n_lang, c.n_heads, c.n_layers, m->lk_all->nb[1],
                                    m->lk_all->nb[2], m->lk_all->nb[3] * (size_t) m->B, m->lk_all->nb[3] * (size_t) cb);
    wamx_build_forward_expand(g, wamx_qk_norm_rope(ctx, b.layer_cols(kv, 0, c.n_layers), m->cnk_all[0], lk, 0, 2, nullptr,
                                                   nullptr, nullptr, c.eps, 10000.0f));
    wamx_tensor * lv = wamx_view_4d(ctx, m->lv_raw_all, c.n_lang, c.head_dim, c.n_heads, c.n_layers,
                                    m->lv_raw_all->nb[1], m->lv_raw_all->nb[2], m->lv_raw_all->nb[3] * (size_t) m->B,
                                    m->lv_raw_all->nb[3] * (size_t) cb);
    wamx_build_forward_expand(g, b.store_v_layers(kv, lv));
    wamx_graph_assign_uid(g);
    m->galloc[gi] = wamx_gallocr_new(m->be);
    return m->galloc[gi] && wamx_gallocr_alloc_graph(m->galloc[gi], g);
}

// Graph 2: prefix pass of chunk cb (cache.cpp:139-485), writing that chunk's
// slice of the prefix cache.
static bool build_prefix_graph(wamx_gwp_model * m, int64_t cb) {
    const wamx_gwp_config & c = m->cfg;
    const int64_t d = (int64_t) c.n_heads * c.head_dim, da = c.action_hidden, dh = c.head_dim, H = c.n_heads;
    const int64_t nimg = m->nimg, P = m->P;
    const int gi = m->prefix_graph(cb);
    wamx_context * ctx = m->gctx[gi] = wamx_init(180 * c.n_layers + 512);
    Builder b(m, ctx);
    wamx_cgraph * g = m->graph[gi] = wamx_new_graph(ctx, 160 * c.n_layers + 512);
    wamx_tensor * state = wamx_view_2d(ctx, m->in_state, c.action_dim, 1, m->in_state->nb[1],
                                       m->in_state->nb[1] * (size_t) cb);
    wamx_tensor * latent = wamx_view_4d(ctx, m->in_latent, m->in_latent->ne[0], m->in_latent->ne[1],
                                        m->in_latent->ne[2], 1, m->in_latent->nb[1], m->in_latent->nb[2],
                                        m->in_latent->nb[3], m->in_latent->nb[3] * (size_t) cb);
    wamx_tensor * prompt = wamx_view_2d(ctx, m->in_prompt, c.t5_hidden, c.n_lang, m->in_prompt->nb[1],
                                        m->in_prompt->nb[2] * (size_t) cb);

    // The state token's chain (its expert projections, row ops and attention
    // query) runs on lane 1, concurrently with the visual tokens' on lane 0;
    // the two meet only through the prefix K/V cache of each layer.
    wamx_set_lane(ctx, 1);
    wamx_tensor * sh = b.mlp3(m->state_enc, state);  // [da, 1]
    wamx_tensor *stemb, *smod;
    b.condition(m->acond, m->in_freq0, &stemb, &smod);
    wamx_tensor * amods = wamx_modulation(ctx, smod, m->a_tables);  // [da, 6, L] f32
    wamx_set_lane(ctx, 0);
    // Patch embedding: conv 2x2 stride 2 as im2col + bf16 MUL_MAT + bias (cache.cpp:203-218).
    wamx_tensor * cols = wamx_im2col(ctx, m->patch_w, latent, 2, 2, 0, 0, 1, 1, WAMX_TYPE_BF16);
    cols = wamx_reshape_2d(ctx, cols, cols->ne[0], nimg);
    wamx_tensor * pw = wamx_reshape_2d(ctx, m->patch_w, 4 * (int64_t) c.z_dim, d);
    wamx_tensor * vh = b.lin(pw, m->patch_b, cols);  // [d, nimg]

    wamx_tensor *vtemb, *vmod;
    // Every visual token has the timestep-0 embedding; its condition rows are
    // identical, so one row is computed and broadcast (bit-identical).
    b.condition(m->vcond, m->in_freq0, &vtemb, &vmod);
    wamx_tensor * vtext = b.text(m->vcond, prompt);
    wamx_tensor * vkv = b.lin(m->kv_w[1], m->kv_b[1], vtext);  // every layer's text K/V [2·L·d, NL]
    // The text keys (RMSNorm by each layer's norm_k, as hi/lo planes) and
    // their V^T for the visual cross-attention of layers 0 .. L-2, one launch
    // each; layer l's are views at planes 2l, 2l + 1 and column block l.
    const int64_t NL = c.n_lang, XL = std::max<int64_t>(1, c.n_layers - 1);
    wamx_tensor * tk = wamx_new_tensor_4d(ctx, WAMX_TYPE_BF16, dh, NL, H, 2 * XL);
    wamx_tensor * tcnk = wamx_view_2d(ctx, m->cnk_all[1], d, XL, m->cnk_all[1]->nb[1], 0);
    tk = wamx_qk_norm_rope_hilo(ctx, b.layer_cols(vkv, 0, XL), tcnk, tk, 0, 2, nullptr, nullptr, nullptr, c.eps,
                                10000.0f);
    wamx_tensor * tv_raw = wamx_new_tensor_4d(ctx, WAMX_TYPE_BF16, round_up(NL, 8), dh, H, XL);
    wamx_tensor * tv = b.store_v_layers(vkv, wamx_view_4d(ctx, tv_raw, NL, dh, H, XL, tv_raw->nb[1], tv_raw->nb[2],
                                                          tv_raw->nb[3], 0));
    wamx_tensor * vmods = wamx_modulation(ctx, vmod, m->v_tables);  // [d, 6, L] f32

    for (int l = 0; l < c.n_layers; ++l) {
        const ExpertLayer & ea = m->act[l];
        const ExpertLayer & ev = m->vis[l];
        wamx_tensor * pk = b.chunk(m->pk[l], cb);       // [dh, P, H]
        wamx_tensor * pv_raw = b.chunk(m->pv_raw[l], cb);
        // State token (lane 1): its Q, and row 0 of the layer's K / V^T cache
        // (1-D rope at position 0).
        wamx_set_lane(ctx, 1);
        wamx_tensor * sn = wamx_norm_modulation_bf16(ctx, sh, b.part(amods, da, l, 1), b.part(amods, da, l, 0), c.eps);
        wamx_tensor * sqkv = b.lin(ea.qkv_w, ea.qkv_b, sn);
        wamx_tensor * Qs = wamx_new_tensor_3d(ctx, WAMX_TYPE_BF16, dh, 1, H);
        Qs = wamx_qk_norm_rope(ctx, b.cols(sqkv, d, 0), ea.norm_q, Qs, 0, 0, m->in_spos, nullptr, nullptr, c.eps,
                               10000.0f);
        wamx_tensor * K = wamx_qk_norm_rope(ctx, b.cols(sqkv, d, d), ea.norm_k, pk, 0, 0, m->in_spos, nullptr, nullptr,
                                            c.eps, 10000.0f);
        wamx_tensor * v0 = b.store_v(sqkv, 2 * d, b.vt_view(pv_raw, 0, 1));
        // Visual tokens (lane 0): their Q, and rows 1..P of the cache (3-D
        // {44,42,42} rope).
        wamx_set_lane(ctx, 0);
        wamx_tensor * vn = wamx_norm_modulation_bf16(ctx, vh, b.part(vmods, d, l, 1), b.part(vmods, d, l, 0), c.eps);
        wamx_tensor * vqkv = b.lin(ev.qkv_w, ev.qkv_b, vn);
        wamx_tensor * Qv = wamx_new_tensor_3d(ctx, WAMX_TYPE_BF16, dh, nimg, H);
        Qv = wamx_qk_norm_rope(ctx, b.cols(vqkv, d, 0), ev.norm_q, Qv, 0, 3, m->vis_rope, nullptr, nullptr, c.eps,
                               10000.0f);
        K = wamx_qk_norm_rope(ctx, b.cols(vqkv, d, d), ev.norm_k, K, 1, 3, m->vis_rope, nullptr, nullptr, c.eps,
                              10000.0f);
        wamx_tensor * v1 = b.store_v(vqkv, 2 * d, after(b.vt_view(pv_raw, 1, nimg), v0));
        wamx_tensor * V = after(b.vt_view(pv_raw, 0, P), v1);
        wamx_set_output(K);
        wamx_set_output(V);
        wamx_build_forward_expand(g, K);
        wamx_build_forward_expand(g, V);
        if (l + 1 == c.n_layers) break;  // the last layer's K/V are the outputs
        // Joint attention over [state, visual] keys, per query set: a query's
        // output does not depend on the other queries.
        wamx_tensor * vatt = wamx_joint_attn(ctx, Qv, K, V, nullptr, nullptr, 0, b.scale);  // [d, nimg]
        vh = b.lin(ev.o_w, ev.o_b, vatt, WAMX_EPI_BIAS_GATED, vh, b.part(vmods, d, l, 2));
        wamx_tensor * tk_l = wamx_view_4d(ctx, tk, dh, NL, H, 2, tk->nb[1], tk->nb[2], tk->nb[3],
                                          tk->nb[3] * (size_t) (2 * l));
        wamx_tensor * tv_l = wamx_view_3d(ctx, tv, NL, dh, H, tv->nb[1], tv->nb[2], tv->nb[3] * (size_t) l);
        vh = b.cross_ffn_uncached(ev, vh, tk_l, tv_l, b.part(vmods, d, l, 3), b.part(vmods, d, l, 4),
                                  b.part(vmods, d, l, 5));
        wamx_set_lane(ctx, 1);
        wamx_tensor * satt = wamx_joint_attn(ctx, Qs, K, V, nullptr, nullptr, 0, b.scale);  // [d, 1]
        sh = b.lin(ea.o_w, ea.o_b, satt, WAMX_EPI_BIAS_GATED, sh, b.part(amods, da, l, 2));
        sh = b.cross_ffn_cached(ea, sh, b.chunk(m->lk[l], cb), b.chunk(m->lv[l], cb), b.part(amods, da, l, 3),
                                b.part(amods, da, l, 4), b.part(amods, da, l, 5));
        wamx_set_lane(ctx, 0);
    }
    wamx_set_lane(ctx, 0);
    wamx_graph_assign_uid(g);
    m->galloc[gi] = wamx_gallocr_new(m->be);
    return m->galloc[gi] && wamx_gallocr_alloc_graph(m->galloc[gi], g);
}

// Graph 3: unrolled denoise (mot.cpp:498-594 over build_cached_action_body).
// The B chunks' tokens are the rows of every projection (B*T rows, chunk
// after chunk); each chunk's queries attend its own prefix and prompt caches.
static bool build_denoise_graph(wamx_gwp_model * m) {
    const wamx_gwp_config & c = m->cfg;
    const int64_t da = c.action_hidden, dh = c.head_dim, H = c.n_heads, T = c.action_chunk, B = m->B;
    const int64_t d = dh * H;
    const int gi = m->denoise_graph();
    wamx_context * ctx = m->gctx[gi] = wamx_init((size_t) (48 * c.n_layers + 64) * c.num_steps + 64);
    Builder b(m, ctx);
    wamx_cgraph * g = m->graph[gi] = wamx_new_graph(ctx, (size_t) (40 * c.n_layers + 64) * c.num_steps + 64);
    wamx_tensor * action = m->in_action;  // bf16 [A, B*T]
    // The time branch of build_condition (mot.cpp:69-82), the per-layer
    // modulation (mot.cpp:130-145) and the output modulation (mot.cpp:468-486)
    // depend on the step's timestep only: they are computed for every step at
    // once, each step's timestep embedding a column of in_freqs.
    wamx_tensor *temb_all, *mod_all;
    b.condition(m->acond, m->in_freqs, &temb_all, &mod_all);             // [da, S], [6 da, S]
    wamx_tensor * mods = wamx_modulation(ctx, mod_all, m->a_tables);     // [da, 6, L, S] f32
    wamx_tensor * tab = wamx_reshape_3d(ctx, m->action_sst, da, 1, 2);
    wamx_tensor * om = wamx_modulation(ctx, temb_all, tab);              // [da, 1, 2, S]: shift, scale
    for (int s = 0; s < c.num_steps; ++s) {
        wamx_tensor * dt = wamx_view_1d(ctx, m->in_dts, 1, (size_t) s * 4);
        wamx_tensor * h = b.mlp3(m->action_enc, action);  // [da, T]
        for (int l = 0; l < c.n_layers; ++l) {
            const ExpertLayer & e = m->act[l];
            wamx_tensor * n = wamx_norm_modulation_bf16(ctx, h, b.part(mods, da, l, 1, s), b.part(mods, da, l, 0, s),
                                                        c.eps);
            wamx_tensor * qkv = b.lin(e.qkv_w, e.qkv_b, n);
            wamx_tensor * Q = wamx_new_tensor_4d(ctx, WAMX_TYPE_BF16, dh, T, H, B);
            Q = wamx_qk_norm_rope(ctx, b.cols(qkv, d, 0), e.norm_q, Q, 0, 0, m->in_apos, nullptr, nullptr, c.eps,
                                  10000.0f);
            wamx_tensor * Ka = wamx_new_tensor_4d(ctx, WAMX_TYPE_BF16, dh, T, H, B);
            Ka = wamx_qk_norm_rope(ctx, b.cols(qkv, d, d), e.norm_k, Ka, 0, 0, m->in_apos, nullptr, nullptr, c.eps,
                                   10000.0f);
            wamx_tensor * vraw = wamx_new_tensor_4d(ctx, WAMX_TYPE_BF16, m->Tpad, dh, H, B);
            wamx_tensor * Va = b.store_v(qkv, 2 * d, b.vt_view(vraw, 0, T));
            // Keys [state, action, reference]: prefix cache split after the state token.
            wamx_tensor * att = b.rows(wamx_joint_attn(ctx, Q, m->pk[l], m->pv[l], Ka, Va, 1, b.scale));
            h = b.lin(e.o_w, e.o_b, att, WAMX_EPI_BIAS_GATED, h, b.part(mods, da, l, 2, s));
            h = b.cross_ffn_cached(e, h, m->lk[l], m->lv[l], b.part(mods, da, l, 3, s), b.part(mods, da, l, 4, s),
                                   b.part(mods, da, l, 5, s));
        }
        // Output modulation: f32(action_scale_shift_table) + f32(temb) (mot.cpp:468-486).
        wamx_tensor * oshift = wamx_view_1d(ctx, om, da, (size_t) (2 * s) * da * 4);
        wamx_tensor * oscale = wamx_view_1d(ctx, om, da, (size_t) (2 * s + 1) * da * 4);
        wamx_tensor * n = wamx_norm_modulation_bf16(ctx, h, oscale, oshift, c.eps);
        wamx_tensor * pred = b.mlp3(m->action_dec, n);  // bf16 [A, T]
        wamx_set_output(pred);
        m->velocity.push_back(pred);
        // scheduler_step (weights.cpp:885-902): bf16(f32(a) + f32(v) * dt).
        action = wamx_euler_step(ctx, action, pred, dt);
    }
    m->action_out = action;
    wamx_set_output(action);
    wamx_build_forward_expand(g, action);
    wamx_graph_assign_uid(g);
    m->galloc[gi] = wamx_gallocr_new(m->be);
    return m->galloc[gi] && wamx_gallocr_alloc_graph(m->galloc[gi], g);
}

// Index of the first Inf or NaN of v[0, n) (n when there is none).  An
// all-ones exponent is tested on the bit patterns a block at a time so the
// scan vectorises (AVX2 where the CPU has it); a block that has one is
// scanned again for the first such element.
template <int kUnused = 0>
static inline size_t first_non_finite_impl(const float * v, size_t n) {
    constexpr size_t kBlock = 4096;
    for (size_t b = 0; b < n; b += kBlock) {
        const size_t e = std::min(n, b + kBlock);
        uint32_t bad = 0;
        for (size_t i = b; i < e; ++i) {
            uint32_t u;
            memcpy(&u, v + i, sizeof u);
            bad |= (uint32_t) ((u & 0x7f800000u) == 0x7f800000u);
        }
        if (bad)
            for (size_t i = b; i < e; ++i)
                if (!isfinite(v[i])) return i;
    }
    return n;
}
__attribute__((target("avx2"))) static size_t first_non_finite_avx2(const float * v, size_t n) {
    return first_non_finite_impl<1>(v, n);
}
static size_t first_non_finite(const float * v, size_t n) {
    static const bool avx2 = __builtin_cpu_supports("avx2");
    return avx2 ? first_non_finite_avx2(v, n) : first_non_finite_impl<0>(v, n);
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

wamx_gwp_config wamx_gwp_default_config(void) {
    wamx_gwp_config c{};
    c.n_layers = 30;
    c.hidden = 3072;
    c.n_heads = 24;
    c.head_dim = 128;
    c.ffn_dim = 14336;
    c.action_hidden = 3072;
    c.action_ffn_dim = 14336;
    c.action_chunk = 48;
    c.action_dim = 32;
    c.grid_h = 32;  // 3 camera views of 32x32 visual tokens side by side
    c.grid_w = 96;
    c.n_lang = 512;
    c.t5_hidden = 4096;
    c.z_dim = 48;
    c.num_steps = 10;
    c.enc_hidden = 128;
    c.shift = 5.0f;
    c.eps = 1e-6f;
    c.batch = 1;
    return c;
}

wamx_gwp_t wamx_gwp_create(wamx_backend_t be, const wamx_gwp_config * cfg) {
    clear_error();
    if (!be || !cfg) {
        set_error("wamx_gwp_create: null argument");
        return nullptr;
    }
    const wamx_gwp_config & c = *cfg;
    if (c.n_layers < 1 || c.n_heads < 1 || c.head_dim != 128 || c.hidden != c.n_heads * c.head_dim ||
        c.action_hidden < 1 || c.ffn_dim < 1 || c.action_ffn_dim < 1 || c.action_chunk < 1 || c.action_chunk > 64 ||
        c.action_dim < 1 || c.grid_h < 1 || c.grid_w < 1 || c.n_lang < 1 || c.t5_hidden < 1 || c.z_dim < 1 ||
        c.num_steps < 1 || c.enc_hidden < 1 || !(c.shift > 0.0f) || !(c.eps >= 0.0f) || c.batch < 0 ||
        c.batch > 64) {
        set_error("wamx_gwp_create: invalid configuration (head_dim 128, hidden = heads*128, chunk <= 64, "
                  "batch <= 64)");
        return nullptr;
    }
    auto m = std::make_unique<wamx_gwp_model>();
    m->be = be;
    m->cfg = c;
    m->B = c.batch > 1 ? c.batch : 1;
    m->cfg.batch = (int32_t) m->B;
    m->gctx.assign(m->n_graphs(), nullptr);
    m->graph.assign(m->n_graphs(), nullptr);
    m->galloc.assign(m->n_graphs(), nullptr);
    m->nimg = (int64_t) c.grid_h * c.grid_w;
    m->P = 1 + m->nimg;
    // V^T rows padded to 64 keys (128 bytes), so every 64-key block of a row
    // the attention kernels copy is one aligned 128-byte segment.
    m->Ppad = round_up(m->P, 64);
    m->NLpad = round_up(c.n_lang, 64);
    m->Tpad = round_up(c.action_chunk, 64);
    if (!create_weights(m.get())) {
        set_errorf("wamx_gwp_create: weight allocation failed: %s", wamx_last_error());
        return nullptr;
    }
    if (!create_storage(m.get())) {
        set_errorf("wamx_gwp_create: cache allocation failed: %s", wamx_last_error());
        return nullptr;
    }
    bool ok = true;
    for (int64_t cb = 0; cb < m->B && ok; ++cb) ok = build_prompt_graph(m.get(), cb) && build_prefix_graph(m.get(), cb);
    if (!ok || !build_denoise_graph(m.get())) {
        set_errorf("wamx_gwp_create: graph construction failed: %s", wamx_last_error());
        return nullptr;
    }
    m->timer = wamx_timer_new(be);
    return m.release();
}

void wamx_gwp_free(wamx_gwp_t m) { delete m; }
int wamx_gwp_n_weights(wamx_gwp_t m) { return m ? (int) m->weights.size() : 0; }
const char * wamx_gwp_weight_name(wamx_gwp_t m, int i) {
    return (m && i >= 0 && i < (int) m->weights.size()) ? m->weights[i].first.c_str() : nullptr;
}
// A weight handle may be written through (the GGUF loader does), so handing
// one out marks the projected prompt stale: the next request projects it
// again with the new weights.
wamx_tensor * wamx_gwp_weight(wamx_gwp_t m, const char * name) {
    if (!m || !name) return nullptr;
    auto it = m->by_name.find(name);
    if (it == m->by_name.end()) return nullptr;
    m->prompt_stale = true;
    return it->second;
}
uint64_t wamx_gwp_param_count(wamx_gwp_t m) {
    uint64_t n = 0;
    if (m)
        for (auto & kv : m->weights) n += (uint64_t) wamx_nelements(kv.second);
    return n;
}

wamx_status wamx_gwp_init_synthetic(wamx_gwp_t m, uint64_t seed, float wstd) {
    WAMX_REQUIRE(m, "wamx_gwp_init_synthetic: null model");
    // Tiled weights are generated row-major into a staging buffer and then
    // written in their layout, so every weight holds the same values as the
    // row-major fill of the same seed.
    size_t stage_bytes = 0;
    for (auto & kv : m->weights)
        if (tensor_is_tiled(kv.second)) stage_bytes = std::max(stage_bytes, wamx_nbytes(kv.second));
    void * stage = stage_bytes ? wamx_device_malloc(m->be, stage_bytes) : nullptr;
    WAMX_REQUIRE(!stage_bytes || stage, "wamx_gwp_init_synthetic: staging allocation failed");
    for (auto & kv : m->weights) {
        const std::string & n = kv.first;
        float mean = 0.0f, sd = wstd;
        auto ends = [&](const char * s) {
            const size_t k = strlen(s);
            return n.size() >= k && n.compare(n.size() - k, k, s) == 0;
        };
        if (ends(".bias")) {
            sd = 0.02f;
        } else if (ends("norm_q.weight") || ends("norm_k.weight") || ends("norm2.weight")) {
            mean = 1.0f;
            sd = 0.02f;
        } else if (n.find("scale_shift_table") != std::string::npos) {
            sd = 0.1f;
        }
        const bool tiled = tensor_is_tiled(kv.second);
        wamx_status st = wamx_fill_normal(m->be, tiled ? stage : kv.second->data, WAMX_TYPE_BF16,
                                          wamx_nelements(kv.second), seed ^ fnv1a(n), mean, sd);
        if (st == WAMX_STATUS_SUCCESS && tiled &&
            tensor_set_from_device(kv.second, stage, (hipStream_t) wamx_backend_stream(m->be)) != hipSuccess) {
            set_errorf("wamx_gwp_init_synthetic: tiling %s failed", n.c_str());
            st = WAMX_STATUS_FAILED;
        }
        if (st != WAMX_STATUS_SUCCESS) {
            wamx_backend_synchronize(m->be);
            if (stage) wamx_device_free(m->be, stage);
            return st;
        }
    }
    wamx_backend_synchronize(m->be);
    if (stage) wamx_device_free(m->be, stage);
    m->prompt_stale = true;  // new weights: the prompt caches no longer hold its projection
    return WAMX_STATUS_SUCCESS;
}

wamx_status wamx_check_finite_f32(const float * values, size_t n, const char * field) {
    WAMX_REQUIRE(values || n == 0, "%s: null array", field ? field : "tensor");
    // Large arrays (the 2.1M-value prompt, the latent) are scanned by several
    // threads: one core's memory bandwidth makes a 10 MB scan ~1 ms.
    size_t nthreads = 1;
    if (n >= (size_t) 1 << 20) nthreads = std::min<size_t>(8, std::max(1u, std::thread::hardware_concurrency()));
    std::vector<size_t> first(nthreads, n);
    auto scan = [&](size_t t) {
        const size_t b = n * t / nthreads, e = n * (t + 1) / nthreads;
        first[t] = first_non_finite(values + b, e - b) + b;
    };
    if (nthreads == 1) {
        scan(0);
    } else {
        std::vector<std::thread> pool;
        for (size_t t = 1; t < nthreads; ++t) pool.emplace_back(scan, t);
        scan(0);
        for (auto & th : pool) th.join();
    }
    for (size_t t = 0; t < nthreads; ++t)
        WAMX_REQUIRE(first[t] >= n * (t + 1) / nthreads, "%s contains NaN or Inf (element %zu)",
                     field ? field : "tensor", first[t]);
    return WAMX_STATUS_SUCCESS;
}

wamx_status wamx_gwp_set_inputs(wamx_gwp_t m, const float * state, const float * latent, const float * prompt,
                                const float * noise) {
    WAMX_REQUIRE(m && state && latent && prompt && noise, "wamx_gwp_set_inputs: null argument");
    // Non-finite inputs are refused and the model's inputs left as they were,
    // as the reference refuses them before its graphs run (engine.cpp:238-247
    // state, :274 reference latent, :320 prompt, :350-357 noise).  The small
    // state and noise are checked on the host; the latent and the prompt
    // (10.6 MB of f32 at batch 1) are uploaded to a staging area, scanned
    // there, and copied into the inputs only when finite.
    const size_t ns = (size_t) wamx_nelements(m->in_state), na = (size_t) wamx_nelements(m->in_action);
    const size_t nl = (size_t) wamx_nelements(m->in_latent), np = (size_t) wamx_nelements(m->in_prompt);
    wamx_status st = wamx_check_finite_f32(state, ns, "wamx_gwp_set_inputs: state");
    if (st == WAMX_STATUS_SUCCESS) st = wamx_check_finite_f32(noise, na, "wamx_gwp_set_inputs: noise");
    if (st != WAMX_STATUS_SUCCESS) return st;
    const bool hit = m->prompt_cache_capacity > 0 && !m->prompt_stale && m->prompt_sig.size() == np &&
                     memcmp(m->prompt_sig.data(), prompt, np * sizeof(float)) == 0;
    hipStream_t s = (hipStream_t) wamx_backend_stream(m->be);
    if (!m->stage) {
        m->stage = wamx_device_malloc(m->be, (nl + np) * sizeof(float) + 256);
        WAMX_REQUIRE(m->stage, "wamx_gwp_set_inputs: staging allocation failed");
        m->flags = (uint32_t *) ((char *) m->stage + (nl + np) * sizeof(float));
    }
    float * sl = (float *) m->stage;
    float * sp = sl + nl;
    WAMX_HIP_TRY(hipMemcpy(sl, latent, nl * sizeof(float), hipMemcpyHostToDevice));
    if (!hit) WAMX_HIP_TRY(hipMemcpy(sp, prompt, np * sizeof(float), hipMemcpyHostToDevice));
    uint32_t first[2] = {UINT32_MAX, UINT32_MAX};
    WAMX_HIP_TRY(hipMemcpyAsync(m->flags, first, sizeof first, hipMemcpyHostToDevice, s));
    WAMX_HIP_TRY(launch_nonfinite_scan(sl, (int64_t) nl, m->flags, s));
    if (!hit) WAMX_HIP_TRY(launch_nonfinite_scan(sp, (int64_t) np, m->flags + 1, s));
    WAMX_HIP_TRY(hipMemcpyAsync(first, m->flags, sizeof first, hipMemcpyDeviceToHost, s));
    WAMX_HIP_TRY(hipStreamSynchronize(s));
    WAMX_REQUIRE(first[0] == UINT32_MAX, "wamx_gwp_set_inputs: latent contains NaN or Inf (element %u)", first[0]);
    WAMX_REQUIRE(first[1] == UINT32_MAX, "wamx_gwp_set_inputs: prompt contains NaN or Inf (element %u)", first[1]);
    if (m->prompt_cache_capacity > 0) ++(hit ? m->prompt_hits : m->prompt_misses);
    WAMX_HIP_TRY(hipMemcpyAsync(m->in_latent->data, sl, nl * sizeof(float), hipMemcpyDeviceToDevice, s));
    if (!hit) {
        m->prompt_stale = true;
        WAMX_HIP_TRY(hipMemcpyAsync(m->in_prompt->data, sp, np * sizeof(float), hipMemcpyDeviceToDevice, s));
        if (m->prompt_cache_capacity > 0) m->prompt_sig.assign(prompt, prompt + np);
    }
    st = wamx_backend_tensor_set(m->in_state, state, 0, ns * sizeof(float));
    if (st != WAMX_STATUS_SUCCESS) return st;
    // The action state is bf16 in the native profile (mot.cpp:523-525, set_f32_tensor).
    std::vector<uint16_t> a(na);
    for (size_t i = 0; i < na; ++i) a[i] = f32_to_bf16_host(noise[i]);
    return wamx_backend_tensor_set(m->in_action, a.data(), 0, na * 2);
}

static wamx_status run_graph(wamx_gwp_t m, int which) {
    WAMX_REQUIRE(m && which >= 0 && which < m->n_graphs() && m->graph[which], "wamx_gwp: graph %d missing", which);
    return wamx_backend_graph_compute(m->be, m->graph[which]);
}
// Phase p (0 prompt, 1 prefix, 2 denoise) of every chunk.
static wamx_status run_phase(wamx_gwp_t m, int phase) {
    WAMX_REQUIRE(m, "wamx_gwp: null model");
    if (phase == 2) return run_graph(m, m->denoise_graph());
    for (int64_t cb = 0; cb < m->B; ++cb) {
        const wamx_status st = run_graph(m, phase == 0 ? m->prompt_graph(cb) : m->prefix_graph(cb));
        if (st != WAMX_STATUS_SUCCESS) return st;
    }
    return WAMX_STATUS_SUCCESS;
}
wamx_status wamx_gwp_set_prompt_cache(wamx_gwp_t m, size_t capacity) {
    WAMX_REQUIRE(m, "wamx_gwp_set_prompt_cache: null model");
    m->prompt_cache_capacity = capacity;
    if (capacity == 0) {
        m->prompt_sig.clear();
        m->prompt_sig.shrink_to_fit();
    }
    return WAMX_STATUS_SUCCESS;
}
wamx_status wamx_gwp_prompt_cache_stats(wamx_gwp_t m, uint64_t * hits, uint64_t * misses) {
    WAMX_REQUIRE(m && hits && misses, "wamx_gwp_prompt_cache_stats: null argument");
    *hits = m->prompt_hits;
    *misses = m->prompt_misses;
    return WAMX_STATUS_SUCCESS;
}
wamx_status wamx_gwp_run_prompt(wamx_gwp_t m) {
    WAMX_REQUIRE(m, "wamx_gwp_run_prompt: null model");
    const wamx_status st = run_phase(m, 0);
    if (st == WAMX_STATUS_SUCCESS) m->prompt_stale = false;
    return st;
}
wamx_status wamx_gwp_run_prefix(wamx_gwp_t m) { return run_phase(m, 1); }
wamx_status wamx_gwp_run_denoise(wamx_gwp_t m) { return run_phase(m, 2); }

wamx_status wamx_gwp_predict(wamx_gwp_t m, wamx_gwp_timing * timing) {
    WAMX_REQUIRE(m, "wamx_gwp_predict: null model");
    float ms[3] = {0, 0, 0};
    for (int i = 0; i < 3; ++i) {
        if (timing) wamx_timer_start(m->timer);
        // The prompt graphs run unless the prompt caches already hold the
        // projection of the uploaded prompt (a projected-prompt cache hit).
        const bool skip = i == 0 && m->prompt_cache_capacity > 0 && !m->prompt_stale;
        const wamx_status st = skip ? WAMX_STATUS_SUCCESS : i == 0 ? wamx_gwp_run_prompt(m) : run_phase(m, i);
        if (st != WAMX_STATUS_SUCCESS) return st;
        if (timing) ms[i] = wamx_timer_stop_ms(m->timer);
    }
    if (timing) {
        timing->prompt_ms = ms[0];
        timing->prefix_ms = ms[1];
        timing->denoise_ms = ms[2];
        timing->total_ms = ms[0] + ms[1] + ms[2];
    }
    return WAMX_STATUS_SUCCESS;
}

wamx_status wamx_gwp_get_action(wamx_gwp_t m, float * out) {
    WAMX_REQUIRE(m && out && m->action_out && m->action_out->data, "wamx_gwp_get_action: no action");
    wamx_backend_synchronize(m->be);
    const int64_t n = wamx_nelements(m->action_out);
    std::vector<uint16_t> a(n);
    const wamx_status st = wamx_backend_tensor_get(m->action_out, a.data(), 0, n * 2);
    if (st != WAMX_STATUS_SUCCESS) return st;
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32_host(a[i]);
    // A non-finite action is an inference failure (model.cpp:246-251); the
    // values are still written for inspection.
    return wamx_check_finite_f32(out, (size_t) n, "wamx_gwp_get_action: action");
}

wamx_status wamx_gwp_get_velocity(wamx_gwp_t m, int step, float * out) {
    WAMX_REQUIRE(m && out, "wamx_gwp_get_velocity: null argument");
    WAMX_REQUIRE(step >= 0 && step < (int) m->velocity.size() && m->velocity[step]->data,
                 "wamx_gwp_get_velocity: step %d outside 0..%d", step, (int) m->velocity.size() - 1);
    wamx_backend_synchronize(m->be);
    wamx_tensor * v = m->velocity[step];
    const int64_t n = wamx_nelements(v);
    std::vector<uint16_t> a(n);
    const wamx_status st = wamx_backend_tensor_get(v, a.data(), 0, n * 2);
    if (st != WAMX_STATUS_SUCCESS) return st;
    for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_f32_host(a[i]);
    return WAMX_STATUS_SUCCESS;
}

wamx_tensor * wamx_gwp_prefix_key(wamx_gwp_t m, int layer) {
    return (m && layer >= 0 && layer < m->cfg.n_layers) ? m->pk[layer] : nullptr;
}
wamx_tensor * wamx_gwp_prefix_value(wamx_gwp_t m, int layer) {
    return (m && layer >= 0 && layer < m->cfg.n_layers) ? m->pv[layer] : nullptr;
}
int wamx_gwp_graph_nodes(wamx_gwp_t m, int which) {
    if (!m || which < 0 || which > 2) return 0;
    const int gi = which == 0 ? m->prompt_graph(0) : which == 1 ? m->prefix_graph(0) : m->denoise_graph();
    return wamx_graph_n_nodes(m->graph[gi]);
}

}  // extern "C"
