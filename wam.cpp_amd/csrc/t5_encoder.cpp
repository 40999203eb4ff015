// UMT5 text encoder: prompt tokens -> the [n_lang][t5_hidden] f32 prompt
// embedding the prompt-projection graph consumes, for requests that send
// tokens instead of an embedding (the reference's `resident` / `fixed`
// language policies, engine.cpp:186-193, :306-314).
//
// The graph is the reference's run_t5 (src/models/gwp05/engine/text_encoder.cpp
// :112-204) op for op on this backend's IR: token rows by GET_ROWS from the
// bf16 table (f32 out); per layer the relative-position bias gathered by
// GET_ROWS and permuted into a [key, query, head] f32 SOFT_MAX mask, RMSNorm
// (RMS_NORM, then MUL by the f32 weight, weights.cpp:904-917), the attention
// of build_attention (:26-73) with no biases and scale 1 (bf16 W x f32 x
// MUL_MATs, f32 K.Q at PREC_F32, SOFT_MAX_EXT, f32 V.P), the residual ADD, and
// the gated-GELU FFN GELU(wi_0 x) * (wi_1 x) -> wo, residual ADD; a final
// RMSNorm.  Only the valid (mask) prefix of the tokens is encoded; the rows
// past it are zero, as the reference returns them.
#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <list>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"

namespace {

constexpr int kBuckets = 32;       // text_encoder.cpp:151-152
constexpr int kMaxDistance = 128;

// The bidirectional relative-position bucket of T5 (text_encoder.cpp:13-24):
// half the buckets per direction (key after query in the upper half), exact
// buckets for |d| < half/2, then logarithmic up to max_distance.
int bucket_of(int relative, int buckets, int max_distance) {
    const int half = buckets / 2;
    const int base = relative > 0 ? half : 0;
    const int d = std::abs(relative);
    const int exact = half / 2;
    if (d < exact) return base + d;
    const float r = std::log((float) d / (float) exact) / std::log((float) max_distance / (float) exact);
    return base + std::min(half - 1, exact + (int) (r * (float) (half - exact)));
}

// Initial capacity of the prompt-embedding cache, read as the reference
// reads WAM_GWP05_PROMPT_CACHE_SIZE (weights.cpp:305-317): unset or empty 4;
// any '-', a non-number, trailing characters or overflow 0 (off).
size_t prompt_cache_capacity_env() {
    const char * v = std::getenv("WAM_GWP05_PROMPT_CACHE_SIZE");
    if (!v || !*v) return 4;
    if (std::strchr(v, '-')) return 0;
    errno = 0;
    char * end = nullptr;
    const unsigned long long n = std::strtoull(v, &end, 10);
    if (errno == ERANGE || end == v || !end || *end) return 0;
    return (size_t) n;
}

// A cached prompt: the request's tokens and mask (all ones when the request
// has none, as prompt_mask does, weights.cpp:412-417) and its embedding
// ([max_tokens][hidden], rows past the valid prefix zero).
struct PromptEntry {
    std::vector<int32_t> tokens, mask;
    std::vector<float> emb;
    bool same(const std::vector<int32_t> & t, const std::vector<int32_t> & m) const { return tokens == t && mask == m; }
};

}  // namespace

struct wamx_t5 {
    wamx_backend_t be = nullptr;
    wamx_t5_config cfg{};
    wamx_context * wctx = nullptr;
    wamx_buffer_t wbuf = nullptr;
    std::vector<std::pair<std::string, wamx_tensor *>> weights;
    std::unordered_map<std::string, wamx_tensor *> by_name;
    wamx_gallocr_t galloc = nullptr;
    // Prompt-embedding LRU (weights.cpp:394-451): most recent first.
    std::list<PromptEntry> cache;
    size_t cache_limit = prompt_cache_capacity_env();
    uint64_t hits = 0, misses = 0;
    bool last_hit = false;
    // The `fixed` language policy: one prompt, encoded up front; the weights
    // are released after it (engine.cpp:180-199).
    bool fixed = false;
    PromptEntry fixed_prompt;

    wamx_tensor * add(const std::string & name, int64_t ne0, int64_t ne1 = 1) {
        wamx_tensor * t = wamx_new_tensor_2d(wctx, WAMX_TYPE_BF16, ne0, ne1);
        if (!t) return nullptr;
        wamx_set_name(t, name.c_str());
        weights.push_back({name, t});
        by_name[name] = t;
        return t;
    }
    wamx_tensor * w(const std::string & name) const {
        auto it = by_name.find(name);
        return it == by_name.end() ? nullptr : it->second;
    }
    ~wamx_t5() {
        wamx_gallocr_free(galloc);
        wamx_buffer_free(wbuf);
        wamx_free(wctx);
    }
};

namespace {

std::string layer_prefix(int64_t l) { return "t5.encoder.block." + std::to_string(l) + ".layer"; }

// RMSNorm of an f32 row by a bf16 weight, as the engine's rms_norm does for
// f32 input (weights.cpp:904-917).
wamx_tensor * rms_norm_w(wamx_context * ctx, wamx_tensor * x, wamx_tensor * w, float eps) {
    return wamx_mul(ctx, wamx_rms_norm(ctx, x, eps), wamx_cast(ctx, w, WAMX_TYPE_F32));
}

}  // namespace

extern "C" {

int32_t wamx_t5_relative_bucket(int32_t relative, int32_t buckets, int32_t max_distance) {
    if (buckets < 4 || max_distance <= buckets / 4) return -1;
    return bucket_of(relative, buckets, max_distance);
}

wamx_t5_t wamx_t5_create(wamx_backend_t be, const wamx_t5_config * c) {
    wamx::clear_error();
    if (!be || !c) {
        wamx::set_error("wamx_t5_create: null argument");
        return nullptr;
    }
    if (c->vocab <= 0 || c->hidden <= 0 || c->ffn_dim <= 0 || c->heads <= 0 || c->head_dim <= 0 || c->layers <= 0 ||
        c->max_tokens <= 0 || !(c->eps > 0.0f) || c->hidden % 8 != 0 || c->ffn_dim % 8 != 0 ||
        (c->heads * c->head_dim) % 8 != 0) {
        wamx::set_error("wamx_t5_create: invalid configuration (positive sizes, widths multiples of 8)");
        return nullptr;
    }
    auto * t = new (std::nothrow) wamx_t5();
    if (!t) return nullptr;
    t->be = be;
    t->cfg = *c;
    const int64_t d = c->hidden, inner = (int64_t) c->heads * c->head_dim, F = c->ffn_dim;
    t->wctx = wamx_init(16 * c->layers + 16);
    bool ok = t->wctx != nullptr;
    if (ok) ok = t->add("t5.shared.weight", d, c->vocab) != nullptr;
    for (int64_t l = 0; ok && l < c->layers; ++l) {
        const std::string p = layer_prefix(l);
        const std::string a = p + ".0.SelfAttention";
        ok = t->add(a + ".q.weight", d, inner) && t->add(a + ".k.weight", d, inner) &&
             t->add(a + ".v.weight", d, inner) && t->add(a + ".o.weight", inner, d) &&
             t->add(a + ".relative_attention_bias.weight", c->heads, kBuckets) &&
             t->add(p + ".0.layer_norm.weight", d) && t->add(p + ".1.DenseReluDense.wi_0.weight", d, F) &&
             t->add(p + ".1.DenseReluDense.wi_1.weight", d, F) && t->add(p + ".1.DenseReluDense.wo.weight", F, d) &&
             t->add(p + ".1.layer_norm.weight", d);
    }
    if (ok) ok = t->add("t5.encoder.final_layer_norm.weight", d) != nullptr;
    if (ok) {
        t->wbuf = wamx_backend_alloc_ctx_tensors(t->wctx, be);
        t->galloc = wamx_gallocr_new(be);
        ok = t->wbuf && t->galloc;
    }
    if (!ok) {
        if (!wamx_last_error()[0]) wamx::set_error("wamx_t5_create: allocation failed");
        delete t;
        return nullptr;
    }
    return t;
}

void wamx_t5_free(wamx_t5_t t) { delete t; }
int wamx_t5_n_weights(wamx_t5_t t) { return t ? (int) t->weights.size() : 0; }
const char * wamx_t5_weight_name(wamx_t5_t t, int i) {
    return t && i >= 0 && i < (int) t->weights.size() ? t->weights[(size_t) i].first.c_str() : nullptr;
}
// A weight handle may be written through, so handing one out empties the
// prompt cache (its embeddings were made with the old weights).  None after
// wamx_t5_fix_prompt released the weights.
wamx_tensor * wamx_t5_weight(wamx_t5_t t, const char * name) {
    if (!t || !name || t->fixed) return nullptr;
    t->cache.clear();
    return t->w(name);
}

wamx_status wamx_t5_load_gguf(wamx_t5_t t, wamx_gguf_t g) {
    WAMX_REQUIRE(t && g, "wamx_t5_load_gguf: null argument");
    WAMX_REQUIRE(!t->fixed, "wamx_t5_load_gguf: the encoder serves a fixed prompt; its weights were released");
    t->cache.clear();
    std::vector<uint16_t> buf;
    char cname[128];
    for (auto & kv : t->weights) {
        const int32_t n = wamx_gguf_compact_name(kv.first.c_str(), cname, (int32_t) sizeof cname);
        WAMX_REQUIRE(n > 0 && n <= (int32_t) sizeof cname, "wamx_t5_load_gguf: no compact name for %s",
                     kv.first.c_str());
        const int64_t i = wamx_gguf_find_tensor(g, cname);
        WAMX_REQUIRE(i >= 0, "wamx_t5_load_gguf: required GGUF tensor %s is missing", cname);
        WAMX_REQUIRE(wamx_gguf_tensor_type(g, i) == 30, "wamx_t5_load_gguf: GGUF tensor %s is not BF16", cname);
        const wamx_tensor * w = kv.second;
        for (int k = 0; k < 4; ++k)
            WAMX_REQUIRE(wamx_gguf_tensor_ne(g, i, k) == w->ne[k], "wamx_t5_load_gguf: GGUF tensor %s has the wrong shape",
                         cname);
        buf.resize((size_t) wamx_nelements(w));
        if (wamx_gguf_read_tensor(g, i, buf.data(), buf.size() * 2) != WAMX_STATUS_SUCCESS) return WAMX_STATUS_FAILED;
        if (wamx_backend_tensor_set(kv.second, buf.data(), 0, buf.size() * 2) != WAMX_STATUS_SUCCESS)
            return WAMX_STATUS_FAILED;
    }
    return WAMX_STATUS_SUCCESS;
}

wamx_t5_t wamx_t5_create_from_gguf(wamx_backend_t be, wamx_gguf_t g) {
    wamx::clear_error();
    uint32_t vocab, hidden, ffn, heads, head_dim, layers;
    if (!be || !g) {
        wamx::set_error("wamx_t5_create_from_gguf: null argument");
        return nullptr;
    }
    if (wamx_gguf_get_u32(g, "gwp05.t5_vocab_size", &vocab) || wamx_gguf_get_u32(g, "gwp05.t5_hidden", &hidden) ||
        wamx_gguf_get_u32(g, "gwp05.t5_ffn_dim", &ffn) || wamx_gguf_get_u32(g, "gwp05.t5_heads", &heads) ||
        wamx_gguf_get_u32(g, "gwp05.t5_head_dim", &head_dim) || wamx_gguf_get_u32(g, "gwp05.t5_layers", &layers))
        return nullptr;
    if (hidden != heads * head_dim) {
        wamx::set_error("wamx_t5_create_from_gguf: t5_hidden must equal t5_heads x t5_head_dim");
        return nullptr;
    }
    wamx_t5_config c{};
    c.vocab = (int32_t) vocab;
    c.hidden = (int32_t) hidden;
    c.ffn_dim = (int32_t) ffn;
    c.heads = (int32_t) heads;
    c.head_dim = (int32_t) head_dim;
    c.layers = (int32_t) layers;
    c.max_tokens = 64;  // the GWP prompt (semantics.h:11)
    c.eps = 1e-6f;      // text_encoder.cpp:166, :184, :196
    wamx_t5_t t = wamx_t5_create(be, &c);
    if (!t) return nullptr;
    if (wamx_t5_load_gguf(t, g) != WAMX_STATUS_SUCCESS) {
        const std::string err = wamx_last_error();
        wamx_t5_free(t);
        wamx::set_errorf("%s", err.c_str());
        return nullptr;
    }
    return t;
}

}  // extern "C"

namespace {

// run_t5 on the valid prefix of a validated request (tokens in the
// vocabulary); out [max_tokens][hidden] with the rows past it zero.
wamx_status encode_graph(wamx_t5_t t5, const int32_t * tokens, int valid, float * out) {
    const wamx_t5_config & c = t5->cfg;
    const int64_t V = valid, d = c.hidden, H = c.heads, dh = c.head_dim, inner = H * dh;
    wamx_context * ctx = wamx_init(64 * c.layers + 64);
    WAMX_REQUIRE(ctx, "wamx_t5_encode: context allocation failed");
    struct Ctx {
        wamx_context * p;
        ~Ctx() { wamx_free(p); }
    } guard{ctx};
    wamx_tensor * ids = wamx_new_tensor_1d(ctx, WAMX_TYPE_I32, V);
    wamx_tensor * bk = wamx_new_tensor_1d(ctx, WAMX_TYPE_I32, V * V);
    WAMX_REQUIRE(ids && bk, "wamx_t5_encode: %s", wamx_last_error());
    wamx_set_input(ids);
    wamx_set_input(bk);
    wamx_tensor * h = wamx_get_rows(ctx, t5->w("t5.shared.weight"), ids);  // f32 [d, V]
    for (int64_t l = 0; l < c.layers && h; ++l) {
        const std::string p = layer_prefix(l), a = p + ".0.SelfAttention";
        // position bias [H, V key, V query] -> mask [V key, V query, H]
        wamx_tensor * pb = wamx_get_rows(ctx, t5->w(a + ".relative_attention_bias.weight"), bk);
        pb = wamx_cont(ctx, wamx_permute(ctx, wamx_reshape_3d(ctx, pb, H, V, V), 2, 0, 1, 3));
        wamx_tensor * x = rms_norm_w(ctx, h, t5->w(p + ".0.layer_norm.weight"), 1e-6f);
        wamx_tensor * q = wamx_mul_mat(ctx, t5->w(a + ".q.weight"), x);
        wamx_tensor * k = wamx_mul_mat(ctx, t5->w(a + ".k.weight"), x);
        wamx_tensor * v = wamx_mul_mat(ctx, t5->w(a + ".v.weight"), x);
        wamx_tensor * Q = wamx_cont(ctx, wamx_permute(ctx, wamx_reshape_3d(ctx, q, dh, H, V), 0, 2, 1, 3));
        wamx_tensor * K = wamx_cont(ctx, wamx_permute(ctx, wamx_reshape_3d(ctx, k, dh, H, V), 0, 2, 1, 3));
        wamx_tensor * Vt = wamx_cont(ctx, wamx_permute(ctx, wamx_reshape_3d(ctx, v, dh, H, V), 1, 2, 0, 3));
        wamx_tensor * s = wamx_mul_mat(ctx, K, Q);
        if (s) wamx_mul_mat_set_prec(s, 10);  // GGML_PREC_F32
        wamx_tensor * pr = wamx_soft_max_ext(ctx, s, pb, 1.0f, 0.0f);
        wamx_tensor * at = wamx_mul_mat(ctx, Vt, pr);  // [dh, V query, H]
        at = wamx_reshape_2d(ctx, wamx_cont(ctx, wamx_permute(ctx, at, 0, 2, 1, 3)), inner, V);
        h = wamx_add(ctx, h, wamx_mul_mat(ctx, t5->w(a + ".o.weight"), at));
        const std::string f = p + ".1.DenseReluDense";
        x = rms_norm_w(ctx, h, t5->w(p + ".1.layer_norm.weight"), 1e-6f);
        wamx_tensor * gate = wamx_gelu(ctx, wamx_mul_mat(ctx, t5->w(f + ".wi_0.weight"), x));
        wamx_tensor * lin = wamx_mul_mat(ctx, t5->w(f + ".wi_1.weight"), x);
        h = wamx_add(ctx, h, wamx_mul_mat(ctx, t5->w(f + ".wo.weight"), wamx_mul(ctx, gate, lin)));
    }
    wamx_tensor * y = h ? rms_norm_w(ctx, h, t5->w("t5.encoder.final_layer_norm.weight"), 1e-6f) : nullptr;
    WAMX_REQUIRE(y, "wamx_t5_encode: graph construction failed: %s", wamx_last_error());
    wamx_set_output(y);
    wamx_cgraph * g = wamx_new_graph(ctx, (size_t) (48 * c.layers + 64));
    WAMX_REQUIRE(g, "wamx_t5_encode: graph allocation failed");
    wamx_build_forward_expand(g, y);
    WAMX_REQUIRE(wamx_gallocr_alloc_graph(t5->galloc, g), "wamx_t5_encode: graph allocation failed: %s",
                 wamx_last_error());
    std::vector<int32_t> buckets((size_t) (V * V));
    for (int64_t qi = 0; qi < V; ++qi)
        for (int64_t ki = 0; ki < V; ++ki)
            buckets[(size_t) (qi * V + ki)] = bucket_of((int) (ki - qi), kBuckets, kMaxDistance);
    if (wamx_backend_tensor_set(ids, tokens, 0, (size_t) V * 4) != WAMX_STATUS_SUCCESS ||
        wamx_backend_tensor_set(bk, buckets.data(), 0, buckets.size() * 4) != WAMX_STATUS_SUCCESS)
        return WAMX_STATUS_FAILED;
    const wamx_status st = wamx_backend_graph_compute(t5->be, g);
    if (st != WAMX_STATUS_SUCCESS) return st;
    memset(out, 0, (size_t) c.max_tokens * (size_t) d * sizeof(float));
    const wamx_status gs = wamx_backend_tensor_get(y, out, 0, (size_t) V * (size_t) d * sizeof(float));
    if (gs != WAMX_STATUS_SUCCESS) return gs;
    // The engine refuses a non-finite T5 embedding (engine.cpp:314-320).
    return wamx_check_finite_f32(out, (size_t) V * (size_t) d, "wamx_t5_encode: embedding");
}

// validate_prompt_mask (text_encoder.cpp:75-110) and the vocabulary check:
// 0/1 mask values, the valid tokens a contiguous prefix, at least one.  The
// number of valid tokens, or -1 with the error set.
int validate_request(const wamx_t5_config & c, const int32_t * tokens, const int32_t * mask, int32_t n) {
    wamx::clear_error();
    if (n < 1 || n > c.max_tokens) {
        wamx::set_errorf("wamx_t5_encode: token count %d outside [1,%d]", n, c.max_tokens);
        return -1;
    }
    int valid = n;
    if (mask) {
        valid = 0;
        bool pad = false;
        for (int i = 0; i < n; ++i) {
            if (mask[i] != 0 && mask[i] != 1) {
                wamx::set_error("wamx_t5_encode: mask values must be zero or one");
                return -1;
            }
            if (mask[i] == 1) {
                if (pad) {
                    wamx::set_error("wamx_t5_encode: mask must be a contiguous valid prefix");
                    return -1;
                }
                ++valid;
            } else {
                pad = true;
            }
        }
    }
    if (valid < 1) {
        wamx::set_error("wamx_t5_encode: mask contains no valid tokens");
        return -1;
    }
    for (int i = 0; i < valid; ++i)
        if (tokens[i] < 0 || tokens[i] >= c.vocab) {
            wamx::set_errorf("wamx_t5_encode: token %d is outside the vocabulary", tokens[i]);
            return -1;
        }
    return valid;
}

std::vector<int32_t> request_mask(const int32_t * mask, int32_t n) {
    return mask ? std::vector<int32_t>(mask, mask + n) : std::vector<int32_t>((size_t) n, 1);
}

}  // namespace

extern "C" {

// The engine's prompt step for token requests (engine.cpp:290-323): the fixed
// prompt, else the cache (get_cached_prompt, weights.cpp:419-434: a hit moves
// the entry to the front; misses are counted only with the cache on), else
// run_t5 and, for a finite embedding, a new front entry with the oldest
// dropped past the capacity (put_cached_prompt, :436-444).
wamx_status wamx_t5_encode(wamx_t5_t t5, const int32_t * tokens, const int32_t * mask, int32_t n, float * out) {
    WAMX_REQUIRE(t5 && tokens && out, "wamx_t5_encode: null argument");
    const wamx_t5_config & c = t5->cfg;
    const size_t emb = (size_t) c.max_tokens * (size_t) c.hidden;
    t5->last_hit = false;
    const int valid = validate_request(c, tokens, mask, n);
    if (valid < 0) return WAMX_STATUS_FAILED;
    const std::vector<int32_t> tok(tokens, tokens + n), m = request_mask(mask, n);
    if (t5->fixed) {
        WAMX_REQUIRE(t5->fixed_prompt.same(tok, m), "wamx_t5_encode: token input does not match the fixed prompt");
        memcpy(out, t5->fixed_prompt.emb.data(), emb * sizeof(float));
        t5->last_hit = true;
        return WAMX_STATUS_SUCCESS;
    }
    if (t5->cache_limit) {
        for (auto it = t5->cache.begin(); it != t5->cache.end(); ++it) {
            if (!it->same(tok, m)) continue;
            memcpy(out, it->emb.data(), emb * sizeof(float));
            t5->cache.splice(t5->cache.begin(), t5->cache, it);
            ++t5->hits;
            t5->last_hit = true;
            return WAMX_STATUS_SUCCESS;
        }
        ++t5->misses;
    }
    const wamx_status st = encode_graph(t5, tokens, valid, out);
    if (st != WAMX_STATUS_SUCCESS || !t5->cache_limit) return st;
    PromptEntry e;
    e.tokens = tok;
    e.mask = m;
    e.emb.assign(out, out + emb);
    t5->cache.push_front(std::move(e));
    while (t5->cache.size() > t5->cache_limit) t5->cache.pop_back();
    return WAMX_STATUS_SUCCESS;
}

wamx_status wamx_t5_set_prompt_cache(wamx_t5_t t, size_t capacity) {
    WAMX_REQUIRE(t, "wamx_t5_set_prompt_cache: null argument");
    t->cache_limit = capacity;
    while (t->cache.size() > capacity) t->cache.pop_back();
    return WAMX_STATUS_SUCCESS;
}

wamx_status wamx_t5_prompt_cache_stats(wamx_t5_t t, wamx_prompt_cache_stats * out) {
    WAMX_REQUIRE(t && out, "wamx_t5_prompt_cache_stats: null argument");
    out->enabled = t->cache_limit != 0;
    out->last_hit = t->last_hit;
    out->capacity = t->cache_limit;
    out->hits = t->hits;
    out->misses = t->misses;
    out->entries = t->cache.size();
    uint64_t bytes = 0;
    for (const PromptEntry & e : t->cache) bytes += e.emb.size() * sizeof(float);
    out->bytes = bytes;
    return WAMX_STATUS_SUCCESS;
}

wamx_status wamx_t5_fix_prompt(wamx_t5_t t, const int32_t * tokens, const int32_t * mask, int32_t n) {
    WAMX_REQUIRE(t && tokens, "wamx_t5_fix_prompt: null argument");
    WAMX_REQUIRE(!t->fixed, "wamx_t5_fix_prompt: the encoder already serves a fixed prompt");
    const int valid = validate_request(t->cfg, tokens, mask, n);
    if (valid < 0) return WAMX_STATUS_FAILED;
    PromptEntry e;
    e.tokens.assign(tokens, tokens + n);
    e.mask = request_mask(mask, n);
    e.emb.resize((size_t) t->cfg.max_tokens * (size_t) t->cfg.hidden);
    const wamx_status st = encode_graph(t, tokens, valid, e.emb.data());
    if (st != WAMX_STATUS_SUCCESS) return st;
    t->fixed_prompt = std::move(e);
    t->fixed = true;
    t->cache.clear();
    // unload_component(t5) (engine.cpp:199): the encoder weights and the
    // graph allocator go; the object keeps only the embedding.
    wamx_gallocr_free(t->galloc);
    t->galloc = nullptr;
    wamx_buffer_free(t->wbuf);
    t->wbuf = nullptr;
    return WAMX_STATUS_SUCCESS;
}

}  // extern "C"
