/*
 * oracle_mot — CPU restatement of the synthetic GWP-0.5 MoT action step
 * (test infrastructure only; see oracle.h).
 *
 * Follows the reference's BF16 latency profile op by op:
 *   prompt projection   src/models/gwp05/engine/cache.cpp:53-137,
 *                       build_cross_kv mot.cpp:101-128
 *   prefix pass         cache.cpp:139-485 (expert_qkv mot.cpp:204-267,
 *                       expert_cross_ffn mot.cpp:284-347, build_attention
 *                       text_encoder.cpp:26-73 for the uncached visual text)
 *   denoise             build_cached_action_body mot.cpp:358-496,
 *                       run_unrolled_action_denoise mot.cpp:498-594,
 *                       scheduler_step weights.cpp:885-902
 * using the per-op restatements of oracle.c.  Weights are fetched by name
 * through a callback so the caller can hand over any bf16 arrays.
 */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "oracle_mot.h"

#ifdef _OPENMP
#include <omp.h>
#endif

struct orc_gwp {
    orc_gwp_config c;
    orc_weight_fn wf;
    void * user;
    int64_t d, nimg, P;
    uint16_t * action_prompt;        /* [n_lang][da] */
    uint16_t ** pk;                  /* [L] -> [H][P][dh] */
    uint16_t ** pv;                  /* [L] -> [H][dh][P] (V^T) */
    uint16_t ** lk;                  /* [L] -> [H][n_lang][dh] */
    uint16_t ** lv;                  /* [L] -> [H][dh][n_lang] */
    uint16_t * state_in;             /* [da]: state encoder output (prefix_state_hidden_in) */
    uint16_t * visual_in;            /* [nimg][d]: patch embedding output (prefix_visual_hidden_in) */
    int32_t * vpos[3];               /* visual (t, h, w) positions, NULL: the grid's */
    float * velocity;                /* [num_steps][T][A]: the decoder output of each denoise step */
    int missing;
};

static inline float b2f(uint16_t h) { return orc_bf16_to_f32(h); }
static inline uint16_t f2b(float f) { return orc_f32_to_bf16(f); }

static const uint16_t * W(orc_gwp * g, const char * fmt, ...) __attribute__((format(printf, 2, 3)));
static const uint16_t * W(orc_gwp * g, const char * fmt, ...) {
    char name[256];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(name, sizeof name, fmt, ap);
    va_end(ap);
    const uint16_t * p = g->wf(g->user, name);
    if (!p) {
        fprintf(stderr, "oracle_mot: missing weight %s\n", name);
        g->missing = 1;
    }
    return p;
}

static uint16_t * alloc16(int64_t n) { return (uint16_t *) calloc((size_t) n, 2); }
static float * alloc32(int64_t n) { return (float *) calloc((size_t) n, 4); }

/* linear_with_activation: bf16 GEMM + bf16 bias ADD; y [N][M]. */
static uint16_t * lin(orc_gwp * g, const char * base, const void * x, int x_type, int64_t N, int64_t K, int64_t M,
                      int epi, const uint16_t * res, const float * gate) {
    char nw[256], nb[256];
    snprintf(nw, sizeof nw, "%s.weight", base);
    snprintf(nb, sizeof nb, "%s.bias", base);
    const uint16_t * w = W(g, "%s", nw);
    const uint16_t * b = W(g, "%s", nb);
    uint16_t * y = alloc16(N * M);
    if (w && b) orc_linear(w, x, x_type, b, epi, res, gate, y, M, N, K);
    return y;
}

/* Unary ops on bf16 tensors: y = bf16(op(f32(x))). */
static void unary_bf16(uint16_t * x, int64_t n, int op) {
    for (int64_t i = 0; i < n; ++i) {
        const float v = b2f(x[i]);
        float r;
        if (op == 0) r = orc_gelu_tanh(v);
        else if (op == 1) r = orc_gelu_erf(v);
        else r = (float) ((double) v / (1.0 + exp(-(double) v)));
        x[i] = f2b(r);
    }
}

/* action_encoder / action_decoder: linear, GELU_ERF, linear, GELU_ERF, linear. */
static uint16_t * mlp3(orc_gwp * g, const char * p, const void * x, int x_type, int64_t N, int64_t in,
                       int64_t out) {
    const int64_t E = g->c.enc_hidden;
    char b[256];
    snprintf(b, sizeof b, "%s.in_proj", p);
    uint16_t * h = lin(g, b, x, x_type, N, in, E, ORC_EPI_BIAS, NULL, NULL);
    unary_bf16(h, N * E, 1);
    snprintf(b, sizeof b, "%s.mid_proj", p);
    uint16_t * h2 = lin(g, b, h, ORC_BF16, N, E, E, ORC_EPI_BIAS, NULL, NULL);
    free(h);
    unary_bf16(h2, N * E, 1);
    snprintf(b, sizeof b, "%s.out_proj", p);
    uint16_t * o = lin(g, b, h2, ORC_BF16, N, E, out, ORC_EPI_BIAS, NULL, NULL);
    free(h2);
    return o;
}

/* build_condition time branch: temb [w], modulation [6w] (bf16). */
static void condition(orc_gwp * g, const char * p, const float * freq, int64_t w, uint16_t ** temb,
                      uint16_t ** mod) {
    char b[256];
    snprintf(b, sizeof b, "%s.time_embedder.linear_1", p);
    uint16_t * t = lin(g, b, freq, ORC_F32, 1, 256, w, ORC_EPI_BIAS, NULL, NULL);
    unary_bf16(t, w, 2);
    snprintf(b, sizeof b, "%s.time_embedder.linear_2", p);
    *temb = lin(g, b, t, ORC_BF16, 1, w, w, ORC_EPI_BIAS, NULL, NULL);
    free(t);
    uint16_t * s = alloc16(w);
    memcpy(s, *temb, (size_t) w * 2);
    unary_bf16(s, w, 2);
    snprintf(b, sizeof b, "%s.time_proj", p);
    *mod = lin(g, b, s, ORC_BF16, 1, w, 6 * w, ORC_EPI_BIAS, NULL, NULL);
    free(s);
}

/* build_condition text branch: linear, GELU (tanh), linear. */
static uint16_t * text(orc_gwp * g, const char * p, const float * prompt, int64_t w) {
    char b[256];
    const int64_t NL = g->c.n_lang;
    snprintf(b, sizeof b, "%s.text_embedder.linear_1", p);
    uint16_t * t = lin(g, b, prompt, ORC_F32, NL, g->c.t5_hidden, w, ORC_EPI_BIAS, NULL, NULL);
    unary_bf16(t, NL * w, 0);
    snprintf(b, sizeof b, "%s.text_embedder.linear_2", p);
    uint16_t * o = lin(g, b, t, ORC_BF16, NL, w, w, ORC_EPI_BIAS, NULL, NULL);
    free(t);
    return o;
}

/* modulation_add for layer l: out[6][w] = f32(mod) + f32(table_l). */
static void modulation(orc_gwp * g, const char * expert, int l, const uint16_t * mod, int64_t w, float * out) {
    const uint16_t * tab = W(g, "gwp.blocks.%s.scale_shift_table", expert);
    if (!tab) return;
    orc_modulation(mod, tab + (int64_t) l * 6 * w, out, 6 * w, 1);
}

/* Transposed V write: v part of rows [N][ld] (column offset off) into
 * vt [H][dh][ldv] at key columns k0... */
static void store_vt(const uint16_t * rows, int64_t N, int64_t ld, int64_t off, int64_t H, int64_t dh, uint16_t * vt,
                     int64_t ldv, int64_t k0) {
    for (int64_t t = 0; t < N; ++t)
        for (int64_t h = 0; h < H; ++h)
            for (int64_t e = 0; e < dh; ++e) vt[(h * dh + e) * ldv + k0 + t] = rows[t * ld + off + h * dh + e];
}

/* build_attention's f32 Q.K path: q, k f32 [T][d] (rms_norm output, no bf16
 * cast), V^T bf16; probabilities rounded to bf16 for the V.P MUL_MAT;
 * output bf16 [T][d] (the O projection's input cast). */
static void attention_f32qk(const float * q, int64_t T, const float * k, int64_t NL, const uint16_t * vt,
                            int64_t H, int64_t dh, float scale, uint16_t * out) {
    if (orc_get_port()) {
        orc_port_attention_f32qk(q, T, k, NL, vt, H, dh, scale, out);
        return;
    }
    const int64_t d = H * dh;
#pragma omp parallel for collapse(2)
    for (int64_t h = 0; h < H; ++h)
        for (int64_t i = 0; i < T; ++i) {
            float * s = (float *) malloc(sizeof(float) * (size_t) NL);
            for (int64_t j = 0; j < NL; ++j) {
                double acc = 0.0;
                for (int64_t e = 0; e < dh; ++e) acc += (double) q[i * d + h * dh + e] * (double) k[j * d + h * dh + e];
                s[j] = (float) acc;
            }
            orc_softmax_f32(s, s, 1, NL, scale);
            for (int64_t e = 0; e < dh; ++e) {
                double acc = 0.0;
                for (int64_t j = 0; j < NL; ++j)
                    acc += (double) b2f(f2b(s[j])) * (double) b2f(vt[(h * dh + e) * NL + j]);
                out[i * d + h * dh + e] = f2b((float) acc);
            }
            free(s);
        }
}

/* FFN half: modulated norm, up + bias + GELU-tanh, down + bias + gated residual. */
static uint16_t * ffn(orc_gwp * g, const char * p, uint16_t * h, int64_t N, int64_t w, int64_t F, const float * mods) {
    const float * cshift = mods + 3 * w;
    const float * cscale = mods + 4 * w;
    const float * cgate = mods + 5 * w;
    uint16_t * n = alloc16(N * w);
    orc_norm_mod_bf16(h, w, cscale, cshift, 0, n, N, w, g->c.eps);
    char b[256];
    snprintf(b, sizeof b, "%s.ffn.net.0.proj", p);
    uint16_t * u = lin(g, b, n, ORC_BF16, N, w, F, ORC_EPI_BIAS_GELU, NULL, NULL);
    free(n);
    snprintf(b, sizeof b, "%s.ffn.net.2", p);
    uint16_t * o = lin(g, b, u, ORC_BF16, N, F, w, ORC_EPI_BIAS_GATED, h, cgate);
    free(u);
    free(h);
    return o;
}

/* expert_cross_ffn with the cached prompt K/V. */
static uint16_t * cross_ffn_cached(orc_gwp * g, const char * p, int l, uint16_t * h, int64_t N, int64_t w, int64_t F,
                                   const float * mods) {
    const int64_t d = g->d, H = g->c.n_heads, dh = g->c.head_dim;
    uint16_t * n = alloc16(N * w);
    char b[256];
    snprintf(b, sizeof b, "%s.norm2.weight", p);
    const uint16_t * n2w = W(g, "%s", b);
    snprintf(b, sizeof b, "%s.norm2.bias", p);
    const uint16_t * n2b = W(g, "%s", b);
    if (n2w && n2b) orc_layer_norm_bf16(h, w, n2w, n2b, n, N, w, g->c.eps);
    snprintf(b, sizeof b, "%s.attn2.to_q", p);
    uint16_t * q = lin(g, b, n, ORC_BF16, N, w, d, ORC_EPI_BIAS, NULL, NULL);
    free(n);
    uint16_t * Q = alloc16(H * N * dh);
    const uint16_t * cnq = W(g, "%s.attn2.norm_q.weight", p);
    if (cnq) orc_qk_norm_rope(q, d, cnq, Q, H, dh, N, N, 0, 2, NULL, NULL, NULL, g->c.eps, 10000.0f);
    free(q);
    uint16_t * att = alloc16(N * d);
    orc_attention(Q, g->lk[l], g->lv[l], g->c.n_lang, g->c.n_lang, NULL, NULL, 0, 0, 0, att, H, dh, N,
                  1.0f / sqrtf((float) dh));
    free(Q);
    snprintf(b, sizeof b, "%s.attn2.to_out.0", p);
    uint16_t * h2 = lin(g, b, att, ORC_BF16, N, d, w, ORC_EPI_BIAS_RESIDUAL, h, NULL);
    free(att);
    free(h);
    return ffn(g, p, h2, N, w, F, mods);
}

/* expert_cross_ffn against uncached text embeddings (visual expert, prefix). */
static uint16_t * cross_ffn_uncached(orc_gwp * g, const char * p, uint16_t * h, int64_t N, int64_t w, int64_t F,
                                     const uint16_t * txt, const float * mods) {
    const int64_t d = g->d, H = g->c.n_heads, dh = g->c.head_dim, NL = g->c.n_lang;
    uint16_t * n = alloc16(N * w);
    const uint16_t * n2w = W(g, "%s.norm2.weight", p);
    const uint16_t * n2b = W(g, "%s.norm2.bias", p);
    if (n2w && n2b) orc_layer_norm_bf16(h, w, n2w, n2b, n, N, w, g->c.eps);
    char b[256];
    snprintf(b, sizeof b, "%s.attn2.to_q", p);
    uint16_t * q = lin(g, b, n, ORC_BF16, N, w, d, ORC_EPI_BIAS, NULL, NULL);
    free(n);
    snprintf(b, sizeof b, "%s.attn2.to_k", p);
    uint16_t * k = lin(g, b, txt, ORC_BF16, NL, w, d, ORC_EPI_BIAS, NULL, NULL);
    snprintf(b, sizeof b, "%s.attn2.to_v", p);
    uint16_t * v = lin(g, b, txt, ORC_BF16, NL, w, d, ORC_EPI_BIAS, NULL, NULL);
    float * qf = alloc32(N * d);
    float * kf = alloc32(NL * d);
    const uint16_t * cnq = W(g, "%s.attn2.norm_q.weight", p);
    const uint16_t * cnk = W(g, "%s.attn2.norm_k.weight", p);
    if (cnq) orc_rms_norm_bf16_f32(q, d, cnq, qf, N, d, g->c.eps);
    if (cnk) orc_rms_norm_bf16_f32(k, d, cnk, kf, NL, d, g->c.eps);
    uint16_t * vt = alloc16(H * dh * NL);
    store_vt(v, NL, d, 0, H, dh, vt, NL, 0);
    uint16_t * att = alloc16(N * d);
    attention_f32qk(qf, N, kf, NL, vt, H, dh, 1.0f / sqrtf((float) dh), att);
    free(q);
    free(k);
    free(v);
    free(qf);
    free(kf);
    free(vt);
    snprintf(b, sizeof b, "%s.attn2.to_out.0", p);
    uint16_t * h2 = lin(g, b, att, ORC_BF16, N, d, w, ORC_EPI_BIAS_RESIDUAL, h, NULL);
    free(att);
    free(h);
    return ffn(g, p, h2, N, w, F, mods);
}

orc_gwp * orc_gwp_new(const orc_gwp_config * cfg, orc_weight_fn wf, void * user) {
    orc_gwp * g = (orc_gwp *) calloc(1, sizeof(orc_gwp));
    g->c = *cfg;
    g->wf = wf;
    g->user = user;
    g->d = (int64_t) cfg->n_heads * cfg->head_dim;
    g->nimg = (int64_t) cfg->grid_h * cfg->grid_w;
    g->P = 1 + g->nimg;
    const int64_t L = cfg->n_layers, H = cfg->n_heads, dh = cfg->head_dim;
    g->action_prompt = alloc16((int64_t) cfg->n_lang * cfg->action_hidden);
    g->pk = (uint16_t **) calloc((size_t) L, sizeof(void *));
    g->pv = (uint16_t **) calloc((size_t) L, sizeof(void *));
    g->lk = (uint16_t **) calloc((size_t) L, sizeof(void *));
    g->lv = (uint16_t **) calloc((size_t) L, sizeof(void *));
    g->state_in = alloc16(cfg->action_hidden);
    g->visual_in = alloc16(g->nimg * g->d);
    for (int64_t l = 0; l < L; ++l) {
        g->pk[l] = alloc16(H * g->P * dh);
        g->pv[l] = alloc16(H * dh * g->P);
        g->lk[l] = alloc16(H * (int64_t) cfg->n_lang * dh);
        g->lv[l] = alloc16(H * dh * (int64_t) cfg->n_lang);
    }
    return g;
}

void orc_gwp_free(orc_gwp * g) {
    if (!g) return;
    for (int l = 0; l < g->c.n_layers; ++l) {
        free(g->pk[l]);
        free(g->pv[l]);
        free(g->lk[l]);
        free(g->lv[l]);
    }
    free(g->pk);
    free(g->pv);
    free(g->lk);
    free(g->lv);
    free(g->action_prompt);
    free(g->state_in);
    free(g->visual_in);
    for (int i = 0; i < 3; ++i) free(g->vpos[i]);
    free(g->velocity);
    free(g);
}

int orc_gwp_set_visual_positions(orc_gwp * g, const int32_t * t, const int32_t * h, const int32_t * w) {
    for (int i = 0; i < 3; ++i) {
        free(g->vpos[i]);
        g->vpos[i] = NULL;
    }
    if (!t || !h || !w) return 0;
    const int32_t * src[3] = {t, h, w};
    for (int i = 0; i < 3; ++i) {
        g->vpos[i] = (int32_t *) malloc((size_t) g->nimg * 4);
        memcpy(g->vpos[i], src[i], (size_t) g->nimg * 4);
    }
    return 0;
}

int orc_gwp_prompt(orc_gwp * g, const float * prompt, int layers) {
    const int64_t da = g->c.action_hidden, d = g->d, NL = g->c.n_lang, H = g->c.n_heads, dh = g->c.head_dim;
    uint16_t * txt = text(g, "gwp.action_condition_embedder", prompt, da);
    memcpy(g->action_prompt, txt, (size_t) NL * da * 2);
    const int L = layers > 0 && layers < g->c.n_layers ? layers : g->c.n_layers;
    for (int l = 0; l < L; ++l) {
        char b[256];
        snprintf(b, sizeof b, "gwp.blocks.%d.action_expert.attn2.to_k", l);
        uint16_t * k = lin(g, b, txt, ORC_BF16, NL, da, d, ORC_EPI_BIAS, NULL, NULL);
        snprintf(b, sizeof b, "gwp.blocks.%d.action_expert.attn2.to_v", l);
        uint16_t * v = lin(g, b, txt, ORC_BF16, NL, da, d, ORC_EPI_BIAS, NULL, NULL);
        const uint16_t * cnk = W(g, "gwp.blocks.%d.action_expert.attn2.norm_k.weight", l);
        if (cnk) orc_qk_norm_rope(k, d, cnk, g->lk[l], H, dh, NL, NL, 0, 2, NULL, NULL, NULL, g->c.eps, 10000.0f);
        store_vt(v, NL, d, 0, H, dh, g->lv[l], NL, 0);
        free(k);
        free(v);
    }
    free(txt);
    return g->missing ? -1 : 0;
}

int orc_gwp_prefix(orc_gwp * g, const float * state, const float * latent, const float * prompt, int layers) {
    const orc_gwp_config * c = &g->c;
    const int64_t da = c->action_hidden, d = g->d, H = c->n_heads, dh = c->head_dim, nimg = g->nimg, P = g->P;
    const int64_t A = c->action_dim, Z = c->z_dim, gh = c->grid_h, gw = c->grid_w;
    const int L = layers > 0 && layers < c->n_layers ? layers : c->n_layers;
    uint16_t * sh = mlp3(g, "gwp.state_encoder", state, ORC_F32, 1, A, da);
    /* Patch embedding: conv 2x2 / stride 2 = im2col (ic, kh, kw) + GEMM + bias. */
    uint16_t * cols = alloc16(nimg * Z * 4);
    for (int64_t y = 0; y < gh; ++y)
        for (int64_t x = 0; x < gw; ++x)
            for (int64_t ic = 0; ic < Z; ++ic)
                for (int64_t kh = 0; kh < 2; ++kh)
                    for (int64_t kw = 0; kw < 2; ++kw)
                        cols[(y * gw + x) * Z * 4 + ic * 4 + kh * 2 + kw] =
                            f2b(latent[(ic * 2 * gh + 2 * y + kh) * 2 * gw + 2 * x + kw]);
    uint16_t * vh = lin(g, "gwp.patch_embedding", cols, ORC_BF16, nimg, Z * 4, d, ORC_EPI_BIAS, NULL, NULL);
    free(cols);
    float freq0[256];
    orc_timestep_embedding(0.0f, 256, freq0);
    uint16_t *stemb, *smod, *vtemb, *vmod;
    condition(g, "gwp.action_condition_embedder", freq0, da, &stemb, &smod);
    condition(g, "gwp.condition_embedder", freq0, d, &vtemb, &vmod);
    uint16_t * vtext = text(g, "gwp.condition_embedder", prompt, d);
    int32_t spos = 0;
    int32_t * vt = (int32_t *) calloc((size_t) nimg, 4);
    int32_t * vhp = (int32_t *) calloc((size_t) nimg, 4);
    int32_t * vwp = (int32_t *) calloc((size_t) nimg, 4);
    /* visual_positions (semantics.cpp:235-257): t = 0, h = y, w = x. */
    for (int64_t y = 0; y < gh; ++y)
        for (int64_t x = 0; x < gw; ++x) {
            vhp[y * gw + x] = (int32_t) y;
            vwp[y * gw + x] = (int32_t) x;
        }
    if (g->vpos[0]) {
        memcpy(vt, g->vpos[0], (size_t) nimg * 4);
        memcpy(vhp, g->vpos[1], (size_t) nimg * 4);
        memcpy(vwp, g->vpos[2], (size_t) nimg * 4);
    }
    memcpy(g->state_in, sh, (size_t) da * 2);
    memcpy(g->visual_in, vh, (size_t) nimg * d * 2);
    float * am = alloc32(6 * da);
    float * vm = alloc32(6 * d);
    const float scale = 1.0f / sqrtf((float) dh);
    for (int l = 0; l < L; ++l) {
        char pa[128], pv[128];
        snprintf(pa, sizeof pa, "gwp.blocks.%d.action_expert", l);
        snprintf(pv, sizeof pv, "gwp.blocks.%d.visual_expert", l);
        modulation(g, "action_expert", l, smod, da, am);
        modulation(g, "visual_expert", l, vmod, d, vm);
        uint16_t * sn = alloc16(da);
        orc_norm_mod_bf16(sh, da, am + da, am, 0, sn, 1, da, c->eps);
        char b[256];
        snprintf(b, sizeof b, "%s.attn1.to_qkv", pa);
        uint16_t * sqkv = lin(g, b, sn, ORC_BF16, 1, da, 3 * d, ORC_EPI_BIAS, NULL, NULL);
        free(sn);
        uint16_t * vn = alloc16(nimg * d);
        orc_norm_mod_bf16(vh, d, vm + d, vm, 0, vn, nimg, d, c->eps);
        snprintf(b, sizeof b, "%s.attn1.to_qkv", pv);
        uint16_t * vqkv = lin(g, b, vn, ORC_BF16, nimg, d, 3 * d, ORC_EPI_BIAS, NULL, NULL);
        free(vn);
        uint16_t * Q = alloc16(H * P * dh);
        const uint16_t *anq = W(g, "%s.attn1.norm_q.weight", pa), *ank = W(g, "%s.attn1.norm_k.weight", pa);
        const uint16_t *vnq = W(g, "%s.attn1.norm_q.weight", pv), *vnk = W(g, "%s.attn1.norm_k.weight", pv);
        if (g->missing) break;
        orc_qk_norm_rope(sqkv, 3 * d, anq, Q, H, dh, 1, P, 0, 0, &spos, NULL, NULL, c->eps, 10000.0f);
        orc_qk_norm_rope(vqkv, 3 * d, vnq, Q, H, dh, nimg, P, 1, 1, vt, vhp, vwp, c->eps, 10000.0f);
        orc_qk_norm_rope(sqkv + d, 3 * d, ank, g->pk[l], H, dh, 1, P, 0, 0, &spos, NULL, NULL, c->eps, 10000.0f);
        orc_qk_norm_rope(vqkv + d, 3 * d, vnk, g->pk[l], H, dh, nimg, P, 1, 1, vt, vhp, vwp, c->eps, 10000.0f);
        store_vt(sqkv, 1, 3 * d, 2 * d, H, dh, g->pv[l], P, 0);
        store_vt(vqkv, nimg, 3 * d, 2 * d, H, dh, g->pv[l], P, 1);
        free(sqkv);
        free(vqkv);
        if (l + 1 == c->n_layers) {
            free(Q);
            break;
        }
        uint16_t * att = alloc16(P * d);
        orc_attention(Q, g->pk[l], g->pv[l], P, P, NULL, NULL, 0, 0, 0, att, H, dh, P, scale);
        free(Q);
        snprintf(b, sizeof b, "%s.attn1.to_out.0", pa);
        uint16_t * sh2 = lin(g, b, att, ORC_BF16, 1, d, da, ORC_EPI_BIAS_GATED, sh, am + 2 * da);
        snprintf(b, sizeof b, "%s.attn1.to_out.0", pv);
        uint16_t * vh2 = lin(g, b, att + d, ORC_BF16, nimg, d, d, ORC_EPI_BIAS_GATED, vh, vm + 2 * d);
        free(att);
        free(sh);
        free(vh);
        sh = cross_ffn_cached(g, pa, l, sh2, 1, da, c->action_ffn_dim, am);
        vh = cross_ffn_uncached(g, pv, vh2, nimg, d, c->ffn_dim, vtext, vm);
    }
    free(sh);
    free(vh);
    free(stemb);
    free(smod);
    free(vtemb);
    free(vmod);
    free(vtext);
    free(vt);
    free(vhp);
    free(vwp);
    free(am);
    free(vm);
    return g->missing ? -1 : 0;
}

int orc_gwp_denoise(orc_gwp * g, const float * noise, float * action_out, int layers, int steps) {
    const orc_gwp_config * c = &g->c;
    const int64_t da = c->action_hidden, d = g->d, H = c->n_heads, dh = c->head_dim, T = c->action_chunk;
    const int64_t A = c->action_dim, P = g->P;
    const int L = layers > 0 && layers < c->n_layers ? layers : c->n_layers;
    const int S = steps > 0 && steps < c->num_steps ? steps : c->num_steps;
    float * ts = alloc32(c->num_steps);
    float * sig = alloc32(c->num_steps + 1);
    orc_flow_schedule(c->num_steps, c->shift, ts, sig);
    uint16_t * action = alloc16(T * A);
    for (int64_t i = 0; i < T * A; ++i) action[i] = f2b(noise[i]);
    int32_t * apos = (int32_t *) calloc((size_t) T, 4);
    for (int64_t i = 0; i < T; ++i) apos[i] = (int32_t) (i + 1);
    float * mods = alloc32(6 * da);
    free(g->velocity);
    g->velocity = (float *) calloc((size_t) (c->num_steps * T * A), sizeof(float));
    const float scale = 1.0f / sqrtf((float) dh);
    for (int s = 0; s < S; ++s) {
        float freq[256];
        orc_timestep_embedding(ts[s], 256, freq);
        uint16_t * h = mlp3(g, "gwp.action_encoder", action, ORC_BF16, T, A, da);
        uint16_t *temb, *mod;
        condition(g, "gwp.action_condition_embedder", freq, da, &temb, &mod);
        for (int l = 0; l < L; ++l) {
            char p[128], b[256];
            snprintf(p, sizeof p, "gwp.blocks.%d.action_expert", l);
            modulation(g, "action_expert", l, mod, da, mods);
            uint16_t * n = alloc16(T * da);
            orc_norm_mod_bf16(h, da, mods + da, mods, 0, n, T, da, c->eps);
            snprintf(b, sizeof b, "%s.attn1.to_qkv", p);
            uint16_t * qkv = lin(g, b, n, ORC_BF16, T, da, 3 * d, ORC_EPI_BIAS, NULL, NULL);
            free(n);
            const uint16_t *nq = W(g, "%s.attn1.norm_q.weight", p), *nk = W(g, "%s.attn1.norm_k.weight", p);
            if (g->missing) break;
            uint16_t * Q = alloc16(H * T * dh);
            uint16_t * Ka = alloc16(H * T * dh);
            uint16_t * Va = alloc16(H * dh * T);
            orc_qk_norm_rope(qkv, 3 * d, nq, Q, H, dh, T, T, 0, 0, apos, NULL, NULL, c->eps, 10000.0f);
            orc_qk_norm_rope(qkv + d, 3 * d, nk, Ka, H, dh, T, T, 0, 0, apos, NULL, NULL, c->eps, 10000.0f);
            store_vt(qkv, T, 3 * d, 2 * d, H, dh, Va, T, 0);
            free(qkv);
            uint16_t * att = alloc16(T * d);
            orc_attention(Q, g->pk[l], g->pv[l], P, P, Ka, Va, T, T, 1, att, H, dh, T, scale);
            free(Q);
            free(Ka);
            free(Va);
            snprintf(b, sizeof b, "%s.attn1.to_out.0", p);
            uint16_t * h2 = lin(g, b, att, ORC_BF16, T, d, da, ORC_EPI_BIAS_GATED, h, mods + 2 * da);
            free(att);
            free(h);
            h = cross_ffn_cached(g, p, l, h2, T, da, c->action_ffn_dim, mods);
        }
        /* Output modulation: f32(action_scale_shift_table) + f32(temb). */
        const uint16_t * sst = W(g, "gwp.action_scale_shift_table");
        if (g->missing) break;
        float * om = alloc32(2 * da);
        for (int r = 0; r < 2; ++r)
            for (int64_t j = 0; j < da; ++j) om[r * da + j] = b2f(sst[r * da + j]) + b2f(temb[j]);
        uint16_t * n = alloc16(T * da);
        orc_norm_mod_bf16(h, da, om + da, om, 0, n, T, da, c->eps);
        uint16_t * pred = mlp3(g, "gwp.action_decoder", n, ORC_BF16, T, da, A);
        /* The velocity of this step (engine.cpp:416-421 dumps it as
           velocity_step0 / denoise_%02d_velocity). */
        for (int64_t i = 0; i < T * A; ++i) g->velocity[(int64_t) s * T * A + i] = b2f(pred[i]);
        const float dt = sig[s + 1] - sig[s];
        for (int64_t i = 0; i < T * A; ++i) {
            volatile float vdt = b2f(pred[i]) * dt;
            volatile float sum = b2f(action[i]) + vdt;
            action[i] = f2b(sum);
        }
        free(om);
        free(n);
        free(pred);
        free(h);
        free(temb);
        free(mod);
    }
    for (int64_t i = 0; i < T * A; ++i) action_out[i] = b2f(action[i]);
    free(ts);
    free(sig);
    free(action);
    free(apos);
    free(mods);
    return g->missing ? -1 : 0;
}

const uint16_t * orc_gwp_prefix_key(orc_gwp * g, int layer) { return g->pk[layer]; }
const uint16_t * orc_gwp_prefix_value(orc_gwp * g, int layer) { return g->pv[layer]; }
const uint16_t * orc_gwp_prompt_key(orc_gwp * g, int layer) { return g->lk[layer]; }
const uint16_t * orc_gwp_prompt_value(orc_gwp * g, int layer) { return g->lv[layer]; }
const uint16_t * orc_gwp_prefix_hidden_in(orc_gwp * g, int which) { return which == 0 ? g->state_in : g->visual_in; }
const uint16_t * orc_gwp_action_prompt(orc_gwp * g) { return g->action_prompt; }

const float * orc_gwp_velocity(orc_gwp * g, int step) {
    if (!g || !g->velocity || step < 0 || step >= g->c.num_steps) return NULL;
    return g->velocity + (int64_t) step * g->c.action_chunk * g->c.action_dim;
}
