/*
 * oracle_mot — CPU restatement of the synthetic GWP-0.5 MoT action step
 * (test infrastructure only; see oracle.h for the rules).
 */
#ifndef WAMX_ORACLE_MOT_H
#define WAMX_ORACLE_MOT_H

#include <stdarg.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same fields and meaning as wamx_gwp_config. */
typedef struct orc_gwp_config {
    int32_t n_layers, hidden, n_heads, head_dim, ffn_dim, action_hidden, action_ffn_dim, action_chunk, action_dim;
    int32_t grid_h, grid_w, n_lang, t5_hidden, z_dim, num_steps, enc_hidden;
    float shift, eps;
} orc_gwp_config;

/* Returns the bf16 array of the named weight (names as in the wamx driver:
 * gwp.blocks.<l>.<expert>.attn1.to_qkv.weight, ...), or NULL. */
typedef const uint16_t * (*orc_weight_fn)(void * user, const char * name);

typedef struct orc_gwp orc_gwp;

orc_gwp * orc_gwp_new(const orc_gwp_config * cfg, orc_weight_fn wf, void * user);
void      orc_gwp_free(orc_gwp * g);
/* prompt f32 [n_lang][t5_hidden] -> action prompt and per-layer prompt K/V. */
/* layers > 0 limits the per-layer prompt K/V to the first `layers` blocks. */
int orc_gwp_prompt(orc_gwp * g, const float * prompt, int layers);
/* state f32 [action_dim], latent f32 [z][2gh][2gw], prompt as above.
 * layers > 0 limits the pass to the first `layers` blocks (timing samples). */
int orc_gwp_prefix(orc_gwp * g, const float * state, const float * latent, const float * prompt, int layers);
/* noise f32 [chunk][action_dim] -> action f32; layers/steps > 0 limit the work. */
int orc_gwp_denoise(orc_gwp * g, const float * noise, float * action_out, int layers, int steps);
const uint16_t * orc_gwp_prefix_key(orc_gwp * g, int layer);    /* [H][P][dh] */
const uint16_t * orc_gwp_prefix_value(orc_gwp * g, int layer);  /* [H][dh][P] */
const uint16_t * orc_gwp_prompt_key(orc_gwp * g, int layer);    /* [H][n_lang][dh] */
const uint16_t * orc_gwp_prompt_value(orc_gwp * g, int layer);  /* [H][dh][n_lang] (V^T) */
/* The prefix pass's inputs to the first layer, as the reference dumps them
 * (prefix_state_hidden_in / prefix_visual_hidden_in, cache.cpp:441-469):
 * which 0: state encoder output [action_hidden]; 1: patch embedding output
 * [nimg][hidden]. */
const uint16_t * orc_gwp_prefix_hidden_in(orc_gwp * g, int which);
/* Visual token positions (t, h, w), each [nimg], for the next prefix pass in
 * place of visual_positions' grid (semantics.cpp:235-257); NULLs restore it. */
int orc_gwp_set_visual_positions(orc_gwp * g, const int32_t * t, const int32_t * h, const int32_t * w);
const uint16_t * orc_gwp_action_prompt(orc_gwp * g);            /* [n_lang][action_hidden] */
/* Velocity (action decoder output, bf16 widened) of denoise step `step` of
   the last orc_gwp_denoise: [T][A]; NULL before a denoise or out of range. */
const float * orc_gwp_velocity(orc_gwp * g, int step);

#ifdef __cplusplus
}
#endif

#endif
