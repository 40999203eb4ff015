"""Pins the oracle's full-step composition (oracle/oracle_mot.c: prompt
projection, prefix pass, unrolled denoise) on the CPU.

The per-op functions are pinned in test_oracle.py.  Here the composition is
checked by properties the mathematics fixes and by rebuilding pieces of the
step from those per-op functions, following the reference files directly:

* a zero action decoder output makes every Euler step add 0, so the chunk
  must stay bf16(noise) exactly; a zero decoder weight with a constant bias
  makes the velocity constant, so the chunk follows the scheduler recursion
  (scheduler_step, weights.cpp:885-902, on the pinned flow schedule);
* with every gate slice and the cross-attention output zeroed, each block is
  the identity, so the velocity must be decoder(norm_mod(encoder(a))) with the
  output modulation table + temb (mot.cpp:468-488) - bit for bit;
* the prefix pass's layer-0 inputs (state encoder, patch embedding) and the
  layer-0 prefix K/V must equal their composition from the per-op functions
  (cache.cpp:196-287, mot.cpp:204-267), and a single nonzero latent entry
  must land in the patch-embedding column ic*KH*KW + kh*KW + kw of
  PyTorch's conv weight [OC][IC][KH][KW];
* permuting the visual tokens together with their (h, w) positions permutes
  the prefix K/V rows of every layer (attention is equivariant);
* the prompt K/V and the projected action prompt equal their composition
  (cache.cpp:53-137, mot.cpp:101-128);
* one denoise step over one layer equals the composition of the pinned ops in
  mot.cpp's order (the same layer the GPU drop-in test builds op for op);
* the prefix layer-1 K equals the composition through a whole layer-0 block
  (joint attention, both cross-attentions, both FFNs).
"""
from __future__ import annotations

from math import erf

import numpy as np
import pytest

from test_gpu_dropin import oracle_action_layer

CFG = dict(n_layers=2, hidden=256, n_heads=2, head_dim=128, ffn_dim=512, action_hidden=256, action_ffn_dim=384,
           action_chunk=48, action_dim=32, grid_h=4, grid_w=8, n_lang=16, t5_hidden=64, z_dim=16, num_steps=3,
           enc_hidden=32, shift=5.0, eps=1e-6)
SEED = 0x5EED0A00
EPS = CFG["eps"]


def f32(h):
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


@pytest.fixture(scope="module")
def base(orc):
    return orc.gwp_synthetic_weights(CFG, SEED)


def inputs(orc, seed=3):
    c = CFG
    return (orc.fill_normal(c["action_dim"], seed + 1),
            orc.fill_normal(c["z_dim"] * 4 * c["grid_h"] * c["grid_w"], seed + 2),
            orc.fill_normal(c["n_lang"] * c["t5_hidden"], seed + 3),
            orc.fill_normal(c["action_chunk"] * c["action_dim"], seed + 4))


def run(orc, w, ins, positions=None):
    g = orc.Gwp(CFG, w)
    state, latent, prompt, noise = ins
    g.prompt(prompt)
    if positions is not None:
        g.set_visual_positions(*positions)
    g.prefix(state, latent, prompt)
    return g


# --- composition helpers from the pinned per-op functions ---------------------
class Ops:
    def __init__(self, orc, w):
        self.orc, self.w = orc, w
        c = CFG
        self.d = c["n_heads"] * c["head_dim"]
        self.da, self.E, self.A = c["action_hidden"], c["enc_hidden"], c["action_dim"]

    def W(self, name, rows):
        a = self.w[name]
        return a.reshape(rows, a.size // rows)

    def lin(self, p, x, out, epi=None, res=None, gate=None):
        o = self.orc
        return o.linear(self.W(p + ".weight", out), x, self.w[p + ".bias"], o.EPI_BIAS if epi is None else epi, res,
                        gate)

    def unary(self, h, fn):
        v = f32(h).astype(np.float64).ravel()
        r = np.array([fn(t) for t in v], np.float32).reshape(h.shape)
        return self.orc.f32_to_bf16(r)

    def gelu_erf(self, h):          # ggml_gelu_erf on bf16, in double then f32
        return self.unary(h, lambda t: 0.5 * t * (1.0 + erf(t / np.sqrt(2.0))))

    def gelu_tanh(self, h):
        return self.unary(h, lambda t: self.orc.gelu_tanh(float(t)))

    def silu(self, h):
        return self.unary(h, lambda t: t / (1.0 + np.exp(-t)))

    def mlp3(self, p, x, out):       # action_encoder / action_decoder, mot.cpp:16-55
        h = self.gelu_erf(self.lin(p + ".in_proj", x, self.E))
        h = self.gelu_erf(self.lin(p + ".mid_proj", h, self.E))
        return self.lin(p + ".out_proj", h, out)

    def condition(self, p, freq, w):  # build_condition time branch, mot.cpp:69-82
        t = self.silu(self.lin(p + ".time_embedder.linear_1", freq[None].astype(np.float32), w))
        temb = self.lin(p + ".time_embedder.linear_2", t, w)
        return temb, self.lin(p + ".time_proj", self.silu(temb), 6 * w)

    def text(self, p, prompt, w):     # build_condition text branch, mot.cpp:84-92
        t = self.gelu_tanh(self.lin(p + ".text_embedder.linear_1", prompt, w))
        return self.lin(p + ".text_embedder.linear_2", t, w)

    def mods(self, expert, l, mod, w):  # modulation_add, mot.cpp:137-145 -> [6][w]
        tab = self.w[f"gwp.blocks.{expert}.scale_shift_table"].reshape(-1, 6 * w)[l]
        return f32(mod).reshape(6, w) + f32(tab).reshape(6, w)

    def patch(self, latent):         # ggml_conv_2d(2x2, stride 2): im2col (ic, kh, kw) + GEMM + bias
        c = CFG
        Z, gh, gw = c["z_dim"], c["grid_h"], c["grid_w"]
        lat = latent.reshape(Z, 2 * gh, 2 * gw)
        cols = np.stack([lat[:, 2 * y:2 * y + 2, 2 * x:2 * x + 2].reshape(-1) for y in range(gh) for x in range(gw)])
        return self.lin("gwp.patch_embedding", self.orc.f32_to_bf16(cols), self.d)

    def grid_positions(self):
        c = CFG
        gh, gw = c["grid_h"], c["grid_w"]
        return (np.zeros(gh * gw, np.int32), np.repeat(np.arange(gh, dtype=np.int32), gw),
                np.tile(np.arange(gw, dtype=np.int32), gh))


def layer_weights(w, prefix):
    n = len(prefix) + 1
    return {k[n:]: v for k, v in w.items() if k.startswith(prefix + ".")}


# --- tests ---------------------------------------------------------------------
def test_zero_velocity_keeps_the_noise(orc, base):
    w = dict(base)
    for k in ("gwp.action_decoder.out_proj.weight", "gwp.action_decoder.out_proj.bias"):
        w[k] = np.zeros_like(w[k])
    ins = inputs(orc)
    out = run(orc, w, ins).denoise(ins[3])
    assert np.array_equal(out, f32(orc.f32_to_bf16(ins[3])))


def test_constant_velocity_follows_the_scheduler(orc, base):
    w = dict(base)
    w["gwp.action_decoder.out_proj.weight"] = np.zeros_like(w["gwp.action_decoder.out_proj.weight"])
    w["gwp.action_decoder.out_proj.bias"] = orc.f32_to_bf16(np.full(CFG["action_dim"], 0.8125, np.float32))
    ins = inputs(orc)
    out = run(orc, w, ins).denoise(ins[3])
    _, sig = orc.flow_schedule(CFG["num_steps"], CFG["shift"])
    a = f32(orc.f32_to_bf16(ins[3]))
    for s in range(CFG["num_steps"]):
        dt = np.float32(sig[s + 1] - sig[s])
        a = f32(orc.f32_to_bf16((a + (np.float32(0.8125) * dt).astype(np.float32)).astype(np.float32)))
    assert np.array_equal(out, a)
    assert not np.array_equal(out, f32(orc.f32_to_bf16(ins[3])))


def test_identity_blocks_leave_encoder_to_decoder(orc, base):
    """Gates (modulation rows 2 and 5 of time_proj and of every layer's table)
    and the cross-attention output projection zeroed: hidden after the blocks
    is the action encoder's output."""
    c, w = CFG, dict(base)
    da, L = c["action_hidden"], c["n_layers"]
    tp_w = w["gwp.action_condition_embedder.time_proj.weight"].reshape(6 * da, da).copy()
    tp_b = w["gwp.action_condition_embedder.time_proj.bias"].copy()
    tab = w["gwp.blocks.action_expert.scale_shift_table"].reshape(L, 6, da).copy()
    for r in (2, 5):
        tp_w[r * da:(r + 1) * da] = 0
        tp_b[r * da:(r + 1) * da] = 0
        tab[:, r] = 0
    w["gwp.action_condition_embedder.time_proj.weight"] = tp_w.reshape(-1)
    w["gwp.action_condition_embedder.time_proj.bias"] = tp_b
    w["gwp.blocks.action_expert.scale_shift_table"] = tab.reshape(-1)
    for l in range(L):
        for s in ("weight", "bias"):
            k = f"gwp.blocks.{l}.action_expert.attn2.to_out.0.{s}"
            w[k] = np.zeros_like(w[k])
    ins = inputs(orc)
    out = run(orc, w, ins).denoise(ins[3])

    ops = Ops(orc, w)
    ts, sig = orc.flow_schedule(c["num_steps"], c["shift"])
    sst = f32(w["gwp.action_scale_shift_table"]).reshape(2, da)
    a = orc.f32_to_bf16(ins[3]).reshape(c["action_chunk"], c["action_dim"])
    for s in range(c["num_steps"]):
        h = ops.mlp3("gwp.action_encoder", a, da)
        temb, _ = ops.condition("gwp.action_condition_embedder", orc.timestep_embedding(float(ts[s])), da)
        om = sst + f32(temb)                 # row 0 shift, row 1 scale (mot.cpp:468-486)
        n = orc.norm_mod_bf16(h, om[1], om[0], EPS)
        v = ops.mlp3("gwp.action_decoder", n, c["action_dim"])
        dt = np.float32(sig[s + 1] - sig[s])
        a = orc.f32_to_bf16((f32(a) + (f32(v) * dt).astype(np.float32)).astype(np.float32))
    assert np.array_equal(out.reshape(a.shape), f32(a))


def test_prefix_inputs_and_layer0_kv(orc, base):
    c, w = CFG, base
    ins = inputs(orc)
    state, latent, prompt, _ = ins
    g = run(orc, w, ins)
    ops = Ops(orc, w)
    d, da, H, dh = ops.d, c["action_hidden"], c["n_heads"], c["head_dim"]
    nimg, P = c["grid_h"] * c["grid_w"], 1 + c["grid_h"] * c["grid_w"]
    sh = ops.mlp3("gwp.state_encoder", state[None], da)
    vh = ops.patch(latent)
    assert np.array_equal(g.prefix_hidden_in(0), sh)
    assert np.array_equal(g.prefix_hidden_in(1), vh)
    freq0 = orc.timestep_embedding(0.0)
    _, smod = ops.condition("gwp.action_condition_embedder", freq0, da)
    _, vmod = ops.condition("gwp.condition_embedder", freq0, d)
    am, vm = ops.mods("action_expert", 0, smod, da), ops.mods("visual_expert", 0, vmod, d)
    sqkv = ops.lin("gwp.blocks.0.action_expert.attn1.to_qkv", orc.norm_mod_bf16(sh, am[1], am[0], EPS), 3 * d)
    vqkv = ops.lin("gwp.blocks.0.visual_expert.attn1.to_qkv", orc.norm_mod_bf16(vh, vm[1], vm[0], EPS), 3 * d)
    K = np.zeros((H, P, dh), np.uint16)
    orc.qk_norm_rope(sqkv[:, d:2 * d], w["gwp.blocks.0.action_expert.attn1.norm_k.weight"], H, dh, 0,
                     pos0=np.zeros(1, np.int32), eps=EPS, dst=K, tok0=0)
    t, hh, ww = ops.grid_positions()
    orc.qk_norm_rope(vqkv[:, d:2 * d], w["gwp.blocks.0.visual_expert.attn1.norm_k.weight"], H, dh, 1, pos0=t,
                     pos1=hh, pos2=ww, eps=EPS, dst=K, tok0=1)
    Vt = np.concatenate([sqkv[:, 2 * d:], vqkv[:, 2 * d:]]).reshape(P, H, dh).transpose(1, 2, 0)
    assert np.array_equal(g.prefix_key(0), K)
    assert np.array_equal(g.prefix_value(0), Vt)


@pytest.mark.parametrize("ic,y,x", [(0, 0, 0), (3, 1, 0), (7, 2, 5), (15, 7, 15)])
def test_patch_embedding_column_order(orc, base, ic, y, x):
    """A single 1 at latent (ic, y, x) selects weight column
    ic*4 + (y%2)*2 + (x%2) of patch token (y//2, x//2) (conv2d over the
    PyTorch weight [OC][IC][KH][KW]); every other token is the bias."""
    c = CFG
    state, latent, prompt, noise = inputs(orc)
    lat = np.zeros_like(latent).reshape(c["z_dim"], 2 * c["grid_h"], 2 * c["grid_w"])
    lat[ic, y, x] = 1.0
    g = run(orc, base, (state, lat.reshape(-1), prompt, noise))
    vh = g.prefix_hidden_in(1)
    d = c["n_heads"] * c["head_dim"]
    wcol = base["gwp.patch_embedding.weight"].reshape(d, c["z_dim"] * 4)[:, ic * 4 + (y % 2) * 2 + (x % 2)]
    b = base["gwp.patch_embedding.bias"]
    tok = (y // 2) * c["grid_w"] + x // 2
    assert np.array_equal(vh[tok], orc.f32_to_bf16(f32(wcol) + f32(b)))
    others = np.delete(vh, tok, axis=0)
    assert np.array_equal(others, np.broadcast_to(b, others.shape))


def test_visual_permutation_permutes_prefix_kv(orc, base):
    c = CFG
    gh, gw, Z = c["grid_h"], c["grid_w"], c["z_dim"]
    nimg = gh * gw
    ins = inputs(orc)
    state, latent, prompt, noise = ins
    ops = Ops(orc, base)
    t, hh, ww = ops.grid_positions()
    g0 = run(orc, base, ins)
    perm = np.random.default_rng(5).permutation(nimg)
    lat = latent.reshape(Z, gh, 2, gw, 2).transpose(1, 3, 0, 2, 4).reshape(nimg, Z, 2, 2)
    # token i of the new latent grid holds the patch of token perm[i]
    lat2 = lat[perm].reshape(gh, gw, Z, 2, 2).transpose(2, 0, 3, 1, 4).reshape(-1)
    g1 = run(orc, base, (state, lat2, prompt, noise), positions=(t[perm], hh[perm], ww[perm]))
    rows = np.concatenate([[0], 1 + perm])
    for l in range(c["n_layers"]):
        k0, k1 = f32(g0.prefix_key(l)), f32(g1.prefix_key(l))
        v0, v1 = f32(g0.prefix_value(l)), f32(g1.prefix_value(l))
        if l == 0:      # no attention before layer 0's K/V: exact
            assert np.array_equal(k1, k0[:, rows]) and np.array_equal(v1, v0[:, :, rows])
        else:           # key order changes only the f64 summation order of layer 0's attention
            for a, b in ((k1, k0[:, rows]), (v1, v0[:, :, rows])):
                diff = np.abs(a - b) > 1e-2 * np.abs(b) + 1e-6
                assert diff.mean() < 1e-3
    # the action chunk does not depend on the key order either
    assert np.allclose(g1.denoise(noise), g0.denoise(noise), rtol=0, atol=2e-2)


def test_prompt_kv_composition(orc, base):
    c = CFG
    ins = inputs(orc)
    g = run(orc, base, ins)
    ops = Ops(orc, base)
    d, da, H, dh, NL = ops.d, c["action_hidden"], c["n_heads"], c["head_dim"], c["n_lang"]
    prompt = ins[2].reshape(NL, c["t5_hidden"])
    txt = ops.text("gwp.action_condition_embedder", prompt, da)
    assert np.array_equal(g.action_prompt(), txt)
    for l in range(c["n_layers"]):
        p = f"gwp.blocks.{l}.action_expert.attn2"
        k = ops.lin(p + ".to_k", txt, d)
        v = ops.lin(p + ".to_v", txt, d)
        K = orc.qk_norm_rope(k, base[p + ".norm_k.weight"], H, dh, 2, eps=EPS)
        assert np.array_equal(g.prompt_key(l), K)
        assert np.array_equal(g.prompt_value(l), v.reshape(NL, H, dh).transpose(1, 2, 0))


def test_one_denoise_step_composition(orc, base):
    c = CFG
    ins = inputs(orc)
    g = run(orc, base, ins)
    out = g.denoise(ins[3], layers=1, steps=1)
    ops = Ops(orc, base)
    d, da, H, dh, T, A = ops.d, c["action_hidden"], c["n_heads"], c["head_dim"], c["action_chunk"], c["action_dim"]
    ts, sig = orc.flow_schedule(c["num_steps"], c["shift"])
    a = orc.f32_to_bf16(ins[3]).reshape(T, A)
    h = ops.mlp3("gwp.action_encoder", a, da)
    temb, mod = ops.condition("gwp.action_condition_embedder", orc.timestep_embedding(float(ts[0])), da)
    table = base["gwp.blocks.action_expert.scale_shift_table"].reshape(-1, 6 * da)[0]
    F = c["action_ffn_dim"]
    Wm = layer_weights(base, "gwp.blocks.0.action_expert")
    for k, shape in (("attn1.to_qkv.weight", (3 * d, da)), ("attn1.to_out.0.weight", (da, d)),
                     ("attn2.to_q.weight", (d, da)), ("attn2.to_out.0.weight", (da, d)),
                     ("ffn.net.0.proj.weight", (F, da)), ("ffn.net.2.weight", (da, F))):
        Wm[k] = Wm[k].reshape(shape)
    apos = np.arange(1, T + 1, dtype=np.int32)
    h = oracle_action_layer(orc, Wm, h, mod.reshape(6, da), table.reshape(6, da), apos, g.prefix_key(0),
                            g.prefix_value(0), g.prompt_key(0), g.prompt_value(0), d, H, T)
    om = f32(base["gwp.action_scale_shift_table"]).reshape(2, da) + f32(temb)
    v = ops.mlp3("gwp.action_decoder", orc.norm_mod_bf16(h, om[1], om[0], EPS), A)
    dt = np.float32(sig[1] - sig[0])
    a = orc.f32_to_bf16((f32(a) + (f32(v) * dt).astype(np.float32)).astype(np.float32))
    assert np.array_equal(out.reshape(T, A), f32(a))


def test_prefix_layer1_key_through_a_whole_block(orc, base):
    """Layer 1's prefix K from the composition of a whole layer-0 block:
    joint self-attention over [state, visual], the state's cross-attention over
    the cached prompt K/V, the visual tokens' over the uncached text with f32
    Q.K (build_attention, text_encoder.cpp:26-73), gated residuals and both
    FFNs (cache.cpp:242-345, mot.cpp:284-347)."""
    c = CFG
    ins = inputs(orc)
    state, latent, prompt, _ = ins
    g = run(orc, base, ins)
    ops = Ops(orc, base)
    d, da, H, dh, NL = ops.d, c["action_hidden"], c["n_heads"], c["head_dim"], c["n_lang"]
    nimg, P = c["grid_h"] * c["grid_w"], 1 + c["grid_h"] * c["grid_w"]
    A0, V0 = "gwp.blocks.0.action_expert", "gwp.blocks.0.visual_expert"
    sh, vh = ops.mlp3("gwp.state_encoder", state[None], da), ops.patch(latent)
    freq0 = orc.timestep_embedding(0.0)
    _, smod = ops.condition("gwp.action_condition_embedder", freq0, da)
    _, vmod = ops.condition("gwp.condition_embedder", freq0, d)
    am, vm = ops.mods("action_expert", 0, smod, da), ops.mods("visual_expert", 0, vmod, d)
    sqkv = ops.lin(A0 + ".attn1.to_qkv", orc.norm_mod_bf16(sh, am[1], am[0], EPS), 3 * d)
    vqkv = ops.lin(V0 + ".attn1.to_qkv", orc.norm_mod_bf16(vh, vm[1], vm[0], EPS), 3 * d)
    t, hh, ww = ops.grid_positions()
    Q = np.zeros((H, P, dh), np.uint16)
    orc.qk_norm_rope(sqkv[:, :d], base[A0 + ".attn1.norm_q.weight"], H, dh, 0, pos0=np.zeros(1, np.int32), eps=EPS,
                     dst=Q, tok0=0)
    orc.qk_norm_rope(vqkv[:, :d], base[V0 + ".attn1.norm_q.weight"], H, dh, 1, pos0=t, pos1=hh, pos2=ww, eps=EPS,
                     dst=Q, tok0=1)
    att = orc.attention(Q, g.prefix_key(0), g.prefix_value(0))
    sh = ops.lin(A0 + ".attn1.to_out.0", att[:1], da, orc.EPI_BIAS_GATED, sh, am[2])
    vh = ops.lin(V0 + ".attn1.to_out.0", att[1:], d, orc.EPI_BIAS_GATED, vh, vm[2])

    def ffn(p, h, m, width, F):
        n = orc.norm_mod_bf16(h, m[4], m[3], EPS)
        u = ops.lin(p + ".ffn.net.0.proj", n, F, orc.EPI_BIAS_GELU)
        return ops.lin(p + ".ffn.net.2", u, width, orc.EPI_BIAS_GATED, h, m[5])

    # state: cross-attention over the cached prompt K/V of layer 0
    n = orc.layer_norm_bf16(sh, base[A0 + ".norm2.weight"], base[A0 + ".norm2.bias"], EPS)
    q = orc.qk_norm_rope(ops.lin(A0 + ".attn2.to_q", n, d), base[A0 + ".attn2.norm_q.weight"], H, dh, 2, eps=EPS)
    sh = ops.lin(A0 + ".attn2.to_out.0", orc.attention(q, g.prompt_key(0), g.prompt_value(0)), da,
                 orc.EPI_BIAS_RESIDUAL, sh)
    sh = ffn(A0, sh, am, da, c["action_ffn_dim"])
    # visual: cross-attention over the uncached text, f32 Q and K
    vtext = ops.text("gwp.condition_embedder", prompt.reshape(NL, c["t5_hidden"]), d)
    n = orc.layer_norm_bf16(vh, base[V0 + ".norm2.weight"], base[V0 + ".norm2.bias"], EPS)
    qf = orc.rms_norm_bf16_f32(ops.lin(V0 + ".attn2.to_q", n, d), base[V0 + ".attn2.norm_q.weight"], EPS)
    kf = orc.rms_norm_bf16_f32(ops.lin(V0 + ".attn2.to_k", vtext, d), base[V0 + ".attn2.norm_k.weight"], EPS)
    vv = f32(ops.lin(V0 + ".attn2.to_v", vtext, d)).astype(np.float64)
    out = np.zeros((nimg, d), np.float32)
    for hd in range(H):
        sl = slice(hd * dh, (hd + 1) * dh)
        s = (qf[:, sl].astype(np.float64) @ kf[:, sl].astype(np.float64).T).astype(np.float32) / np.sqrt(dh)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p = f32(orc.f32_to_bf16((p / p.sum(axis=1, keepdims=True)).astype(np.float32))).astype(np.float64)
        out[:, sl] = p @ vv[:, sl]
    vh = ops.lin(V0 + ".attn2.to_out.0", orc.f32_to_bf16(out), d, orc.EPI_BIAS_RESIDUAL, vh)
    vh = ffn(V0, vh, vm, d, c["ffn_dim"])
    # layer 1's K
    A1, V1 = "gwp.blocks.1.action_expert", "gwp.blocks.1.visual_expert"
    am1, vm1 = ops.mods("action_expert", 1, smod, da), ops.mods("visual_expert", 1, vmod, d)
    sqkv = ops.lin(A1 + ".attn1.to_qkv", orc.norm_mod_bf16(sh, am1[1], am1[0], EPS), 3 * d)
    vqkv = ops.lin(V1 + ".attn1.to_qkv", orc.norm_mod_bf16(vh, vm1[1], vm1[0], EPS), 3 * d)
    K = np.zeros((H, P, dh), np.uint16)
    orc.qk_norm_rope(sqkv[:, d:2 * d], base[A1 + ".attn1.norm_k.weight"], H, dh, 0, pos0=np.zeros(1, np.int32),
                     eps=EPS, dst=K, tok0=0)
    orc.qk_norm_rope(vqkv[:, d:2 * d], base[V1 + ".attn1.norm_k.weight"], H, dh, 1, pos0=t, pos1=hh, pos2=ww,
                     eps=EPS, dst=K, tok0=1)
    got, ref = f32(g.prefix_key(1)).astype(np.float64), f32(K).astype(np.float64)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= 1e-2
    assert (got.ravel() @ ref.ravel()) / (np.linalg.norm(got) * np.linalg.norm(ref)) >= 0.99999
    assert np.mean(got != ref) < 0.02


def test_small_parity_weights_are_input_sensitive(orc):
    """The small-geometry GPU parity tests compare velocities under the
    velocity bar (cosine >= 0.9999, max-rel <= 3e-2).  That comparison only
    binds the inputs if each input moves the velocity past the bar: at the
    synthetic weight std those tests use (0.05), changing the latent, the
    prompt or the noise must fail it at every step.  The state token (1 of 33
    prefix keys) moves the velocity past the per-op bar (1e-2) only; the GPU
    tests pin it through the prefix K/V (its row 0 of every layer) at the
    per-op bar.  At std 0.02 the 32-wide encoder and decoder MLPs squash the
    inputs: the velocity moves by under 1e-2."""
    from conftest import COS_TOL, REL_TOL, cosine, rel_err
    from test_gpu_gwp import SMALL, SMALL_WSTD, VEL_REL_TOL
    from test_gpu_gwp import inputs as gwp_inputs
    w = orc.gwp_synthetic_weights(SMALL, 0x5EED0003, SMALL_WSTD)

    def velocities(ins):
        g = orc.Gwp(SMALL, w)
        state, latent, prompt, noise = ins
        g.prompt(prompt)
        g.prefix(state, latent, prompt)
        g.denoise(noise)
        return [g.velocity(s) for s in range(SMALL["num_steps"])]

    base_in = gwp_inputs(SMALL, 7)
    v0 = velocities(base_in)
    for k, name in enumerate(("state", "latent", "prompt", "noise")):
        ins = list(base_in)
        ins[k] = gwp_inputs(SMALL, 30 + k)[k]
        v1 = velocities(ins)
        bar = REL_TOL if name == "state" else VEL_REL_TOL
        for s in range(SMALL["num_steps"]):
            r, c = rel_err(v1[s], v0[s]), cosine(v1[s], v0[s])
            assert r > bar or c < COS_TOL, f"{name} step {s}: rel {r:.2e} cos {c:.6f} passes the bar"
