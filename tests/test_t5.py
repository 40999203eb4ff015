"""The UMT5 encoder's host pieces and its oracle, on the CPU.

* The relative-position bucket (text_encoder.cpp:13-24) of libwamx equals the
  oracle's over [-300, 300] and is pinned by its closed form: exact buckets
  below 8, 8 + 2j at distance 8 * 2^j (j = 0..3), 15 from 128 on, the upper
  half for keys after the query.
* The oracle's vectorised bf16 rounding equals orc_f32_to_bf16.
* The oracle encoder (oracle.t5_encode, run_t5 of text_encoder.cpp:112-204)
  is pinned by properties a misreading would fail:
    - zero attention and FFN output projections make every block the
      identity: the output is the final RMSNorm of the embedding rows;
    - a constant added to every relative-bias entry changes nothing
      (softmax invariance: the bias is a pre-softmax mask);
    - the scores are not scaled (scale 1, text_encoder.cpp:174-177): a
      score margin of about 40 is one-hot at scale 1 and would leak
      e^(-40/8) of the other key at 1/sqrt(64);
    - the bias direction: with the upper-half buckets (key after query)
      raised, query 0 attends only to later keys, in equal shares.
"""
from __future__ import annotations

import numpy as np
import pytest


@pytest.fixture(scope="module")
def lib(wx):
    return wx.load()


def test_bucket_matches_oracle_and_closed_form(lib, orc):
    for r in range(-300, 301):
        assert lib.wamx_t5_relative_bucket(r, 32, 128) == orc.t5_relative_bucket(r), r
    b = orc.t5_relative_bucket
    for d in range(8):
        assert b(d) == (16 + d if d > 0 else 0) and b(-d) == d
    for j in range(4):
        assert b(8 << j) == 16 + 8 + 2 * j and b(-(8 << j)) == 8 + 2 * j
    for d in (128, 129, 500, 10**6):
        assert b(d) == 31 and b(-d) == 15
    assert lib.wamx_t5_relative_bucket(5, 2, 128) == -1


def test_vectorised_bf16_rounding(orc):
    orc.load()
    rng = np.random.default_rng(5)
    x = np.concatenate([(rng.standard_normal(4000) * 10.0 ** rng.integers(-30, 30, 4000)).astype(np.float32),
                        np.array([np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-42, 3.3e38, 1.00390625, 1.01171875],
                                 np.float32)])
    assert np.array_equal(orc.bf16_rne(x), orc.f32_to_bf16(x))


CFG = dict(vocab=40, hidden=64, ffn_dim=96, heads=2, head_dim=32, layers=2, max_tokens=12)


def weights(orc, cfg, rng, std=0.05):
    out = {}
    for name, ne in orc.t5_weight_specs(cfg):
        n = int(np.prod(ne))
        a = rng.standard_normal(n) * std
        if name.endswith("layer_norm.weight"):
            a = 1.0 + a
        if name == "t5.shared.weight":
            a = rng.standard_normal(n)
        out[name] = orc.bf16_rne(a.astype(np.float32))
    return out


def test_identity_blocks(orc):
    rng = np.random.default_rng(1)
    w = weights(orc, CFG, rng)
    for l in range(CFG["layers"]):
        p = f"t5.encoder.block.{l}.layer"
        w[p + ".0.SelfAttention.o.weight"][:] = 0
        w[p + ".1.DenseReluDense.wo.weight"][:] = 0
    tokens = [3, 17, 5, 39, 0, 8, 8]
    y = orc.t5_encode(CFG, w, tokens)
    E = orc._bf(w["t5.shared.weight"]).reshape(CFG["vocab"], CFG["hidden"])[tokens]
    wf = orc._bf(w["t5.encoder.final_layer_norm.weight"])
    want = E / np.sqrt(np.mean(E * E, axis=1, keepdims=True) + 1e-6) * wf
    assert np.allclose(y[:len(tokens)], want, rtol=0, atol=1e-12)
    assert not y[len(tokens):].any()


def test_bias_offset_invariance_and_mask_prefix(orc):
    rng = np.random.default_rng(2)
    w = weights(orc, CFG, rng)
    w2 = dict(w)
    for l in range(CFG["layers"]):
        k = f"t5.encoder.block.{l}.layer.0.SelfAttention.relative_attention_bias.weight"
        grid = np.round(rng.uniform(-1, 1, w[k].size) * 16) / 16     # 1/16 steps: +2 stays exact in bf16
        w[k] = orc.bf16_rne(grid.astype(np.float32))
        w2[k] = orc.bf16_rne((grid + 2.0).astype(np.float32))
        assert np.array_equal(orc._bf(w2[k]) - orc._bf(w[k]), np.full(w[k].size, 2.0))
    tokens = rng.integers(0, CFG["vocab"], 10)
    y = orc.t5_encode(CFG, w, tokens)
    assert np.allclose(orc.t5_encode(CFG, w2, tokens), y, rtol=0, atol=1e-12)
    # a mask keeps only the valid prefix: the same as encoding the prefix alone
    mask = np.array([1] * 6 + [0] * 4)
    assert np.allclose(orc.t5_encode(CFG, w, tokens, mask), orc.t5_encode(CFG, w, tokens[:6]), atol=0)


def _probe(orc, wq_scale, bias_upper):
    """One layer, one head of 64 dims; token i's embedding is 8 e_i; V = O = I;
    Q = K = wq_scale I; FFN output 0; bias_upper added to the buckets of keys
    after the query."""
    c = dict(vocab=8, hidden=64, ffn_dim=8, heads=1, head_dim=64, layers=1, max_tokens=8)
    w = {name: np.zeros(int(np.prod(ne)), np.uint16) for name, ne in orc.t5_weight_specs(c)}
    eye = orc.bf16_rne(np.eye(64, dtype=np.float32)).ravel()
    emb = np.zeros((8, 64), np.float32)
    emb[np.arange(8), np.arange(8)] = 8.0
    w["t5.shared.weight"] = orc.bf16_rne(emb).ravel()
    a = "t5.encoder.block.0.layer.0.SelfAttention"
    w[a + ".q.weight"] = w[a + ".k.weight"] = orc.bf16_rne(np.eye(64, dtype=np.float32) * wq_scale).ravel()
    w[a + ".v.weight"] = w[a + ".o.weight"] = eye
    bias = np.zeros((32, 1), np.float32)
    bias[17:, 0] = bias_upper       # upper half = key after the query; bucket 16 is never used
    w[a + ".relative_attention_bias.weight"] = orc.bf16_rne(bias).ravel()
    for k in ("t5.encoder.block.0.layer.0.layer_norm.weight", "t5.encoder.block.0.layer.1.layer_norm.weight",
              "t5.encoder.final_layer_norm.weight"):
        w[k] = orc.bf16_rne(np.ones(64, np.float32))
    return c, w


def test_scores_are_not_scaled(orc):
    # x_i = rmsnorm(8 e_i) = 8 e_i (1 / sqrt(1 + eps)); q.k = 64 s^2 for the same token, 0 otherwise.
    c, w = _probe(orc, 0.7890625, 0.0)          # 64 * 0.789^2 ~ 39.8
    y = orc.t5_encode(c, w, [0, 1])
    # token 0 attends to itself only: y_0 is a multiple of e_0 (the leak at
    # scale 1/8 would put ~e^-5 of e_1 into it)
    assert y[0, 0] > 1.0 and abs(y[0, 1]) < 1e-12 and abs(y[1, 0]) < 1e-12


def test_bias_direction(orc):
    # zero Q/K scores, +60 on keys after the query: query 0 of 4 attends to
    # keys 1, 2, 3 in equal shares and not to itself.
    c, w = _probe(orc, 0.0, 60.0)
    y = orc.t5_encode(c, w, [0, 1, 2, 3])
    assert y[0, 1] > 0 and np.allclose(y[0, 1:4], y[0, 1], rtol=1e-12)
    x = 8.0 / np.sqrt(1.0 + 1e-6)                     # rmsnorm(8 e_i)
    v = orc._bf(orc.bf16_rne(np.float32(x)))[()]      # V's bf16 input: 8
    att = orc._bf(orc.bf16_rne(np.float32(v / 3.0)))[()]  # the attention output, rounded for the O MUL_MAT
    assert np.isclose(y[0, 0] / y[0, 1], 8.0 / att, rtol=1e-9)
    # the last query has no later key: uniform over all four
    assert np.allclose(y[3, 0:3], y[3, 0], rtol=1e-12)
