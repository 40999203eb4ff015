"""The UMT5 encoder on the GPU (wamx_t5_encode) against the oracle
(oracle.t5_encode, pinned in test_t5.py), with the per-op bar (max-rel <=
1e-2, cosine >= 0.9999) on the f32 prompt embedding:

* a small encoder (2 layers, 2 x 32 heads) and one at UMT5-XXL's widths
  (d = 4096, 64 heads x 64, FFN 10240; 1 layer, a 512-token vocabulary),
  on 64 prompt tokens with and without a mask (valid prefix of 37);
* the t5.* tensors of a GGUF artifact (compact names) give the same
  embedding as the weights set by name;
* refused inputs: a mask with a hole, a token outside the vocabulary, no
  valid token, too many tokens.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import gguf_io as gi
from conftest import assert_parity

pytestmark = pytest.mark.gpu

SMALL = dict(vocab=64, hidden=64, ffn_dim=96, heads=2, head_dim=32, layers=2, max_tokens=64)
XXL = dict(vocab=512, hidden=4096, ffn_dim=10240, heads=64, head_dim=64, layers=1, max_tokens=64)


def make(wx, be, cfg):
    t = be.lib.wamx_t5_create(be.ptr, C.byref(wx.T5Config(**cfg, eps=1e-6)))
    assert t, wx.last_error()
    return t


def synth(orc, cfg, seed):
    rng = np.random.default_rng(seed)
    out = {}
    for name, ne in orc.t5_weight_specs(cfg):
        n = int(np.prod(ne))
        if name == "t5.shared.weight":
            a = rng.standard_normal(n)
        elif name.endswith("layer_norm.weight"):
            a = 1.0 + 0.05 * rng.standard_normal(n)
        elif "relative_attention_bias" in name:
            a = rng.standard_normal(n)
        else:
            fan_in = ne[0]
            a = rng.standard_normal(n) / np.sqrt(fan_in)
        out[name] = orc.bf16_rne(a.astype(np.float32))
    return out


def upload(wx, be, t, w):
    for name, a in w.items():
        wt = be.lib.wamx_t5_weight(t, name.encode())
        assert wt, name
        wx.check(be.lib.wamx_backend_tensor_set(wt, a.ctypes.data, 0, a.nbytes), name)


def encode(wx, be, t, cfg, tokens, mask=None):
    tok = np.ascontiguousarray(tokens, np.int32)
    m = None if mask is None else np.ascontiguousarray(mask, np.int32)
    out = np.empty((cfg["max_tokens"], cfg["hidden"]), np.float32)
    st = be.lib.wamx_t5_encode(t, tok.ctypes.data, None if m is None else m.ctypes.data, tok.size, out.ctypes.data)
    return st, out


@pytest.mark.parametrize("which", ["small", "xxl_width"])
def test_encoder_matches_oracle(wx, be, orc, which):
    cfg = SMALL if which == "small" else XXL
    print(f"t5 encoder {which}", flush=True)
    w = synth(orc, cfg, 0x5EED0B00)
    t = make(wx, be, cfg)
    try:
        upload(wx, be, t, w)
        rng = np.random.default_rng(9)
        tokens = rng.integers(0, cfg["vocab"], 64)
        for mask in (None, np.array([1] * 37 + [0] * 27)):
            st, got = encode(wx, be, t, cfg, tokens, mask)
            wx.check(st, "t5_encode")
            ref = orc.t5_encode(cfg, w, tokens, mask)
            n = 64 if mask is None else 37
            assert not got[n:].any()
            assert_parity(got[:n], ref[:n].astype(np.float32), what=f"t5 {which} mask={mask is not None}")
    finally:
        be.lib.wamx_t5_free(t)


def test_encoder_from_gguf_and_refusals(wx, be, orc, tmp_path):
    print("t5 encoder from gguf", flush=True)
    cfg = SMALL
    lib = be.lib
    w = synth(orc, cfg, 0x5EED0B01)
    wr = gi.GgufWriter()
    for k, v in (("t5_vocab_size", cfg["vocab"]), ("t5_hidden", cfg["hidden"]), ("t5_ffn_dim", cfg["ffn_dim"]),
                 ("t5_heads", cfg["heads"]), ("t5_head_dim", cfg["head_dim"]), ("t5_layers", cfg["layers"])):
        wr.u32("gwp05." + k, v)
    out = C.create_string_buffer(128)
    for name, ne in orc.t5_weight_specs(cfg):
        assert lib.wamx_gguf_compact_name(name.encode(), out, 128) > 0
        wr.tensor(out.value.decode(), w[name], gi.GGML_BF16, ne)
    path = wr.write(tmp_path / "t5.gguf")
    g = lib.wamx_gguf_open(str(path).encode())
    assert g, wx.last_error()
    t1 = lib.wamx_t5_create_from_gguf(be.ptr, g)
    lib.wamx_gguf_close(g)
    assert t1, wx.last_error()
    t2 = make(wx, be, cfg)
    try:
        upload(wx, be, t2, w)
        tokens = np.arange(64) % cfg["vocab"]
        a, b = encode(wx, be, t1, cfg, tokens), encode(wx, be, t2, cfg, tokens)
        wx.check(a[0], "t5_encode (artifact)")
        wx.check(b[0], "t5_encode (by name)")
        assert np.array_equal(a[1], b[1])
        # refusals, with their messages
        for toks, mask, why in (
                (tokens, np.array([1, 0, 1] + [0] * 61), "contiguous valid prefix"),
                (np.array([cfg["vocab"]] + [0] * 63), None, "outside the vocabulary"),
                (tokens, np.zeros(64, np.int32), "no valid tokens"),
                (np.zeros(65, np.int32), None, "outside [1,64]")):
            st, _ = encode(wx, be, t2, cfg, toks, mask)
            assert st != 0 and why in wx.last_error(), (why, wx.last_error())
    finally:
        lib.wamx_t5_free(t1)
        lib.wamx_t5_free(t2)
