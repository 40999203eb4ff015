"""The UMT5 encoder on the GPU (wamx_t5_encode) against the oracle
(oracle.t5_encode, pinned in test_t5.py), with the per-op bar (max-rel <=
1e-2, cosine >= 0.9999) on the f32 prompt embedding:

* a small encoder (2 layers, 2 x 32 heads) and one at UMT5-XXL's widths
  (d = 4096, 64 heads x 64, FFN 10240; 1 layer, a 512-token vocabulary),
  on 64 prompt tokens with and without a mask (valid prefix of 37);
* the t5.* tensors of a GGUF artifact (compact names) give the same
  embedding as the weights set by name;
* refused inputs: a mask with a hole, a token outside the vocabulary, no
  valid token, too many tokens;
* the prompt-embedding cache and the fixed-prompt policy.
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


def stats(wx, be, t):
    s = wx.PromptCacheStats()
    wx.check(be.lib.wamx_t5_prompt_cache_stats(t, C.byref(s)), "prompt_cache_stats")
    return s


def test_prompt_cache_lru_and_fixed_policy(wx, be, orc, monkeypatch):
    """The prompt-embedding LRU of the reference's engine (weights.cpp:305-317,
    :419-451; engine.cpp:306-331) and its `fixed` policy (engine.cpp:180-199,
    :290-300): hits return the encoded embedding bit for bit, the least
    recently used entry goes first, a different mask is a different prompt,
    misses count only with the cache on, weight handles empty the cache, and
    a fixed prompt refuses every other prompt."""
    print("t5 prompt cache", flush=True)
    cfg = SMALL
    lib = be.lib
    w = synth(orc, cfg, 0x5EED0B02)
    rng = np.random.default_rng(11)
    A, B, Cc = (rng.integers(0, cfg["vocab"], 64) for _ in range(3))
    half = np.array([1] * 40 + [0] * 24)
    # initial capacity from WAM_GWP05_PROMPT_CACHE_SIZE, read at creation
    for value, cap in ((None, 4), ("", 4), ("7", 7), ("0", 0), ("-1", 0), ("abc", 0), ("3x", 0)):
        if value is None:
            monkeypatch.delenv("WAM_GWP05_PROMPT_CACHE_SIZE", raising=False)
        else:
            monkeypatch.setenv("WAM_GWP05_PROMPT_CACHE_SIZE", value)
        t = make(wx, be, cfg)
        s = stats(wx, be, t)
        lib.wamx_t5_free(t)
        assert (s.capacity, s.enabled) == (cap, int(cap != 0)), value
    monkeypatch.delenv("WAM_GWP05_PROMPT_CACHE_SIZE", raising=False)

    t = make(wx, be, cfg)
    try:
        upload(wx, be, t, w)
        wx.check(lib.wamx_t5_set_prompt_cache(t, 2), "capacity 2")

        def enc(tokens, mask=None):
            st, out = encode(wx, be, t, cfg, tokens, mask)
            wx.check(st, "t5_encode")
            return out, stats(wx, be, t)

        a0, s = enc(A)
        assert (s.hits, s.misses, s.entries, s.last_hit) == (0, 1, 1, 0)
        ref = orc.t5_encode(cfg, w, A, None)
        assert_parity(a0, ref.astype(np.float32), what="t5 through the cache")
        b0, s = enc(B)
        a1, s = enc(A)                          # hit; order now A, B
        assert (s.hits, s.misses, s.entries, s.last_hit) == (1, 2, 2, 1)
        assert np.array_equal(a1, a0)
        assert s.bytes == 2 * cfg["max_tokens"] * cfg["hidden"] * 4
        _, s = enc(Cc)                          # miss; B, the oldest, goes
        assert (s.hits, s.misses, s.entries) == (1, 3, 2)
        _, s = enc(A)                           # still cached
        assert (s.hits, s.misses) == (2, 3)
        b1, s = enc(B)                          # evicted: encoded again
        assert (s.hits, s.misses, s.last_hit) == (2, 4, 0)
        assert np.array_equal(b1, b0)
        _, s = enc(A, np.ones(64, np.int32))    # the all-ones mask is the null mask
        assert (s.hits, s.misses) == (3, 4)
        h0, s = enc(A, half)                    # same tokens, another mask
        assert (s.hits, s.misses) == (3, 5) and not h0[40:].any()
        # a weight handle empties the cache
        assert lib.wamx_t5_weight(t, b"t5.shared.weight")
        assert stats(wx, be, t).entries == 0
        _, s = enc(A)
        assert (s.hits, s.misses, s.entries) == (3, 6, 1)
        # capacity 0: off, emptied, no counting
        wx.check(lib.wamx_t5_set_prompt_cache(t, 0), "capacity 0")
        _, s = enc(A)
        assert (s.enabled, s.entries, s.hits, s.misses, s.last_hit) == (0, 0, 3, 6, 0)
        # a refused request leaves the counters alone
        st, _ = encode(wx, be, t, cfg, A, np.array([1, 0, 1] + [0] * 61))
        assert st != 0 and "contiguous" in wx.last_error()

        # the fixed policy
        mk = np.ascontiguousarray(half, np.int32)
        tk = np.ascontiguousarray(A, np.int32)
        wx.check(lib.wamx_t5_fix_prompt(t, tk.ctypes.data, mk.ctypes.data, 64), "fix_prompt")
        assert not lib.wamx_t5_weight(t, b"t5.shared.weight")
        f, s = enc(A, half)
        assert s.last_hit == 1 and np.array_equal(f, h0)
        for toks, mask in ((A, None), (B, half)):
            st, _ = encode(wx, be, t, cfg, toks, mask)
            assert st != 0 and "does not match the fixed prompt" in wx.last_error()
        assert lib.wamx_t5_fix_prompt(t, tk.ctypes.data, mk.ctypes.data, 64) != 0
    finally:
        lib.wamx_t5_free(t)
