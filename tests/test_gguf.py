"""The GGUF reader (wamx_gguf_*, no GPU needed) and the artifact tensor-name
ABI.

* A container written by tests/gguf_io.py from the published GGUF v3 layout
  reads back: every scalar and array key type, strings, a non-default
  alignment, tensors of 1..4 dimensions and of F32 / F16 / BF16, payload
  bytes and aligned offsets.
* Corrupt or truncated files fail with a message at open (bad magic,
  unsupported version, truncated header or payload, misaligned offsets,
  duplicate keys, five dimensions), and typed getters refuse missing keys and
  other types, as the reference's GgufReader::require_* do
  (src/models/common/gguf_reader.cpp:104-227).
* The compact-name ABI maps the framework names the reference validates by
  their compact form (artifact.cpp:101-117: gwp.patch.weight,
  gwp.state.in.weight, gwp.decode.out.weight, t5.token_embd.weight,
  vae.enc.in.weight, gwp.blk.{l}.{a,v}.sa.{qkv,q}.weight) and keeps every
  weight name of the model distinct and under 64 bytes (the converter's
  collision and length checks, convert_gwp05.py:134-150).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import gguf_io as gi


@pytest.fixture(scope="module")
def lib(wx):
    return wx.load()


def opened(lib, wx, path):
    g = lib.wamx_gguf_open(str(path).encode())
    assert g, wx.last_error()
    return g


def test_round_trip(lib, wx, tmp_path):
    rng = np.random.default_rng(3)
    w = gi.GgufWriter(alignment=64)
    w.add("k.u8", gi.U8, 200).add("k.i8", gi.I8, -5).add("k.u16", gi.U16, 65000).add("k.i16", gi.I16, -300)
    w.u32("k.u32", 4000000000).add("k.i32", gi.I32, -7).f32("k.f32", 1.5).add("k.bool", gi.BOOL, True)
    w.string("k.str", "gwp05 é").u64("k.u64", 1 << 40).add("k.i64", gi.I64, -(1 << 40)).add("k.f64", gi.F64, 0.25)
    w.array("k.af32", gi.F32, [1.0, -2.0, 3.5]).array("k.af64", gi.F64, [0.5, 0.125])
    w.array("k.astr", gi.STR, ["a", "bc"]).array("k.au32", gi.U32, [1, 2, 3])
    t1 = rng.integers(0, 1 << 16, 3 * 5, dtype=np.uint16)
    t2 = rng.standard_normal(7).astype(np.float32)
    t3 = rng.integers(0, 1 << 16, 2 * 3 * 4 * 5, dtype=np.uint16)
    t4 = rng.standard_normal(9).astype(np.float16)
    w.tensor("a.bf16", t1, gi.GGML_BF16, (5, 3)).tensor("b.f32", t2, gi.GGML_F32, (7,))
    w.tensor("c.bf16.4d", t3, gi.GGML_BF16, (5, 4, 3, 2)).tensor("d.f16", t4, gi.GGML_F16, (9,))
    p = w.write(tmp_path / "rt.gguf")
    g = opened(lib, wx, p)
    try:
        assert lib.wamx_gguf_version(g) == 3
        assert lib.wamx_gguf_data_offset(g) % 64 == 0
        keys = [lib.wamx_gguf_key(g, i).decode() for i in range(lib.wamx_gguf_n_keys(g))]
        assert keys[:4] == ["k.u8", "k.i8", "k.u16", "k.i16"] and "general.alignment" in keys
        assert lib.wamx_gguf_key_type(g, b"k.f64") == gi.F64 and lib.wamx_gguf_key_type(g, b"nope") == -1
        u32, u64, f = C.c_uint32(), C.c_uint64(), C.c_float()
        wx.check(lib.wamx_gguf_get_u32(g, b"k.u32", C.byref(u32)))
        wx.check(lib.wamx_gguf_get_u64(g, b"k.u64", C.byref(u64)))
        wx.check(lib.wamx_gguf_get_f32(g, b"k.f32", C.byref(f)))
        assert (u32.value, u64.value, f.value) == (4000000000, 1 << 40, 1.5)
        assert lib.wamx_gguf_get_str(g, b"k.str").decode() == "gwp05 é"
        buf = (C.c_float * 8)()
        assert lib.wamx_gguf_get_f32_array(g, b"k.af32", buf, 8) == 3 and list(buf)[:3] == [1.0, -2.0, 3.5]
        assert lib.wamx_gguf_get_f32_array(g, b"k.af64", buf, 8) == 2 and list(buf)[:2] == [0.5, 0.125]
        assert lib.wamx_gguf_get_f32_array(g, b"k.astr", buf, 8) == -1
        # typed getters refuse other types and missing keys, with a message
        assert lib.wamx_gguf_get_u32(g, b"k.f32", C.byref(u32)) != 0 and "type" in wx.last_error()
        assert lib.wamx_gguf_get_u32(g, b"missing.key", C.byref(u32)) != 0 and "missing.key" in wx.last_error()
        assert lib.wamx_gguf_get_str(g, b"k.u32") is None
        assert lib.wamx_gguf_n_tensors(g) == 4 and lib.wamx_gguf_find_tensor(g, b"zz") == -1
        for name, arr, gtype, ne in (("a.bf16", t1, 30, (5, 3)), ("b.f32", t2, 0, (7,)),
                                     ("c.bf16.4d", t3, 30, (5, 4, 3, 2)), ("d.f16", t4, 1, (9,))):
            i = lib.wamx_gguf_find_tensor(g, name.encode())
            assert lib.wamx_gguf_tensor_name(g, i).decode() == name
            assert lib.wamx_gguf_tensor_type(g, i) == gtype and lib.wamx_gguf_tensor_n_dims(g, i) == len(ne)
            assert [lib.wamx_gguf_tensor_ne(g, i, k) for k in range(4)] == list(ne) + [1] * (4 - len(ne))
            assert lib.wamx_gguf_tensor_bytes(g, i) == arr.nbytes
            assert lib.wamx_gguf_tensor_offset(g, i) % 64 == 0
            out = np.empty_like(arr)
            wx.check(lib.wamx_gguf_read_tensor(g, i, out.ctypes.data, out.nbytes), name)
            assert np.array_equal(out.view(np.uint8), arr.view(np.uint8))
        assert lib.wamx_gguf_read_tensor(g, 0, out.ctypes.data, 3) != 0   # wrong byte count
    finally:
        lib.wamx_gguf_close(g)


def _base() -> bytes:
    w = gi.GgufWriter().u32("x", 1)
    w.tensor("t", np.arange(64, dtype=np.uint16), gi.GGML_BF16, (64,))
    return w.to_bytes()


@pytest.mark.parametrize("case", ["magic", "version", "truncated_payload", "truncated_header", "misaligned",
                                  "duplicate_key", "five_dims", "empty"])
def test_corrupt_files_are_refused(lib, wx, tmp_path, case):
    b = bytearray(_base())
    if case == "magic":
        b[0:4] = b"GGUG"
    elif case == "version":
        b[4:8] = (1).to_bytes(4, "little")
    elif case == "truncated_payload":
        b = b[:-10]
    elif case == "truncated_header":
        b = b[:30]
    elif case == "misaligned":
        w = gi.GgufWriter().u32("x", 1)
        w.tensor("t", np.arange(64, dtype=np.uint16), gi.GGML_BF16, (64,))
        raw = bytearray(w.to_bytes())
        pos = raw.index(b"t\x01\x00\x00\x00") + 5 + 8 + 4        # name, n_dims, ne[0], type -> offset
        raw[pos:pos + 8] = (3).to_bytes(8, "little")
        b = raw
    elif case == "duplicate_key":
        b = bytearray(gi.GgufWriter().u32("x", 1).u32("x", 2).to_bytes())
    elif case == "five_dims":
        w = gi.GgufWriter()
        w.tensor("t", np.arange(32, dtype=np.uint16), gi.GGML_BF16, (2, 2, 2, 2, 2))
        b = bytearray(w.to_bytes())
    elif case == "empty":
        b = bytearray()
    p = tmp_path / f"{case}.gguf"
    p.write_bytes(bytes(b))
    assert not lib.wamx_gguf_open(str(p).encode())
    why = {"magic": "bad magic", "version": "unsupported GGUF version 1", "truncated_payload": "outside the file",
           "truncated_header": "corrupt GGUF header", "misaligned": "not aligned", "duplicate_key": "duplicate GGUF key",
           "five_dims": "5 dimensions", "empty": "too short"}[case]
    assert why in wx.last_error(), (case, wx.last_error())
    assert not lib.wamx_gguf_open(str(tmp_path / "absent.gguf").encode())


def compact(lib, name: str) -> str:
    out = C.create_string_buffer(128)
    n = lib.wamx_gguf_compact_name(name.encode(), out, 128)
    assert n > 0, name
    return out.value.decode()


def test_compact_names_match_the_reference_schema(lib):
    # The compact names artifact.cpp:101-117 requires, from their framework names.
    pairs = {
        "gwp.patch_embedding.weight": "gwp.patch.weight",
        "gwp.state_encoder.in_proj.weight": "gwp.state.in.weight",
        "gwp.action_decoder.out_proj.weight": "gwp.decode.out.weight",
        "t5.shared.weight": "t5.token_embd.weight",
        "vae.encoder.conv_in.weight": "vae.enc.in.weight",
        "gwp.blocks.7.action_expert.attn1.to_qkv.weight": "gwp.blk.7.a.sa.qkv.weight",
        "gwp.blocks.12.visual_expert.attn1.to_q.weight": "gwp.blk.12.v.sa.q.weight",
        "gwp.blocks.0.action_expert.scale_shift_table": "gwp.blk.0.a.mod",
        "gwp.action_condition_embedder.time_embedder.linear_1.bias": "gwp.acond.time.0.bias",
        "gwp.blocks.3.visual_expert.attn2.to_v.weight": "gwp.blk.3.v.ca.vproj.weight",
    }
    for long_name, short in pairs.items():
        assert compact(lib, long_name) == short
        if long_name.startswith("gwp."):
            assert gi.compact_name(long_name) == short
    assert lib.wamx_gguf_compact_name(b"other.x", None, 0) == -1


def test_model_names_compact_uniquely(lib, orc):
    cfg = dict(n_layers=30, hidden=3072, n_heads=24, head_dim=128, ffn_dim=14336, action_hidden=3072,
               action_ffn_dim=14336, action_chunk=48, action_dim=32, grid_h=8, grid_w=32, n_lang=512, t5_hidden=4096,
               z_dim=48, num_steps=10, enc_hidden=128, shift=5.0, eps=1e-6)
    names = [n for n, _ in orc.gwp_weight_specs(cfg) if not n.endswith(".scale_shift_table") or "blocks." not in n]
    for x in ("action_expert", "visual_expert"):
        names += [f"gwp.blocks.{l}.{x}.scale_shift_table" for l in range(cfg["n_layers"])]
    short = [compact(lib, n) for n in names]
    assert len(set(short)) == len(short)
    assert max(len(s.encode()) for s in short) < 64
    assert short == [gi.compact_name(n) for n in names]
