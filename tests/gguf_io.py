"""A minimal GGUF v3 writer for test artifacts, from the published container
layout (u32 magic "GGUF", u32 version, u64 tensor count, u64 key/value count,
the key/values, the tensor descriptors, padding to general.alignment, the
tensor data).  Used to build GWP-0.5 artifacts in the reference's layout for
the loader tests; the reference's own converter writes through the gguf
Python package (scripts/convert/convert_gwp05.py), which is not installed.

Also: `gwp_artifact`, which lays a synthetic GWP-0.5 weight set (this model's
names and layout, as oracle.gwp_synthetic_weights returns it) out the way the
reference's converter stores it.
"""
from __future__ import annotations

import struct
from pathlib import Path

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
           I64: "<q", F64: "<d"}
GGML_F32, GGML_F16, GGML_BF16 = 0, 1, 30


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


class GgufWriter:
    def __init__(self, alignment: int = 32, version: int = 3):
        self.alignment, self.version = alignment, version
        self.kv: list[tuple[str, int, object, int | None]] = []
        self.tensors: list[tuple[str, int, tuple[int, ...], bytes]] = []

    def add(self, key: str, vtype: int, value, elem_type: int | None = None):
        self.kv.append((key, vtype, value, elem_type))
        return self

    def u32(self, key, v): return self.add(key, U32, int(v))
    def u64(self, key, v): return self.add(key, U64, int(v))
    def f32(self, key, v): return self.add(key, F32, float(v))
    def string(self, key, v): return self.add(key, STR, str(v))
    def array(self, key, elem_type, values): return self.add(key, ARR, list(values), elem_type)

    def tensor(self, name: str, data: np.ndarray, ggml_type: int, ne: tuple[int, ...]):
        """ne in ggml order (ne[0] contiguous); data holds prod(ne) elements."""
        assert int(np.prod(ne)) == data.size, (name, ne, data.size)
        self.tensors.append((name, ggml_type, tuple(int(x) for x in ne), np.ascontiguousarray(data).tobytes()))
        return self

    def _value(self, vtype, value, elem_type) -> bytes:
        if vtype == STR:
            return _str(value)
        if vtype == ARR:
            out = struct.pack("<IQ", elem_type, len(value))
            for v in value:
                out += self._value(elem_type, v, None)
            return out
        return struct.pack(_SCALAR[vtype], value)

    def to_bytes(self) -> bytes:
        kv = list(self.kv)
        if self.alignment != 32:
            kv.append(("general.alignment", U32, self.alignment, None))
        head = b"GGUF" + struct.pack("<IQQ", self.version, len(self.tensors), len(kv))
        for key, vtype, value, et in kv:
            head += _str(key) + struct.pack("<I", vtype) + self._value(vtype, value, et)
        offsets, off = [], 0
        for _, _, _, payload in self.tensors:
            offsets.append(off)
            off += -(-len(payload) // self.alignment) * self.alignment
        for (name, gtype, ne, _), o in zip(self.tensors, offsets):
            head += _str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne)
            head += struct.pack("<IQ", gtype, o)
        head += b"\0" * (-len(head) % self.alignment)
        body = b""
        for (_, _, _, payload), o in zip(self.tensors, offsets):
            body += b"\0" * (o - len(body)) + payload
        return head + body

    def write(self, path: Path) -> Path:
        Path(path).write_bytes(self.to_bytes())
        return Path(path)


# ---------------------------------------------------------------------------
# GWP-0.5 artifacts in the reference's layout.
# ---------------------------------------------------------------------------
def compact_name(name: str) -> str:
    """The GGUF tensor-name ABI for the gwp component (convert_gwp05.py:57-90),
    restated for the test writer."""
    reps = (("action_condition_embedder.", "acond."), ("condition_embedder.", "cond."),
            ("patch_embedding.", "patch."), ("state_encoder.", "state."), ("action_encoder.", "action."),
            ("action_decoder.", "decode."), ("blocks.", "blk."), (".action_expert.", ".a."),
            (".visual_expert.", ".v."), ("time_embedder.linear_1.", "time.0."),
            ("time_embedder.linear_2.", "time.1."), ("text_embedder.linear_1.", "text.0."),
            ("text_embedder.linear_2.", "text.1."), ("time_proj.", "time.out."), (".ffn.net.0.proj.", ".ffn.in."),
            (".ffn.net.2.", ".ffn.out."), (".attn1.", ".sa."), (".attn2.", ".ca."), (".to_out.0.", ".o."),
            (".to_qkv.", ".qkv."), (".to_q.", ".q."), (".to_k.", ".k."), (".to_v.", ".vproj."),
            (".norm_q.", ".qn."), (".norm_k.", ".kn."), (".norm2.", ".ca_norm."), ("in_proj.", "in."),
            ("mid_proj.", "mid."), ("out_proj.", "out."), ("scale_shift_table", "mod"))
    comp, rest = name.split(".", 1)
    assert comp == "gwp"
    for a, b in reps:
        rest = rest.replace(a, b)
    return comp + "." + rest


CATEGORY = ("gwp.state_encoder.in_proj", "gwp.action_encoder.in_proj", "gwp.action_decoder.out_proj")


def geometry_keys(w: GgufWriter, cfg: dict, policy: str, num_embodiments: int, embodiment_id: int, **over):
    """The gwp05.* metadata the reference's inspect_artifact reads
    (artifact.cpp:20-56, 232-268) for a model of config `cfg`."""
    keys = {
        "hidden": cfg["n_heads"] * cfg["head_dim"], "n_layers": cfg["n_layers"], "n_heads": cfg["n_heads"],
        "head_dim": cfg["head_dim"], "ffn_dim": cfg["ffn_dim"], "action_hidden": cfg["action_hidden"],
        "action_ffn_dim": cfg["action_ffn_dim"], "action_dim": cfg["action_dim"], "real_state_dim": 14,
        "real_action_dim": 14, "num_embodiments": num_embodiments, "embodiment_id": embodiment_id,
        "image_height": 32 * cfg["grid_h"], "image_width": 32 * cfg["grid_w"], "num_views": 3,
        "action_chunk": cfg["action_chunk"], "inference_steps": cfg["num_steps"], "t5_vocab_size": 256,
        "t5_hidden": cfg["t5_hidden"], "t5_ffn_dim": 128, "t5_heads": cfg["t5_hidden"] // 64 or 1,
        "t5_head_dim": 64 if cfg["t5_hidden"] >= 64 else cfg["t5_hidden"], "t5_layers": 1,
        "vae_z_dim": cfg["z_dim"],
    }
    keys.update({k: v for k, v in over.items() if k not in ("flow_shift", "norm_eps")})
    for k, v in keys.items():
        w.u32("gwp05." + k, v)
    w.f32("gwp05.flow_shift", over.get("flow_shift", cfg["shift"]))
    w.f32("gwp05.norm_eps", over.get("norm_eps", cfg["eps"]))
    w.string("gwp05.architecture", "gwp05")
    if policy:
        w.string("gwp05.conversion_policy", policy)
        w.string("gwp05.converter_revision", "gwp05-native-bf16-v1")
        w.string("gwp05.weight_policy", policy)


def gwp_artifact(cfg: dict, weights: dict, shapes: dict, *, packed_qkv: bool, num_embodiments: int = 3,
                 embodiment_id: int = 1, policy: str | None = None, seed: int = 7) -> GgufWriter:
    """weights: this model's name -> flat bf16 (uint16) array; shapes: name ->
    the model tensor's ggml ne.  Returns a writer holding the reference's
    layout: per-layer adaLN tables, category-specific projections as
    [num_embodiments][in][out] (the other embodiments' slices random), packed
    or split self-attention q / k / v, plus T5 / VAE / statistic tensors the
    MoT loader must skip."""
    rng = np.random.default_rng(seed)
    policy = policy or ("mot-vae-bf16-qkv-v1" if packed_qkv else "mot-vae-bf16-v1")
    w = GgufWriter()
    geometry_keys(w, cfg, policy, num_embodiments, embodiment_id)
    L = cfg["n_layers"]
    junk = lambda n: rng.integers(0, 1 << 16, n, dtype=np.uint16)  # noqa: E731
    for name, a in weights.items():
        ne = tuple(shapes[name])
        if name.endswith(".scale_shift_table") and name.startswith("gwp.blocks."):
            expert = name[len("gwp.blocks."):]
            width = ne[0]
            per = a.reshape(L, 6 * width)
            for l in range(L):
                w.tensor(compact_name(f"gwp.blocks.{l}.{expert}"), per[l], GGML_BF16, (width, 6, 1))
            continue
        base = name.rsplit(".", 1)[0]
        if base in CATEGORY:
            if name.endswith(".weight"):
                n_in, n_out = ne[0], ne[1]
                t = np.stack([junk(n_in * n_out).reshape(n_in, n_out) for _ in range(num_embodiments)])
                t[embodiment_id] = a.reshape(n_out, n_in).T
                w.tensor(compact_name(name), t, GGML_BF16, (n_out, n_in, num_embodiments))
            else:
                t = np.stack([junk(ne[0]) for _ in range(num_embodiments)])
                t[embodiment_id] = a
                w.tensor(compact_name(name), t, GGML_BF16, (ne[0], num_embodiments))
            continue
        if not packed_qkv and ".attn1.to_qkv." in name:
            is_w = name.endswith(".weight")
            parts = np.split(a.reshape(-1, ne[0]) if is_w else a, 3)
            for p, part in zip(("to_q", "to_k", "to_v"), parts):
                pn = name.replace(".to_qkv.", f".{p}.")
                w.tensor(compact_name(pn), part, GGML_BF16, (ne[0], ne[1] // 3) if is_w else (ne[0] // 3,))
            continue
        w.tensor(compact_name(name), a, GGML_BF16, ne)
    # Tensors of the other components and an unused MoT output head.
    w.tensor("gwp.proj_out.weight", junk(16 * 8), GGML_BF16, (16, 8))
    w.tensor("t5.token_embd.weight", junk(64 * 8), GGML_BF16, (64, 8))
    w.tensor("vae.enc.in.weight", junk(3 * 3 * 12 * 4), GGML_BF16, (3, 3, 12, 4))
    w.tensor("state_q01", np.zeros(cfg["action_dim"], np.float32), GGML_F32, (cfg["action_dim"],))
    return w
