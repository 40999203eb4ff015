// A GWP-0.5 model from a GGUF artifact: geometry and schema checks, then the
// MoT weights made resident on the backend in the layout the model holds.
//
// The artifact addresses weights by compact names (the GGUF tensor-name ABI,
// at most 63 bytes); the engine addresses them by framework names and maps
// one to the other with a fixed list of substring replacements applied in
// order (src/models/gwp05/engine/weights.cpp:116-167, the same list as
// scripts/convert/convert_gwp05.py:57-140).  The lists below are that ABI.
//
// Layout differences between the artifact and this model, undone at load:
//   * adaLN tables: one [6][width] table per layer and expert in the artifact
//     (gwp.blk.{l}.{a,v}.mod), one packed [width, 6, L] tensor per expert
//     here (the denoise graph views layer l's slice);
//   * category-specific projections (state / action encoder in_proj, action
//     decoder out_proj): [num_embodiments][in][out] in the artifact, of which
//     the engine takes the embodiment_id slice and transposes it every graph
//     (mot.cpp:1-53); here that slice is transposed once to [out][in];
//   * self-attention q / k / v: packed [3d][w] in the qkv policy
//     (convert_gwp05.py:182-207, rows q then k then v), separate otherwise;
//     the model always holds the packed form.
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "common.h"

namespace {

struct Rep {
    const char * from;
    const char * to;
};

// The GGUF tensor-name ABI (weights.cpp:122-159; convert_gwp05.py:60-133).
const Rep kGwpNames[] = {
    {"action_condition_embedder.", "acond."}, {"condition_embedder.", "cond."},
    {"patch_embedding.", "patch."},           {"state_encoder.", "state."},
    {"action_encoder.", "action."},           {"action_decoder.", "decode."},
    {"blocks.", "blk."},                      {".action_expert.", ".a."},
    {".visual_expert.", ".v."},               {"time_embedder.linear_1.", "time.0."},
    {"time_embedder.linear_2.", "time.1."},   {"text_embedder.linear_1.", "text.0."},
    {"text_embedder.linear_2.", "text.1."},   {"time_proj.", "time.out."},
    {".ffn.net.0.proj.", ".ffn.in."},         {".ffn.net.2.", ".ffn.out."},
    {".attn1.", ".sa."},                      {".attn2.", ".ca."},
    {".to_out.0.", ".o."},                    {".to_qkv.", ".qkv."},
    {".to_q.", ".q."},                        {".to_k.", ".k."},
    {".to_v.", ".vproj."},                    {".norm_q.", ".qn."},
    {".norm_k.", ".kn."},                     {".norm2.", ".ca_norm."},
    {"in_proj.", "in."},                      {"mid_proj.", "mid."},
    {"out_proj.", "out."},                    {"scale_shift_table", "mod"},
};
const Rep kT5Names[] = {
    {"shared.", "token_embd."},
    {"encoder.final_layer_norm.", "final_norm."},
    {"encoder.block.", "blk."},
    {".layer.0.SelfAttention.", ".sa."},
    {".layer.0.layer_norm.", ".sa_norm."},
    {".layer.1.DenseReluDense.", ".ffn."},
    {".layer.1.layer_norm.", ".ffn_norm."},
    {"relative_attention_bias.", "rel."},
    {"wi_0.", "wi0."},
    {"wi_1.", "wi1."},
};
const Rep kVaeNames[] = {
    {"encoder.", "enc."},        {"down_blocks.", "down."},  {"downsampler.resample.1.", "ds."},
    {"resnets.", "res."},        {"mid_block.", "mid."},     {"attentions.0.", "attn."},
    {"conv_shortcut.", "skip."}, {"conv_in.", "in."},        {"conv_out.", "out."},
    {"norm_out.gamma", "out_norm"}, {"to_qkv.", "qkv."},     {"quant_conv.", "quant."},
    {"norm1.gamma", "n1"},       {"norm2.gamma", "n2"},      {"norm.gamma", "norm"},
    {"conv1.", "c1."},           {"conv2.", "c2."},
};

template <size_t N>
void apply(std::string & s, const Rep (&reps)[N]) {
    for (const Rep & r : reps) {
        const size_t fl = strlen(r.from), tl = strlen(r.to);
        for (size_t pos = 0; (pos = s.find(r.from, pos)) != std::string::npos; pos += tl) s.replace(pos, fl, r.to);
    }
}

bool compact(const std::string & full, std::string & out) {
    const size_t dot = full.find('.');
    if (dot == std::string::npos) return false;
    const std::string comp = full.substr(0, dot);
    std::string rest = full.substr(dot + 1);
    if (comp == "gwp") apply(rest, kGwpNames);
    else if (comp == "t5") apply(rest, kT5Names);
    else if (comp == "vae") apply(rest, kVaeNames);
    else return false;
    out = comp + "." + rest;
    return true;
}

constexpr int32_t kGgmlBf16 = 30;

// GWP geometry keys of artifact.cpp:20-56.
struct Geometry {
    uint32_t hidden, layers, heads, head_dim, ffn_dim, action_hidden, action_ffn_dim, action_dim;
    uint32_t real_state_dim, real_action_dim, num_embodiments, embodiment_id;
    uint32_t image_height, image_width, num_views, action_chunk, inference_steps;
    float flow_shift, norm_eps;
    uint32_t t5_vocab_size, t5_hidden, t5_ffn_dim, t5_heads, t5_head_dim, t5_layers, t5_max_length, vae_z_dim;
};

bool read_geometry(wamx_gguf_t g, Geometry & v) {
    struct U {
        const char * key;
        uint32_t * dst;
    } us[] = {
        {"gwp05.hidden", &v.hidden},
        {"gwp05.n_layers", &v.layers},
        {"gwp05.n_heads", &v.heads},
        {"gwp05.head_dim", &v.head_dim},
        {"gwp05.ffn_dim", &v.ffn_dim},
        {"gwp05.action_hidden", &v.action_hidden},
        {"gwp05.action_ffn_dim", &v.action_ffn_dim},
        {"gwp05.action_dim", &v.action_dim},
        {"gwp05.real_state_dim", &v.real_state_dim},
        {"gwp05.real_action_dim", &v.real_action_dim},
        {"gwp05.num_embodiments", &v.num_embodiments},
        {"gwp05.embodiment_id", &v.embodiment_id},
        {"gwp05.image_height", &v.image_height},
        {"gwp05.image_width", &v.image_width},
        {"gwp05.num_views", &v.num_views},
        {"gwp05.action_chunk", &v.action_chunk},
        {"gwp05.inference_steps", &v.inference_steps},
        {"gwp05.t5_vocab_size", &v.t5_vocab_size},
        {"gwp05.t5_hidden", &v.t5_hidden},
        {"gwp05.t5_ffn_dim", &v.t5_ffn_dim},
        {"gwp05.t5_heads", &v.t5_heads},
        {"gwp05.t5_head_dim", &v.t5_head_dim},
        {"gwp05.t5_layers", &v.t5_layers},
        {"gwp05.vae_z_dim", &v.vae_z_dim},
    };
    for (const U & u : us)
        if (wamx_gguf_get_u32(g, u.key, u.dst) != WAMX_STATUS_SUCCESS) return false;
    if (wamx_gguf_get_f32(g, "gwp05.flow_shift", &v.flow_shift) != WAMX_STATUS_SUCCESS ||
        wamx_gguf_get_f32(g, "gwp05.norm_eps", &v.norm_eps) != WAMX_STATUS_SUCCESS)
        return false;
    v.t5_max_length = 512;
    if (wamx_gguf_has(g, "gwp05.t5_max_length") &&
        wamx_gguf_get_u32(g, "gwp05.t5_max_length", &v.t5_max_length) != WAMX_STATUS_SUCCESS)
        return false;
    return true;
}

// The checks of artifact.cpp:57-95 and semantics.cpp:35-56 that bear on the
// MoT path.
bool check_geometry(const Geometry & v) {
    const bool zero = v.hidden == 0 || v.layers == 0 || v.heads == 0 || v.head_dim == 0 || v.ffn_dim == 0 ||
                      v.action_hidden == 0 || v.action_ffn_dim == 0 || v.action_dim == 0 || v.num_embodiments == 0 ||
                      v.image_height == 0 || v.image_width == 0 || v.action_chunk == 0 || v.inference_steps == 0 ||
                      v.t5_vocab_size == 0 || v.t5_hidden == 0 || v.t5_ffn_dim == 0 || v.t5_heads == 0 ||
                      v.t5_head_dim == 0 || v.t5_layers == 0 || v.vae_z_dim == 0;
    if (zero) {
        wamx::set_error("GWP geometry contains a zero dimension");
        return false;
    }
    if (v.hidden != v.heads * v.head_dim || v.t5_hidden != v.t5_heads * v.t5_head_dim) {
        wamx::set_error("GWP attention geometry is inconsistent: hidden must equal heads x head_dim");
        return false;
    }
    if (v.head_dim != 128) {
        wamx::set_errorf("unsupported GWP attention geometry: head_dim %u (128-wide heads expected)", v.head_dim);
        return false;
    }
    if (v.real_state_dim > v.action_dim || v.real_action_dim > v.action_dim) {
        wamx::set_error("GWP action geometry is inconsistent: real dimensions exceed the padded action dimension");
        return false;
    }
    if (v.num_views != 3) {
        wamx::set_errorf("GWP-0.5 requires three camera views (gwp05.num_views = %u)", v.num_views);
        return false;
    }
    if (v.embodiment_id >= v.num_embodiments) {
        wamx::set_errorf("GWP embodiment id %u is out of range (%u embodiments)", v.embodiment_id, v.num_embodiments);
        return false;
    }
    if (v.image_height % 32 != 0 || v.image_width % 32 != 0) {
        wamx::set_errorf("GWP image geometry %ux%u must be divisible by 32", v.image_height, v.image_width);
        return false;
    }
    if (!std::isfinite(v.flow_shift) || v.flow_shift <= 0.0f || !std::isfinite(v.norm_eps) || v.norm_eps <= 0.0f) {
        wamx::set_error("GWP floating-point metadata is invalid: flow_shift and norm_eps must be finite and positive");
        return false;
    }
    if (v.t5_max_length < 64) {
        wamx::set_errorf("T5 capacity %u is smaller than the GWP prompt (64 tokens)", v.t5_max_length);
        return false;
    }
    return true;
}

// The conversion policy (artifact.cpp:245-268): only the BF16 MoT policies
// run on this backend.  *packed: the self-attention q / k / v are one tensor.
bool check_policy(wamx_gguf_t g, bool * packed) {
    const char * arch = wamx_gguf_get_str(g, "gwp05.architecture");
    if (!arch || strcmp(arch, "gwp05") != 0) {
        wamx::set_error("wrong GWP architecture marker (gwp05.architecture must be \"gwp05\")");
        return false;
    }
    if (!wamx_gguf_has(g, "gwp05.conversion_policy")) {
        wamx::set_error("GWP artifact without a conversion policy stores the source F32 weights; this backend runs the "
                        "BF16 latency profile and needs a BF16 MoT policy");
        return false;
    }
    const char * pol = wamx_gguf_get_str(g, "gwp05.conversion_policy");
    if (!pol) return false;
    const std::string policy = pol;
    if (policy != "mot-bf16-v1" && policy != "mot-vae-bf16-v1" && policy != "mot-vae-bf16-qkv-v1") {
        wamx::set_errorf("unsupported GWP conversion policy %s for the BF16 latency profile", policy.c_str());
        return false;
    }
    const char * rev = wamx_gguf_get_str(g, "gwp05.converter_revision");
    const char * wp = wamx_gguf_get_str(g, "gwp05.weight_policy");
    if (!rev || !wp || strcmp(rev, "gwp05-native-bf16-v1") != 0 || policy != wp) {
        wamx::set_error("GWP conversion metadata is inconsistent (converter revision or weight policy mismatch)");
        return false;
    }
    *packed = policy == "mot-vae-bf16-qkv-v1";
    return true;
}

// Reads artifact tensor `name` (compact form) as bf16 with the given shape
// (ggml ne, trailing 1s ignored on both sides).
bool read_bf16(wamx_gguf_t g, const std::string & name, const int64_t (&ne)[4], std::vector<uint16_t> & out) {
    const int64_t i = wamx_gguf_find_tensor(g, name.c_str());
    if (i < 0) {
        wamx::set_errorf("required GGUF tensor %s is missing", name.c_str());
        return false;
    }
    if (wamx_gguf_tensor_type(g, i) != kGgmlBf16) {
        wamx::set_errorf("GGUF tensor %s has ggml type %d, the BF16 policy stores 30", name.c_str(),
                         wamx_gguf_tensor_type(g, i));
        return false;
    }
    for (int k = 0; k < 4; ++k)
        if (wamx_gguf_tensor_ne(g, i, k) != ne[k]) {
            wamx::set_errorf("GGUF tensor %s has the wrong shape: expected [%lld,%lld,%lld,%lld], got "
                             "[%lld,%lld,%lld,%lld]",
                             name.c_str(), (long long) ne[0], (long long) ne[1], (long long) ne[2], (long long) ne[3],
                             (long long) wamx_gguf_tensor_ne(g, i, 0), (long long) wamx_gguf_tensor_ne(g, i, 1),
                             (long long) wamx_gguf_tensor_ne(g, i, 2), (long long) wamx_gguf_tensor_ne(g, i, 3));
            return false;
        }
    out.resize((size_t) (ne[0] * ne[1] * ne[2] * ne[3]));
    return wamx_gguf_read_tensor(g, i, out.data(), out.size() * 2) == WAMX_STATUS_SUCCESS;
}

bool ends_with(const std::string & s, const char * suf) {
    const size_t n = strlen(suf);
    return s.size() >= n && s.compare(s.size() - n, n, suf) == 0;
}

bool load_weights(wamx_gguf_t g, wamx_gwp_t m, const Geometry & geo, bool packed) {
    const int64_t L = geo.layers, emb = geo.embodiment_id, NE = geo.num_embodiments;
    std::vector<uint16_t> buf, part;
    auto set = [&](wamx_tensor * t, const std::vector<uint16_t> & a, size_t off, const std::string & what) {
        if (wamx_backend_tensor_set(t, a.data(), off, a.size() * 2) != WAMX_STATUS_SUCCESS) {
            wamx::set_errorf("upload of %s failed: %s", what.c_str(), wamx_last_error());
            return false;
        }
        return true;
    };
    const int n = wamx_gwp_n_weights(m);
    for (int wi = 0; wi < n; ++wi) {
        const std::string name = wamx_gwp_weight_name(m, wi);
        wamx_tensor * t = wamx_gwp_weight(m, name.c_str());
        if (!t) return false;
        const int64_t ne[4] = {t->ne[0], t->ne[1], t->ne[2], t->ne[3]};
        std::string cn;
        // Packed per-expert adaLN tables: one artifact table per layer.
        if (ends_with(name, ".scale_shift_table") && name.rfind("gwp.blocks.", 0) == 0) {
            const std::string expert = name.substr(strlen("gwp.blocks."));  // "{action,visual}_expert.scale_shift_table"
            const int64_t layer_ne[4] = {ne[0], ne[1], 1, 1};
            for (int64_t l = 0; l < L; ++l) {
                compact("gwp.blocks." + std::to_string(l) + "." + expert, cn);
                if (!read_bf16(g, cn, layer_ne, buf) || !set(t, buf, (size_t) (l * ne[0] * ne[1] * 2), cn)) return false;
            }
            continue;
        }
        // Category-specific projections: the embodiment's [in][out] slice, transposed.
        const bool cat_w = name == "gwp.state_encoder.in_proj.weight" || name == "gwp.action_encoder.in_proj.weight" ||
                           name == "gwp.action_decoder.out_proj.weight";
        const bool cat_b = name == "gwp.state_encoder.in_proj.bias" || name == "gwp.action_encoder.in_proj.bias" ||
                           name == "gwp.action_decoder.out_proj.bias";
        compact(name, cn);
        if (cat_w) {
            const int64_t in = ne[0], out = ne[1];
            const int64_t art[4] = {out, in, NE, 1};
            if (!read_bf16(g, cn, art, part)) return false;
            buf.resize((size_t) (in * out));
            const uint16_t * s = part.data() + emb * in * out;  // [in][out] of embodiment emb
            for (int64_t o = 0; o < out; ++o)
                for (int64_t k = 0; k < in; ++k) buf[(size_t) (o * in + k)] = s[k * out + o];
            if (!set(t, buf, 0, cn)) return false;
            continue;
        }
        if (cat_b) {
            const int64_t out = ne[0];
            const int64_t art[4] = {out, NE, 1, 1};
            if (!read_bf16(g, cn, art, part)) return false;
            buf.assign(part.begin() + emb * out, part.begin() + (emb + 1) * out);
            if (!set(t, buf, 0, cn)) return false;
            continue;
        }
        // Self-attention q / k / v stored separately: rows of the packed QKV.
        if (!packed && (ends_with(name, ".attn1.to_qkv.weight") || ends_with(name, ".attn1.to_qkv.bias"))) {
            const bool is_w = ends_with(name, ".weight");
            const std::string base = name.substr(0, name.size() - strlen(is_w ? ".to_qkv.weight" : ".to_qkv.bias"));
            const int64_t rows = is_w ? ne[1] / 3 : ne[0] / 3, cols = is_w ? ne[0] : 1;
            const int64_t one[4] = {is_w ? cols : rows, is_w ? rows : 1, 1, 1};
            buf.clear();
            for (const char * part_name : {".to_q.", ".to_k.", ".to_v."}) {
                compact(base + part_name + (is_w ? "weight" : "bias"), cn);
                if (!read_bf16(g, cn, one, part)) return false;
                buf.insert(buf.end(), part.begin(), part.end());
            }
            if (!set(t, buf, 0, name)) return false;
            continue;
        }
        if (!read_bf16(g, cn, ne, buf) || !set(t, buf, 0, cn)) return false;
    }
    return true;
}

}  // namespace

extern "C" {

int32_t wamx_gguf_compact_name(const char * name, char * out, int32_t cap) {
    std::string c;
    if (!name || !compact(name, c)) return -1;
    if (out && cap > 0) {
        const size_t n = std::min<size_t>(c.size(), (size_t) cap - 1);
        memcpy(out, c.data(), n);
        out[n] = '\0';
    }
    return (int32_t) c.size() + 1;
}

wamx_gwp_t wamx_gwp_create_from_gguf(wamx_backend_t be, wamx_gguf_t g, int32_t n_lang, int32_t batch) {
    wamx::clear_error();
    if (!be || !g) {
        wamx::set_error("wamx_gwp_create_from_gguf: null backend or artifact");
        return nullptr;
    }
    Geometry geo{};
    bool packed = false;
    if (!read_geometry(g, geo) || !check_geometry(geo) || !check_policy(g, &packed)) return nullptr;
    wamx_gwp_config c = wamx_gwp_default_config();
    c.n_layers = (int32_t) geo.layers;
    c.hidden = (int32_t) geo.hidden;
    c.n_heads = (int32_t) geo.heads;
    c.head_dim = (int32_t) geo.head_dim;
    c.ffn_dim = (int32_t) geo.ffn_dim;
    c.action_hidden = (int32_t) geo.action_hidden;
    c.action_ffn_dim = (int32_t) geo.action_ffn_dim;
    c.action_chunk = (int32_t) geo.action_chunk;
    c.action_dim = (int32_t) geo.action_dim;
    c.grid_h = (int32_t) (geo.image_height / 32);
    c.grid_w = (int32_t) (geo.image_width / 32);
    c.n_lang = n_lang > 0 ? n_lang : 64;
    c.t5_hidden = (int32_t) geo.t5_hidden;
    c.z_dim = (int32_t) geo.vae_z_dim;
    c.num_steps = (int32_t) geo.inference_steps;
    c.enc_hidden = 128;  // the category-specific MLP width (mot.cpp:23-26)
    c.shift = geo.flow_shift;
    c.eps = geo.norm_eps;
    c.batch = batch;
    wamx_gwp_t m = wamx_gwp_create(be, &c);
    if (!m) return nullptr;
    if (!load_weights(g, m, geo, packed)) {
        const std::string err = wamx_last_error();
        wamx_gwp_free(m);
        wamx::set_errorf("wamx_gwp_create_from_gguf: %s", err.c_str());
        return nullptr;
    }
    return m;
}

}  // extern "C"
