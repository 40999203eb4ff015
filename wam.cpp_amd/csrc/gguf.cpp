// GGUF reader: the model artifact's container (the role of wam.cpp's
// GgufReader, src/models/common/gguf_reader.{h,cpp}, which parses through
// ggml's gguf library).  Written from the published GGUF v3 layout:
//
//   u32 magic "GGUF" | u32 version | u64 n_tensors | u64 n_kv
//   n_kv x  { string key | u32 type | value }
//   n_tensors x { string name | u32 n_dims | u64 ne[n_dims] | u32 ggml type |
//                 u64 offset (from the data section, aligned) }
//   padding to `general.alignment` (default 32) | tensor data
//
// strings are u64 length + bytes; arrays are u32 element type + u64 count +
// elements.  The header is read into memory once; tensor payloads are read
// on request with pread (the artifact is 20+ GB and is never loaded whole).
// Every count, length and offset is checked against the file size, so a
// truncated or corrupt file fails with a message instead of reading past it.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "common.h"
#include "internal.h"

namespace {

enum GgufType : uint32_t {
    kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64, kTypeCount
};

struct GgufValue {
    uint32_t type = kTypeCount;
    uint64_t u = 0;       // unsigned / bool / bit pattern of signed values
    double f = 0.0;       // f32 / f64
    std::string s;
    uint32_t arr_type = kTypeCount;
    uint64_t arr_n = 0;
    std::vector<double> arr_num;          // numeric arrays, widened
    std::vector<std::string> arr_str;     // string arrays
};

struct GgufTensor {
    std::string name;
    int32_t type = -1;
    int32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;  // absolute file offset
    uint64_t bytes = 0;   // 0 when the type's size is unknown here
};

// Bytes per element of the ggml types a GWP artifact can hold unquantised
// (F32 0, F16 1, I8 24, I16 25, I32 26, I64 27, F64 28, BF16 30).
int64_t type_size(int32_t t) {
    switch (t) {
        case 0: case 26: return 4;
        case 1: case 25: case 30: return 2;
        case 24: return 1;
        case 27: case 28: return 8;
        default: return 0;
    }
}

}  // namespace

struct wamx_gguf {
    int fd = -1;
    std::string path;
    uint64_t file_size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32;
    uint64_t data_offset = 0;
    std::vector<std::string> keys;
    std::unordered_map<std::string, GgufValue> kv;
    std::vector<GgufTensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
    std::string error;
};

namespace {

// Sequential reader over the header bytes with bounds checks.
struct Cursor {
    const std::vector<uint8_t> & b;
    size_t pos = 0;
    bool ok = true;
    std::string why;
    explicit Cursor(const std::vector<uint8_t> & buf) : b(buf) {}
    bool need(size_t n, const char * what) {
        if (!ok) return false;
        if (n > b.size() - pos) {
            ok = false;
            why = std::string("truncated ") + what;
        }
        return ok;
    }
    template <typename T>
    T get(const char * what) {
        T v{};
        if (need(sizeof(T), what)) {
            memcpy(&v, b.data() + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    std::string str(const char * what) {
        const uint64_t n = get<uint64_t>(what);
        if (!ok) return {};
        if (n > (uint64_t) 1 << 20) {
            ok = false;
            why = std::string("implausible string length in ") + what;
            return {};
        }
        if (!need((size_t) n, what)) return {};
        std::string s((const char *) b.data() + pos, (size_t) n);
        pos += (size_t) n;
        return s;
    }
};

bool read_scalar(Cursor & c, uint32_t t, GgufValue & v, const char * what) {
    switch (t) {
        case kU8: v.u = c.get<uint8_t>(what); break;
        case kI8: v.u = (uint64_t) (int64_t) c.get<int8_t>(what); break;
        case kU16: v.u = c.get<uint16_t>(what); break;
        case kI16: v.u = (uint64_t) (int64_t) c.get<int16_t>(what); break;
        case kU32: v.u = c.get<uint32_t>(what); break;
        case kI32: v.u = (uint64_t) (int64_t) c.get<int32_t>(what); break;
        case kF32: v.f = c.get<float>(what); break;
        case kBool: v.u = c.get<uint8_t>(what) != 0; break;
        case kStr: v.s = c.str(what); break;
        case kU64: v.u = c.get<uint64_t>(what); break;
        case kI64: v.u = (uint64_t) c.get<int64_t>(what); break;
        case kF64: v.f = c.get<double>(what); break;
        default:
            c.ok = false;
            c.why = std::string("unknown value type in ") + what;
    }
    return c.ok;
}

double numeric(const GgufValue & v, uint32_t t) {
    switch (t) {
        case kF32: case kF64: return v.f;
        case kI8: case kI16: case kI32: case kI64: return (double) (int64_t) v.u;
        default: return (double) v.u;
    }
}

bool parse(wamx_gguf & g) {
    // The header (key/values and tensor infos) is read in growing chunks
    // until it parses; the payload is left on disk.
    std::vector<uint8_t> buf;
    size_t want = std::min<uint64_t>(g.file_size, 1 << 20);
    for (;;) {
        buf.resize(want);
        const ssize_t r = pread(g.fd, buf.data(), want, 0);
        if (r < 0 || (size_t) r != want) {
            g.error = "cannot read the GGUF header";
            return false;
        }
        Cursor c(buf);
        const uint32_t magic = c.get<uint32_t>("magic");
        if (c.ok && magic != 0x46554747u) {
            g.error = "not a GGUF file (bad magic)";
            return false;
        }
        g.version = c.get<uint32_t>("version");
        if (c.ok && g.version != 2 && g.version != 3) {
            g.error = "unsupported GGUF version " + std::to_string(g.version);
            return false;
        }
        const uint64_t n_t = c.get<uint64_t>("tensor count");
        const uint64_t n_kv = c.get<uint64_t>("key/value count");
        if (c.ok && (n_t > (uint64_t) 1 << 24 || n_kv > (uint64_t) 1 << 24)) {
            g.error = "implausible GGUF tensor or key/value count";
            return false;
        }
        g.keys.clear();
        g.kv.clear();
        g.tensors.clear();
        g.by_name.clear();
        for (uint64_t i = 0; c.ok && i < n_kv; ++i) {
            std::string key = c.str("key");
            GgufValue v;
            v.type = c.get<uint32_t>("value type");
            if (!c.ok) break;
            if (v.type == kArr) {
                v.arr_type = c.get<uint32_t>("array type");
                v.arr_n = c.get<uint64_t>("array length");
                if (c.ok && (v.arr_type == kArr || v.arr_type >= kTypeCount || v.arr_n > (uint64_t) 1 << 28)) {
                    c.ok = false;
                    c.why = "unsupported or implausible array in key " + key;
                    break;
                }
                for (uint64_t k = 0; c.ok && k < v.arr_n; ++k) {
                    GgufValue e;
                    read_scalar(c, v.arr_type, e, "array element");
                    if (v.arr_type == kStr) v.arr_str.push_back(std::move(e.s));
                    else v.arr_num.push_back(numeric(e, v.arr_type));
                }
            } else {
                read_scalar(c, v.type, v, "value");
            }
            if (!c.ok) break;
            if (g.kv.count(key)) {
                g.error = "duplicate GGUF key " + key;
                return false;
            }
            g.keys.push_back(key);
            g.kv.emplace(std::move(key), std::move(v));
        }
        std::vector<GgufTensor> infos;
        for (uint64_t i = 0; c.ok && i < n_t; ++i) {
            GgufTensor t;
            t.name = c.str("tensor name");
            const uint32_t nd = c.get<uint32_t>("tensor dims");
            if (c.ok && (nd == 0 || nd > 4)) {
                g.error = "tensor " + t.name + " has " + std::to_string(nd) + " dimensions (1..4 supported)";
                return false;
            }
            t.n_dims = (int32_t) nd;
            for (uint32_t k = 0; c.ok && k < nd; ++k) t.ne[k] = (int64_t) c.get<uint64_t>("tensor shape");
            t.type = (int32_t) c.get<uint32_t>("tensor type");
            t.offset = c.get<uint64_t>("tensor offset");
            if (!c.ok) break;
            infos.push_back(std::move(t));
        }
        if (!c.ok) {
            // The header may just be longer than the chunk read so far; a
            // GWP artifact's is a few hundred KB, so past kMaxHeader it is
            // corrupt.
            constexpr uint64_t kMaxHeader = 256ull << 20;
            if (want < g.file_size && want < kMaxHeader) {
                want = (size_t) std::min<uint64_t>(std::min<uint64_t>(g.file_size, kMaxHeader), (uint64_t) want * 4);
                continue;
            }
            g.error = "corrupt GGUF header: " + c.why;
            return false;
        }
        auto al = g.kv.find("general.alignment");
        if (al != g.kv.end()) {
            if (al->second.type != kU32 || al->second.u == 0 || (al->second.u & (al->second.u - 1))) {
                g.error = "general.alignment must be a power-of-two u32";
                return false;
            }
            g.alignment = al->second.u;
        }
        g.data_offset = (c.pos + g.alignment - 1) / g.alignment * g.alignment;
        for (auto & t : infos) {
            int64_t n = 1;
            for (int k = 0; k < 4; ++k) {
                if (t.ne[k] <= 0 || (n > 0 && t.ne[k] > ((int64_t) 1 << 40) / n)) {
                    g.error = "tensor " + t.name + " has an invalid shape";
                    return false;
                }
                n *= t.ne[k];
            }
            const int64_t es = type_size(t.type);
            t.bytes = es > 0 ? (uint64_t) n * (uint64_t) es : 0;
            if (t.offset % g.alignment != 0) {
                g.error = "tensor " + t.name + " data is not aligned";
                return false;
            }
            if (t.offset > g.file_size || g.data_offset > g.file_size - t.offset ||
                t.bytes > g.file_size - g.data_offset - t.offset) {
                g.error = "tensor " + t.name + " data lies outside the file (truncated artifact)";
                return false;
            }
            t.offset += g.data_offset;
            if (g.by_name.count(t.name)) {
                g.error = "duplicate GGUF tensor " + t.name;
                return false;
            }
            g.by_name[t.name] = g.tensors.size();
            g.tensors.push_back(std::move(t));
        }
        return true;
    }
}

const GgufValue * find_typed(wamx_gguf_t g, const char * key, uint32_t type) {
    if (!g || !key) return nullptr;
    auto it = g->kv.find(key);
    if (it == g->kv.end()) {
        wamx::set_errorf("GGUF metadata key %s is required", key);
        return nullptr;
    }
    if (it->second.type != type) {
        wamx::set_errorf("GGUF metadata key %s has type %u, expected %u", key, it->second.type, type);
        return nullptr;
    }
    return &it->second;
}

const GgufTensor * tensor_at(wamx_gguf_t g, int64_t i) {
    return g && i >= 0 && i < (int64_t) g->tensors.size() ? &g->tensors[(size_t) i] : nullptr;
}

}  // namespace

extern "C" {

wamx_gguf_t wamx_gguf_open(const char * path) {
    wamx::clear_error();
    if (!path) {
        wamx::set_error("wamx_gguf_open: null path");
        return nullptr;
    }
    auto * g = new (std::nothrow) wamx_gguf();
    if (!g) return nullptr;
    g->path = path;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (g->fd < 0 || fstat(g->fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        wamx::set_errorf("wamx_gguf_open: %s is not a readable regular file", path);
        wamx_gguf_close(g);
        return nullptr;
    }
    g->file_size = (uint64_t) st.st_size;
    if (g->file_size < 24 || !parse(*g)) {
        wamx::set_errorf("wamx_gguf_open: %s: %s", path, g->error.empty() ? "file too short" : g->error.c_str());
        wamx_gguf_close(g);
        return nullptr;
    }
    return g;
}

void wamx_gguf_close(wamx_gguf_t g) {
    if (!g) return;
    if (g->fd >= 0) close(g->fd);
    delete g;
}

uint32_t wamx_gguf_version(wamx_gguf_t g) { return g ? g->version : 0; }
uint64_t wamx_gguf_data_offset(wamx_gguf_t g) { return g ? g->data_offset : 0; }
int64_t wamx_gguf_n_keys(wamx_gguf_t g) { return g ? (int64_t) g->keys.size() : 0; }
const char * wamx_gguf_key(wamx_gguf_t g, int64_t i) {
    return g && i >= 0 && i < (int64_t) g->keys.size() ? g->keys[(size_t) i].c_str() : nullptr;
}
int32_t wamx_gguf_key_type(wamx_gguf_t g, const char * key) {
    if (!g || !key) return -1;
    auto it = g->kv.find(key);
    return it == g->kv.end() ? -1 : (int32_t) it->second.type;
}
bool wamx_gguf_has(wamx_gguf_t g, const char * key) { return wamx_gguf_key_type(g, key) >= 0; }

wamx_status wamx_gguf_get_u32(wamx_gguf_t g, const char * key, uint32_t * out) {
    const GgufValue * v = find_typed(g, key, kU32);
    if (!v || !out) return WAMX_STATUS_FAILED;
    *out = (uint32_t) v->u;
    return WAMX_STATUS_SUCCESS;
}
wamx_status wamx_gguf_get_u64(wamx_gguf_t g, const char * key, uint64_t * out) {
    const GgufValue * v = find_typed(g, key, kU64);
    if (!v || !out) return WAMX_STATUS_FAILED;
    *out = v->u;
    return WAMX_STATUS_SUCCESS;
}
wamx_status wamx_gguf_get_f32(wamx_gguf_t g, const char * key, float * out) {
    const GgufValue * v = find_typed(g, key, kF32);
    if (!v || !out) return WAMX_STATUS_FAILED;
    *out = (float) v->f;
    return WAMX_STATUS_SUCCESS;
}
const char * wamx_gguf_get_str(wamx_gguf_t g, const char * key) {
    const GgufValue * v = find_typed(g, key, kStr);
    return v ? v->s.c_str() : nullptr;
}
int64_t wamx_gguf_get_f32_array(wamx_gguf_t g, const char * key, float * out, int64_t cap) {
    const GgufValue * v = find_typed(g, key, kArr);
    if (!v) return -1;
    if (v->arr_type != kF32 && v->arr_type != kF64) {
        wamx::set_errorf("GGUF metadata array %s is not F32 or F64", key);
        return -1;
    }
    const int64_t n = (int64_t) v->arr_num.size();
    for (int64_t i = 0; out && i < std::min(n, cap); ++i) out[i] = (float) v->arr_num[(size_t) i];
    return n;
}

int64_t wamx_gguf_n_tensors(wamx_gguf_t g) { return g ? (int64_t) g->tensors.size() : 0; }
int64_t wamx_gguf_find_tensor(wamx_gguf_t g, const char * name) {
    if (!g || !name) return -1;
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? -1 : (int64_t) it->second;
}
const char * wamx_gguf_tensor_name(wamx_gguf_t g, int64_t i) {
    const GgufTensor * t = tensor_at(g, i);
    return t ? t->name.c_str() : nullptr;
}
int32_t wamx_gguf_tensor_type(wamx_gguf_t g, int64_t i) {
    const GgufTensor * t = tensor_at(g, i);
    return t ? t->type : -1;
}
int32_t wamx_gguf_tensor_n_dims(wamx_gguf_t g, int64_t i) {
    const GgufTensor * t = tensor_at(g, i);
    return t ? t->n_dims : 0;
}
int64_t wamx_gguf_tensor_ne(wamx_gguf_t g, int64_t i, int32_t dim) {
    const GgufTensor * t = tensor_at(g, i);
    return t && dim >= 0 && dim < 4 ? t->ne[dim] : 0;
}
uint64_t wamx_gguf_tensor_offset(wamx_gguf_t g, int64_t i) {
    const GgufTensor * t = tensor_at(g, i);
    return t ? t->offset : 0;
}
uint64_t wamx_gguf_tensor_bytes(wamx_gguf_t g, int64_t i) {
    const GgufTensor * t = tensor_at(g, i);
    return t ? t->bytes : 0;
}

wamx_status wamx_gguf_read_tensor(wamx_gguf_t g, int64_t i, void * dst, uint64_t bytes) {
    const GgufTensor * t = tensor_at(g, i);
    WAMX_REQUIRE(t && dst, "wamx_gguf_read_tensor: bad tensor index or destination");
    WAMX_REQUIRE(t->bytes > 0, "wamx_gguf_read_tensor: tensor %s has a type (%d) this reader does not size",
                 t->name.c_str(), t->type);
    WAMX_REQUIRE(bytes == t->bytes, "wamx_gguf_read_tensor: tensor %s holds %llu bytes, not %llu", t->name.c_str(),
                 (unsigned long long) t->bytes, (unsigned long long) bytes);
    uint64_t done = 0;
    while (done < bytes) {
        const size_t chunk = (size_t) std::min<uint64_t>(bytes - done, (uint64_t) 1 << 30);
        const ssize_t r = pread(g->fd, (char *) dst + done, chunk, (off_t) (t->offset + done));
        WAMX_REQUIRE(r > 0, "wamx_gguf_read_tensor: read of %s failed", t->name.c_str());
        done += (uint64_t) r;
    }
    return WAMX_STATUS_SUCCESS;
}

}  // extern "C"
