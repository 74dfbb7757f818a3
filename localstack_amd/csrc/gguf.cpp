// gguf.cpp - memory-mapped GGUF reader (include/lstk_gguf.h).
//
// The reference reads GGUF through ggml's gguf library (src/gguf_model.cpp:14-103), which this library
// does not link; this is a reader written from the published GGUF layout (versions 2 and 3):
//   "GGUF" | u32 version | u64 n_tensors | u64 n_kv
//   n_kv x   { string key | u32 value type | value }
//   n_tensors x { string name | u32 n_dims | u64 ne[n_dims] | u32 ggml type | u64 offset }
//   padding to general.alignment (default 32) | tensor data, each tensor at data start + offset
// where a string is { u64 length | bytes } and an array value is { u32 element type | u64 count |
// elements }. The same layout is what the reference's own writer produces (tools/make_tiny_moe.py:37-77).
// Every read goes through a bounds-checked cursor over the mapping.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/lstk_gguf.h"
#include "formats.h"
#include "internal.h"

namespace {

using lstk::set_error;

enum : uint32_t {
    kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7, kStr = 8, kArr = 9,
    kU64 = 10, kI64 = 11, kF64 = 12,
};

// ggml type id -> (values per block, bytes per block); types this reader can size.
struct TypeTraits {
    int32_t id;
    int32_t block;
    int32_t bytes;
    const char *name;
};
constexpr TypeTraits kTypes[] = {
    {0, 1, 4, "F32"},     {1, 1, 2, "F16"},      {2, 32, 18, "Q4_0"},   {3, 32, 20, "Q4_1"},  {6, 32, 22, "Q5_0"},
    {7, 32, 24, "Q5_1"},  {8, 32, 34, "Q8_0"},   {9, 32, 36, "Q8_1"},   {10, 256, 84, "Q2_K"}, {11, 256, 110, "Q3_K"},
    {12, 256, 144, "Q4_K"}, {13, 256, 176, "Q5_K"}, {14, 256, 210, "Q6_K"}, {15, 256, 292, "Q8_K"}, {24, 1, 1, "I8"},
    {25, 1, 2, "I16"},    {26, 1, 4, "I32"},     {27, 1, 8, "I64"},     {28, 1, 8, "F64"},    {30, 1, 2, "BF16"},
};

const TypeTraits *traits(int32_t id) {
    for (const TypeTraits &t : kTypes)
        if (t.id == id) return &t;
    return nullptr;
}

std::string type_name(int32_t id) {
    const TypeTraits *t = traits(id);
    return t ? t->name : "type " + std::to_string(id);
}

struct Value {
    uint32_t type = 0;
    int64_t i = 0;  // integers and bool
    double f = 0.0; // floats
    std::string s;  // strings
    uint32_t arr_type = 0;
    uint64_t arr_n = 0;
};

struct Tensor {
    std::string name;
    int32_t type = 0, n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0; // offset from the start of the file
};

// Bounds-checked little-endian reader over [p, end).
struct Cursor {
    const uint8_t *base, *p, *end;
    bool ok = true;
    bool take(void *dst, size_t n) {
        if (!ok || (size_t) (end - p) < n) return ok = false;
        std::memcpy(dst, p, n);
        p += n;
        return true;
    }
    bool skip(uint64_t n) {
        if (!ok || (uint64_t) (end - p) < n) return ok = false;
        p += n;
        return true;
    }
    template <typename T>
    T get() {
        T v{};
        take(&v, sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || (uint64_t) (end - p) < n) {
            ok = false;
            return {};
        }
        std::string s(reinterpret_cast<const char *>(p), (size_t) n);
        p += n;
        return s;
    }
    size_t pos() const { return (size_t) (p - base); }
};

size_t scalar_size(uint32_t t) {
    switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
    }
}

bool read_scalar(Cursor &c, uint32_t t, Value &v) {
    switch (t) {
    case kU8: v.i = c.get<uint8_t>(); break;
    case kI8: v.i = c.get<int8_t>(); break;
    case kU16: v.i = c.get<uint16_t>(); break;
    case kI16: v.i = c.get<int16_t>(); break;
    case kU32: v.i = c.get<uint32_t>(); break;
    case kI32: v.i = c.get<int32_t>(); break;
    case kU64: v.i = (int64_t) c.get<uint64_t>(); break;
    case kI64: v.i = c.get<int64_t>(); break;
    case kBool: v.i = c.get<uint8_t>() != 0; break;
    case kF32: v.f = c.get<float>(); break;
    case kF64: v.f = c.get<double>(); break;
    case kStr: v.s = c.str(); break;
    default: return false;
    }
    return c.ok;
}

}  // namespace

struct lstk_gguf {
    int fd = -1;
    void *map = nullptr;
    size_t size = 0;
    uint32_t version = 0, alignment = 32;
    std::string arch;
    std::vector<std::pair<std::string, Value>> kv;
    std::unordered_map<std::string, size_t> kv_index;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> t_index;
    uint64_t data_offset = 0;
};

namespace {

void destroy(lstk_gguf *g) {
    if (!g) return;
    if (g->map && g->map != MAP_FAILED) munmap(g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

int parse(lstk_gguf *g, const std::string &path) {
    const uint8_t *base = static_cast<const uint8_t *>(g->map);
    Cursor c{base, base, base + g->size};
    char magic[4];
    if (!c.take(magic, 4) || std::memcmp(magic, "GGUF", 4) != 0) return set_error(LSTK_E_INVALID, "not a GGUF file (bad magic): " + path);
    g->version = c.get<uint32_t>();
    if (!c.ok || g->version < 2 || g->version > 3)
        return set_error(LSTK_E_INVALID, "unsupported GGUF version " + std::to_string(g->version) + ": " + path);
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    // every entry takes at least 8 bytes, so counts beyond the file size are malformed
    if (!c.ok || n_tensors > g->size / 8 || n_kv > g->size / 8) return set_error(LSTK_E_INVALID, "truncated or malformed GGUF header: " + path);
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = c.str();
        Value v;
        v.type = c.get<uint32_t>();
        if (!c.ok) break;
        if (v.type == kArr) {
            v.arr_type = c.get<uint32_t>();
            v.arr_n = c.get<uint64_t>();
            if (!c.ok) break;
            if (v.arr_type == kStr) {
                for (uint64_t i = 0; i < v.arr_n && c.ok; i++) c.skip(c.get<uint64_t>());
            } else {
                const size_t es = scalar_size(v.arr_type);
                if (es == 0 || v.arr_n > g->size / es)
                    return set_error(LSTK_E_INVALID, "bad array type in metadata key " + key + ": " + path);
                c.skip(v.arr_n * es);
            }
        } else if (!read_scalar(c, v.type, v)) {
            if (c.ok) return set_error(LSTK_E_INVALID, "unknown value type " + std::to_string(v.type) + " of key " + key);
            break;
        }
        if (!c.ok) break;
        g->kv_index[key] = g->kv.size();
        g->kv.emplace_back(std::move(key), std::move(v));
    }
    if (!c.ok) return set_error(LSTK_E_INVALID, "truncated GGUF metadata: " + path);
    auto al = g->kv_index.find("general.alignment");
    if (al != g->kv_index.end()) {
        const Value &v = g->kv[al->second].second;
        if (v.type != kU32 || v.i <= 0 || (v.i & (v.i - 1))) return set_error(LSTK_E_INVALID, "bad general.alignment: " + path);
        g->alignment = (uint32_t) v.i;
    }
    g->tensors.resize((size_t) n_tensors);
    for (uint64_t i = 0; i < n_tensors && c.ok; i++) {
        Tensor &t = g->tensors[(size_t) i];
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok) break;
        if (nd < 1 || nd > 4) return set_error(LSTK_E_INVALID, "tensor " + t.name + " has " + std::to_string(nd) + " dimensions");
        t.n_dims = (int32_t) nd;
        for (uint32_t d = 0; d < nd; d++) t.ne[d] = (int64_t) c.get<uint64_t>();
        t.type = (int32_t) c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
    }
    if (!c.ok) return set_error(LSTK_E_INVALID, "truncated GGUF tensor index: " + path);
    g->data_offset = (c.pos() + g->alignment - 1) / g->alignment * g->alignment;
    for (Tensor &t : g->tensors) {
        const TypeTraits *tt = traits(t.type);
        if (!tt) return set_error(LSTK_E_INVALID, "tensor " + t.name + " has an unknown type " + std::to_string(t.type));
        for (int d = 0; d < 4; d++)
            if (t.ne[d] < 0 || (t.ne[d] > 0 && (uint64_t) t.ne[d] > g->size * 8))
                return set_error(LSTK_E_INVALID, "tensor " + t.name + " has an impossible shape");
        if (t.ne[0] % tt->block) return set_error(LSTK_E_INVALID, "tensor " + t.name + ": ne[0] is not a multiple of its block");
        // bytes = blocks * bytes per block, each partial product checked: a product of four dims near
        // size * 8 can pass 2^64 (and would wrap any fixed-width integer)
        uint64_t n = 0;
        bool over = false;
        if (t.ne[0] > 0 && t.ne[1] > 0 && t.ne[2] > 0 && t.ne[3] > 0) {
            n = (uint64_t) t.ne[0] / tt->block;
            for (int d = 1; d < 4 && !over; d++) over = __builtin_mul_overflow(n, (uint64_t) t.ne[d], &n) || n > g->size;
            over = over || __builtin_mul_overflow(n, (uint64_t) tt->bytes, &n);
        }
        if (over || t.offset % g->alignment || n > g->size || t.offset > g->size || g->data_offset + t.offset + n > g->size)
            return set_error(LSTK_E_INVALID, "tensor " + t.name + " lies outside the file (truncated?): " + path);
        t.nbytes = n;
        t.offset += g->data_offset;
        g->t_index[t.name] = (size_t) (&t - g->tensors.data());
    }
    g->arch = lstk_gguf_get_str(g, "general.architecture", "");
    if (g->arch.empty()) return set_error(LSTK_E_INVALID, "GGUF has no general.architecture");
    return LSTK_OK;
}

const Value *find(const lstk_gguf *g, const char *key) {
    if (!g || !key) return nullptr;
    auto it = g->kv_index.find(key);
    return it == g->kv_index.end() ? nullptr : &g->kv[it->second].second;
}

void fill(const lstk_gguf *g, const Tensor &t, lstk_gguf_tensor *out) {
    out->name = t.name.c_str();
    out->type = t.type;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) out->ne[d] = t.ne[d];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->data = static_cast<const uint8_t *>(g->map) + t.offset;
}

}  // namespace

extern "C" {

int lstk_gguf_open(const char *path, lstk_gguf **out) {
    if (!path || !out) return set_error(LSTK_E_INVALID, "null argument");
    *out = nullptr;
    lstk_gguf *g = new lstk_gguf();
    g->fd = open(path, O_RDONLY);
    if (g->fd < 0) {
        destroy(g);
        return set_error(LSTK_E_IO, std::string("cannot open ") + path);
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0 || st.st_size < 24) {
        destroy(g);
        return set_error(LSTK_E_INVALID, std::string("not a readable GGUF file: ") + path);
    }
    g->size = (size_t) st.st_size;
    g->map = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (g->map == MAP_FAILED) {
        g->map = nullptr;
        destroy(g);
        return set_error(LSTK_E_IO, std::string("cannot map ") + path);
    }
    int rc;
    try {
        rc = parse(g, path);
    } catch (const std::exception &ex) {
        rc = set_error(LSTK_E_NOMEM, std::string("lstk_gguf_open: ") + ex.what());
    }
    if (rc != LSTK_OK) {
        destroy(g);
        return rc;
    }
    *out = g;
    return LSTK_OK;
}

void lstk_gguf_close(lstk_gguf *g) { destroy(g); }

const char *lstk_gguf_arch(const lstk_gguf *g) { return g ? g->arch.c_str() : ""; }
int lstk_gguf_version(const lstk_gguf *g) { return g ? (int) g->version : 0; }
int lstk_gguf_alignment(const lstk_gguf *g) { return g ? (int) g->alignment : 0; }

int lstk_gguf_has(const lstk_gguf *g, const char *key) { return find(g, key) != nullptr; }

int64_t lstk_gguf_get_int(const lstk_gguf *g, const char *key, int64_t def) {
    const Value *v = find(g, key);
    if (!v) return def;
    switch (v->type) {
    case kU8: case kI8: case kU16: case kI16: case kU32: case kI32: case kU64: case kI64: case kBool: return v->i;
    default: return def;
    }
}

double lstk_gguf_get_float(const lstk_gguf *g, const char *key, double def) {
    const Value *v = find(g, key);
    if (!v) return def;
    if (v->type == kF32 || v->type == kF64) return v->f;
    return (double) lstk_gguf_get_int(g, key, (int64_t) def);
}

const char *lstk_gguf_get_str(const lstk_gguf *g, const char *key, const char *def) {
    const Value *v = find(g, key);
    return v && v->type == kStr ? v->s.c_str() : def;
}

int lstk_gguf_n_tensors(const lstk_gguf *g) { return g ? (int) g->tensors.size() : 0; }

int lstk_gguf_tensor_at(const lstk_gguf *g, int i, lstk_gguf_tensor *out) {
    if (!g || !out || i < 0 || i >= (int) g->tensors.size()) return set_error(LSTK_E_INVALID, "tensor index out of range");
    fill(g, g->tensors[(size_t) i], out);
    return LSTK_OK;
}

int lstk_gguf_find_tensor(const lstk_gguf *g, const char *name, lstk_gguf_tensor *out) {
    if (!g || !name || !out) return set_error(LSTK_E_INVALID, "null argument");
    auto it = g->t_index.find(name);
    if (it == g->t_index.end()) return set_error(LSTK_E_INVALID, std::string("missing tensor ") + name);
    fill(g, g->tensors[it->second], out);
    return LSTK_OK;
}

int lstk_gguf_qwen3_hparams(const lstk_gguf *g, lstk_qwen3_hparams *hp) {
    if (!g || !hp) return set_error(LSTK_E_INVALID, "null argument");
    if (g->arch != "qwen3moe")
        return set_error(LSTK_E_INVALID, "unsupported architecture: " + g->arch + " (this path runs qwen3moe)");
    const std::string a = g->arch + ".";
    auto gi = [&](const std::string &k, int64_t def) { return lstk_gguf_get_int(g, k.c_str(), def); };
    auto gf = [&](const std::string &k, double def) { return lstk_gguf_get_float(g, k.c_str(), def); };
    lstk_qwen3_hparams h{};
    h.n_layer = (int32_t) gi(a + "block_count", 0);
    h.n_embd = (int32_t) gi(a + "embedding_length", 0);
    const int64_t n_ff = gi(a + "feed_forward_length", 0);
    h.n_head = (int32_t) gi(a + "attention.head_count", 0);
    h.n_head_kv = (int32_t) gi(a + "attention.head_count_kv", h.n_head);
    h.head_dim = (int32_t) gi(a + "attention.key_length", h.n_head ? h.n_embd / h.n_head : 0);
    h.n_ctx_train = (int32_t) gi(a + "context_length", 32768);
    h.rms_eps = (float) gf(a + "attention.layer_norm_rms_epsilon", 1e-6);
    h.rope_freq_base = (float) gf(a + "rope.freq_base", 10000.0);
    h.n_expert = (int32_t) gi(a + "expert_count", 0);
    h.n_expert_used = (int32_t) gi(a + "expert_used_count", 0);
    h.n_ff_exp = (int32_t) gi(a + "expert_feed_forward_length", h.n_expert_used ? n_ff / h.n_expert_used : 0);
    if (!h.n_expert || !h.n_expert_used || !h.n_ff_exp) return set_error(LSTK_E_INVALID, "incomplete MoE hyperparameters in GGUF");
    if (!h.n_layer || !h.n_embd || !n_ff || !h.n_head || !h.n_head_kv || !h.head_dim)
        return set_error(LSTK_E_INVALID, "incomplete hyperparameters in GGUF");
    lstk_gguf_tensor emb;
    if (lstk_gguf_find_tensor(g, "token_embd.weight", &emb) != LSTK_OK) return LSTK_E_INVALID;
    h.n_vocab = (int32_t) emb.ne[1];
    *hp = h;
    return LSTK_OK;
}

int lstk_gguf_qwen3_experts(const lstk_gguf *g, const lstk_qwen3_hparams *hp, lstk_expert_layer *layers) {
    if (!g || !hp || !layers) return set_error(LSTK_E_INVALID, "null argument");
    for (int l = 0; l < hp->n_layer; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        const char *names[3] = {"ffn_up_exps.weight", "ffn_gate_exps.weight", "ffn_down_exps.weight"};
        lstk_gguf_tensor t[3];
        for (int m = 0; m < 3; m++) {
            auto it = g->t_index.find(p + names[m]);
            if (it == g->t_index.end()) return set_error(LSTK_E_INVALID, "missing expert tensors for layer " + std::to_string(l));
            fill(g, g->tensors[it->second], &t[m]);
        }
        const bool shape_ok = t[0].ne[0] == hp->n_embd && t[0].ne[1] == hp->n_ff_exp && t[0].ne[2] == hp->n_expert &&
                              t[1].ne[0] == hp->n_embd && t[1].ne[1] == hp->n_ff_exp && t[1].ne[2] == hp->n_expert &&
                              t[2].ne[0] == hp->n_ff_exp && t[2].ne[1] == hp->n_embd && t[2].ne[2] == hp->n_expert;
        if (!shape_ok) return set_error(LSTK_E_INVALID, "expert tensor shapes do not match the hyperparameters for layer " + std::to_string(l));
        for (int m = 0; m < 3; m++)
            if (!lstk::supported_weight_type(t[m].type))
                return set_error(LSTK_E_INVALID, "layer " + std::to_string(l) + ": " + p + names[m] + " is " + type_name(t[m].type) +
                                                     "; the expert pool stores Q8_0, Q2_K, Q3_K, Q4_K, Q5_K and Q6_K");
        layers[l].type_up = t[0].type;
        layers[l].type_gate = t[1].type;
        layers[l].type_down = t[2].type;
        layers[l].host_up = t[0].data;
        layers[l].host_gate = t[1].data;
        layers[l].host_down = t[2].data;
    }
    return LSTK_OK;
}

}  // extern "C"

namespace {

float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t) (h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else { // subnormal: normalise
            int ee = -1;
            uint32_t mm = m;
            do {
                ee++;
                mm <<= 1;
            } while ((mm & 0x400u) == 0);
            bits = sign | ((uint32_t) (127 - 15 - ee) << 23) | ((mm & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// f32 -> fp16, round to nearest even (overflow to infinity, NaN kept quiet)
uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    x &= 0x7fffffffu;
    if (x > 0x7f800000u) return (uint16_t) (sign | 0x7e00u);
    if (x >= 0x477ff000u) return (uint16_t) (sign | 0x7c00u); // rounds to above 65504
    if (x < 0x38800000u) {                                      // subnormal or zero in fp16
        if (x < 0x33000000u) return (uint16_t) sign;            // below half the smallest subnormal
        const uint32_t m = (x & 0x7fffffu) | 0x800000u;
        const int shift = 126 - (int) (x >> 23); // 14 .. 24
        const uint32_t q = m >> shift, rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        return (uint16_t) (sign | (q + (rem > half || (rem == half && (q & 1u)))));
    }
    const uint32_t q = ((x - 0x38000000u) >> 13), rem = x & 0x1fffu;
    return (uint16_t) (sign | (q + (rem > 0x1000u || (rem == 0x1000u && (q & 1u)))));
}

void scale_min_k4(int j, const uint8_t *q, int &sc, int &m) {
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

}  // namespace

extern "C" int lstk_dequant_f16(int type, const void *src, size_t n, uint16_t *dst) {
    if (!src || !dst) return set_error(LSTK_E_INVALID, "lstk_dequant_f16: null argument");
    const uint8_t *b = static_cast<const uint8_t *>(src);
    auto h16 = [](const uint8_t *p) { return (uint16_t) (p[0] | (p[1] << 8)); };
    switch (type) {
    case 0: // F32
        for (size_t i = 0; i < n; i++) {
            float f;
            std::memcpy(&f, b + 4 * i, 4);
            dst[i] = float_to_half(f);
        }
        return LSTK_OK;
    case 1: // F16
        std::memcpy(dst, src, n * 2);
        return LSTK_OK;
    case 8: // Q8_0: {fp16 d, int8 q[32]}
        if (n % 32) break;
        for (size_t blk = 0; blk < n / 32; blk++, b += 34) {
            const float d = half_to_float(h16(b));
            for (int i = 0; i < 32; i++) dst[blk * 32 + i] = float_to_half((float) (int8_t) b[2 + i] * d);
        }
        return LSTK_OK;
    case 12: // Q4_K: {fp16 d, dmin, scales[12], qs[128]}
        if (n % 256) break;
        for (size_t blk = 0; blk < n / 256; blk++, b += 144) {
            const float d = half_to_float(h16(b)), dmin = half_to_float(h16(b + 2));
            const uint8_t *sc = b + 4, *qs = b + 16;
            uint16_t *y = dst + blk * 256;
            for (int c = 0; c < 4; c++) { // 64 values: sub-blocks 2c (low nibbles) and 2c + 1 (high)
                int s0, m0, s1, m1;
                scale_min_k4(2 * c, sc, s0, m0);
                scale_min_k4(2 * c + 1, sc, s1, m1);
                const float d1 = d * (float) s0, mm1 = dmin * (float) m0, d2 = d * (float) s1, mm2 = dmin * (float) m1;
                for (int l = 0; l < 32; l++) {
                    y[64 * c + l] = float_to_half(d1 * (float) (qs[32 * c + l] & 0xF) - mm1);
                    y[64 * c + 32 + l] = float_to_half(d2 * (float) (qs[32 * c + l] >> 4) - mm2);
                }
            }
        }
        return LSTK_OK;
    case 10: // Q2_K, Q3_K, Q5_K, Q6_K: the block as integers (kq8_unpack), then (d sc) q - dmin m as ggml forms it
    case 11:
    case 13:
    case 14: {
        const size_t bb = (size_t) lstk::gguf_superblock_bytes(type);
        if (n % 256) break;
        const bool mins = type == 10 || type == 13;
        lstk::KQ8Block k;
        for (size_t blk = 0; blk < n / 256; blk++, b += bb) {
            lstk::kq8_unpack(type, b, k);
            uint16_t *y = dst + blk * 256;
            for (int v = 0; v < 256; v++) {
                const float dl = k.d * (float) k.sc[v / 16], yv = dl * (float) k.q[v];
                y[v] = float_to_half(mins ? yv - k.dmin * (float) k.m[v / 16] : yv);
            }
        }
        return LSTK_OK;
    }
    default:
        return set_error(LSTK_E_INVALID, "lstk_dequant_f16: unsupported type " + std::to_string(type));
    }
    return set_error(LSTK_E_INVALID, "lstk_dequant_f16: n is not a multiple of the type's block");
}
