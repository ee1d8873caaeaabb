// gguf.hip -- GGUF container reader (host code) and the upload path that
// turns a mapped model file into device weights and a resident decoder.
//
//   ParseGGUF        gguf.go:493-568 (header, metadata, tensor table,
//                    DataOffset = divCeil(pos, general.alignment) * alignment)
//   cursor           gguf.go:609-767 (bounds-checked little-endian reads,
//                    value kinds 0..12, arrays of any kind)
//   MetaValue.As*    gguf.go:303-431 (AsU32 widens every integer kind)
//   DataSize         gguf.go:241-297; inferTensorSizes model.go:2272-2310
//   OpenMmap         mmap.go:11-14 (read-only mapping, read copy otherwise)
//   loadWeight       model.go:2357-2476 (rows = dims[1], cols = dims[0];
//                    a short quantised tensor is zero-padded)
//   LoadModel        model.go:1872-1930 + ConfigFromGGUF model.go:328-420
//                    (llama: token_embd, output or tied, output_norm, blk.N.*)
//
// Nothing here touches the device except the weight uploads; the parser runs
// on any host.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "gllm_common.h"

namespace gllm {
int model_adopt_weight(gllm_hip_model* m, gllm_hip_weight* w);
void model_set_attn_scale(gllm_hip_model* m, float scale);
}

namespace {

using gllm::fail;

// One decoded metadata value, pointing into the file bytes: scalars decoded
// (u / i / f), a string as (off, len), an array as its element kind and
// count plus, for scalar elements, the offset of the packed elements, for
// strings their (off, len) list, and for nested arrays the decoded items.
struct MetaVal {
    uint32_t kind = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    size_t off = 0, len = 0;  // kStr: bytes [off, off + len); scalar arrays: elements at off
    uint32_t elem = 0;
    uint64_t count = 0;
    std::vector<std::pair<size_t, size_t>> strs;
    std::vector<MetaVal> items;
};

constexpr uint32_t kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7,
                   kStr = 8, kArr = 9, kU64 = 10, kI64 = 11, kF64 = 12;

bool is_int_kind(uint32_t k) {
    return k == kU8 || k == kI8 || k == kU16 || k == kI16 || k == kU32 || k == kI32 || k == kU64 ||
           k == kI64;
}

// Wire size of a scalar kind; 0 for strings, arrays and unknown kinds.
size_t scalar_size(uint32_t k) {
    switch (k) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
    }
}

// Decode one scalar of kind k at p into v.
void decode_scalar(uint32_t k, const uint8_t* p, MetaVal* v) {
    v->kind = k;
    switch (k) {
    case kU8: v->u = p[0]; v->i = p[0]; break;
    case kI8: v->i = (int8_t)p[0]; v->u = (uint64_t)v->i; break;
    case kBool: v->u = p[0] != 0; break;
    case kU16: { uint16_t x; memcpy(&x, p, 2); v->u = x; v->i = x; break; }
    case kI16: { int16_t x; memcpy(&x, p, 2); v->i = x; v->u = (uint64_t)v->i; break; }
    case kU32: { uint32_t x; memcpy(&x, p, 4); v->u = x; v->i = x; break; }
    case kI32: { int32_t x; memcpy(&x, p, 4); v->i = x; v->u = (uint64_t)v->i; break; }
    case kF32: { float x; memcpy(&x, p, 4); v->f = x; break; }
    case kU64: { uint64_t x; memcpy(&x, p, 8); v->u = x; v->i = (int64_t)x; break; }
    case kI64: { int64_t x; memcpy(&x, p, 8); v->i = x; v->u = (uint64_t)x; break; }
    case kF64: { double x; memcpy(&x, p, 8); v->f = x; break; }
    default: break;
    }
}

// Bounds-checked little-endian reader; every failure names the byte where
// the data ran out.
struct Reader {
    const uint8_t* p;
    size_t n, pos = 0;
    std::string err;

    bool need(uint64_t k) {
        if (k > n || pos > n - k) {
            if (err.empty()) err = "unexpected EOF at byte " + std::to_string(pos);
            return false;
        }
        return true;
    }
    template <class T>
    bool get(T* v) {
        if (!need(sizeof(T))) return false;
        memcpy(v, p + pos, sizeof(T));
        pos += sizeof(T);
        return true;
    }
    bool str(size_t* off, size_t* len) {
        uint64_t l;
        if (!get(&l) || !need(l)) return false;
        *off = pos;
        *len = (size_t)l;
        pos += (size_t)l;
        return true;
    }
    bool value(uint32_t kind, MetaVal* v, int depth) {
        v->kind = kind;
        if (const size_t w = scalar_size(kind)) {
            if (!need(w)) return false;
            decode_scalar(kind, p + pos, v);
            pos += w;
            return true;
        }
        if (kind == kStr) return str(&v->off, &v->len);
        if (kind != kArr) {
            err = "unknown GGUF value type " + std::to_string(kind);
            return false;
        }
        if (!get(&v->elem) || !get(&v->count)) return false;
        if (const size_t w = scalar_size(v->elem)) {
            if (v->count > (n - pos) / w) return need(n - pos + 1);  // EOF error
            v->off = pos;
            pos += (size_t)v->count * w;
            return true;
        }
        if (v->elem != kStr && v->elem != kArr) {
            if (v->count == 0) return true;  // no element to decode
            err = "unknown GGUF value type " + std::to_string(v->elem);
            return false;
        }
        // a string costs at least its 8-byte length, a nested array 12 bytes
        const uint64_t least = v->elem == kStr ? 8 : 12;
        if (v->count > (n - pos) / least) return need(n - pos + 1);
        if (v->elem == kStr) {
            v->strs.resize((size_t)v->count);
            for (auto& sp : v->strs)
                if (!str(&sp.first, &sp.second)) return false;
            return true;
        }
        if (depth >= 8) {
            err = "GGUF arrays nested too deeply";
            return false;
        }
        v->items.resize((size_t)v->count);
        for (auto& it : v->items)
            if (!value(kArr, &it, depth + 1)) return false;
        return true;
    }
};

}  // namespace

struct gllm_hip_gguf {
    const uint8_t* data = nullptr;
    size_t size = 0;
    bool mapped = false;   // data is an mmap of the file
    bool owned = false;    // data is a heap copy (read fallback)
    uint32_t version = 0;
    size_t data_offset = 0;
    std::unordered_map<std::string, MetaVal> meta;
    std::vector<std::string> meta_keys;  // file order (first occurrence)
    struct Tensor {
        std::string name;
        std::vector<uint64_t> dims;
        uint32_t type;
        uint64_t offset;  // relative to data_offset
        uint64_t bytes;   // DataSize, or the gap to the next tensor
    };
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, int> index;
};

namespace {

// GGMLType.DataSize (gguf.go:241-297); 0 for a type it cannot size.
uint64_t data_size(uint32_t t, uint64_t n) {
    switch (t) {
    case 0: return n * 4;                        // F32
    case 28: return n * 8;                       // F64
    case 1: case 30: return n * 2;               // F16, BF16
    case 2: case 20: return n / 32 * 18;         // Q4_0, IQ4_NL
    case 3: return n / 32 * 20;                  // Q4_1
    case 6: return n / 32 * 22;                  // Q5_0
    case 7: return n / 32 * 24;                  // Q5_1
    case 8: return n / 32 * 34;                  // Q8_0
    case 9: return n / 32 * 36;                  // Q8_1
    case 10: return n / 256 * 84;                // Q2_K
    case 11: return n / 256 * 110;               // Q3_K
    case 12: return n / 256 * 144;               // Q4_K
    case 13: return n / 256 * 176;               // Q5_K
    case 14: return n / 256 * 210;               // Q6_K
    case 15: return n / 256 * 292;               // Q8_K
    case 23: return n / 256 * 136;               // IQ4_XS
    case 22: return n / 256 * 82;                // IQ2_S
    case 21: return n / 256 * 110;               // IQ3_S
    case 16: return n / 256 * 66;                // IQ2_XXS
    case 17: return n / 256 * 74;                // IQ2_XS
    case 18: return n / 256 * 98;                // IQ3_XXS
    case 19: return n / 256 * 50;                // IQ1_S
    case 29: return n / 256 * 56;                // IQ1_M
    case 34: return n / 256 * 54;                // TQ1_0
    case 35: return n / 256 * 66;                // TQ2_0
    case 39: return n / 32 * 17;                 // MXFP4
    case 41: return n / 128 * 18;                // Q1_0
    case 42: return n / 64 * 18;                 // Q2_0
    default: return 0;
    }
}

// ggmlTypeFromUint32 (gguf.go:66-77): ids outside the known set become 255.
uint32_t known_type(uint32_t v) {
    static const uint32_t ids[] = {0, 1, 2, 3, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15, 16,
                                   17, 18, 19, 20, 21, 22, 23, 28, 29, 30, 34, 35, 39, 41, 42};
    for (uint32_t id : ids)
        if (id == v) return v;
    return 255;
}

const MetaVal* find_meta(const gllm_hip_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

bool parse(gllm_hip_gguf* g) {
    Reader r{g->data, g->size};
    if (g->size < 4) {
        fail(GLLM_EINVAL, "file too small for GGUF header");
        return false;
    }
    if (memcmp(g->data, "GGUF", 4) != 0) {
        uint32_t m;
        memcpy(&m, g->data, 4);
        fail(GLLM_EINVAL, "invalid GGUF magic: 0x%08X", m);
        return false;
    }
    r.pos = 4;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!r.get(&g->version) || !r.get(&n_tensors) || !r.get(&n_kv)) {
        fail(GLLM_EINVAL, "%s", r.err.c_str());
        return false;
    }
    for (uint64_t k = 0; k < n_kv; k++) {
        size_t ko, kl;
        uint32_t kind;
        MetaVal v;
        if (!r.str(&ko, &kl) || !r.get(&kind)) {
            fail(GLLM_EINVAL, "%s", r.err.c_str());
            return false;
        }
        const std::string key((const char*)g->data + ko, kl);
        if (!r.value(kind, &v, 0)) {
            fail(GLLM_EINVAL, "%s: %s", key.c_str(), r.err.c_str());
            return false;
        }
        if (!g->meta.count(key)) g->meta_keys.push_back(key);
        g->meta[key] = std::move(v);  // a repeated key keeps its last value
    }
    for (uint64_t k = 0; k < n_tensors; k++) {
        gllm_hip_gguf::Tensor t;
        uint32_t nd;
        size_t no, nl;
        if (!r.str(&no, &nl) || !r.get(&nd)) {
            fail(GLLM_EINVAL, "%s", r.err.c_str());
            return false;
        }
        t.name.assign((const char*)g->data + no, nl);
        if (nd > 8) {
            fail(GLLM_EINVAL, "tensor %s: %u dimensions", t.name.c_str(), nd);
            return false;
        }
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; d++)
            if (!r.get(&t.dims[d])) {
                fail(GLLM_EINVAL, "%s", r.err.c_str());
                return false;
            }
        uint32_t raw_type;
        if (!r.get(&raw_type) || !r.get(&t.offset)) {
            fail(GLLM_EINVAL, "%s", r.err.c_str());
            return false;
        }
        t.type = known_type(raw_type);
        g->tensors.push_back(std::move(t));
    }
    uint64_t align = 32;
    if (const MetaVal* a = find_meta(g, "general.alignment"))
        if (is_int_kind(a->kind) && (uint32_t)a->u > 0) align = (uint32_t)a->u;
    g->data_offset = (size_t)((r.pos + align - 1) / align * align);
    // byte sizes: DataSize, else the gap to the next tensor's offset (the
    // last one runs to the end of the file)
    std::vector<int> order(g->tensors.size());
    for (size_t k = 0; k < order.size(); k++) order[k] = (int)k;
    std::sort(order.begin(), order.end(),
              [&](int a, int b) { return g->tensors[a].offset < g->tensors[b].offset; });
    const uint64_t limit = g->size > g->data_offset ? g->size - g->data_offset : 0;
    for (size_t k = 0; k < order.size(); k++) {
        auto& t = g->tensors[order[k]];
        const uint64_t next = k + 1 < order.size() ? g->tensors[order[k + 1]].offset : limit;
        const uint64_t gap = next > t.offset ? next - t.offset : 0;
        uint64_t numel = 1;
        for (uint64_t d : t.dims) numel *= d;
        const uint64_t ds = data_size(t.type, numel);
        t.bytes = ds ? ds : gap;
    }
    for (size_t k = 0; k < g->tensors.size(); k++) g->index[g->tensors[k].name] = (int)k;
    return true;
}

gllm_hip_gguf* finish(gllm_hip_gguf* g) {
    if (parse(g)) return g;
    gllm_hip_gguf_close(g);
    return nullptr;
}

int tensor_index(const gllm_hip_gguf* g, const char* name) {
    if (!g || !name) return -1;
    auto it = g->index.find(name);
    return it == g->index.end() ? -1 : it->second;
}

// The tensor's bytes: borrowed from the mapping, or (when the file ends
// early) a zero-padded copy in `pad`, as loadWeight pads short quantised
// tensors.  Returns null when the offset lies outside the file.
const uint8_t* tensor_bytes(const gllm_hip_gguf* g, const gllm_hip_gguf::Tensor& t,
                            std::vector<uint8_t>* pad) {
    const uint64_t start = (uint64_t)g->data_offset + t.offset;
    if (start > g->size) return nullptr;
    const uint64_t have = std::min<uint64_t>(t.bytes, g->size - start);
    if (have == t.bytes) return g->data + start;
    pad->assign((size_t)t.bytes, 0);
    memcpy(pad->data(), g->data + start, (size_t)have);
    return pad->data();
}

// F16ToF32: exact widening of IEEE half bits.
float half_to_float(uint16_t h) {
    _Float16 v;
    memcpy(&v, &h, 2);
    return (float)v;
}

// loadF32Vec (model.go:2519-2528) for norm vectors: F32, F16, BF16 and F64
// storage to host floats.
int load_f32_vec(const gllm_hip_gguf* g, const char* name, std::vector<float>* out, size_t want) {
    const int i = tensor_index(g, name);
    if (i < 0) return fail(GLLM_EINVAL, "missing tensor: %s", name);
    const auto& t = g->tensors[i];
    uint64_t numel = 1;
    for (uint64_t d : t.dims) numel *= d;
    if (numel != want) return fail(GLLM_EINVAL, "tensor %s: %llu elements, want %zu", name,
                                   (unsigned long long)numel, want);
    const uint64_t start = (uint64_t)g->data_offset + t.offset;
    if (t.bytes == 0 || start > g->size || g->size - start < t.bytes)
        return fail(GLLM_EINVAL, "tensor %s exceeds file length", name);
    const uint8_t* p = g->data + start;
    out->resize(want);
    for (size_t k = 0; k < want; k++) {
        switch (t.type) {
        case 0: memcpy(&(*out)[k], p + 4 * k, 4); break;
        case 1: {
            uint16_t h;
            memcpy(&h, p + 2 * k, 2);
            (*out)[k] = half_to_float(h);
            break;
        }
        case 30: {
            uint16_t h;
            memcpy(&h, p + 2 * k, 2);
            const uint32_t b = (uint32_t)h << 16;
            memcpy(&(*out)[k], &b, 4);
            break;
        }
        case 28: {
            double d;
            memcpy(&d, p + 8 * k, 8);
            (*out)[k] = (float)d;
            break;
        }
        default: return fail(GLLM_EUNSUP, "tensor %s: type %u is not a float vector", name, t.type);
        }
    }
    return GLLM_OK;
}

}  // namespace

extern "C" {

gllm_hip_gguf* gllm_hip_gguf_open(const char* path) {
    if (!path) {
        fail(GLLM_EINVAL, "gllm_hip_gguf_open: null path");
        return nullptr;
    }
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        fail(GLLM_EINVAL, "open %s: %s", path, strerror(errno));
        return nullptr;
    }
    struct stat st;
    if (fstat(fd, &st) != 0) {
        fail(GLLM_EINVAL, "stat %s: %s", path, strerror(errno));
        close(fd);
        return nullptr;
    }
    auto* g = new gllm_hip_gguf();
    g->size = (size_t)st.st_size;
    if (g->size > 0) {
        void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m != MAP_FAILED) {
            g->data = (const uint8_t*)m;
            g->mapped = true;
        } else {
            // no mapping for this file: read it into memory instead
            auto* buf = new (std::nothrow) uint8_t[g->size];
            size_t got = 0;
            while (buf && got < g->size) {
                const ssize_t k = pread(fd, buf + got, g->size - got, (off_t)got);
                if (k <= 0) break;
                got += (size_t)k;
            }
            if (!buf || got != g->size) {
                delete[] buf;
                close(fd);
                delete g;
                fail(GLLM_EINVAL, "read %s failed", path);
                return nullptr;
            }
            g->data = buf;
            g->owned = true;
        }
    }
    close(fd);
    return finish(g);
}

gllm_hip_gguf* gllm_hip_gguf_parse(const void* data, size_t len) {
    if (!data && len) {
        fail(GLLM_EINVAL, "gllm_hip_gguf_parse: null data");
        return nullptr;
    }
    auto* g = new gllm_hip_gguf();
    g->data = (const uint8_t*)data;
    g->size = len;
    return finish(g);
}

void gllm_hip_gguf_close(gllm_hip_gguf* g) {
    if (!g) return;
    if (g->mapped) munmap((void*)g->data, g->size);
    if (g->owned) delete[] g->data;
    delete g;
}

uint32_t gllm_hip_gguf_version(const gllm_hip_gguf* g) { return g ? g->version : 0; }
size_t gllm_hip_gguf_data_offset(const gllm_hip_gguf* g) { return g ? g->data_offset : 0; }
int gllm_hip_gguf_n_tensors(const gllm_hip_gguf* g) { return g ? (int)g->tensors.size() : 0; }
int gllm_hip_gguf_n_metadata(const gllm_hip_gguf* g) { return g ? (int)g->meta_keys.size() : 0; }

const char* gllm_hip_gguf_metadata_key(const gllm_hip_gguf* g, int i) {
    if (!g || i < 0 || i >= (int)g->meta_keys.size()) return nullptr;
    return g->meta_keys[i].c_str();
}

int gllm_hip_gguf_find_tensor(const gllm_hip_gguf* g, const char* name) { return tensor_index(g, name); }

int gllm_hip_gguf_tensor(const gllm_hip_gguf* g, int i, const char** name, int* n_dims,
                         uint64_t* dims, int* type, uint64_t* offset, uint64_t* bytes) {
    if (!g || i < 0 || i >= (int)g->tensors.size())
        return fail(GLLM_EINVAL, "gllm_hip_gguf_tensor: index %d out of range", i);
    const auto& t = g->tensors[i];
    if (name) *name = t.name.c_str();
    if (n_dims) *n_dims = (int)t.dims.size();
    if (dims)
        for (size_t d = 0; d < t.dims.size(); d++) dims[d] = t.dims[d];
    if (type) *type = (int)t.type;
    if (offset) *offset = t.offset;
    if (bytes) *bytes = t.bytes;
    return GLLM_OK;
}

const void* gllm_hip_gguf_tensor_data(const gllm_hip_gguf* g, int i) {
    if (!g || i < 0 || i >= (int)g->tensors.size()) return nullptr;
    const uint64_t start = (uint64_t)g->data_offset + g->tensors[i].offset;
    return start <= g->size ? g->data + start : nullptr;
}

int gllm_hip_gguf_meta_kind(const gllm_hip_gguf* g, const char* key, int* kind, int* elem,
                            uint64_t* count) {
    const MetaVal* v = find_meta(g, key);
    if (!v) return fail(GLLM_EINVAL, "metadata %s not present", key ? key : "(null)");
    if (kind) *kind = (int)v->kind;
    if (elem) *elem = v->kind == kArr ? (int)v->elem : -1;
    if (count) *count = v->kind == kArr ? v->count : 1;
    return GLLM_OK;
}

// AsU32 (gguf.go:308-329): every integer kind, cast to uint32.
static bool as_u32(const MetaVal& v, uint32_t* out) {
    if (!is_int_kind(v.kind)) return false;
    *out = (uint32_t)v.u;
    return true;
}

// AsF32 (gguf.go:331-340): f32 and f64.
static bool as_f32(const MetaVal& v, float* out) {
    if (v.kind == kF32 || v.kind == kF64) {
        *out = (float)v.f;
        return true;
    }
    return false;
}

// The value under key (idx < 0) or element idx of the array under key.
static bool element(const gllm_hip_gguf* g, const char* key, int idx, MetaVal* out) {
    const MetaVal* v = find_meta(g, key);
    if (!v) return false;
    if (idx < 0) {
        *out = *v;
        return true;
    }
    if (v->kind != kArr || (uint64_t)idx >= v->count) return false;
    if (const size_t w = scalar_size(v->elem)) {
        decode_scalar(v->elem, g->data + v->off + (size_t)idx * w, out);
    } else if (v->elem == kStr) {
        out->kind = kStr;
        out->off = v->strs[idx].first;
        out->len = v->strs[idx].second;
    } else {
        *out = v->items[idx];
    }
    return true;
}

int gllm_hip_gguf_get_u32(const gllm_hip_gguf* g, const char* key, int idx, uint32_t* out) {
    MetaVal v;
    if (!out || !element(g, key, idx, &v) || !as_u32(v, out))
        return fail(GLLM_EINVAL, "metadata %s[%d]: no integer value", key ? key : "(null)", idx);
    return GLLM_OK;
}

int gllm_hip_gguf_get_u64(const gllm_hip_gguf* g, const char* key, int idx, uint64_t* out) {
    MetaVal v;
    if (!out || !element(g, key, idx, &v) || !is_int_kind(v.kind))
        return fail(GLLM_EINVAL, "metadata %s[%d]: no integer value", key ? key : "(null)", idx);
    *out = v.u;
    return GLLM_OK;
}

int gllm_hip_gguf_get_f32(const gllm_hip_gguf* g, const char* key, int idx, float* out) {
    MetaVal v;
    if (!out || !element(g, key, idx, &v) || !as_f32(v, out))
        return fail(GLLM_EINVAL, "metadata %s[%d]: no float value", key ? key : "(null)", idx);
    return GLLM_OK;
}

int gllm_hip_gguf_get_f64(const gllm_hip_gguf* g, const char* key, int idx, double* out) {
    MetaVal v;
    if (!out || !element(g, key, idx, &v) || (v.kind != kF32 && v.kind != kF64))
        return fail(GLLM_EINVAL, "metadata %s[%d]: no float value", key ? key : "(null)", idx);
    *out = v.f;
    return GLLM_OK;
}

int gllm_hip_gguf_get_bool(const gllm_hip_gguf* g, const char* key, int idx, int* out) {
    MetaVal v;
    if (!out || !element(g, key, idx, &v) || v.kind != kBool)
        return fail(GLLM_EINVAL, "metadata %s[%d]: no bool value", key ? key : "(null)", idx);
    *out = (int)v.u;
    return GLLM_OK;
}

int gllm_hip_gguf_get_str(const gllm_hip_gguf* g, const char* key, int idx, const char** out,
                          size_t* len) {
    MetaVal v;
    if (!out || !element(g, key, idx, &v) || v.kind != kStr)
        return fail(GLLM_EINVAL, "metadata %s[%d]: no string value", key ? key : "(null)", idx);
    *out = (const char*)g->data + v.off;
    if (len) *len = v.len;
    return GLLM_OK;
}

uint64_t gllm_hip_ggml_data_size(int type, uint64_t n) {
    return type < 0 ? 0 : data_size((uint32_t)type, n);
}

gllm_hip_weight* gllm_hip_gguf_load_weight(const gllm_hip_gguf* g, const char* name) {
    const int i = tensor_index(g, name);
    if (i < 0) {
        fail(GLLM_EINVAL, "missing tensor: %s", name ? name : "(null)");
        return nullptr;
    }
    const auto& t = g->tensors[i];
    if (t.dims.size() < 1 || t.dims.size() > 2) {
        fail(GLLM_EUNSUP, "tensor %s: %zu dimensions (a weight matrix has 1 or 2)", name,
             t.dims.size());
        return nullptr;
    }
    const uint64_t cols = t.dims[0], rows = t.dims.size() == 2 ? t.dims[1] : 1;
    if (cols > (1u << 30) || rows > (1u << 30)) {
        fail(GLLM_EINVAL, "tensor %s: %llux%llu too large", name, (unsigned long long)rows,
             (unsigned long long)cols);
        return nullptr;
    }
    std::vector<uint8_t> pad;
    const uint8_t* p = tensor_bytes(g, t, &pad);
    if (!p) {
        fail(GLLM_EINVAL, "tensor %s offset out of range", name);
        return nullptr;
    }
    return gllm_hip_weight_new(p, (size_t)t.bytes, (int)t.type, (int)rows, (int)cols);
}

gllm_hip_model* gllm_hip_model_from_gguf(const gllm_hip_gguf* g, int max_len) {
    if (!g) {
        fail(GLLM_EINVAL, "gllm_hip_model_from_gguf: null file");
        return nullptr;
    }
    const char* arch = nullptr;
    size_t alen = 0;
    if (gllm_hip_gguf_get_str(g, "general.architecture", -1, &arch, &alen) != GLLM_OK ||
        std::string(arch, alen) != "llama") {
        fail(GLLM_EUNSUP, "gllm_hip_model_from_gguf: only general.architecture = llama is supported");
        return nullptr;
    }
    // ConfigFromGGUF (model.go:328-420) for the llama.* keys this decoder uses
    auto u32 = [&](const char* k, uint32_t def) {
        uint32_t v;
        const MetaVal* m = find_meta(g, k);
        return m && as_u32(*m, &v) ? v : def;
    };
    auto f32 = [&](const char* k, float def) {
        float v;
        const MetaVal* m = find_meta(g, k);
        return m && as_f32(*m, &v) ? v : def;
    };
    gllm_hip_model_config c{};
    c.dim = (int)u32("llama.embedding_length", 0);
    c.n_heads = (int)u32("llama.attention.head_count", 0);
    c.n_kv_heads = (int)u32("llama.attention.head_count_kv", (uint32_t)std::max(1, c.n_heads));
    c.head_dim = (int)u32("llama.attention.key_length", 0);
    if (c.n_heads > 0) c.head_dim = std::max(c.head_dim, c.dim / c.n_heads);
    c.hidden = (int)u32("llama.feed_forward_length", 0);
    c.n_layers = (int)u32("llama.block_count", 0);
    c.rms_eps = f32("llama.attention.layer_norm_rms_epsilon", 1e-5f);
    c.rope_theta = f32("llama.rope.freq_base", 10000.0f);
    c.max_len = max_len > 0 ? max_len : (int)u32("llama.context_length", 2048);
    const int te = tensor_index(g, "token_embd.weight");
    if (te < 0 || g->tensors[te].dims.size() != 2) {
        fail(GLLM_EINVAL, "missing tensor: token_embd.weight");
        return nullptr;
    }
    c.vocab = (int)g->tensors[te].dims[1];
    // ConfigFromGGUF / LoadModel (model.go:400-452, 1728-1756, 1866-1869)
    // read further llama keys that change the graph.  This decoder runs the
    // plain llama graph only, so a file that sets any of them to a
    // non-default value is refused rather than decoded into other tokens.
    auto present = [&](const char* k) { return find_meta(g, k) != nullptr; };
    const char* why = nullptr;
    // buildRopeInvFreq (model.go:1729-1732) rotates the whole head when the
    // count is <= 0 or above head_dim; only 0 < count < head_dim (partial
    // rotary) changes the graph
    const int rope_dim = (int)u32("llama.rope.dimension_count", 0);
    if (present("llama.rope.dimension_count") && rope_dim > 0 && rope_dim < c.head_dim)
        why = "llama.rope.dimension_count below head_dim (partial rotary)";
    else if (present("llama.attention.value_length") &&
             (int)u32("llama.attention.value_length", 0) != c.head_dim)
        why = "llama.attention.value_length != head_dim";
    else if (f32("llama.attention.temperature_scale", 0.0f) != 0.0f)
        why = "llama.attention.temperature_scale";
    else if (u32("llama.attention.sliding_window", 0) > 0 &&
             (int)u32("llama.attention.sliding_window", 0) < c.max_len)
        why = "llama.attention.sliding_window";
    else if (f32("llama.attn_logit_softcapping", 0.0f) != 0.0f)
        why = "llama.attn_logit_softcapping";
    else if (f32("llama.final_logit_softcapping", 0.0f) != 0.0f)
        why = "llama.final_logit_softcapping";
    else if (f32("llama.embedding_scale", 0.0f) != 0.0f && f32("llama.embedding_scale", 0.0f) != 1.0f)
        why = "llama.embedding_scale";
    else if (f32("llama.residual_scale", 1.0f) != 0.0f && f32("llama.residual_scale", 1.0f) != 1.0f)
        why = "llama.residual_scale";
    else if (f32("llama.logit_scale", 1.0f) != 0.0f && f32("llama.logit_scale", 1.0f) != 1.0f)
        why = "llama.logit_scale";
    else if (tensor_index(g, "rope_factors_long.weight") >= 0 ||
             tensor_index(g, "rope_factors_short.weight") >= 0)
        why = "rope_factors_{long,short}.weight";
    else {
        const char* st = nullptr;
        size_t sl = 0;
        if (gllm_hip_gguf_get_str(g, "llama.rope.scaling.type", -1, &st, &sl) == GLLM_OK &&
            std::string(st, sl) == "yarn" && f32("llama.rope.scaling.factor", 1.0f) > 1.0f &&
            u32("llama.rope.scaling.original_context_length", 0) > 0)
            why = "llama.rope.scaling.type = yarn";
    }
    if (why) {
        fail(GLLM_EUNSUP, "gllm_hip_model_from_gguf: %s is not supported by this decoder", why);
        return nullptr;
    }
    gllm_hip_model* m = gllm_hip_model_new(&c);
    if (!m) return nullptr;
    // llama.attention.scale replaces 1/sqrt(head_dim) when set (model.go:2685-2688)
    if (f32("llama.attention.scale", 0.0f) != 0.0f)
        gllm::model_set_attn_scale(m, f32("llama.attention.scale", 0.0f));
    auto load = [&](const std::string& name, int layer, int slot) -> gllm_hip_weight* {
        gllm_hip_weight* w = gllm_hip_gguf_load_weight(g, name.c_str());
        if (!w) return nullptr;
        if (gllm::model_adopt_weight(m, w) != GLLM_OK) {
            gllm_hip_weight_release(w);
            return nullptr;
        }
        if (gllm_hip_model_set_weight(m, layer, slot, w) != GLLM_OK) return nullptr;
        return w;
    };
    auto norm = [&](const std::string& name, int layer, int slot) {
        std::vector<float> v;
        if (load_f32_vec(g, name.c_str(), &v, (size_t)c.dim) != GLLM_OK) return false;
        return gllm_hip_model_set_norm(m, layer, slot, v.data()) == GLLM_OK;
    };
    gllm_hip_weight* emb = load("token_embd.weight", 0, GLLM_T_TOK_EMBD);
    bool ok = emb != nullptr;
    if (ok) {
        if (tensor_index(g, "output.weight") >= 0)
            ok = load("output.weight", 0, GLLM_T_OUTPUT) != nullptr;
        else  // output tied to the embeddings (model.go:1888-1899)
            ok = gllm_hip_model_set_weight(m, 0, GLLM_T_OUTPUT, emb) == GLLM_OK;
    }
    ok = ok && norm("output_norm.weight", 0, GLLM_T_OUT_NORM);
    static const struct {
        const char* name;
        int slot;
    } slots[] = {{"attn_q", GLLM_T_WQ},      {"attn_k", GLLM_T_WK},   {"attn_v", GLLM_T_WV},
                 {"attn_output", GLLM_T_WO}, {"ffn_gate", GLLM_T_W1}, {"ffn_down", GLLM_T_W2},
                 {"ffn_up", GLLM_T_W3}};
    for (int l = 0; ok && l < c.n_layers; l++) {
        const std::string p = "blk." + std::to_string(l) + ".";
        for (const auto& s : slots)
            if (ok) ok = load(p + s.name + ".weight", l, s.slot) != nullptr;
        ok = ok && norm(p + "attn_norm.weight", l, GLLM_T_ATTN_NORM);
        ok = ok && norm(p + "ffn_norm.weight", l, GLLM_T_FFN_NORM);
    }
    if (!ok) {
        const std::string why = gllm_hip_last_error();
        gllm_hip_model_release(m);
        fail(GLLM_EINVAL, "%s", why.c_str());
        return nullptr;
    }
    return m;
}

}  // extern "C"
