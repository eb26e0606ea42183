// GGUF v3 header reader (host code). Behaviour follows GLM-SSD's crates/gguf/src/lib.rs:
// header layout and value types (lib.rs:256-292, 336-378), limits on counts, string and array
// lengths, nesting depth and alignment (lib.rs:19-31, 241-292, 351-358), checked tensor sizes and
// offsets (lib.rs:380-395), split-model discovery (lib.rs:186-231) and the split.tensors.count
// consistency check (lib.rs:153-157). Metadata values are kept as a small tagged tree.
#include <sys/stat.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "../../include/glmssd_gguf.h"

#define GG_EXPORT extern "C" __attribute__((visibility("default")))

namespace {

thread_local std::string g_err;

struct Fail {
    std::string msg;
};
[[noreturn]] void fail(const std::string &m) { throw Fail{m}; }

struct Value {
    int type = -1;      // GS_GGUF_*
    uint64_t u = 0;     // unsigned integers and bool
    int64_t i = 0;      // signed integers
    double f = 0;       // floats
    std::string s;
    int elem = -1;      // arrays: element type
    std::vector<Value> arr;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    int ty;
    int shard;
    uint64_t offset, n_bytes, row_bytes;
};

struct Model {
    std::vector<std::string> shards;
    std::map<std::string, Value> kv;
    std::vector<Tensor> tensors;
    std::map<std::string, int> by_name;
};

// (elements, bytes) per block of every type a GGUF may hold (crates/gguf/src/types.rs:87-116)
bool block_of(uint32_t id, uint64_t &be, uint64_t &bb) {
    switch (id) {
        case 0: case 26: be = 1; bb = 4; return true;     // F32, I32
        case 1: case 30: case 25: be = 1; bb = 2; return true;   // F16, BF16, I16
        case 24: be = 1; bb = 1; return true;             // I8
        case 27: case 28: be = 1; bb = 8; return true;    // I64, F64
        case 2: be = 32; bb = 18; return true;            // Q4_0
        case 3: be = 32; bb = 20; return true;            // Q4_1
        case 6: be = 32; bb = 22; return true;            // Q5_0
        case 7: be = 32; bb = 24; return true;            // Q5_1
        case 8: be = 32; bb = 34; return true;            // Q8_0
        case 20: be = 32; bb = 18; return true;           // IQ4_NL
        case 10: be = 256; bb = 84; return true;          // Q2_K
        case 11: be = 256; bb = 110; return true;         // Q3_K
        case 12: be = 256; bb = 144; return true;         // Q4_K
        case 13: be = 256; bb = 176; return true;         // Q5_K
        case 14: be = 256; bb = 210; return true;         // Q6_K
        case 15: be = 256; bb = 292; return true;         // Q8_K
        case 16: be = 256; bb = 66; return true;          // IQ2_XXS
        case 17: be = 256; bb = 74; return true;          // IQ2_XS
        case 22: be = 256; bb = 82; return true;          // IQ2_S
        case 18: be = 256; bb = 98; return true;          // IQ3_XXS
        case 21: be = 256; bb = 110; return true;         // IQ3_S
        case 19: be = 256; bb = 50; return true;          // IQ1_S
        case 29: be = 256; bb = 56; return true;          // IQ1_M
        case 23: be = 256; bb = 136; return true;         // IQ4_XS
        default: return false;
    }
}

// bytes of a row of n elements; false if n is not whole blocks or the size overflows
bool row_bytes_of(uint32_t ty, uint64_t n, uint64_t &out) {
    uint64_t be, bb;
    if (!block_of(ty, be, bb) || n % be) return false;
    return !__builtin_mul_overflow(n / be, bb, &out);
}

struct Reader {
    FILE *f;
    uint64_t pos = 0, len;
    Reader(FILE *f_, uint64_t len_) : f(f_), len(len_) {}
    uint64_t remaining() const { return len > pos ? len - pos : 0; }
    void bytes(void *p, size_t n) {
        if (n && fread(p, 1, n, f) != n) fail("unexpected end of file");
        pos += n;
    }
    template <class T>
    T get() {
        T v;
        bytes(&v, sizeof v);   // little-endian host
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (n > GS_GGUF_MAX_LEN || n > remaining()) fail("string too long (" + std::to_string(n) + " bytes)");
        std::string s(n, '\0');
        bytes(&s[0], n);
        return s;
    }
    Value value(uint32_t t, int depth) {
        Value v;
        v.type = (int)t;
        switch (t) {
            case GS_GGUF_U8: v.u = get<uint8_t>(); break;
            case GS_GGUF_I8: v.i = get<int8_t>(); break;
            case GS_GGUF_U16: v.u = get<uint16_t>(); break;
            case GS_GGUF_I16: v.i = get<int16_t>(); break;
            case GS_GGUF_U32: v.u = get<uint32_t>(); break;
            case GS_GGUF_I32: v.i = get<int32_t>(); break;
            case GS_GGUF_F32: v.f = get<float>(); break;
            case GS_GGUF_BOOL: v.u = get<uint8_t>() != 0; break;
            case GS_GGUF_STR: v.s = str(); break;
            case GS_GGUF_ARR: {
                if (depth >= 2) fail("metadata arrays nested too deeply");
                const uint32_t et = get<uint32_t>();
                const uint64_t n = get<uint64_t>();
                // every element takes at least one byte of the file
                if (n > GS_GGUF_MAX_ARR || n > remaining())
                    fail("metadata array too long (" + std::to_string(n) + " elements)");
                v.elem = (int)et;
                v.arr.reserve(n < 65536 ? n : 65536);
                for (uint64_t k = 0; k < n; k++) v.arr.push_back(value(et, depth + 1));
                break;
            }
            case GS_GGUF_U64: v.u = get<uint64_t>(); break;
            case GS_GGUF_I64: v.i = get<int64_t>(); break;
            case GS_GGUF_F64: v.f = get<double>(); break;
            default: fail("unknown GGUF value type " + std::to_string(t));
        }
        return v;
    }
};

bool is_signed(int t) { return t == GS_GGUF_I8 || t == GS_GGUF_I16 || t == GS_GGUF_I32 || t == GS_GGUF_I64; }
bool as_u64(const Value &v, uint64_t &out) {
    if (v.type == GS_GGUF_U8 || v.type == GS_GGUF_U16 || v.type == GS_GGUF_U32 || v.type == GS_GGUF_U64 ||
        v.type == GS_GGUF_BOOL) {
        out = v.u;
        return true;
    }
    if (is_signed(v.type) && v.i >= 0) {
        out = (uint64_t)v.i;
        return true;
    }
    return false;
}

// Parse one file's header; tensors get absolute offsets inside this file.
void read_header(const std::string &path, int shard, bool check_len, std::map<std::string, Value> &kv,
                 std::vector<Tensor> &tensors) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) fail("cannot open " + path);
    std::unique_ptr<FILE, int (*)(FILE *)> guard(f, fclose);
    struct stat st;
    if (fstat(fileno(f), &st) != 0) fail("cannot stat " + path);
    Reader r(f, (uint64_t)st.st_size);
    char magic[4];
    r.bytes(magic, 4);
    if (memcmp(magic, "GGUF", 4) != 0) fail("not a GGUF file");
    const uint32_t ver = r.get<uint32_t>();
    if (ver != 3) fail("unsupported GGUF version " + std::to_string(ver));
    const uint64_t n_tensors = r.get<uint64_t>(), n_kv = r.get<uint64_t>();
    if (n_tensors > GS_GGUF_MAX_COUNT || n_kv > GS_GGUF_MAX_COUNT)
        fail("implausible header: " + std::to_string(n_tensors) + " tensors, " + std::to_string(n_kv) +
             " metadata keys");
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = r.str();
        const uint32_t t = r.get<uint32_t>();
        kv[key] = r.value(t, 0);
    }
    uint64_t align = 32;
    auto it = kv.find("general.alignment");
    if (it != kv.end()) {
        uint64_t a;
        if (!as_u64(it->second, a) || a == 0 || (a & (a - 1)) || a > GS_GGUF_MAX_ALIGN)
            fail("invalid general.alignment (must be a power of two <= " + std::to_string(GS_GGUF_MAX_ALIGN) + ")");
        align = a;
    }
    struct Raw {
        std::string name;
        std::vector<uint64_t> dims;
        uint32_t ty;
        uint64_t off;
    };
    std::vector<Raw> raw;
    raw.reserve(n_tensors < 65536 ? n_tensors : 65536);
    for (uint64_t k = 0; k < n_tensors; k++) {
        Raw t;
        t.name = r.str();
        const uint32_t nd = r.get<uint32_t>();
        if (nd < 1 || nd > 4) fail("tensor " + t.name + ": " + std::to_string(nd) + " dimensions (must be 1..=4)");
        for (uint32_t d = 0; d < nd; d++) t.dims.push_back(r.get<uint64_t>());
        for (uint64_t d : t.dims)
            if (d == 0) fail("tensor " + t.name + ": zero dimension");
        t.ty = r.get<uint32_t>();
        uint64_t be, bb;
        if (!block_of(t.ty, be, bb)) fail("tensor " + t.name + ": unsupported ggml type id " + std::to_string(t.ty));
        t.off = r.get<uint64_t>();
        raw.push_back(std::move(t));
    }
    // r.pos <= file length here, so rounding up cannot overflow
    const uint64_t data_start = (r.pos + align - 1) / align * align;
    for (Raw &t : raw) {
        uint64_t rb, nb;
        bool ok = row_bytes_of(t.ty, t.dims[0], rb);
        nb = rb;
        for (size_t d = 1; ok && d < t.dims.size(); d++) ok = !__builtin_mul_overflow(nb, t.dims[d], &nb);
        if (!ok) fail("tensor " + t.name + ": bad shape for its type");
        uint64_t offset, end;
        if (__builtin_add_overflow(data_start, t.off, &offset)) fail("tensor " + t.name + ": offset overflows");
        if (__builtin_add_overflow(offset, nb, &end)) fail("tensor " + t.name + ": end overflows");
        if (check_len && end > r.len) fail("tensor " + t.name + " extends past the end of the file");
        tensors.push_back(Tensor{std::move(t.name), std::move(t.dims), (int)t.ty, shard, offset, nb, rb});
    }
}

// "foo-00002-of-00004" -> ("foo", 4); none when the pattern is absent; error when it is present
// but invalid (lib.rs:188-214)
bool split_pattern(const std::string &stem, std::string &base, int &total) {
    if (stem.size() <= 15) return false;
    const char *t = stem.data() + stem.size() - 15;
    auto digits = [](const char *p, int n) {
        for (int i = 0; i < n; i++)
            if (p[i] < '0' || p[i] > '9') return false;
        return true;
    };
    if (!(t[0] == '-' && memcmp(t + 6, "-of-", 4) == 0 && digits(t + 1, 5) && digits(t + 10, 5))) return false;
    const int idx = atoi(std::string(t + 1, 5).c_str()), tot = atoi(std::string(t + 10, 5).c_str());
    if (tot < 1 || tot > 9999) fail("invalid shard count " + std::to_string(tot) + " in " + stem);
    if (idx < 1 || idx > tot)
        fail("shard index " + std::to_string(idx) + " out of range 1..=" + std::to_string(tot) + " in " + stem);
    base = stem.substr(0, stem.size() - 15);
    total = tot;
    return true;
}

std::vector<std::string> discover_shards(const std::string &path) {
    const size_t slash = path.find_last_of('/');
    const std::string dir = slash == std::string::npos ? "" : path.substr(0, slash + 1);
    std::string name = slash == std::string::npos ? path : path.substr(slash + 1);
    if (name.size() > 5 && name.compare(name.size() - 5, 5, ".gguf") == 0) name.resize(name.size() - 5);
    std::string base;
    int total;
    if (!split_pattern(name, base, total)) return {path};
    std::vector<std::string> v;
    for (int i = 1; i <= total; i++) {
        char tail[32];
        snprintf(tail, sizeof tail, "-%05d-of-%05d.gguf", i, total);
        std::string p = dir + base + tail;
        struct stat st;
        if (stat(p.c_str(), &st) != 0) fail("missing shard " + p);
        v.push_back(p);
    }
    return v;
}

Model *open_model(const std::string &path, int mode) {
    std::unique_ptr<Model> m(new Model);
    m->shards = mode == 2 ? std::vector<std::string>{path} : discover_shards(path);
    for (size_t si = 0; si < m->shards.size(); si++) {
        std::map<std::string, Value> kv;
        read_header(m->shards[si], (int)si, mode != 1, kv, m->tensors);
        if (si == 0) m->kv = std::move(kv);
        if (m->tensors.size() > GS_GGUF_MAX_COUNT) fail("too many tensors across shards");
    }
    auto it = m->kv.find("split.tensors.count");
    uint64_t n;
    if (mode != 2 && it != m->kv.end() && as_u64(it->second, n) && n != m->tensors.size())
        fail("split.tensors.count = " + std::to_string(n) + " but found " + std::to_string(m->tensors.size()) +
             " tensors across shards");
    for (size_t i = 0; i < m->tensors.size(); i++) m->by_name[m->tensors[i].name] = (int)i;
    return m.release();
}

const Value *kv_get(void *h, const char *key) {
    if (!h || !key) return nullptr;
    Model *m = (Model *)h;
    auto it = m->kv.find(key);
    return it == m->kv.end() ? nullptr : &it->second;
}

int err(const std::string &m) {
    g_err = m;
    return GS_GGUF_ERR;
}

}  // namespace

GG_EXPORT const char *gs_gguf_error(void) { return g_err.c_str(); }

GG_EXPORT int gs_gguf_open(const char *path, int mode, void **handle) {
    if (!path || !handle || mode < 0 || mode > 2) return err("invalid argument");
    *handle = nullptr;
    try {
        *handle = open_model(path, mode);
        return 0;
    } catch (const Fail &e) {
        return err(std::string(path) + ": " + e.msg);
    } catch (const std::bad_alloc &) {
        return err(std::string(path) + ": out of memory");
    }
}

GG_EXPORT void gs_gguf_close(void *handle) { delete (Model *)handle; }

GG_EXPORT int gs_gguf_n_shards(void *handle) {
    return handle ? (int)((Model *)handle)->shards.size() : err("invalid argument");
}

GG_EXPORT int gs_gguf_shard_path(void *handle, int i, char *buf, size_t n) {
    if (!handle || !buf) return err("invalid argument");
    Model *m = (Model *)handle;
    if (i < 0 || i >= (int)m->shards.size()) return err("shard index out of range");
    if (m->shards[i].size() + 1 > n) return err("buffer too small");
    memcpy(buf, m->shards[i].c_str(), m->shards[i].size() + 1);
    return 0;
}

GG_EXPORT int gs_gguf_n_tensors(void *handle) {
    return handle ? (int)((Model *)handle)->tensors.size() : err("invalid argument");
}

GG_EXPORT int gs_gguf_tensor(void *handle, int i, GsGgufTensor *out) {
    if (!handle || !out) return err("invalid argument");
    Model *m = (Model *)handle;
    if (i < 0 || i >= (int)m->tensors.size()) return err("tensor index out of range");
    const Tensor &t = m->tensors[i];
    if (t.name.size() + 1 > GS_GGUF_NAME_MAX) return err("tensor name longer than GS_GGUF_NAME_MAX");
    memset(out, 0, sizeof *out);
    memcpy(out->name, t.name.c_str(), t.name.size() + 1);
    out->n_dims = (int)t.dims.size();
    for (size_t d = 0; d < t.dims.size(); d++) out->dims[d] = t.dims[d];
    out->ty = t.ty;
    out->shard = t.shard;
    out->offset = t.offset;
    out->n_bytes = t.n_bytes;
    out->row_bytes = t.row_bytes;
    return 0;
}

GG_EXPORT int gs_gguf_find(void *handle, const char *name) {
    if (!handle || !name) return err("invalid argument");
    Model *m = (Model *)handle;
    auto it = m->by_name.find(name);
    return it == m->by_name.end() ? err(std::string("no tensor ") + name) : it->second;
}

// lib.rs:106-111: the slice of expert e is n_bytes / last_dim bytes at offset + e * that
// (saturating arithmetic, like the reference; the parser guarantees sane inputs)
GG_EXPORT int gs_gguf_slice_range(const GsGgufTensor *t, uint64_t e, uint64_t *offset, uint64_t *n_bytes) {
    if (!t || !offset || !n_bytes) return err("invalid argument");
    uint64_t last = t->n_dims > 0 ? t->dims[t->n_dims - 1] : 1;
    if (last == 0) last = 1;
    const uint64_t per = t->n_bytes / last;
    uint64_t x, o;
    if (__builtin_mul_overflow(e, per, &x)) x = UINT64_MAX;
    if (__builtin_add_overflow(t->offset, x, &o)) o = UINT64_MAX;
    *offset = o;
    *n_bytes = per;
    return 0;
}

GG_EXPORT int gs_gguf_kv_type(void *handle, const char *key) {
    const Value *v = kv_get(handle, key);
    return v ? v->type : err(std::string("missing key ") + (key ? key : ""));
}

GG_EXPORT int gs_gguf_kv_u64(void *handle, const char *key, uint64_t *out) {
    const Value *v = kv_get(handle, key);
    if (!v || !out || !as_u64(*v, *out)) return err(std::string("missing/invalid key ") + (key ? key : ""));
    return 0;
}

GG_EXPORT int gs_gguf_kv_f64(void *handle, const char *key, double *out) {
    const Value *v = kv_get(handle, key);
    if (!v || !out) return err(std::string("missing/invalid key ") + (key ? key : ""));
    uint64_t u;
    if (v->type == GS_GGUF_F32 || v->type == GS_GGUF_F64) *out = v->f;
    else if (as_u64(*v, u)) *out = (double)u;
    else return err(std::string("missing/invalid key ") + key);
    return 0;
}

GG_EXPORT int gs_gguf_kv_str(void *handle, const char *key, char *buf, size_t n) {
    const Value *v = kv_get(handle, key);
    if (!v || !buf || v->type != GS_GGUF_STR) return err(std::string("missing/invalid key ") + (key ? key : ""));
    if (v->s.size() + 1 > n) return err("buffer too small");
    memcpy(buf, v->s.c_str(), v->s.size() + 1);
    return 0;
}

GG_EXPORT int gs_gguf_kv_arr(void *handle, const char *key, int *elem_type, uint64_t *len) {
    const Value *v = kv_get(handle, key);
    if (!v || !elem_type || !len || v->type != GS_GGUF_ARR)
        return err(std::string("missing/invalid key ") + (key ? key : ""));
    *elem_type = v->elem;
    *len = v->arr.size();
    return 0;
}
