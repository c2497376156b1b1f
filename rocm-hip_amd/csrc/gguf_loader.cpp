// gguf_loader.cpp -- GGUF v3 mapping (include/gguf_mmap.h) and the MoE layer binding / HBM upload
// (include/moe_gguf.h).
//
// GGUF v3 layout (little-endian): "GGUF", u32 version, u64 tensor count, u64 key/value count; the key/values
// (string key, u32 value type, value; strings are u64 length + bytes, arrays u32 element type + u64 count +
// elements); the tensor infos (string name, u32 n_dims, n_dims x u64 ne, u32 type, u64 offset); then, at the
// next multiple of general.alignment (32 when absent), the data section the offsets are relative to.
// The reference parses the same layout in src/gguf_mmap.cpp:185-355 (load_gguf) and joins split files in
// :386-425 (load_gguf_splits); this parser reads through a bounds-checked cursor and keeps a name index.

#include "gguf_mmap.h"
#include "moe_gguf.h"

#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "qmatvec.h"

namespace {

enum : uint32_t {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6, KV_BOOL = 7,
    KV_STRING = 8, KV_ARRAY = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12,
};

constexpr uint32_t kVersion = 3;
constexpr size_t kDefaultAlign = 32;
constexpr int kMaxSplits = 256;

// Bytes of one scalar of a numeric key/value type; 0 for string, array or an unknown type
size_t scalar_bytes(uint32_t t) {
    switch (t) {
    case KV_U8: case KV_I8: case KV_BOOL: return 1;
    case KV_U16: case KV_I16: return 2;
    case KV_U32: case KV_I32: case KV_F32: return 4;
    case KV_U64: case KV_I64: case KV_F64: return 8;
    }
    return 0;
}

// (values per block, bytes per block) of a tensor type: the public ggml block layouts, and the reference's
// ROCmFP4 (100) and FAST (101) from src/quant_types.h:46-47 and src/quant_types.cpp's trait table
bool block_layout(int type, int64_t* bv, size_t* bb) {
    struct L { int t; int64_t v; size_t b; };
    static const L tab[] = {
        {0, 1, 4}, {1, 1, 2}, {2, 32, 18}, {3, 32, 20}, {6, 32, 22}, {7, 32, 24}, {8, 32, 34}, {9, 32, 36},
        {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292},
        {16, 256, 66}, {17, 256, 74}, {18, 256, 98}, {19, 256, 50}, {20, 32, 18}, {21, 256, 110},
        {22, 256, 82}, {23, 256, 136}, {24, 1, 1}, {25, 1, 2}, {26, 1, 4}, {27, 1, 8}, {28, 1, 8},
        {29, 256, 56}, {30, 1, 2}, {34, 256, 54}, {35, 256, 66}, {39, 32, 17}, {40, 64, 36},
        {100, 32, 18}, {101, 32, 17},
    };
    for (const L& l : tab)
        if (l.t == type) {
            *bv = l.v;
            *bb = l.b;
            return true;
        }
    return false;
}

struct Tensor {
    std::string name;
    uint32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    int type = -1;
    uint64_t offset = 0;
    int split = 0;
    size_t nbytes = (size_t)-1;  // (size_t)-1: unknown type or size overflow
    const uint8_t* data = nullptr;  // NULL: unknown size or past the end of its file
};

struct Kv {
    std::string key;
    uint32_t type = 0;            // KV_* (KV_ARRAY for arrays)
    uint32_t arr_type = 0;        // element type of an array
    uint64_t arr_n = 0;
    const uint8_t* raw = nullptr;  // the scalar value, or a numeric array's first element, in the mapping
    std::string str;              // a string value
};

struct Map {
    void* base = nullptr;
    size_t size = 0;
    size_t data_off = 0;
};

thread_local std::string g_open_error;
thread_local std::string g_bind_error;

void set_open_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_open_error = buf;
}

// Bounds-checked little-endian reader over one mapped file
struct Cursor {
    const uint8_t* p;
    const uint8_t* end;
    bool ok = true;

    bool need(uint64_t n) {
        if (!ok || (uint64_t)(end - p) < n) ok = false;
        return ok;
    }
    template <typename T>
    T get() {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p, sizeof(T));
            p += sizeof(T);
        }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return std::string();
        std::string s((const char*)p, (size_t)n);
        p += n;
        return s;
    }
    void skip(uint64_t n) {
        if (need(n)) p += n;
    }
};

}  // namespace

struct gguf_model {
    std::vector<Map> maps;
    std::vector<Tensor> tensors;
    std::vector<Kv> kvs;
    std::unordered_map<std::string, int64_t> tensor_index;
    std::unordered_map<std::string, int64_t> kv_index;
    size_t alignment = kDefaultAlign;
    std::string arch;
};

namespace {

void unmap_all(gguf_model* m) {
    for (Map& mp : m->maps)
        if (mp.base) munmap(mp.base, mp.size);
    m->maps.clear();
}

// Parse one file into `kvs` / `tensors` (tensors tagged with split) and append its mapping. false: error set.
bool parse_file(const char* path, int split, gguf_model* m, std::vector<Kv>* kvs, std::vector<Tensor>* tensors,
                size_t* alignment) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) {
        set_open_error("gguf: cannot open '%s': %s", path, strerror(errno));
        return false;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        set_open_error("gguf: '%s' is too short to be GGUF", path);
        close(fd);
        return false;
    }
    const size_t size = (size_t)st.st_size;
    void* base = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (base == MAP_FAILED) {
        set_open_error("gguf: mmap of '%s' failed: %s", path, strerror(errno));
        return false;
    }
    (void)madvise(base, size, MADV_HUGEPAGE);
    m->maps.push_back(Map{base, size, 0});
    Cursor c{(const uint8_t*)base, (const uint8_t*)base + size};
    c.skip(4);  // the magic, compared in place
    const uint32_t version = c.get<uint32_t>();
    if (memcmp(base, "GGUF", 4) != 0 || version != kVersion) {
        set_open_error("gguf: '%s' is not GGUF version %u (bad magic or version %u)", path, kVersion, version);
        return false;
    }
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    // Every entry takes at least 8 bytes, so counts beyond the file size are corruption, not a huge reserve
    if (n_tensors > size / 8 || n_kv > size / 8) {
        set_open_error("gguf: corrupted header in '%s' (%llu tensors, %llu key/values)", path,
                       (unsigned long long)n_tensors, (unsigned long long)n_kv);
        return false;
    }
    size_t align = kDefaultAlign;
    kvs->reserve(kvs->size() + n_kv);
    for (uint64_t i = 0; i < n_kv && c.ok; ++i) {
        Kv kv;
        kv.key = c.str();
        kv.type = c.get<uint32_t>();
        if (kv.type == KV_STRING) {
            kv.str = c.str();
        } else if (kv.type == KV_ARRAY) {
            kv.arr_type = c.get<uint32_t>();
            kv.arr_n = c.get<uint64_t>();
            kv.raw = c.p;
            if (kv.arr_type == KV_STRING) {
                for (uint64_t j = 0; j < kv.arr_n && c.ok; ++j) c.skip(c.get<uint64_t>());
            } else {
                const size_t eb = scalar_bytes(kv.arr_type);
                if (eb == 0 || kv.arr_n > size / eb) c.ok = false;
                else c.skip(kv.arr_n * eb);
            }
        } else {
            const size_t b = scalar_bytes(kv.type);
            if (b == 0) c.ok = false;
            kv.raw = c.p;
            c.skip(b);
        }
        if (!c.ok) break;
        if (kv.key == "general.alignment") {
            // An integer power of two; anything else is a corrupted file
            uint64_t a = 0;
            if (kv.type == KV_U32) a = *(const uint32_t*)kv.raw;
            else if (kv.type == KV_U64) a = *(const uint64_t*)kv.raw;
            if (a == 0 || (a & (a - 1)) || a > (1u << 20)) {
                set_open_error("gguf: '%s' has general.alignment %llu (not a power of two)", path,
                               (unsigned long long)a);
                return false;
            }
            align = (size_t)a;
        }
        kvs->push_back(std::move(kv));
    }
    tensors->reserve(tensors->size() + n_tensors);
    for (uint64_t i = 0; i < n_tensors && c.ok; ++i) {
        Tensor t;
        t.name = c.str();
        t.n_dims = c.get<uint32_t>();
        if (t.n_dims < 1 || t.n_dims > 4) {
            c.ok = false;
            break;
        }
        for (uint32_t d = 0; d < t.n_dims; ++d) t.ne[d] = c.get<int64_t>();
        t.type = (int)c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        t.split = split;
        for (uint32_t d = 0; d < t.n_dims; ++d)
            if (t.ne[d] < 0) c.ok = false;
        tensors->push_back(std::move(t));
    }
    if (!c.ok) {
        set_open_error("gguf: corrupted structure in '%s' (header runs past the end of the file)", path);
        return false;
    }
    const size_t here = (size_t)(c.p - (const uint8_t*)base);
    const size_t data_off = (here + align - 1) / align * align;
    m->maps.back().data_off = data_off;
    if (split == 0) *alignment = align;
    return true;
}

// Sizes and data pointers of every tensor, once all files are mapped
void resolve_tensors(gguf_model* m) {
    for (size_t i = 0; i < m->tensors.size(); ++i) {
        Tensor& t = m->tensors[i];
        m->tensor_index.emplace(t.name, (int64_t)i);
        int64_t bv;
        size_t bb;
        if (!block_layout(t.type, &bv, &bb)) continue;
        // Element count with an overflow guard (a corrupted shape must not wrap to a small size)
        unsigned __int128 n = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) n *= (uint64_t)t.ne[d];
        const unsigned __int128 blocks = (n + (uint64_t)bv - 1) / (uint64_t)bv, bytes = blocks * bb;
        if (bytes > (unsigned __int128)SIZE_MAX / 2) continue;
        t.nbytes = (size_t)bytes;
        const Map& mp = m->maps[t.split];
        if (mp.data_off <= mp.size && t.offset <= mp.size - mp.data_off &&
            t.nbytes <= mp.size - mp.data_off - t.offset)
            t.data = (const uint8_t*)mp.base + mp.data_off + t.offset;
    }
}

int64_t find_kv_index(const gguf_model* m, const char* key) {
    if (!m || !key) return -1;
    const auto it = m->kv_index.find(key);
    return it == m->kv_index.end() ? -1 : it->second;
}

bool kv_as_int(const Kv& kv, int64_t* v) {
    if (kv.type == KV_ARRAY || kv.type == KV_STRING || !kv.raw) return false;
    const uint8_t* r = kv.raw;
    switch (kv.type) {
    case KV_U8: *v = *(const uint8_t*)r; return true;
    case KV_I8: *v = *(const int8_t*)r; return true;
    case KV_BOOL: *v = *(const uint8_t*)r ? 1 : 0; return true;
    case KV_U16: { uint16_t x; memcpy(&x, r, 2); *v = x; return true; }
    case KV_I16: { int16_t x; memcpy(&x, r, 2); *v = x; return true; }
    case KV_U32: { uint32_t x; memcpy(&x, r, 4); *v = x; return true; }
    case KV_I32: { int32_t x; memcpy(&x, r, 4); *v = x; return true; }
    case KV_U64: { uint64_t x; memcpy(&x, r, 8); *v = (int64_t)x; return true; }
    case KV_I64: { int64_t x; memcpy(&x, r, 8); *v = x; return true; }
    }
    return false;
}

int64_t arch_kv(const gguf_model* m, const char* suffix) {
    if (!m || !suffix || m->arch.empty()) return -1;
    return find_kv_index(m, (m->arch + "." + suffix).c_str());
}

int64_t kv_int_or(const gguf_model* m, const char* key, int64_t def) {
    const int64_t i = find_kv_index(m, key);
    int64_t v;
    return i >= 0 && kv_as_int(m->kvs[i], &v) ? v : def;
}

template <typename T>
int32_t kv_get(const gguf_model_t* m, int64_t idx, uint32_t type, T* out) {
    if (!m || !out || idx < 0 || idx >= (int64_t)m->kvs.size()) return -1;
    const Kv& kv = m->kvs[idx];
    if (kv.type != type || !kv.raw) return -1;
    memcpy(out, kv.raw, sizeof(T));
    return 0;
}

const Tensor* tensor_at(const gguf_model_t* m, int64_t idx) {
    return m && idx >= 0 && idx < (int64_t)m->tensors.size() ? &m->tensors[idx] : nullptr;
}

}  // namespace

extern "C" {

const char* gguf_last_error(void) { return g_open_error.c_str(); }

gguf_model_t* gguf_mmap_open(const char* path) {
    g_open_error.clear();
    if (!path) {
        set_open_error("gguf: NULL path");
        return nullptr;
    }
    gguf_model* m = new gguf_model();
    auto fail = [&]() -> gguf_model_t* {
        unmap_all(m);
        delete m;
        return nullptr;
    };
    if (!parse_file(path, 0, m, &m->kvs, &m->tensors, &m->alignment)) return fail();
    for (size_t i = 0; i < m->kvs.size(); ++i) m->kv_index.emplace(m->kvs[i].key, (int64_t)i);
    const int64_t ai = find_kv_index(m, "general.architecture");
    if (ai >= 0 && m->kvs[ai].type == KV_STRING) m->arch = m->kvs[ai].str;
    // A split model: <prefix>-00001-of-<count>.gguf names the first of count files, each with split.no = its index
    const int64_t count = kv_int_or(m, "split.count", 1);
    if (count > 1) {
        char suffix[64];
        snprintf(suffix, sizeof(suffix), "-00001-of-%05d.gguf", (int)count);
        const size_t pl = strlen(path), sl = strlen(suffix);
        if (count > kMaxSplits || pl < sl || strcmp(path + pl - sl, suffix) != 0) {
            set_open_error("gguf: '%s' is split in %lld files: open the first, named <prefix>%s", path,
                           (long long)count, suffix);
            return fail();
        }
        const std::string prefix(path, pl - sl);
        for (int i = 1; i < count; ++i) {
            char part_suffix[64];
            snprintf(part_suffix, sizeof(part_suffix), "-%05d-of-%05d.gguf", i + 1, (int)count);
            const std::string part = prefix + part_suffix;
            std::vector<Kv> kvs;
            size_t unused;
            if (!parse_file(part.c_str(), i, m, &kvs, &m->tensors, &unused)) return fail();
            int64_t no = -1;
            for (const Kv& kv : kvs)
                if (kv.key == "split.no") kv_as_int(kv, &no);
            if (no != i) {
                set_open_error("gguf: split %d of '%s' is not split %d: %s", i + 1, path, i + 1, part.c_str());
                return fail();
            }
        }
    }
    resolve_tensors(m);
    return m;
}

void gguf_mmap_close(gguf_model_t* model) {
    if (!model) return;
    unmap_all(model);
    delete model;
}

const void* gguf_get_tensor_ptr(const gguf_model_t* m, const char* name, size_t* out_bytes) {
    if (!m || !name || !out_bytes) return nullptr;
    const auto it = m->tensor_index.find(name);
    if (it == m->tensor_index.end()) return nullptr;
    const Tensor& t = m->tensors[it->second];
    if (!t.data) return nullptr;
    *out_bytes = t.nbytes;
    return t.data;
}

const void* gguf_mmap_get_tensor(const gguf_model_t* m, const char* name, size_t* out_bytes) {
    return gguf_get_tensor_ptr(m, name, out_bytes);
}

int64_t gguf_n_tensors(const gguf_model_t* m) { return m ? (int64_t)m->tensors.size() : 0; }

const char* gguf_tensor_name(const gguf_model_t* m, int64_t idx) {
    const Tensor* t = tensor_at(m, idx);
    return t ? t->name.c_str() : nullptr;
}

int gguf_tensor_type(const gguf_model_t* m, int64_t idx) {
    const Tensor* t = tensor_at(m, idx);
    return t ? t->type : -1;
}

int64_t* gguf_tensor_ne(const gguf_model_t* m, int64_t idx) {
    const Tensor* t = tensor_at(m, idx);
    return t ? const_cast<int64_t*>(t->ne) : nullptr;
}

uint8_t gguf_tensor_dims(const gguf_model_t* m, int64_t idx) {
    const Tensor* t = tensor_at(m, idx);
    return t ? (uint8_t)t->n_dims : 0;
}

size_t gguf_tensor_block_size(const gguf_model_t* m, int64_t idx) {
    const Tensor* t = tensor_at(m, idx);
    int64_t bv;
    size_t bb;
    return t && block_layout(t->type, &bv, &bb) ? (size_t)bv : (size_t)-1;
}

size_t gguf_tensor_type_size(const gguf_model_t* m, int64_t idx) {
    const Tensor* t = tensor_at(m, idx);
    int64_t bv;
    size_t bb;
    return t && block_layout(t->type, &bv, &bb) ? bb : (size_t)-1;
}

uint64_t gguf_tensor_offset(const gguf_model_t* m, int64_t idx) {
    const Tensor* t = tensor_at(m, idx);
    return t ? t->offset : UINT64_MAX;
}

size_t gguf_tensor_nbytes(const gguf_model_t* m, int64_t idx) {
    const Tensor* t = tensor_at(m, idx);
    return t ? t->nbytes : (size_t)-1;
}

int64_t gguf_n_kv(const gguf_model_t* m) { return m ? (int64_t)m->kvs.size() : 0; }

const char* gguf_kv_key(const gguf_model_t* m, int64_t idx) {
    return m && idx >= 0 && idx < (int64_t)m->kvs.size() ? m->kvs[idx].key.c_str() : "(null)";
}

int gguf_kv_type(const gguf_model_t* m, int64_t idx) {
    return m && idx >= 0 && idx < (int64_t)m->kvs.size() ? (int)m->kvs[idx].type : -1;
}

int32_t gguf_kv_get_u8(const gguf_model_t* m, int64_t i, uint8_t* o) { return kv_get(m, i, KV_U8, o); }
int32_t gguf_kv_get_i8(const gguf_model_t* m, int64_t i, int8_t* o) { return kv_get(m, i, KV_I8, o); }
int32_t gguf_kv_get_u16(const gguf_model_t* m, int64_t i, uint16_t* o) { return kv_get(m, i, KV_U16, o); }
int32_t gguf_kv_get_i16(const gguf_model_t* m, int64_t i, int16_t* o) { return kv_get(m, i, KV_I16, o); }
int32_t gguf_kv_get_u32(const gguf_model_t* m, int64_t i, uint32_t* o) { return kv_get(m, i, KV_U32, o); }
int32_t gguf_kv_get_i32(const gguf_model_t* m, int64_t i, int32_t* o) { return kv_get(m, i, KV_I32, o); }
int32_t gguf_kv_get_f32(const gguf_model_t* m, int64_t i, float* o) { return kv_get(m, i, KV_F32, o); }
int32_t gguf_kv_get_u64(const gguf_model_t* m, int64_t i, uint64_t* o) { return kv_get(m, i, KV_U64, o); }
int32_t gguf_kv_get_i64(const gguf_model_t* m, int64_t i, int64_t* o) { return kv_get(m, i, KV_I64, o); }
int32_t gguf_kv_get_f64(const gguf_model_t* m, int64_t i, double* o) { return kv_get(m, i, KV_F64, o); }

size_t gguf_alignment(const gguf_model_t* m) { return m ? m->alignment : 0; }
size_t gguf_data_offset(const gguf_model_t* m) { return m && !m->maps.empty() ? m->maps[0].data_off : 0; }
uint32_t gguf_version(const gguf_model_t* m) { return m ? kVersion : 0; }
const char* gguf_arch(const gguf_model_t* m) { return m ? m->arch.c_str() : ""; }

int64_t gguf_arch_int(const gguf_model_t* m, const char* suffix, int64_t def) {
    const int64_t i = arch_kv(m, suffix);
    int64_t v;
    return i >= 0 && kv_as_int(m->kvs[i], &v) ? v : def;
}

float gguf_arch_float(const gguf_model_t* m, const char* suffix, float def) {
    const int64_t i = arch_kv(m, suffix);
    if (i < 0) return def;
    const Kv& kv = m->kvs[i];
    if (kv.type == KV_F32) {
        float f;
        memcpy(&f, kv.raw, 4);
        return f;
    }
    if (kv.type == KV_F64) {
        double f;
        memcpy(&f, kv.raw, 8);
        return (float)f;
    }
    int64_t v;
    return kv_as_int(kv, &v) ? (float)v : def;
}

int64_t gguf_block_count(const gguf_model_t* m) { return gguf_arch_int(m, "block_count", 0); }

const char* gguf_kv_str_val(const gguf_model_t* m, int64_t idx) {
    if (!m || idx < 0 || idx >= (int64_t)m->kvs.size() || m->kvs[idx].type != KV_STRING) return nullptr;
    return m->kvs[idx].str.c_str();
}

int64_t gguf_find_kv(const gguf_model_t* m, const char* key) { return find_kv_index(m, key); }

int32_t gguf_kv_get_array(const gguf_model_t* m, const char* key, int32_t* out_type, const void** out_data,
                          size_t* out_count) {
    const int64_t i = find_kv_index(m, key);
    if (i < 0 || !out_type || !out_data || !out_count) return -1;
    const Kv& kv = m->kvs[i];
    if (kv.type != KV_ARRAY || kv.arr_type == KV_STRING) return -1;
    *out_type = (int32_t)kv.arr_type;
    *out_data = kv.raw;
    *out_count = (size_t)kv.arr_n;
    return 0;
}

int gguf_n_maps(const gguf_model_t* m) { return m ? (int)m->maps.size() : 0; }

const void* gguf_map_at(const gguf_model_t* m, int i, size_t* out_size) {
    if (!m || i < 0 || i >= (int)m->maps.size()) return nullptr;
    if (out_size) *out_size = m->maps[i].size;
    return m->maps[i].base;
}

}  // extern "C"

// ---------------------------------------------------------------- MoE layer binding

namespace {

bool bind_fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_bind_error = buf;
    return false;
}

// Bytes of one row of k values of a type, 0 when k is not a whole number of blocks
size_t row_bytes(int type, int64_t k) {
    int64_t bv;
    size_t bb;
    if (!block_layout(type, &bv, &bb) || k <= 0 || k % bv) return 0;
    return (size_t)(k / bv) * bb;
}

struct Bound {
    const void* p = nullptr;
    size_t bytes = 0;
    int type = -1;
    long long N = 0;  // rows: ne[1] * ne[2] (a 3-D expert stack is one matrix of all experts' rows)
    int64_t K = 0;    // ne[0]
};

// src/inference.cpp:234-262 (bind_weight): a 1- to 3-D tensor as a matrix of N rows of K values, its byte size
// checked against rows x row bytes
bool bind_matrix(const gguf_model_t* g, const std::string& name, Bound* w, bool required) {
    const auto it = g->tensor_index.find(name);
    if (it == g->tensor_index.end()) return required ? bind_fail("missing tensor %s", name.c_str()) : true;
    const Tensor& t = g->tensors[it->second];
    if (t.n_dims < 1 || t.n_dims > 3)
        return bind_fail("%s: expected a 2-D or 3-D tensor (n_dims=%u)", name.c_str(), t.n_dims);
    const int64_t K = t.ne[0];
    const long long N = (long long)t.ne[1] * t.ne[2];
    const size_t rb = row_bytes(t.type, K);
    if (rb == 0) return bind_fail("%s: type %d cannot hold rows of %lld values", name.c_str(), t.type,
                                  (long long)K);
    if (!t.data || t.nbytes != rb * (size_t)N)
        return bind_fail("%s: size %zu does not match %lld rows x %zu bytes (type %d)", name.c_str(),
                         t.data ? t.nbytes : (size_t)0, N, rb, t.type);
    w->p = t.data;
    w->bytes = t.nbytes;
    w->type = t.type;
    w->N = N;
    w->K = K;
    return true;
}

// src/inference.cpp:298-302 (check_shape)
bool check_shape(const char* what, int layer, const Bound& w, long long N, long long K) {
    if (w.N == N && w.K == K) return true;
    return bind_fail("blk.%d.%s: shape %lldx%lld, expected %lldx%lld (rows x cols)", layer, what, w.N,
                     (long long)w.K, N, K);
}

bool layer_type_ok(int t) { return t == 8 || t == 12 || t == 100 || t == 101; }

struct LayerBind {
    Bound router, gate, up, down, sgate, sup, sdown, shexp;
    bool shared = false;
    int E = 0, NE = 0, NU = 0, FE = 0, FS = 0;
};

// src/inference.cpp:519-545 plus the layer path's own limits
bool bind_layer(const gguf_model_t* g, int layer, LayerBind* b) {
    g_bind_error.clear();
    if (!g) return bind_fail("NULL model");
    if (layer < 0) return bind_fail("layer %d out of range", layer);
    auto nm = [&](const char* suffix) { return "blk." + std::to_string(layer) + "." + suffix; };
    b->E = (int)gguf_arch_int(g, "embedding_length", 0);
    b->NE = (int)gguf_arch_int(g, "expert_count", 0);
    b->NU = (int)gguf_arch_int(g, "expert_used_count", 0);
    b->FE = (int)gguf_arch_int(g, "expert_feed_forward_length", 0);
    b->FS = (int)gguf_arch_int(g, "expert_shared_feed_forward_length", 0);
    if (g->tensor_index.find(nm("ffn_gate_inp.weight")) == g->tensor_index.end())
        return bind_fail("blk.%d: not a MoE layer (no ffn_gate_inp.weight)", layer);
    b->shared = g->tensor_index.find(nm("ffn_gate_shexp.weight")) != g->tensor_index.end();
    const int E = b->E, NE = b->NE, NU = b->NU, FE = b->FE, FS = b->FS;
    if (E <= 0 || NE <= 0 || NU <= 0 || NU > NE || FE <= 0 || (b->shared ? FS <= 0 : FS != 0))
        return bind_fail("blk.%d: bad MoE hparams (embd %d experts %d used %d ff_exp %d ff_shexp %d)", layer, E, NE,
                         NU, FE, FS);
    if (!bind_matrix(g, nm("ffn_gate_inp.weight"), &b->router, true) ||
        !bind_matrix(g, nm("ffn_gate_exps.weight"), &b->gate, true) ||
        !bind_matrix(g, nm("ffn_up_exps.weight"), &b->up, true) ||
        !bind_matrix(g, nm("ffn_down_exps.weight"), &b->down, true))
        return false;
    if (!check_shape("ffn_gate_inp", layer, b->router, NE, E) ||
        !check_shape("ffn_gate_exps", layer, b->gate, (long long)NE * FE, E) ||
        !check_shape("ffn_up_exps", layer, b->up, (long long)NE * FE, E) ||
        !check_shape("ffn_down_exps", layer, b->down, (long long)NE * E, FE))
        return false;
    if (b->shared) {
        if (!bind_matrix(g, nm("ffn_gate_shexp.weight"), &b->sgate, true) ||
            !bind_matrix(g, nm("ffn_up_shexp.weight"), &b->sup, true) ||
            !bind_matrix(g, nm("ffn_down_shexp.weight"), &b->sdown, true) ||
            !check_shape("ffn_gate_shexp", layer, b->sgate, FS, E) ||
            !check_shape("ffn_up_shexp", layer, b->sup, FS, E) ||
            !check_shape("ffn_down_shexp", layer, b->sdown, E, FS))
            return false;
        // src/inference.cpp:264-296 (bind_norm): an F32 vector of E values
        const std::string gn = nm("ffn_gate_inp_shexp.weight");
        const auto it = g->tensor_index.find(gn);
        if (it == g->tensor_index.end()) return bind_fail("missing tensor %s", gn.c_str());
        const Tensor& t = g->tensors[it->second];
        if (t.type != 0 || !t.data || t.nbytes != (size_t)E * 4 || t.ne[0] != E)
            return bind_fail("%s: expected %d F32 values", gn.c_str(), E);
        b->shexp.p = t.data;
        b->shexp.bytes = t.nbytes;
        b->shexp.type = 0;
    }
    // What moe_layer_forward runs
    if (b->router.type != 0) return bind_fail("blk.%d.ffn_gate_inp: type %d, the router needs F32", layer,
                                              b->router.type);
    const int type = b->gate.type;
    if (!layer_type_ok(type)) return bind_fail("blk.%d.ffn_gate_exps: type %d is not one of 8, 12, 100, 101",
                                               layer, type);
    if (b->up.type != type || b->down.type != type ||
        (b->shared && (b->sgate.type != type || b->sup.type != type || b->sdown.type != type)))
        return bind_fail("blk.%d: expert tensors of different types (gate %d up %d down %d): the layer needs one",
                         layer, type, b->up.type, b->down.type);
    if (b->shared && FS != FE)
        return bind_fail("blk.%d: shared expert width %d differs from the experts' %d", layer, FS, FE);
    if (E % 256 || FE % 256 || NE > 1024 || NU > 64)
        return bind_fail("blk.%d: E %d and FE %d must be multiples of 256, experts <= 1024, used <= 64", layer, E,
                         FE);
    return true;
}

void fill_desc(const LayerBind& b, moe_layer_desc* d, const void* const* p) {
    d->type = b.gate.type;
    d->n_embd = b.E;
    d->n_expert = b.NE;
    d->n_used = b.NU;
    d->n_ff = b.FE;
    d->w_router = (const float*)p[0];
    d->w_gate = p[1];
    d->w_up = p[2];
    d->w_down = p[3];
    d->s_gate = b.shared ? p[4] : nullptr;
    d->s_up = b.shared ? p[5] : nullptr;
    d->s_down = b.shared ? p[6] : nullptr;
    d->w_shexp = b.shared ? (const float*)p[7] : nullptr;
}

constexpr size_t kStage = 32u << 20;  // pinned staging buffer bytes (two of them alternate)

// Copy n bytes of host memory to dst through the two pinned buffers: the memcpy into one overlaps the DMA of
// the other
hipError_t staged_copy(void* dst, const void* src, size_t n, void* const* stage, hipEvent_t* ev, int* turn,
                       hipStream_t s) {
    for (size_t o = 0; o < n; o += kStage) {
        const size_t c = n - o < kStage ? n - o : kStage;
        const int k = (*turn)++ & 1;
        hipError_t e = hipEventSynchronize(ev[k]);  // the buffer's previous copy has finished
        if (e != hipSuccess) return e;
        memcpy(stage[k], (const char*)src + o, c);
        e = hipMemcpyAsync((char*)dst + o, stage[k], c, hipMemcpyHostToDevice, s);
        if (e != hipSuccess) return e;
        e = hipEventRecord(ev[k], s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

extern "C" {

const char* moe_gguf_error(void) { return g_bind_error.c_str(); }

int moe_gguf_layer_bind(const gguf_model_t* g, int layer, moe_layer_desc* desc) {
    LayerBind b;
    if (!desc) return bind_fail("NULL desc"), -1;
    if (!bind_layer(g, layer, &b)) return -1;
    const void* p[8] = {b.router.p, b.gate.p, b.up.p, b.down.p, b.sgate.p, b.sup.p, b.sdown.p, b.shexp.p};
    fill_desc(b, desc, p);
    return 0;
}

void moe_gguf_layer_release(moe_gguf_layer* l) {
    if (!l) return;
    if (l->packed) {
        const void* w[6] = {l->desc.w_gate, l->desc.w_up, l->desc.w_down, l->desc.s_gate, l->desc.s_up,
                            l->desc.s_down};
        for (const void* p : w)
            if (p) (void)qmatvec_unpack_weights(p);  // (the device copy is freed next either way)
    }
    if (l->dev) (void)hipFree(l->dev);
    memset(l, 0, sizeof(*l));
}

hipError_t moe_gguf_layer_upload(const gguf_model_t* g, int layer, int pack, moe_gguf_layer* out,
                                 hipStream_t stream) {
    if (!out) return bind_fail("NULL layer"), hipErrorInvalidValue;
    memset(out, 0, sizeof(*out));
    LayerBind b;
    if (!bind_layer(g, layer, &b)) return hipErrorInvalidValue;
    const Bound* parts[8] = {&b.router, &b.gate, &b.up, &b.down, &b.sgate, &b.sup, &b.sdown, &b.shexp};
    size_t off[8], total = 0;
    for (int i = 0; i < 8; ++i) {
        off[i] = total;
        total += (parts[i]->bytes + 255) & ~(size_t)255;
    }
    hipError_t e = hipMalloc(&out->dev, total);
    if (e != hipSuccess) {
        out->dev = nullptr;
        bind_fail("hipMalloc of %zu bytes failed", total);
        return e;
    }
    out->dev_bytes = total;
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    int turn = 0;
    e = hipHostMalloc(&stage[0], kStage, hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostMalloc(&stage[1], kStage, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[0], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[1], hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(ev[0], stream);
    if (e == hipSuccess) e = hipEventRecord(ev[1], stream);
    for (int i = 0; i < 8 && e == hipSuccess; ++i)
        if (parts[i]->bytes)
            e = staged_copy((char*)out->dev + off[i], parts[i]->p, parts[i]->bytes, stage, ev, &turn, stream);
    const hipError_t es = hipStreamSynchronize(stream);
    if (e == hipSuccess) e = es;
    for (int k = 0; k < 2; ++k) {
        if (ev[k]) (void)hipEventDestroy(ev[k]);
        if (stage[k]) (void)hipHostFree(stage[k]);
    }
    const void* p[8];
    for (int i = 0; i < 8; ++i) p[i] = parts[i]->bytes ? (const char*)out->dev + off[i] : nullptr;
    fill_desc(b, &out->desc, p);
    if (e == hipSuccess && (pack < 0 || pack > 4)) e = hipErrorInvalidValue;
    if (e == hipSuccess && pack) {
        out->packed = 1;
        const Bound* mats[6] = {&b.gate, &b.up, &b.down, &b.sgate, &b.sup, &b.sdown};
        for (int i = 0; i < 6 && e == hipSuccess; ++i)
            if (mats[i]->bytes)
                e = qmatvec_pack_weights_ex(mats[i]->type, (void*)p[1 + i], row_bytes(mats[i]->type, mats[i]->K),
                                            mats[i]->N, (int)mats[i]->K, pack - 1, stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
    }
    if (e != hipSuccess) {
        bind_fail("upload of blk.%d failed: %s", layer, hipGetErrorString(e));
        moe_gguf_layer_release(out);
    }
    return e;
}

}  // extern "C"
