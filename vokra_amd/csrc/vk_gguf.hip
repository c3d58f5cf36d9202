// vk_gguf.hip — GGUF v3 reader over a read-only mmap (host code), and the
// upload of its block-quant tensors into resident device weights.
//
// Format (crates/vokra-core/src/gguf/mod.rs:1-100, reader.rs:333-510): "GGUF",
// u32 version 3, u64 tensor_count, u64 kv_count, kv_count typed key/values,
// tensor_count infos (name, u32 n_dims <= 8, u64 dims, u32 ggml type, u64
// offset), then the data region at the next multiple of general.alignment
// (default 32); every tensor offset is a multiple of it and its payload lies
// inside the file. The checks and their order follow the reference reader;
// the accepted tensor types are the ones this library computes with: F32 (0),
// F16 (1), Q4_0 (2), Q5_0 (6), Q8_0 (8), Q4_K (12). The reference itself
// rejects Q4_0 / Q5_0 / Q8_0 (crates/vokra-core/src/gguf/tensor.rs:85-95);
// loading them is the block-format route its Whisper loader names
// (crates/vokra-models/src/whisper/weights.rs:454-509).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/vokra_hip.h"
#include "vk_launch.h"

namespace {

constexpr uint32_t kGgufVersion = 3;
constexpr uint64_t kDefaultAlignment = 32;
constexpr size_t kMaxDims = 8;
constexpr int kMaxArrayDepth = 64;

struct Meta {
    int type = 0;            // GGUF value type tag
    int64_t i = 0;           // integer types and bool
    double f = 0.0;          // float types
    std::string s;           // string
    uint64_t array_len = 0;  // arrays: element count (elements are skipped)
    int array_type = -1;
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0, nbytes = 0;
};

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return vk::ctx_fail(code, "%s", buf);
}

// Bytes per block and elements per block of the accepted tensor types.
bool type_geometry(uint32_t t, uint64_t* block_elems, uint64_t* block_bytes) {
    switch (t) {
    case 0: *block_elems = 1; *block_bytes = 4; return true;      // F32
    case 1: *block_elems = 1; *block_bytes = 2; return true;      // F16
    case 2: *block_elems = 32; *block_bytes = 18; return true;    // Q4_0
    case 6: *block_elems = 32; *block_bytes = 22; return true;    // Q5_0
    case 8: *block_elems = 32; *block_bytes = 34; return true;    // Q8_0
    case 12: *block_elems = 256; *block_bytes = 144; return true; // Q4_K
    default: return false;
    }
}

struct Reader {
    const uint8_t* p;
    size_t n, pos = 0;
    size_t remaining() const { return n - pos; }
    bool take(size_t k, const uint8_t** out) {
        if (k > remaining()) return false;
        *out = p + pos;
        pos += k;
        return true;
    }
    template <class T>
    bool num(T* v) {
        const uint8_t* b;
        if (!take(sizeof(T), &b)) return false;
        memcpy(v, b, sizeof(T));  // little-endian file on a little-endian host
        return true;
    }
};

}  // namespace

struct vokra_hip_gguf {
    const uint8_t* base = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = kDefaultAlignment, data_offset = 0;
    std::vector<std::pair<std::string, Meta>> meta;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
    void unmap() {
        if (base) munmap(const_cast<uint8_t*>(base), size ? size : 1);
        base = nullptr;
    }
};

namespace {

int read_string(Reader& r, std::string* s, const char* what) {
    uint64_t len;
    const uint8_t* b;
    if (!r.num(&len)) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (%s)", what);
    if (len > r.remaining() || !r.take((size_t)len, &b)) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (%s)", what);
    s->assign((const char*)b, (size_t)len);
    return VOKRA_HIP_OK;
}

// One value payload of type t (reader.rs:454-482). Arrays keep their length
// and element type; their elements are validated and skipped.
int read_value(Reader& r, int t, int depth, Meta* m) {
    m->type = t;
    switch (t) {
    case 0: { uint8_t v; if (!r.num(&v)) break; m->i = v; return VOKRA_HIP_OK; }
    case 1: { int8_t v; if (!r.num(&v)) break; m->i = v; return VOKRA_HIP_OK; }
    case 2: { uint16_t v; if (!r.num(&v)) break; m->i = v; return VOKRA_HIP_OK; }
    case 3: { int16_t v; if (!r.num(&v)) break; m->i = v; return VOKRA_HIP_OK; }
    case 4: { uint32_t v; if (!r.num(&v)) break; m->i = v; return VOKRA_HIP_OK; }
    case 5: { int32_t v; if (!r.num(&v)) break; m->i = v; return VOKRA_HIP_OK; }
    case 6: { float v; if (!r.num(&v)) break; m->f = v; return VOKRA_HIP_OK; }
    case 7: {
        uint8_t v;
        if (!r.num(&v)) break;
        if (v > 1) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: invalid bool %u", v);
        m->i = v;
        return VOKRA_HIP_OK;
    }
    case 8: return read_string(r, &m->s, "string");
    case 9: {
        if (depth >= kMaxArrayDepth) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: array nesting too deep");
        uint32_t et;
        uint64_t len;
        if (!r.num(&et) || !r.num(&len)) break;
        if (et > 12) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: unknown value type %u", et);
        if (len > r.remaining()) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (array length exceeds file size)");
        m->array_len = len;
        m->array_type = (int)et;
        Meta e;
        for (uint64_t i = 0; i < len; ++i) {
            int st = read_value(r, (int)et, depth + 1, &e);
            if (st) return st;
        }
        return VOKRA_HIP_OK;
    }
    case 10: { uint64_t v; if (!r.num(&v)) break; m->i = (int64_t)v; return VOKRA_HIP_OK; }
    case 11: { int64_t v; if (!r.num(&v)) break; m->i = v; return VOKRA_HIP_OK; }
    case 12: { double v; if (!r.num(&v)) break; m->f = v; return VOKRA_HIP_OK; }
    default: return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: unknown value type %d", t);
    }
    return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated value");
}

int parse(vokra_hip_gguf* f) {
    Reader r{f->base, f->size};
    const uint8_t* magic;
    if (!r.take(4, &magic)) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (magic)");
    if (memcmp(magic, "GGUF", 4) != 0) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: bad magic");
    uint64_t n_tensors, n_kv;
    if (!r.num(&f->version)) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (version)");
    if (f->version != kGgufVersion) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: unsupported version %u", f->version);
    if (!r.num(&n_tensors) || !r.num(&n_kv)) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (counts)");
    if (n_tensors > r.remaining() || n_kv > r.remaining())
        return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (declared count exceeds file size)");
    for (uint64_t i = 0; i < n_kv; ++i) {
        std::string key;
        uint32_t t;
        Meta m;
        int st = read_string(r, &key, "metadata key");
        if (st) return st;
        if (!r.num(&t)) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (value type)");
        if ((st = read_value(r, (int)t, 0, &m))) return st;
        f->meta.emplace_back(std::move(key), std::move(m));
    }
    for (const auto& kv : f->meta)  // general.alignment (reader.rs:431-446)
        if (kv.first == "general.alignment") {
            const Meta& m = kv.second;
            const bool integer = m.type <= 5 || m.type == 10 || m.type == 11;
            if (!integer) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: general.alignment is not an integer");
            const uint64_t a = (uint64_t)m.i;
            if (m.i <= 0 || (a & (a - 1))) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: invalid alignment %lld", (long long)m.i);
            f->alignment = a;
            break;
        }
    for (uint64_t i = 0; i < n_tensors; ++i) {
        Tensor t;
        uint32_t nd;
        int st = read_string(r, &t.name, "tensor name");
        if (st) return st;
        if (!r.num(&nd)) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (tensor n_dims)");
        if (nd > kMaxDims) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: tensor '%s' has %u dimensions", t.name.c_str(), nd);
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; ++d)
            if (!r.num(&t.dims[d])) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (tensor dim)");
        if (!r.num(&t.type) || !r.num(&t.offset)) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: truncated (tensor type / offset)");
        uint64_t be, bb;
        if (!type_geometry(t.type, &be, &bb))
            return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: tensor '%s' has unsupported ggml type %u", t.name.c_str(), t.type);
        if (f->by_name.count(t.name)) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: duplicate tensor '%s'", t.name.c_str());
        uint64_t n = 1;
        for (uint64_t d : t.dims) {
            if (d != 0 && n > UINT64_MAX / d) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: tensor size overflows");
            n *= d;
        }
        if (n % be != 0)
            return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: tensor '%s': %llu elements is not a whole number of %llu-element blocks",
                        t.name.c_str(), (unsigned long long)n, (unsigned long long)be);
        if (n / be > UINT64_MAX / bb) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: tensor size overflows");
        t.nbytes = n / be * bb;
        f->by_name[t.name] = f->tensors.size();
        f->tensors.push_back(std::move(t));
    }
    const uint64_t a = f->alignment;
    f->data_offset = (r.pos + a - 1) / a * a;
    if (!f->tensors.empty() && f->data_offset > f->size)
        return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: tensor-data region starts past end of file");
    for (const Tensor& t : f->tensors) {
        if (t.offset % a != 0)
            return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: tensor '%s' offset %llu is not a multiple of %llu", t.name.c_str(),
                        (unsigned long long)t.offset, (unsigned long long)a);
        const uint64_t start = f->data_offset + t.offset;
        if (start < t.offset || start + t.nbytes < start || start + t.nbytes > f->size)
            return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: tensor '%s' lies outside the file", t.name.c_str());
    }
    return VOKRA_HIP_OK;
}

// IEEE binary16 -> f32, exact (crates/vokra-core/src/gguf/quant/mod.rs:108-125).
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, ex = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu, bits;
    if (ex == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: man * 2^-24, renormalised
            int e = -1;
            do {
                ++e;
                man <<= 1;
            } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(112 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

const Tensor* find(const vokra_hip_gguf* f, const char* name) {
    if (!f || !name) return nullptr;
    auto it = f->by_name.find(name);
    return it == f->by_name.end() ? nullptr : &f->tensors[it->second];
}

const Meta* find_meta(const vokra_hip_gguf* f, const char* key) {
    if (!f || !key) return nullptr;
    for (const auto& kv : f->meta)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

}  // namespace

extern "C" {

int vokra_hip_gguf_open(const char* path, vokra_hip_gguf_t** out) {
    if (!path || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf_open: NULL argument");
    *out = nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(VOKRA_HIP_ERROR_IO, "gguf_open: cannot open '%s': %s", path, strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        close(fd);
        return fail(VOKRA_HIP_ERROR_IO, "gguf_open: cannot stat '%s'", path);
    }
    auto* f = new vokra_hip_gguf();
    f->size = (size_t)sb.st_size;
    void* m = mmap(nullptr, f->size ? f->size : 1, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) {
        delete f;
        return fail(VOKRA_HIP_ERROR_IO, "gguf_open: cannot map '%s'", path);
    }
    f->base = (const uint8_t*)m;
    const int st = parse(f);
    if (st) {
        f->unmap();
        delete f;
        return st;
    }
    *out = f;
    return VOKRA_HIP_OK;
}

void vokra_hip_gguf_close(vokra_hip_gguf_t* f) {
    if (!f) return;
    f->unmap();
    delete f;
}

int vokra_hip_gguf_tensor_count(const vokra_hip_gguf_t* f, size_t* n) {
    if (!f || !n) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf_tensor_count: NULL argument");
    *n = f->tensors.size();
    return VOKRA_HIP_OK;
}

int vokra_hip_gguf_tensor_info(const vokra_hip_gguf_t* f, size_t index, const char** name, uint32_t* ggml_type,
                               size_t* n_dims, uint64_t* dims, const void** data, size_t* n_bytes) {
    if (!f) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf_tensor_info: NULL file");
    if (index >= f->tensors.size()) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf_tensor_info: index out of range");
    const Tensor& t = f->tensors[index];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = t.type;
    if (n_dims) *n_dims = t.dims.size();
    if (dims)
        for (size_t d = 0; d < t.dims.size(); ++d) dims[d] = t.dims[d];
    if (data) *data = f->base + f->data_offset + t.offset;
    if (n_bytes) *n_bytes = (size_t)t.nbytes;
    return VOKRA_HIP_OK;
}

int vokra_hip_gguf_find(const vokra_hip_gguf_t* f, const char* name, size_t* index) {
    if (!f || !name || !index) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf_find: NULL argument");
    auto it = f->by_name.find(name);
    if (it == f->by_name.end()) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: missing tensor '%s'", name);
    *index = it->second;
    return VOKRA_HIP_OK;
}

int vokra_hip_gguf_meta_int(const vokra_hip_gguf_t* f, const char* key, int64_t* out) {
    const Meta* m = find_meta(f, key);
    if (!m || !out) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: missing metadata key '%s'", key ? key : "(null)");
    if (!(m->type <= 5 || m->type == 7 || m->type == 10 || m->type == 11))
        return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: metadata '%s' is not an integer", key);
    *out = m->i;
    return VOKRA_HIP_OK;
}

int vokra_hip_gguf_meta_str(const vokra_hip_gguf_t* f, const char* key, const char** out, size_t* len) {
    const Meta* m = find_meta(f, key);
    if (!m || !out) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: missing metadata key '%s'", key ? key : "(null)");
    if (m->type != 8) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: metadata '%s' is not a string", key);
    *out = m->s.c_str();
    if (len) *len = m->s.size();
    return VOKRA_HIP_OK;
}

int vokra_hip_gguf_upload_qweight(vokra_hip_ctx_t* c, const vokra_hip_gguf_t* f, const char* name,
                                  vokra_hip_qweight_t** out) {
    if (!c || !f || !name || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf_upload_qweight: NULL argument");
    const Tensor* t = find(f, name);
    if (!t) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: missing tensor '%s'", name);
    if (t->type != 2 && t->type != 6 && t->type != 8 && t->type != 12)
        return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "gguf: tensor '%s' (ggml type %u) is not a block-quant weight", name,
                    t->type);
    if (t->dims.size() != 2)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf: weight '%s' must be 2-D, has %zu dims", name, t->dims.size());
    // ggml order: dims[0] = row length (in features), dims[1] = rows (out features)
    const size_t k = (size_t)t->dims[0], n = (size_t)t->dims[1];
    return vokra_hip_qweight_upload(c, (int)t->type, n, k, f->base + f->data_offset + t->offset, (size_t)t->nbytes, out);
}

int vokra_hip_gguf_read_f32(const vokra_hip_gguf_t* f, const char* name, float* out, size_t out_len) {
    if (!f || !name || (!out && out_len)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf_read_f32: NULL argument");
    const Tensor* t = find(f, name);
    if (!t) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: missing tensor '%s'", name);
    if (t->type != 0 && t->type != 1)
        return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "gguf: tensor '%s' (ggml type %u) is not F32/F16", name, t->type);
    const size_t n = (size_t)t->nbytes / (t->type == 0 ? 4 : 2);
    if (out_len != n) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf: tensor '%s' has %zu elements, not %zu", name, n, out_len);
    const uint8_t* p = f->base + f->data_offset + t->offset;
    if (t->type == 0) {
        memcpy(out, p, n * 4);
    } else {
        for (size_t i = 0; i < n; ++i) {
            uint16_t h;
            memcpy(&h, p + 2 * i, 2);
            out[i] = f16_to_f32(h);
        }
    }
    return VOKRA_HIP_OK;
}

}  // extern "C"
