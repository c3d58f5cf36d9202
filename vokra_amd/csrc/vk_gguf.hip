// vk_gguf.hip — GGUF v3 reader over a read-only mmap (host code), and the
// upload of its block-quant tensors into resident device weights.
//
// Format (crates/vokra-core/src/gguf/mod.rs:1-100, reader.rs:333-510): "GGUF",
// u32 version 3, u64 tensor_count, u64 kv_count, kv_count typed key/values,
// tensor_count infos (name, u32 n_dims <= 8, u64 dims, u32 ggml type, u64
// offset), then the data region at the next multiple of general.alignment
// (default 32); every tensor offset is a multiple of it and its payload lies
// inside the file. The checks and their order follow the reference reader;
// the accepted tensor types are the reference's (F32 0, F16 1, Q4_K 12, Q5_K
// 13, Q6_K 14, BF16 30; tensor.rs:85-95) and the block formats this library
// also computes with: Q4_0 (2), Q5_0 (6), Q8_0 (8). The reference itself
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
#include <initializer_list>
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
    uint64_t array_len = 0;  // arrays: element count
    int array_type = -1;
    std::vector<int64_t> ints;  // top-level arrays of integers: the elements
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
    case 13: *block_elems = 256; *block_bytes = 176; return true; // Q5_K
    case 14: *block_elems = 256; *block_bytes = 210; return true; // Q6_K
    case 30: *block_elems = 1; *block_bytes = 2; return true;     // BF16
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
        const bool keep = depth == 0 && (et <= 5 || et == 10 || et == 11);
        Meta e;
        for (uint64_t i = 0; i < len; ++i) {
            int st = read_value(r, (int)et, depth + 1, &e);
            if (st) return st;
            if (keep) m->ints.push_back(e.i);
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
    // dims as the reference's loader reads a Linear weight (whisper/weights.rs:460-470):
    // [out_features, in_features], rows of in_features values back to back
    const size_t n = (size_t)t->dims[0], k = (size_t)t->dims[1];
    return vokra_hip_qweight_upload(c, (int)t->type, n, k, f->base + f->data_offset + t->offset, (size_t)t->nbytes, out);
}

int vokra_hip_gguf_read_f32(const vokra_hip_gguf_t* f, const char* name, float* out, size_t out_len) {
    if (!f || !name || (!out && out_len)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf_read_f32: NULL argument");
    const Tensor* t = find(f, name);
    if (!t) return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "gguf: missing tensor '%s'", name);
    if (t->type != 0 && t->type != 1 && t->type != 30)
        return fail(VOKRA_HIP_ERROR_UNSUPPORTED_OP, "gguf: tensor '%s' (ggml type %u) is not F32/F16/BF16", name, t->type);
    const size_t n = (size_t)t->nbytes / (t->type == 0 ? 4 : 2);
    if (out_len != n) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "gguf: tensor '%s' has %zu elements, not %zu", name, n, out_len);
    const uint8_t* p = f->base + f->data_offset + t->offset;
    if (t->type == 0) {
        memcpy(out, p, n * 4);
    } else if (t->type == 30) {
        // bf16 -> f32 is exact: the 16 bits become the high half
        for (size_t i = 0; i < n; ++i) {
            uint16_t h;
            memcpy(&h, p + 2 * i, 2);
            const uint32_t bits = (uint32_t)h << 16;
            memcpy(out + i, &bits, 4);
        }
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

// ---- Whisper sessions straight from a GGUF file ------------------------------
//
// WhisperConfig::from_gguf (crates/vokra-models/src/whisper/config.rs:106-170)
// and WhisperWeights::load_with (whisper/weights.rs:302-378) with
// fused_quant_weights: the tensor names, the expected shapes (PyTorch order,
// [out_features, in_features] for a Linear) and the order in which they are
// checked follow the reference, so the first bad tensor is the one it names.
// A Linear already in the session's block dtype is handed to the session
// straight from the mapping; an F32/F16 Linear is packed to Q8_0/Q4_0/Q5_0 on
// the device (pack_matrix_to_bytes, kv_quant/dequant_gemm.rs:137-186).
// Norms, biases, embeddings and the conv stem decode to f32.

namespace {

bool unsigned_meta(int t) { return t == 0 || t == 2 || t == 4 || t == 10; }

int cfg_bad(const char* fmt, ...) {
    char buf[400];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "whisper config: %s", buf);
}

int req_u32(const vokra_hip_gguf* f, const char* key, size_t* out) {
    const Meta* m = find_meta(f, key);
    if (!m) return cfg_bad("missing metadata key `%s`", key);
    if (!unsigned_meta(m->type) || (uint64_t)m->i > UINT32_MAX)
        return cfg_bad("metadata key `%s` is not a u32-range integer", key);
    *out = (size_t)(uint64_t)m->i;
    return VOKRA_HIP_OK;
}

// A u32 array's length after checking its elements (config.rs:189-203).
int req_u32_array(const vokra_hip_gguf* f, const char* key, size_t* len) {
    const Meta* m = find_meta(f, key);
    if (!m) return cfg_bad("missing metadata key `%s`", key);
    if (m->type != 9) return cfg_bad("metadata key `%s` is not an array", key);
    if (!unsigned_meta(m->array_type) && m->array_len) return cfg_bad("`%s` element is not a u32-range integer", key);
    for (int64_t v : m->ints)
        if ((uint64_t)v > UINT32_MAX) return cfg_bad("`%s` element is not a u32-range integer", key);
    *len = (size_t)m->array_len;
    return VOKRA_HIP_OK;
}

// The optional (layer, head) pairs (config.rs:205-240): absent is fine,
// anything present must be an even-length unsigned array of in-range layers.
int opt_pair_array(const vokra_hip_gguf* f, const char* key, size_t n_layer) {
    const Meta* m = find_meta(f, key);
    if (!m) return VOKRA_HIP_OK;
    if (m->type != 9) return cfg_bad("metadata key `%s` is not an array", key);
    if (m->array_len % 2)
        return cfg_bad("`%s` must be an even-length (layer, head) pair array, got %llu", key,
                       (unsigned long long)m->array_len);
    if (!unsigned_meta(m->array_type) && m->array_len) return cfg_bad("`%s` element is not a usize-range integer", key);
    for (size_t i = 0; i + 1 < m->ints.size(); i += 2)
        if ((uint64_t)m->ints[i] >= n_layer)
            return cfg_bad("`%s` layer index %llu >= n_text_layer %zu", key, (unsigned long long)(uint64_t)m->ints[i],
                           n_layer);
    return VOKRA_HIP_OK;
}

// ---- VoxtralConfig::from_gguf (crates/vokra-models/src/voxtral/config.rs:
// 155-267): required keys fail with "missing metadata key", optional ones
// read as 0 when absent or not of the accessor's type (as_u64 takes the
// unsigned integers, as_f64 the two float types).
int vox_bad(const char* fmt, ...) {
    char buf[400];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "voxtral config: %s", buf);
}

int vox_req_u32(const vokra_hip_gguf* f, const char* key, size_t* out) {
    const Meta* m = find_meta(f, key);
    if (!m) return vox_bad("missing metadata key `%s`", key);
    if (!unsigned_meta(m->type) || (uint64_t)m->i > UINT32_MAX)
        return vox_bad("metadata key `%s` is not a u32-range integer", key);
    *out = (size_t)(uint64_t)m->i;
    return VOKRA_HIP_OK;
}

size_t vox_opt_u32(const vokra_hip_gguf* f, const char* key) {
    const Meta* m = find_meta(f, key);
    return (m && unsigned_meta(m->type) && (uint64_t)m->i <= UINT32_MAX) ? (size_t)(uint64_t)m->i : 0;
}

float vox_opt_f32(const vokra_hip_gguf* f, const char* key) {
    const Meta* m = find_meta(f, key);
    return (m && (m->type == 6 || m->type == 12)) ? (float)m->f : 0.0f;
}

std::string dims_str(const uint64_t* d, size_t n) {
    std::string s = "[";
    for (size_t i = 0; i < n; ++i) {
        if (i) s += ", ";
        s += std::to_string((unsigned long long)d[i]);
    }
    return s + "]";
}

// A tensor error in the wording of the loader being mirrored: Whisper
// (weights.rs: "whisper weight `name`: ...") or the text decoder
// (text_decoder.rs:1486-1496: "voxtral text_decoder: `name` missing from
// GGUF", "... `name` shape [..] != expected [..]", other failures
// "`name`: ...").
int tensor_err(bool vox, int code, const std::string& name, const char* fmt, ...) {
    char buf[400];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    if (!vox) return fail(code, "whisper weight `%s`: %s", name.c_str(), buf);
    const bool bare = !strncmp(buf, "missing", 7) || !strncmp(buf, "shape", 5);
    return fail(code, "voxtral text_decoder: `%s`%s%s", name.c_str(), bare ? " " : ": ", buf);
}

// Owns the f32 decodes and packed weights until the session has uploaded them.
struct Loader {
    vokra_hip_ctx_t* ctx;
    const vokra_hip_gguf* f;
    int wdtype;
    bool vox = false;  // the text decoder's wording (else Whisper's)
    std::vector<std::vector<float>> floats;
    std::vector<std::vector<uint8_t>> packed;
    size_t verbatim = 0, n_packed = 0;

    // Presence and shape, as weights.rs:400-410 / text_decoder.rs:1486-1493 check them.
    int shaped(const std::string& name, std::initializer_list<uint64_t> want, const Tensor** out) {
        const Tensor* t = find(f, name.c_str());
        if (!t) return tensor_err(vox, VOKRA_HIP_ERROR_MODEL_LOAD, name, "missing from GGUF");
        const std::vector<uint64_t> w(want);
        if (t->dims != w)
            return tensor_err(vox, VOKRA_HIP_ERROR_MODEL_LOAD, name, "shape %s != expected %s",
                              dims_str(t->dims.data(), t->dims.size()).c_str(), dims_str(w.data(), w.size()).c_str());
        *out = t;
        return VOKRA_HIP_OK;
    }

    // The tensor widened to f32, as GgufFile::tensor_f32 does: F32 as
    // stored, F16 exactly, Q4_K through the device dequantizer (bit-exact
    // with gguf/quant/q4_k.rs:34-69).
    int f32(const std::string& name, std::initializer_list<uint64_t> want, const float** out) {
        const Tensor* t;
        int st = shaped(name, want, &t);
        if (st) return st;
        if (t->type == VOKRA_HIP_W_Q4_K || t->type == VOKRA_HIP_W_Q5_K || t->type == VOKRA_HIP_W_Q6_K) {
            const size_t bb = t->type == VOKRA_HIP_W_Q4_K ? 144 : t->type == VOKRA_HIP_W_Q5_K ? 176 : 210;
            const size_t n = (size_t)t->nbytes / bb * 256;
            floats.emplace_back(n);
            if ((st = vokra_hip_kquant_dequantize(ctx, (int)t->type, f->base + f->data_offset + t->offset,
                                                  (size_t)t->nbytes, n, floats.back().data())))
                return st;
            *out = floats.back().data();
            return VOKRA_HIP_OK;
        }
        if (t->type != 0 && t->type != 1 && t->type != 30)
            return tensor_err(vox, VOKRA_HIP_ERROR_UNSUPPORTED_OP, name,
                              "ggml type %u where F32, F16, BF16 or a K-quant is needed", t->type);
        const size_t n = (size_t)t->nbytes / (t->type == 0 ? 4 : 2);
        floats.emplace_back(n);
        if ((st = vokra_hip_gguf_read_f32(f, name.c_str(), floats.back().data(), n))) return st;
        *out = floats.back().data();
        return VOKRA_HIP_OK;
    }

    // linear_with (weights.rs:439-521): bias first, then the [out, in] weight
    // (the text decoder's projections have no bias, text_decoder.rs:1498-1524).
    int linear(const std::string& prefix, size_t in, size_t outf, bool has_bias, const uint8_t** w, const float** b) {
        int st;
        *b = nullptr;
        if (has_bias && (st = f32(prefix + ".bias", {outf}, b))) return st;
        const std::string wname = prefix + ".weight";
        const Tensor* t;
        if ((st = shaped(wname, {outf, in}, &t))) return st;
        if ((int)t->type == wdtype) {
            const size_t be = wdtype == VOKRA_HIP_W_Q4_K || wdtype == VOKRA_HIP_W_Q5_K || wdtype == VOKRA_HIP_W_Q6_K
                                  ? 256 : 32;
            if (in % be)
                return tensor_err(vox, VOKRA_HIP_ERROR_UNSUPPORTED_OP, wname,
                                  "in_features %zu is not a multiple of %zu, so a block would straddle two rows", in, be);
            *w = f->base + f->data_offset + t->offset;
            ++verbatim;
            return VOKRA_HIP_OK;
        }
        auto names = [](uint32_t ty) -> const char* {
            switch (ty) {
            case 0: return "F32";
            case 1: return "F16";
            case 2: return "Q4_0";
            case 6: return "Q5_0";
            case 8: return "Q8_0";
            case 12: return "Q4_K";
            case 13: return "Q5_K";
            case 14: return "Q6_K";
            case 30: return "BF16";
            default: return "?";
            }
        };
        const int mode = wdtype == VOKRA_HIP_W_Q8_0 ? VOKRA_HIP_KV_Q8_0
                         : wdtype == VOKRA_HIP_W_Q4_0 ? VOKRA_HIP_KV_Q4_0
                         : wdtype == VOKRA_HIP_W_Q5_0 ? VOKRA_HIP_KV_Q5_0 : -1;
        if ((t->type != 0 && t->type != 1 && t->type != 30) || mode < 0)
            return tensor_err(vox, VOKRA_HIP_ERROR_UNSUPPORTED_OP, wname,
                              "%s on disk, and the session's %s weights cannot be made from it (same block dtype, or "
                              "F32/F16/BF16 packed to Q8_0 / Q4_0 / Q5_0)",
                              names(t->type), names((uint32_t)wdtype));
        if (in % 32)
            return tensor_err(vox, VOKRA_HIP_ERROR_UNSUPPORTED_OP, wname,
                              "in_features %zu is not a multiple of 32, so its rows cannot be packed to %s blocks", in,
                              names((uint32_t)wdtype));
        std::vector<float> x(in * outf);
        if ((st = vokra_hip_gguf_read_f32(f, wname.c_str(), x.data(), x.size()))) return st;
        const size_t bb = wdtype == VOKRA_HIP_W_Q8_0 ? 34 : wdtype == VOKRA_HIP_W_Q4_0 ? 18 : 22;
        packed.emplace_back(x.size() / 32 * bb);
        if ((st = vokra_hip_quantize_bytes(ctx, mode, x.data(), x.size(), packed.back().data(), packed.back().size())))
            return st;
        *w = packed.back().data();
        ++n_packed;
        return VOKRA_HIP_OK;
    }

    // attention_with (weights.rs:540-552): k_proj has no bias.
    int attention(const std::string& p, size_t d, const uint8_t** wq, const uint8_t** wk, const uint8_t** wv,
                  const uint8_t** wo, const float** bq, const float** bk, const float** bv, const float** bo) {
        int st;
        if ((st = linear(p + ".q_proj", d, d, true, wq, bq))) return st;
        if ((st = linear(p + ".k_proj", d, d, false, wk, bk))) return st;
        if ((st = linear(p + ".v_proj", d, d, true, wv, bv))) return st;
        return linear(p + ".out_proj", d, d, true, wo, bo);
    }

    int layer_norm(const std::string& p, size_t d, const float** g, const float** b) {
        int st = f32(p + ".weight", {d}, g);
        return st ? st : f32(p + ".bias", {d}, b);
    }

    void report(vokra_hip_whisper_load_report_t* r) const {
        if (r) {
            r->verbatim = verbatim;
            r->packed = n_packed;
        }
    }
};

bool whisper_wdtype(int w) {
    return w == VOKRA_HIP_W_Q8_0 || w == VOKRA_HIP_W_Q4_0 || w == VOKRA_HIP_W_Q5_0 || w == VOKRA_HIP_W_Q4_K ||
           w == VOKRA_HIP_W_Q5_K || w == VOKRA_HIP_W_Q6_K;
}

}  // namespace

extern "C" {

int vokra_hip_whisper_config_from_gguf(const vokra_hip_gguf_t* f, vokra_hip_whisper_config_t* cfg) {
    if (!f || !cfg) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "whisper_config_from_gguf: NULL argument");
    vokra_hip_whisper_config_t c{};
    size_t n_text_state = 0, eot = 0, n_start = 0;
    int st;
    if ((st = req_u32(f, "vokra.whisper.n_mels", &c.n_mels)) || (st = req_u32(f, "vokra.whisper.n_audio_state", &c.d_model)) ||
        (st = req_u32(f, "vokra.whisper.n_text_state", &n_text_state)) ||
        (st = req_u32(f, "vokra.whisper.n_audio_ctx", &c.n_audio_ctx)) ||
        (st = req_u32(f, "vokra.whisper.n_audio_head", &c.n_audio_head)) ||
        (st = req_u32(f, "vokra.whisper.n_audio_layer", &c.n_audio_layer)) ||
        (st = req_u32(f, "vokra.whisper.n_text_ctx", &c.n_text_ctx)) ||
        (st = req_u32(f, "vokra.whisper.n_text_head", &c.n_text_head)) ||
        (st = req_u32(f, "vokra.whisper.n_text_layer", &c.n_text_layer)) ||
        (st = req_u32(f, "vokra.whisper.n_vocab", &c.n_vocab)) || (st = req_u32(f, "vokra.whisper.ffn_dim", &c.ffn_dim)) ||
        (st = req_u32(f, "vokra.whisper.eot", &eot)) ||
        (st = req_u32_array(f, "vokra.whisper.decoder_start_ids", &n_start)) ||
        (st = opt_pair_array(f, "vokra.whisper.alignment_heads", c.n_text_layer)))
        return st;
    if (n_text_state != c.d_model)
        return cfg_bad("n_text_state (%zu) != n_audio_state (%zu); Whisper shares d_model across encoder and decoder",
                       n_text_state, c.d_model);
    if (c.n_audio_head == 0 || c.d_model % c.n_audio_head)
        return cfg_bad("n_audio_head (%zu) must divide d_model (%zu)", c.n_audio_head, c.d_model);
    if (c.n_text_head == 0 || c.d_model % c.n_text_head)
        return cfg_bad("n_text_head (%zu) must divide d_model (%zu)", c.n_text_head, c.d_model);
    if (!c.n_mels || !c.n_audio_ctx || !c.n_audio_layer || !c.n_text_ctx || !c.n_text_layer || !c.n_vocab || !c.ffn_dim)
        return cfg_bad("a required Whisper hyperparameter was zero");
    if (!n_start) return cfg_bad("decoder_start_ids must not be empty");
    c.eot = (uint32_t)eot;
    *cfg = c;
    return VOKRA_HIP_OK;
}

int vokra_hip_whisper_encoder_from_gguf(vokra_hip_ctx_t* ctx, const vokra_hip_gguf_t* f,
                                        const vokra_hip_whisper_config_t* cfg, int wdtype, size_t max_rows,
                                        vokra_hip_whisper_load_report_t* report, vokra_hip_encoder_t** out) {
    if (!ctx || !f || !cfg || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "whisper_encoder_from_gguf: NULL argument");
    *out = nullptr;
    if (!whisper_wdtype(wdtype)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "whisper_encoder_from_gguf: unknown weight dtype %d", wdtype);
    const size_t d = cfg->d_model, ff = cfg->ffn_dim;
    Loader L{ctx, f, wdtype};
    const float *c1w, *c1b, *c2w, *c2b, *pos, *lg, *lb;
    int st;
    if ((st = L.f32("model.encoder.conv1.weight", {d, cfg->n_mels, 3}, &c1w)) ||
        (st = L.f32("model.encoder.conv1.bias", {d}, &c1b)) || (st = L.f32("model.encoder.conv2.weight", {d, d, 3}, &c2w)) ||
        (st = L.f32("model.encoder.conv2.bias", {d}, &c2b)) ||
        (st = L.f32("model.encoder.embed_positions.weight", {cfg->n_audio_ctx, d}, &pos)))
        return st;
    std::vector<vokra_hip_prenorm_layer_t> layers(cfg->n_audio_layer);
    for (size_t i = 0; i < cfg->n_audio_layer; ++i) {
        const std::string p = "model.encoder.layers." + std::to_string(i);
        vokra_hip_prenorm_layer_t& y = layers[i];
        if ((st = L.layer_norm(p + ".self_attn_layer_norm", d, &y.ln1_gamma, &y.ln1_beta)) ||
            (st = L.attention(p + ".self_attn", d, &y.wq, &y.wk, &y.wv, &y.wo, &y.bq, &y.bk, &y.bv, &y.bo)) ||
            (st = L.layer_norm(p + ".final_layer_norm", d, &y.ln2_gamma, &y.ln2_beta)) ||
            (st = L.linear(p + ".fc1", d, ff, true, &y.w1, &y.b1)) || (st = L.linear(p + ".fc2", ff, d, true, &y.w2, &y.b2)))
            return st;
    }
    if ((st = L.layer_norm("model.encoder.layer_norm", d, &lg, &lb))) return st;
    vokra_hip_encoder_t* enc = nullptr;
    if ((st = vokra_hip_encoder_create(ctx, wdtype, cfg->n_audio_layer, d, cfg->n_audio_head, ff, layers.data(), lg, lb,
                                       max_rows, &enc)))
        return st;
    if ((st = vokra_hip_encoder_set_stem(ctx, enc, cfg->n_mels, 2 * cfg->n_audio_ctx, c1w, c1b, c2w, c2b, pos))) {
        vokra_hip_encoder_destroy(enc);
        return st;
    }
    L.report(report);
    *out = enc;
    return VOKRA_HIP_OK;
}

int vokra_hip_whisper_decoder_from_gguf(vokra_hip_ctx_t* ctx, const vokra_hip_gguf_t* f,
                                        const vokra_hip_whisper_config_t* cfg, int wdtype, size_t n_stream,
                                        size_t block_size, vokra_hip_whisper_load_report_t* report,
                                        vokra_hip_decoder_t** out) {
    if (!ctx || !f || !cfg || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "whisper_decoder_from_gguf: NULL argument");
    *out = nullptr;
    if (!whisper_wdtype(wdtype)) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "whisper_decoder_from_gguf: unknown weight dtype %d", wdtype);
    const size_t d = cfg->d_model, ff = cfg->ffn_dim;
    Loader L{ctx, f, wdtype};
    const float *tok, *pos, *lg, *lb;
    int st;
    if ((st = L.f32("model.decoder.embed_tokens.weight", {cfg->n_vocab, d}, &tok)) ||
        (st = L.f32("model.decoder.embed_positions.weight", {cfg->n_text_ctx, d}, &pos)))
        return st;
    std::vector<vokra_hip_decoder_layer_t> layers(cfg->n_text_layer);
    for (size_t i = 0; i < cfg->n_text_layer; ++i) {
        const std::string p = "model.decoder.layers." + std::to_string(i);
        vokra_hip_decoder_layer_t& y = layers[i];
        if ((st = L.layer_norm(p + ".self_attn_layer_norm", d, &y.ln1_gamma, &y.ln1_beta)) ||
            (st = L.attention(p + ".self_attn", d, &y.wq, &y.wk, &y.wv, &y.wo, &y.bq, &y.bk, &y.bv, &y.bo)) ||
            (st = L.layer_norm(p + ".encoder_attn_layer_norm", d, &y.ln2_gamma, &y.ln2_beta)) ||
            (st = L.attention(p + ".encoder_attn", d, &y.cwq, &y.cwk, &y.cwv, &y.cwo, &y.cbq, &y.cbk, &y.cbv, &y.cbo)) ||
            (st = L.layer_norm(p + ".final_layer_norm", d, &y.ln3_gamma, &y.ln3_beta)) ||
            (st = L.linear(p + ".fc1", d, ff, true, &y.w1, &y.b1)) || (st = L.linear(p + ".fc2", ff, d, true, &y.w2, &y.b2)))
            return st;
    }
    if ((st = L.layer_norm("model.decoder.layer_norm", d, &lg, &lb))) return st;
    vokra_hip_decoder_t* dec = nullptr;
    if ((st = vokra_hip_decoder_create(ctx, wdtype, cfg->n_text_layer, d, cfg->n_text_head, ff, cfg->n_vocab,
                                       cfg->n_text_ctx, cfg->n_audio_ctx, n_stream, block_size, layers.data(), tok, pos,
                                       lg, lb, &dec)))
        return st;
    L.report(report);
    *out = dec;
    return VOKRA_HIP_OK;
}

}  // extern "C"

// ---- the speech-LLM text decoder straight from a GGUF file -------------------
//
// TextDecoder::load (crates/vokra-models/src/voxtral/text_decoder.rs:484-575):
// the tensor prefix picked by which embedding name exists (:1456-1471), the
// per-layer names input_layernorm / self_attn.{q,k,v,o}_proj /
// post_attention_layernorm / mlp.{gate,up,down}_proj with [out, in] shapes,
// the final norm, and an untied lm_head beside the decoder submodule when
// present (:763-768), checked in that order with the reference's messages.
// The reference widens every tensor to f32; these sessions keep the Linears
// quantized, so a Linear is taken from the mapping when it is already in the
// session's dtype and packed when it is F32/F16 and the session's dtype is a
// 32-element block format (anything else is UNSUPPORTED_OP naming it).

namespace {

const char* pick_prefix(const vokra_hip_gguf* f) {
    if (find(f, "language_model.model.embed_tokens.weight")) return "language_model.model.";
    if (find(f, "language_model.embed_tokens.weight")) return "language_model.";
    return "model.";
}

// "language_model.model." -> "language_model.", "model." -> "", anything else
// unchanged (text_decoder.rs:763-768)
std::string lm_head_base(const std::string& prefix) {
    const std::string suf = "model.";
    if (prefix.size() >= suf.size() && prefix.compare(prefix.size() - suf.size(), suf.size(), suf) == 0) {
        const std::string base = prefix.substr(0, prefix.size() - suf.size());
        if (base.empty() || base.back() == '.') return base;
    }
    return prefix;
}

int td_bad(const char* msg) { return fail(VOKRA_HIP_ERROR_MODEL_LOAD, "voxtral text_decoder: %s", msg); }

}  // namespace

extern "C" {

int vokra_hip_voxtral_config_from_gguf(const vokra_hip_gguf_t* f, vokra_hip_voxtral_config_t* cfg) {
    if (!f || !cfg) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "voxtral_config_from_gguf: NULL argument");
    vokra_hip_voxtral_config_t c{};
    int st;
    if ((st = vox_req_u32(f, "vokra.voxtral.audio_encoder.n_layer", &c.audio_n_layer)) ||
        (st = vox_req_u32(f, "vokra.voxtral.audio_encoder.hidden_dim", &c.audio_hidden_dim)) ||
        (st = vox_req_u32(f, "vokra.voxtral.audio_encoder.n_head", &c.audio_n_head)))
        return st;
    c.audio_n_ctx = vox_opt_u32(f, "vokra.voxtral.audio_encoder.n_ctx");
    if ((st = vox_req_u32(f, "vokra.voxtral.audio_encoder.n_mels", &c.audio_n_mels))) return st;
    c.audio_ffn_dim = vox_opt_u32(f, "vokra.voxtral.audio_encoder.ffn_dim");
    if (c.audio_n_head != 0 && c.audio_hidden_dim % c.audio_n_head != 0)
        return vox_bad("audio_encoder.n_head (%zu) must divide audio_encoder.hidden_dim (%zu)", c.audio_n_head,
                       c.audio_hidden_dim);
    if ((st = vox_req_u32(f, "vokra.voxtral.text_decoder.n_layer", &c.n_layer)) ||
        (st = vox_req_u32(f, "vokra.voxtral.text_decoder.hidden_dim", &c.hidden_dim)) ||
        (st = vox_req_u32(f, "vokra.voxtral.text_decoder.ffn_dim", &c.ffn_dim)))
        return st;
    c.vocab_size = vox_opt_u32(f, "vokra.voxtral.text_decoder.vocab_size");
    c.n_ctx = vox_opt_u32(f, "vokra.voxtral.text_decoder.n_ctx");
    c.n_head_q = vox_opt_u32(f, "vokra.voxtral.text_decoder.n_head_q");
    c.n_head_kv = vox_opt_u32(f, "vokra.voxtral.text_decoder.n_head_kv");
    c.head_dim = vox_opt_u32(f, "vokra.voxtral.text_decoder.head_dim");
    c.rope_base = vox_opt_f32(f, "vokra.voxtral.text_decoder.rope_base");
    c.rms_norm_eps = vox_opt_f32(f, "vokra.voxtral.text_decoder.rms_norm_eps");
    if (c.head_dim == 0 && c.n_head_q != 0 && c.hidden_dim != 0 && c.hidden_dim % c.n_head_q != 0)
        return vox_bad("text_decoder.n_head_q (%zu) must divide text_decoder.hidden_dim (%zu) when no explicit "
                       "text_decoder.head_dim is present - re-convert with a converter that writes "
                       "vokra.voxtral.text_decoder.head_dim",
                       c.n_head_q, c.hidden_dim);
    if (c.n_head_kv != 0 && c.n_head_q != 0 && c.n_head_q % c.n_head_kv != 0)
        return vox_bad("text_decoder.n_head_kv (%zu) must divide text_decoder.n_head_q (%zu) for GQA", c.n_head_kv,
                       c.n_head_q);
    c.cross_attn_hidden_dim = vox_opt_u32(f, "vokra.voxtral.cross_attn.hidden_dim");
    *cfg = c;
    return VOKRA_HIP_OK;
}

int vokra_hip_text_decoder_from_gguf(vokra_hip_ctx_t* ctx, const vokra_hip_gguf_t* f,
                                     const vokra_hip_voxtral_config_t* cfg, int wdtype, size_t n_stream, size_t n_ctx,
                                     size_t block_size, vokra_hip_whisper_load_report_t* report,
                                     vokra_hip_text_decoder_t** out) {
    if (!ctx || !f || !cfg || !out) return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_from_gguf: NULL argument");
    *out = nullptr;
    if (!whisper_wdtype(wdtype))
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT, "text_decoder_from_gguf: unknown weight dtype %d", wdtype);
    const size_t d = cfg->hidden_dim, ff = cfg->ffn_dim, vocab = cfg->vocab_size;
    // the converter's shape-only sentinel binds nothing in the reference, and
    // its session refuses it (TextDecoderSession::new)
    if (cfg->n_layer == 0 || d == 0)
        return fail(VOKRA_HIP_ERROR_MODEL_LOAD,
                    "voxtral::TextDecoderSession: config carries 0-sentinel (n_layer, d, vocab, heads, head_dim)");
    const std::string prefix = pick_prefix(f);
    if (vocab == 0) return td_bad("text_decoder.vocab_size must be non-zero");
    Loader L{ctx, f, wdtype, true};
    const float *tok, *fin;
    int st;
    if ((st = L.f32(prefix + "embed_tokens.weight", {vocab, d}, &tok))) return st;
    if (cfg->n_head_q == 0 || cfg->n_head_kv == 0)
        return td_bad("text_decoder.n_head_q and n_head_kv must be non-zero (GQA head split)");
    // TextDecoderConfig::head_dim (config.rs:108-115): explicit, else derived
    const size_t hd = cfg->head_dim ? cfg->head_dim : d / cfg->n_head_q;
    if (hd == 0)
        return td_bad("text_decoder.head_dim resolves to 0 - re-convert with a converter that writes "
                      "vokra.voxtral.text_decoder.head_dim");
    const size_t qh = cfg->n_head_q * hd, kvh = cfg->n_head_kv * hd;
    std::vector<vokra_hip_text_decoder_layer_t> layers(cfg->n_layer);
    const float* none = nullptr;
    for (size_t i = 0; i < cfg->n_layer; ++i) {
        const std::string p = prefix + "layers." + std::to_string(i);
        vokra_hip_text_decoder_layer_t& y = layers[i];
        if ((st = L.f32(p + ".input_layernorm.weight", {d}, &y.attn_norm_gamma)) ||
            (st = L.linear(p + ".self_attn.q_proj", d, qh, false, &y.wq, &none)) ||
            (st = L.linear(p + ".self_attn.k_proj", d, kvh, false, &y.wk, &none)) ||
            (st = L.linear(p + ".self_attn.v_proj", d, kvh, false, &y.wv, &none)) ||
            (st = L.linear(p + ".self_attn.o_proj", qh, d, false, &y.wo, &none)) ||
            (st = L.f32(p + ".post_attention_layernorm.weight", {d}, &y.ffn_norm_gamma)) ||
            (st = L.linear(p + ".mlp.gate_proj", d, ff, false, &y.w_gate, &none)) ||
            (st = L.linear(p + ".mlp.up_proj", d, ff, false, &y.w_up, &none)) ||
            (st = L.linear(p + ".mlp.down_proj", ff, d, false, &y.w_down, &none)))
            return st;
    }
    if ((st = L.f32(prefix + "norm.weight", {d}, &fin))) return st;
    // an untied head is bound when present (a wrong shape is an error, never
    // a silent tie); absent, the token embedding is the head
    const uint8_t* head = nullptr;
    const std::string head_name = lm_head_base(prefix) + "lm_head";
    if (find(f, (head_name + ".weight").c_str()) && (st = L.linear(head_name, d, vocab, false, &head, &none))) return st;
    const size_t ctx_len = n_ctx ? n_ctx : cfg->n_ctx;
    if (ctx_len == 0)
        return fail(VOKRA_HIP_ERROR_INVALID_ARGUMENT,
                    "text_decoder_from_gguf: n_ctx is 0 and the file has no vokra.voxtral.text_decoder.n_ctx");
    if ((st = vokra_hip_text_decoder_create(ctx, wdtype, cfg->n_layer, d, cfg->n_head_q, cfg->n_head_kv, hd, ff, vocab,
                                            ctx_len, n_stream, block_size, cfg->rope_base, cfg->rms_norm_eps,
                                            layers.data(), tok, fin, head, out)))
        return st;
    L.report(report);
    return VOKRA_HIP_OK;
}

}  // extern "C"
