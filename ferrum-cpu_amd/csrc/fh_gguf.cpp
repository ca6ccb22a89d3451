// fh_gguf.cpp — GGUF reader for libferrum_hip (host code).
//
// Parses a GGUF v2/v3 file the way ferrum_core's gguf module does
// (gguf/header.rs:14-75 parse_header, gguf/cursor.rs read_value,
// gguf/format.rs:87-137 type_nbytes / align_up, gguf/header.rs check_extents):
// little-endian header, metadata key/value table, tensor directory, data
// section at the next multiple of general.alignment (default 32).  The file is
// memory-mapped read-only; a Q8_0 tensor goes from the mapping straight to the
// device (fh_gguf_upload_q8_0), never expanded to f32 on the host.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "fh_internal.hpp"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF" little-endian
constexpr uint64_t kDefaultAlignment = 32;
enum : uint32_t {
    VT_U8 = 0, VT_I8 = 1, VT_U16 = 2, VT_I16 = 3, VT_U32 = 4, VT_I32 = 5, VT_F32 = 6, VT_BOOL = 7,
    VT_STRING = 8, VT_ARRAY = 9, VT_U64 = 10, VT_I64 = 11, VT_F64 = 12
};
enum : uint32_t { GGML_F32 = 0, GGML_F16 = 1, GGML_Q4_0 = 2, GGML_Q4_1 = 3, GGML_Q5_0 = 6, GGML_Q5_1 = 7,
                  GGML_Q8_0 = 8, GGML_Q8_1 = 9, GGML_Q2_K = 10, GGML_Q3_K = 11, GGML_Q4_K = 12, GGML_Q5_K = 13,
                  GGML_Q6_K = 14, GGML_I16 = 25, GGML_I32 = 26 };

struct Value {
    uint32_t type = VT_U8;
    uint64_t u = 0;  // unsigned / bool payload
    int64_t i = 0;   // signed payload
    double f = 0.0;  // float payload
    std::string s;
    uint32_t elem = 0;            // array element type
    std::vector<Value> items;     // array of strings (or of other values)
    std::vector<uint8_t> nums;    // array of numbers, raw little-endian
    uint64_t count = 0;           // array length
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;  // relative to the data section
    uint64_t nbytes = 0;  // 0 when the type cannot be sized
    bool sized = false;
};

struct ParseError {
    std::string msg;
};

struct Cursor {
    const uint8_t* b;
    size_t pos = 0, total;
    const uint8_t* take(size_t n) {
        if (n > total - pos)
            throw ParseError{"GGUF truncated at +" + std::to_string(pos) + ": need " + std::to_string(n) +
                             " bytes, file has " + std::to_string(total)};
        const uint8_t* p = b + pos;
        pos += n;
        return p;
    }
    template <typename T>
    T get() {
        T v;
        std::memcpy(&v, take(sizeof(T)), sizeof(T));
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (n > total - pos) take(static_cast<size_t>(std::min<uint64_t>(n, SIZE_MAX)));  // throws
        const uint8_t* p = take(static_cast<size_t>(n));
        return std::string(reinterpret_cast<const char*>(p), static_cast<size_t>(n));
    }
};

size_t num_size(uint32_t t) {
    switch (t) {
        case VT_U8: case VT_I8: case VT_BOOL: return 1;
        case VT_U16: case VT_I16: return 2;
        case VT_U32: case VT_I32: case VT_F32: return 4;
        case VT_U64: case VT_I64: case VT_F64: return 8;
        default: return 0;
    }
}

Value read_value(Cursor& c, uint32_t t) {
    Value v;
    v.type = t;
    switch (t) {
        case VT_U8: v.u = c.get<uint8_t>(); v.i = static_cast<int64_t>(v.u); v.f = static_cast<double>(v.u); break;
        case VT_I8: v.i = c.get<int8_t>(); v.f = static_cast<double>(v.i); break;
        case VT_U16: v.u = c.get<uint16_t>(); v.i = static_cast<int64_t>(v.u); v.f = static_cast<double>(v.u); break;
        case VT_I16: v.i = c.get<int16_t>(); v.f = static_cast<double>(v.i); break;
        case VT_U32: v.u = c.get<uint32_t>(); v.i = static_cast<int64_t>(v.u); v.f = static_cast<double>(v.u); break;
        case VT_I32: v.i = c.get<int32_t>(); v.f = static_cast<double>(v.i); break;
        case VT_F32: v.f = c.get<float>(); break;
        case VT_BOOL: v.u = c.get<uint8_t>() != 0; v.i = static_cast<int64_t>(v.u); break;
        case VT_STRING: v.s = c.str(); break;
        case VT_U64: v.u = c.get<uint64_t>(); v.f = static_cast<double>(v.u); break;
        case VT_I64: v.i = c.get<int64_t>(); v.f = static_cast<double>(v.i); break;
        case VT_F64: v.f = c.get<double>(); break;
        case VT_ARRAY: {
            v.elem = c.get<uint32_t>();
            if (v.elem == VT_ARRAY) throw ParseError{"GGUF nested arrays are not supported"};
            v.count = c.get<uint64_t>();
            if (v.count == 0) break;
            const size_t ns = num_size(v.elem);
            const size_t min = v.elem == VT_STRING ? 8 : ns;
            if (min == 0) throw ParseError{"GGUF unknown metadata value type " + std::to_string(v.elem)};
            if (v.count > (c.total - c.pos) / min) throw ParseError{"GGUF array count exceeds the file size"};
            if (ns) {
                const uint8_t* p = c.take(static_cast<size_t>(v.count) * ns);
                v.nums.assign(p, p + static_cast<size_t>(v.count) * ns);
            } else {
                v.items.reserve(static_cast<size_t>(std::min<uint64_t>(v.count, 1u << 20)));
                for (uint64_t k = 0; k < v.count; k++) v.items.push_back(read_value(c, v.elem));
            }
            break;
        }
        default: throw ParseError{"GGUF unknown metadata value type " + std::to_string(t)};
    }
    return v;
}

// gguf/format.rs:87-129: bytes of n elements of a GGML type (false: unsized).
bool type_nbytes(uint32_t t, uint64_t n, uint64_t* out) {
    auto blocks = [&](uint64_t qk, uint64_t bytes) {
        if (n % qk) return false;
        *out = n / qk * bytes;
        return true;
    };
    switch (t) {
        case GGML_F32: case GGML_I32: *out = n * 4; return true;
        case GGML_F16: case GGML_I16: *out = n * 2; return true;
        case GGML_Q8_0: return blocks(32, 34);
        case GGML_Q8_1: return blocks(32, 36);
        case GGML_Q4_0: return blocks(32, 18);
        case GGML_Q4_1: return blocks(32, 20);
        case GGML_Q5_0: return blocks(32, 22);
        case GGML_Q5_1: return blocks(32, 24);
        case GGML_Q2_K: return blocks(256, 84);
        case GGML_Q3_K: return blocks(256, 110);
        case GGML_Q4_K: return blocks(256, 144);
        case GGML_Q5_K: return blocks(256, 176);
        case GGML_Q6_K: return blocks(256, 210);
        default: return false;
    }
}

}  // namespace

struct fh_gguf {
    std::string err;
    void* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    std::map<std::string, Value> meta;
    std::vector<Tensor> tensors;
    uint64_t data_offset = 0;
};

namespace {

void parse(fh_gguf* g) {
    Cursor c{static_cast<const uint8_t*>(g->map), 0, g->size};
    if (c.get<uint32_t>() != kMagic) throw ParseError{"not a GGUF file (bad magic)"};
    g->version = c.get<uint32_t>();
    if (g->version != 2 && g->version != 3)
        throw ParseError{"unsupported GGUF version " + std::to_string(g->version) + " (need 2 or 3)"};
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        Value v = read_value(c, t);
        g->meta[key] = std::move(v);  // a repeated key keeps its last value, as the reference's map does
    }
    for (uint64_t k = 0; k < n_tensors; k++) {
        Tensor t;
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (nd > 8) throw ParseError{"tensor '" + t.name + "' has implausible " + std::to_string(nd) + " dims"};
        for (uint32_t d = 0; d < nd; d++) t.dims.push_back(c.get<uint64_t>());
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        g->tensors.push_back(std::move(t));
    }
    uint64_t align = kDefaultAlignment;
    auto a = g->meta.find("general.alignment");
    if (a != g->meta.end() && a->second.type != VT_STRING && a->second.type != VT_ARRAY && a->second.u > 0)
        align = a->second.u;
    g->data_offset = (c.pos + align - 1) / align * align;
    // check_extents (gguf/header.rs): every sized tensor inside the file, none overlapping
    const uint64_t avail = g->size > g->data_offset ? g->size - g->data_offset : 0;
    std::vector<std::pair<uint64_t, size_t>> spans;
    for (size_t k = 0; k < g->tensors.size(); k++) {
        Tensor& t = g->tensors[k];
        uint64_t n = 1;
        for (uint64_t d : t.dims) {
            if (d && n > UINT64_MAX / d) throw ParseError{"tensor '" + t.name + "' element count overflows"};
            n *= d;
        }
        if (n == 0 && !(t.dims.size() == 1 && t.dims[0] == 0))
            throw ParseError{"tensor '" + t.name + "' has an empty shape; only a 1-D [0] tensor may be empty"};
        if (n > avail * 8) throw ParseError{"GGUF tensor '" + t.name + "' element count exceeds what the file can hold"};
        t.sized = type_nbytes(t.type, n, &t.nbytes);
        if (!t.sized || t.nbytes == 0) continue;
        if (t.offset > avail || t.nbytes > avail - t.offset)
            throw ParseError{"tensor '" + t.name + "' data runs past EOF"};
        spans.push_back({t.offset, k});
    }
    std::sort(spans.begin(), spans.end());
    for (size_t k = 1; k < spans.size(); k++) {
        const Tensor& p = g->tensors[spans[k - 1].second];
        const Tensor& q = g->tensors[spans[k].second];
        if (q.offset < p.offset + p.nbytes)
            throw ParseError{"tensors '" + p.name + "' and '" + q.name + "' overlap"};
    }
}

// The status, with the message kept in ctx when there is one (reads are
// host-only and may run without a context).
int read_fail(fh_ctx* ctx, int code, const std::string& msg) { return ctx ? fh_fail(ctx, code, msg) : code; }

const Value* find_meta(const fh_gguf* g, const char* key) {
    if (!g || !key) return nullptr;
    auto it = g->meta.find(key);
    return it == g->meta.end() ? nullptr : &it->second;
}

}  // namespace

extern "C" {

int fh_gguf_open(const char* path, fh_gguf** out) {
    if (!out) return FH_ERR_INVALID;
    fh_gguf* g = new fh_gguf();
    *out = g;
    if (!path) {
        g->err = "fh_gguf_open: path is NULL";
        return FH_ERR_INVALID;
    }
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) {
        g->err = std::string("cannot open ") + path + ": " + std::strerror(errno);
        return FH_ERR_INVALID;
    }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        g->err = std::string("cannot read ") + path;
        ::close(fd);
        return FH_ERR_INVALID;
    }
    g->size = static_cast<size_t>(st.st_size);
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (m == MAP_FAILED) {
        g->err = std::string("cannot map ") + path + ": " + std::strerror(errno);
        g->size = 0;
        return FH_ERR_INVALID;
    }
    g->map = m;
    try {
        parse(g);
    } catch (const ParseError& e) {
        g->err = e.msg;
        return FH_ERR_FORMAT;
    } catch (const std::bad_alloc&) {
        g->err = "fh_gguf_open: out of host memory";
        return FH_ERR_OOM;
    }
    return FH_OK;
}

void fh_gguf_close(fh_gguf* g) {
    if (!g) return;
    if (g->map) munmap(g->map, g->size);
    delete g;
}

const char* fh_gguf_error(const fh_gguf* g) { return g ? g->err.c_str() : "fh_gguf: NULL handle"; }

uint32_t fh_gguf_version(const fh_gguf* g) { return g ? g->version : 0; }

size_t fh_gguf_tensor_count(const fh_gguf* g) { return g ? g->tensors.size() : 0; }

long fh_gguf_find_tensor(const fh_gguf* g, const char* name) {
    if (!g || !name) return -1;
    for (size_t k = 0; k < g->tensors.size(); k++)
        if (g->tensors[k].name == name) return static_cast<long>(k);  // first match, as the reference
    return -1;
}

int fh_gguf_tensor_info(const fh_gguf* g, size_t i, const char** name, uint32_t* n_dims, uint64_t* dims,
                        uint32_t* ggml_type, uint64_t* nbytes) {
    if (!g || i >= g->tensors.size()) return FH_ERR_INVALID;
    const Tensor& t = g->tensors[i];
    if (name) *name = t.name.c_str();
    if (n_dims) *n_dims = static_cast<uint32_t>(t.dims.size());
    if (dims)
        for (size_t d = 0; d < t.dims.size(); d++) dims[d] = t.dims[d];
    if (ggml_type) *ggml_type = t.type;
    if (nbytes) *nbytes = t.sized ? t.nbytes : 0;
    return FH_OK;
}

const void* fh_gguf_tensor_data(const fh_gguf* g, size_t i) {
    if (!g || i >= g->tensors.size() || !g->tensors[i].sized) return nullptr;
    return static_cast<const uint8_t*>(g->map) + g->data_offset + g->tensors[i].offset;
}

int fh_gguf_meta_type(const fh_gguf* g, const char* key, uint32_t* type, uint32_t* elem_type, uint64_t* count) {
    const Value* v = find_meta(g, key);
    if (!v) return FH_ERR_INVALID;
    if (type) *type = v->type;
    if (elem_type) *elem_type = v->type == VT_ARRAY ? v->elem : 0;
    if (count) *count = v->type == VT_ARRAY ? v->count : 1;
    return FH_OK;
}

int fh_gguf_meta_u64(const fh_gguf* g, const char* key, uint64_t* out) {
    const Value* v = find_meta(g, key);
    if (!v || !out) return FH_ERR_INVALID;
    switch (v->type) {
        case VT_U8: case VT_U16: case VT_U32: case VT_U64: case VT_BOOL: *out = v->u; return FH_OK;
        case VT_I8: case VT_I16: case VT_I32: case VT_I64:
            if (v->i < 0) return FH_ERR_INVALID;
            *out = static_cast<uint64_t>(v->i);
            return FH_OK;
        default: return FH_ERR_INVALID;
    }
}

int fh_gguf_meta_f64(const fh_gguf* g, const char* key, double* out) {
    const Value* v = find_meta(g, key);
    if (!v || !out || v->type == VT_STRING || v->type == VT_ARRAY || v->type == VT_BOOL) return FH_ERR_INVALID;
    *out = v->f;
    return FH_OK;
}

int fh_gguf_meta_str(const fh_gguf* g, const char* key, size_t index, const char** out, size_t* len) {
    const Value* v = find_meta(g, key);
    if (!v || !out) return FH_ERR_INVALID;
    const std::string* s = nullptr;
    if (v->type == VT_STRING && index == 0) s = &v->s;
    else if (v->type == VT_ARRAY && v->elem == VT_STRING && index < v->items.size()) s = &v->items[index].s;
    if (!s) return FH_ERR_INVALID;
    *out = s->c_str();
    if (len) *len = s->size();
    return FH_OK;
}

int fh_gguf_meta_array_data(const fh_gguf* g, const char* key, const void** data, size_t* elem_size) {
    const Value* v = find_meta(g, key);
    if (!v || !data || v->type != VT_ARRAY || v->elem == VT_STRING) return FH_ERR_INVALID;
    *data = v->nums.empty() ? nullptr : v->nums.data();
    if (elem_size) *elem_size = num_size(v->elem);
    return FH_OK;
}

int fh_gguf_read_f32(fh_ctx* ctx, const fh_gguf* g, const char* name, float* out, size_t n) {
    if (ctx) ctx->err.clear();
    const long i = fh_gguf_find_tensor(g, name);
    if (i < 0 || !out) return read_fail(ctx, FH_ERR_INVALID, std::string("GGUF missing ") + (name ? name : "(null)"));
    const Tensor& t = g->tensors[static_cast<size_t>(i)];
    uint64_t elems = 1;
    for (uint64_t d : t.dims) elems *= d;
    if (elems != n)
        return read_fail(ctx, FH_ERR_DIM, "tensor '" + t.name + "' has " + std::to_string(elems) + " elements, not " +
                                            std::to_string(n));
    const uint8_t* p = static_cast<const uint8_t*>(fh_gguf_tensor_data(g, static_cast<size_t>(i)));
    if (t.type == GGML_F32) {
        std::memcpy(out, p, n * sizeof(float));
        return FH_OK;
    }
    if (t.type == GGML_F16) {  // IEEE half -> float, exact (gguf/dequant.rs:7-35)
        for (size_t k = 0; k < n; k++) {
            uint16_t h;
            std::memcpy(&h, p + 2 * k, 2);
            const uint32_t sign = (h & 0x8000u) << 16, e = (h >> 10) & 0x1F, m = h & 0x3FF;
            uint32_t bits;
            if (e == 0x1F) bits = sign | 0x7F800000u | (m << 13);
            else if (e != 0) bits = sign | ((e + 112) << 23) | (m << 13);
            else if (m == 0) bits = sign;
            else {  // subnormal: normalise
                int sh = 0;
                uint32_t mm = m;
                while (!(mm & 0x400)) mm <<= 1, sh++;
                bits = sign | (static_cast<uint32_t>(113 - sh) << 23) | ((mm & 0x3FF) << 13);
            }
            std::memcpy(out + k, &bits, 4);
        }
        return FH_OK;
    }
    return read_fail(ctx, FH_ERR_INVALID, "tensor '" + t.name + "' is GGML type " + std::to_string(t.type) +
                                            ", not F32 or F16");
}

int fh_gguf_upload_q8_0(fh_ctx* ctx, const fh_gguf* g, const char* name, fh_q8_0** out) {
    if (!ctx || !out) return FH_ERR_INVALID;
    ctx->err.clear();
    const long i = fh_gguf_find_tensor(g, name);
    if (i < 0) return fh_fail(ctx, FH_ERR_INVALID, std::string("GGUF missing ") + (name ? name : "(null)"));
    const Tensor& t = g->tensors[static_cast<size_t>(i)];
    if (t.type != GGML_Q8_0)
        return fh_fail(ctx, FH_ERR_INVALID, "tensor '" + t.name + "' is GGML type " + std::to_string(t.type) +
                                                ", not Q8_0");
    if (t.dims.empty() || t.dims.size() > 2)
        return fh_fail(ctx, FH_ERR_DIM, "tensor '" + t.name + "' is not a matrix");
    const uint64_t k = t.dims[0], n = t.dims.size() == 2 ? t.dims[1] : 1;
    // GGUF [ne0 = k, ne1 = n]: n rows of k quants (loader/decode.rs:57-81)
    return fh_q8_0_upload(ctx, static_cast<const uint8_t*>(fh_gguf_tensor_data(g, static_cast<size_t>(i))),
                          static_cast<size_t>(n), static_cast<size_t>(k), out);
}

}  // extern "C"
