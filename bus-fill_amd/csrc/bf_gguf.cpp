// GGUF reader: llama.cpp's model file format (versions 2 and 3), memory-mapped.
//
// Layout (little-endian), from the public GGUF specification:
//   "GGUF" u32 version, u64 tensor_count, u64 kv_count,
//   kv_count x { string key, u32 value_type, value },
//   tensor_count x { string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset },
//   padding to `general.alignment` (default 32), then the tensor data; each
//   tensor's offset is relative to the start of the data and aligned.
// A string is u64 length + bytes (no NUL); an array value is u32 element type,
// u64 count, elements.  ne[0] is the contiguous dimension: a weight matrix of N
// rows of K weights has ne = {K, N}, each row K / block_size blocks.
//
// The Q4_0 and Q4_K tensors are stored in exactly the block layouts bf_gemm
// takes (block_q4_0: fp16 d + 16 code bytes; block_q4_K: fp16 d, dmin, 12
// scale bytes, 128 code bytes), so the reader hands out the mapped bytes as
// they are and bf_gguf_upload copies them to the device unchanged.  The file
// is untrusted input: every length and offset is checked against the file
// size before it is used.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "busfill.h"
#include "bf_host.h"

namespace {

bf_status gguf_fail(const char* fmt, ...) {
    char text[256];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(text, sizeof text, fmt, ap);
    va_end(ap);
    bf::set_last_error(text);
    return BF_ERR_INVALID;
}

enum : uint32_t {
    KV_U8 = 0, KV_I8 = 1, KV_U16 = 2, KV_I16 = 3, KV_U32 = 4, KV_I32 = 5, KV_F32 = 6, KV_BOOL = 7,
    KV_STRING = 8, KV_ARRAY = 9, KV_U64 = 10, KV_I64 = 11, KV_F64 = 12
};

// Bytes of one scalar metadata value (0: not a fixed-size scalar).
size_t scalar_size(uint32_t t) {
    switch (t) {
        case KV_U8: case KV_I8: case KV_BOOL: return 1;
        case KV_U16: case KV_I16: return 2;
        case KV_U32: case KV_I32: case KV_F32: return 4;
        case KV_U64: case KV_I64: case KV_F64: return 8;
        default: return 0;
    }
}

// ggml type -> (block size, bytes per block); {0, 0} when unknown.
struct TypeSize {
    uint32_t blck, bytes;
};
TypeSize ggml_type_size(uint32_t t) {
    switch (t) {
        case 0: return {1, 4};       // F32
        case 1: return {1, 2};       // F16
        case 2: return {32, 18};     // Q4_0
        case 3: return {32, 20};     // Q4_1
        case 6: return {32, 22};     // Q5_0
        case 7: return {32, 24};     // Q5_1
        case 8: return {32, 34};     // Q8_0
        case 9: return {32, 36};     // Q8_1
        case 10: return {256, 84};   // Q2_K
        case 11: return {256, 110};  // Q3_K
        case 12: return {256, 144};  // Q4_K
        case 13: return {256, 176};  // Q5_K
        case 14: return {256, 210};  // Q6_K
        case 15: return {256, 292};  // Q8_K
        case 30: return {1, 2};      // BF16
        default: return {0, 0};
    }
}

struct Cursor {
    const uint8_t* base;
    size_t size, pos;
    bool take(void* dst, size_t n) {
        if (n > size - pos) return false;
        memcpy(dst, base + pos, n);
        pos += n;
        return true;
    }
    bool skip(size_t n) {
        if (n > size - pos) return false;
        pos += n;
        return true;
    }
    bool str(std::string* out) {
        uint64_t n;
        if (!take(&n, 8) || n > size - pos) return false;
        if (out) out->assign((const char*)base + pos, (size_t)n);
        pos += (size_t)n;
        return true;
    }
};

struct Kv {
    std::string key;
    uint32_t type;
    size_t pos;        // file offset of the value
};

struct Tensor {
    std::string name;
    uint32_t type, n_dims;
    uint64_t dims[4];
    uint64_t offset, nbytes;   // offset from the start of the file
};

}  // namespace

struct bf_gguf {
    int fd = -1;
    const uint8_t* map = nullptr;
    size_t size = 0;
    uint32_t version = 0;
    std::vector<Kv> kv;
    std::vector<Tensor> tensors;
};

namespace {

bf_status parse(bf_gguf* g) {
    Cursor c{g->map, g->size, 0};
    uint32_t magic = 0;
    if (!c.take(&magic, 4) || memcmp(&magic, "GGUF", 4) != 0) return gguf_fail("not a GGUF file (magic)");
    if (!c.take(&g->version, 4)) return gguf_fail("truncated header");
    if (g->version != 2 && g->version != 3) return gguf_fail("GGUF version %u is not supported (2, 3)", g->version);
    uint64_t n_tensors = 0, n_kv = 0;
    if (!c.take(&n_tensors, 8) || !c.take(&n_kv, 8)) return gguf_fail("truncated header");
    // every entry takes at least 8 bytes of the file: bounds the counts before reserving
    if (n_tensors > g->size / 8 || n_kv > g->size / 8) return gguf_fail("implausible counts");
    uint64_t alignment = 32;
    g->kv.reserve((size_t)n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
        Kv e;
        if (!c.str(&e.key) || !c.take(&e.type, 4)) return gguf_fail("truncated metadata entry %llu", (unsigned long long)i);
        e.pos = c.pos;
        if (e.type == KV_STRING) {
            if (!c.str(nullptr)) return gguf_fail("truncated string value of %s", e.key.c_str());
        } else if (e.type == KV_ARRAY) {
            uint32_t et;
            uint64_t n;
            if (!c.take(&et, 4) || !c.take(&n, 8)) return gguf_fail("truncated array header of %s", e.key.c_str());
            if (et == KV_STRING) {
                for (uint64_t k = 0; k < n; k++)
                    if (!c.str(nullptr)) return gguf_fail("truncated string array %s", e.key.c_str());
            } else {
                const size_t es = scalar_size(et);
                if (!es || n > (c.size - c.pos) / es || !c.skip((size_t)(n * es)))
                    return gguf_fail("bad array %s (element type %u)", e.key.c_str(), et);
            }
        } else {
            const size_t es = scalar_size(e.type);
            if (!es || !c.skip(es)) return gguf_fail("bad value type %u of %s", e.type, e.key.c_str());
        }
        if (e.key == "general.alignment") {
            uint32_t a = 0;
            if (e.type != KV_U32) return gguf_fail("general.alignment is not a u32");
            memcpy(&a, g->map + e.pos, 4);
            if (a == 0 || (a & (a - 1))) return gguf_fail("general.alignment %u is not a power of two", a);
            alignment = a;
        }
        g->kv.push_back(std::move(e));
    }
    g->tensors.reserve((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor t{};
        if (!c.str(&t.name) || !c.take(&t.n_dims, 4)) return gguf_fail("truncated tensor info %llu", (unsigned long long)i);
        if (t.n_dims < 1 || t.n_dims > 4) return gguf_fail("tensor %s: %u dimensions", t.name.c_str(), t.n_dims);
        for (uint32_t d = 0; d < 4; d++) t.dims[d] = 1;
        for (uint32_t d = 0; d < t.n_dims; d++)
            if (!c.take(&t.dims[d], 8)) return gguf_fail("truncated tensor info %s", t.name.c_str());
        if (!c.take(&t.type, 4) || !c.take(&t.offset, 8)) return gguf_fail("truncated tensor info %s", t.name.c_str());
        if (t.offset % alignment) return gguf_fail("tensor %s: offset not aligned", t.name.c_str());
        const TypeSize ts = ggml_type_size(t.type);
        t.nbytes = 0;
        if (ts.blck) {
            if (t.dims[0] % ts.blck) return gguf_fail("tensor %s: row of %llu not whole blocks", t.name.c_str(),
                                                     (unsigned long long)t.dims[0]);
            unsigned __int128 b = (unsigned __int128)(t.dims[0] / ts.blck) * ts.bytes;   // < 2^73
            for (uint32_t d = 1; d < 4; d++) {
                if (t.dims[d] && b > (unsigned __int128)g->size / t.dims[d])
                    return gguf_fail("tensor %s larger than the file", t.name.c_str());
                b *= t.dims[d];
            }
            if (b > g->size) return gguf_fail("tensor %s larger than the file", t.name.c_str());
            t.nbytes = (uint64_t)b;
        }
        g->tensors.push_back(std::move(t));
    }
    const uint64_t data0 = (c.pos + alignment - 1) / alignment * alignment;
    for (Tensor& t : g->tensors) {
        if (t.offset > g->size || data0 > g->size - t.offset || t.nbytes > g->size - data0 - t.offset)
            return gguf_fail("tensor %s: data past the end of the file", t.name.c_str());
        t.offset += data0;
    }
    return BF_OK;
}

void fill(const bf_gguf* g, const Tensor& t, bf_gguf_tensor* out) {
    out->name = t.name.c_str();
    out->ggml_type = t.type;
    out->qtype = t.type == 2 ? BF_Q4_0 : t.type == 12 ? BF_Q4_K : -1;
    out->n_dims = t.n_dims;
    for (int d = 0; d < 4; d++) out->dims[d] = t.dims[d];
    out->offset = t.offset;
    out->nbytes = t.nbytes;
    out->data = t.nbytes ? g->map + t.offset : nullptr;
}

const Kv* find_kv(const bf_gguf* g, const char* key) {
    for (const Kv& e : g->kv)
        if (e.key == key) return &e;
    return nullptr;
}

}  // namespace

extern "C" {

bf_status bf_gguf_open(const char* path, bf_gguf** out) {
    bf::set_last_error("");
    if (!path || !out) return gguf_fail("path or out is NULL");
    *out = nullptr;
    auto* g = new bf_gguf;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) {
        delete g;
        return gguf_fail("cannot open %s", path);
    }
    struct stat sb;
    if (fstat(g->fd, &sb) != 0 || sb.st_size < 24) {
        close(g->fd);
        delete g;
        return gguf_fail("%s: too short for a GGUF header", path);
    }
    g->size = (size_t)sb.st_size;
    void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        close(g->fd);
        delete g;
        return gguf_fail("cannot map %s", path);
    }
    g->map = (const uint8_t*)m;
    const bf_status st = parse(g);
    if (st != BF_OK) {
        bf_gguf_close(g);
        return st;
    }
    *out = g;
    return BF_OK;
}

void bf_gguf_close(bf_gguf* g) {
    if (!g) return;
    if (g->map) munmap((void*)g->map, g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

int64_t bf_gguf_tensor_count(const bf_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }

bf_status bf_gguf_tensor_at(const bf_gguf* g, int64_t i, bf_gguf_tensor* out) {
    if (!g || !out) return gguf_fail("handle or out is NULL");
    if (i < 0 || i >= (int64_t)g->tensors.size()) return gguf_fail("tensor index %lld out of range", (long long)i);
    fill(g, g->tensors[(size_t)i], out);
    return BF_OK;
}

bf_status bf_gguf_find(const bf_gguf* g, const char* name, bf_gguf_tensor* out) {
    if (!g || !name || !out) return gguf_fail("handle, name or out is NULL");
    for (const Tensor& t : g->tensors)
        if (t.name == name) {
            fill(g, t, out);
            return BF_OK;
        }
    return gguf_fail("no tensor named %s", name);
}

bf_status bf_gguf_get_u64(const bf_gguf* g, const char* key, uint64_t* out) {
    if (!g || !key || !out) return gguf_fail("handle, key or out is NULL");
    const Kv* e = find_kv(g, key);
    if (!e) return gguf_fail("no metadata key %s", key);
    const uint8_t* p = g->map + e->pos;
    switch (e->type) {
        case KV_U8: case KV_BOOL: *out = p[0]; return BF_OK;
        case KV_I8: { int8_t v; memcpy(&v, p, 1); if (v < 0) break; *out = (uint64_t)v; return BF_OK; }
        case KV_U16: { uint16_t v; memcpy(&v, p, 2); *out = v; return BF_OK; }
        case KV_I16: { int16_t v; memcpy(&v, p, 2); if (v < 0) break; *out = (uint64_t)v; return BF_OK; }
        case KV_U32: { uint32_t v; memcpy(&v, p, 4); *out = v; return BF_OK; }
        case KV_I32: { int32_t v; memcpy(&v, p, 4); if (v < 0) break; *out = (uint64_t)v; return BF_OK; }
        case KV_U64: { uint64_t v; memcpy(&v, p, 8); *out = v; return BF_OK; }
        case KV_I64: { int64_t v; memcpy(&v, p, 8); if (v < 0) break; *out = (uint64_t)v; return BF_OK; }
        default: return gguf_fail("metadata %s is not an integer", key);
    }
    return gguf_fail("metadata %s is negative", key);
}

bf_status bf_gguf_get_str(const bf_gguf* g, const char* key, const char** out, uint64_t* len) {
    if (!g || !key || !out || !len) return gguf_fail("handle, key or out is NULL");
    const Kv* e = find_kv(g, key);
    if (!e) return gguf_fail("no metadata key %s", key);
    if (e->type != KV_STRING) return gguf_fail("metadata %s is not a string", key);
    memcpy(len, g->map + e->pos, 8);
    *out = (const char*)g->map + e->pos + 8;
    return BF_OK;
}

bf_status bf_gguf_upload(const bf_gguf* g, const bf_gguf_tensor* t, void* dst, void* stream) {
    if (!g || !t || !dst) return gguf_fail("handle, tensor or dst is NULL");
    if (!t->data || !t->nbytes) return gguf_fail("tensor %s has no known byte size", t->name ? t->name : "?");
    if ((const uint8_t*)t->data < g->map || t->nbytes > g->size ||
        (const uint8_t*)t->data - g->map > (ptrdiff_t)(g->size - t->nbytes))
        return gguf_fail("tensor does not belong to this file");
    return bf::copy_to_device(dst, t->data, t->nbytes, stream) ? BF_OK : BF_ERR_HIP;
}

}  // extern "C"
