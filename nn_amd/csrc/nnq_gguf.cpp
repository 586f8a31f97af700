// GGUF ingest: a memory-mapped GGUF v3 reader whose tensor bytes go straight into device
// weights (no f32 detour).  It follows nn-gguf's GgufFile::open
// (crates/nn-gguf/src/reader.rs:68-141): header (header.rs:47-80), metadata key-value
// pairs (metadata.rs:86-222), tensor infos (tensor_info.rs:36-82), the data section at
// the next multiple of 32 bytes after the tensor infos (the reference fixes the alignment
// at 32 and ignores general.alignment), and every tensor's byte range checked against
// the file before any access.  Limits and error kinds are the reference's.
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

#include "nnq_internal.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint64_t kMaxString = 16ull << 20;
constexpr uint64_t kMaxTensorBytes = 8ull << 30;
constexpr uint64_t kMaxTensors = 100000;
constexpr uint64_t kMaxKv = 100000;
constexpr uint64_t kMaxArray = 10000000;
constexpr uint32_t kMaxDims = 8;
constexpr uint64_t kAlign = 32;

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    uint32_t dtype = 0;
    uint64_t offset = 0, nbytes = 0;
};

struct Meta {
    uint32_t type = 0;
    uint64_t u = 0;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    uint32_t arr_type = 0;
    uint64_t arr_count = 0;
};

// GgufDType::block_size / type_size (crates/nn-gguf/src/dequant.rs:84-114); unknown ids
// are rejected, the IQ types keep the reference's sizes (block 1, 0 bytes)
bool dtype_sizes(uint32_t t, uint64_t *bs, uint64_t *ts) {
    switch (t) {
    case 0: *bs = 1, *ts = 4; return true;     // F32
    case 1: *bs = 1, *ts = 2; return true;     // F16
    case 2: *bs = 32, *ts = 18; return true;   // Q4_0
    case 3: *bs = 32, *ts = 20; return true;   // Q4_1
    case 6: *bs = 32, *ts = 22; return true;   // Q5_0
    case 7: *bs = 32, *ts = 24; return true;   // Q5_1
    case 8: *bs = 32, *ts = 34; return true;   // Q8_0
    case 9: *bs = 32, *ts = 40; return true;   // Q8_1
    case 10: *bs = 256, *ts = 84; return true;  // Q2_K
    case 11: *bs = 256, *ts = 110; return true; // Q3_K
    case 12: *bs = 256, *ts = 144; return true; // Q4_K
    case 13: *bs = 256, *ts = 176; return true; // Q5_K
    case 14: *bs = 256, *ts = 210; return true; // Q6_K
    case 16: case 17: case 18: case 19: case 20: case 21: case 22: case 23: case 29:
        *bs = 1, *ts = 0; return true;          // IQ*
    case 24: *bs = 1, *ts = 1; return true;     // I8
    case 25: *bs = 1, *ts = 2; return true;     // I16
    case 26: *bs = 1, *ts = 4; return true;     // I32
    case 27: case 28: *bs = 1, *ts = 8; return true;  // I64, F64
    case 30: *bs = 1, *ts = 2; return true;     // BF16
    }
    return false;
}

struct Cursor {
    const uint8_t *p;
    uint64_t n, pos = 0;
    bool take(uint64_t k, const uint8_t **out) {
        if (k > n - pos) return false;
        *out = p + pos;
        pos += k;
        return true;
    }
    template <class T>
    bool get(T *v) {
        const uint8_t *q;
        if (!take(sizeof(T), &q)) return false;
        std::memcpy(v, q, sizeof(T));
        return true;
    }
};

}  // namespace

struct nnq_gguf {
    int fd = -1;
    const uint8_t *map = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t data_offset = 0;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> index;  // last entry of a name wins (HashMap insert)
    std::unordered_map<std::string, Meta> meta;
    ~nnq_gguf() {
        if (map) munmap(const_cast<uint8_t *>(map), size);
        if (fd >= 0) close(fd);
    }
};

namespace {

int gfail(int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return nnq::set_error(code, buf);
}

// read_string (header.rs:120-131)
int read_string(Cursor &c, std::string *s) {
    uint64_t len;
    if (!c.get(&len)) return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (string length)");
    if (len > kMaxString)
        return gfail(NNQ_ERR_INVALID_SHAPE, "GGUF: string length %llu exceeds %llu", (unsigned long long)len,
                     (unsigned long long)kMaxString);
    const uint8_t *q;
    if (!c.take(len, &q)) return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (string)");
    s->assign(reinterpret_cast<const char *>(q), len);
    return NNQ_OK;
}

// read_typed_value (metadata.rs:139-222); arrays are walked (each element parsed and
// checked) and kept as their element type and count
int read_value(Cursor &c, uint32_t type, Meta *m, int depth) {
    m->type = type;
    switch (type) {
    case 0: { uint8_t v; if (!c.get(&v)) break; m->u = v; return NNQ_OK; }
    case 1: { int8_t v; if (!c.get(&v)) break; m->i = v; return NNQ_OK; }
    case 2: { uint16_t v; if (!c.get(&v)) break; m->u = v; return NNQ_OK; }
    case 3: { int16_t v; if (!c.get(&v)) break; m->i = v; return NNQ_OK; }
    case 4: { uint32_t v; if (!c.get(&v)) break; m->u = v; return NNQ_OK; }
    case 5: { int32_t v; if (!c.get(&v)) break; m->i = v; return NNQ_OK; }
    case 6: { float v; if (!c.get(&v)) break; m->f = v; return NNQ_OK; }
    case 7: { uint8_t v; if (!c.get(&v)) break; m->u = v != 0; return NNQ_OK; }
    case 8: return read_string(c, &m->s);
    case 9: {
        uint32_t et;
        uint64_t cnt;
        if (!c.get(&et) || !c.get(&cnt)) break;
        if (cnt > kMaxArray)
            return gfail(NNQ_ERR_INVALID_SHAPE, "GGUF: array length %llu exceeds %llu", (unsigned long long)cnt,
                         (unsigned long long)kMaxArray);
        if (depth > 16) return gfail(NNQ_ERR_WRONG_FORMAT, "GGUF: arrays nested too deeply");
        m->arr_type = et;
        m->arr_count = cnt;
        Meta tmp;
        for (uint64_t k = 0; k < cnt; k++) {
            tmp = Meta{};
            int rc = read_value(c, et, &tmp, depth + 1);
            if (rc) return rc;
        }
        return NNQ_OK;
    }
    case 10: { uint64_t v; if (!c.get(&v)) break; m->u = v; return NNQ_OK; }
    case 11: { int64_t v; if (!c.get(&v)) break; m->i = v; return NNQ_OK; }
    case 12: { double v; if (!c.get(&v)) break; m->f = v; return NNQ_OK; }
    default:
        return gfail(NNQ_ERR_WRONG_FORMAT, "GGUF: unknown metadata type %u", type);
    }
    return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (metadata value)");
}

int parse(nnq_gguf *g) {
    Cursor c{g->map, g->size};
    uint32_t magic;
    if (!c.get(&magic)) return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (magic)");
    if (magic != kMagic) return gfail(NNQ_ERR_WRONG_FORMAT, "GGUF: invalid magic 0x%08x", magic);
    if (!c.get(&g->version)) return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (version)");
    if (g->version != 3) return gfail(NNQ_ERR_WRONG_FORMAT, "GGUF: unsupported version %u", g->version);
    uint64_t nt, nkv;
    if (!c.get(&nt) || !c.get(&nkv)) return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (counts)");
    if (nt > kMaxTensors)
        return gfail(NNQ_ERR_INVALID_SHAPE, "GGUF: tensor count %llu exceeds %llu", (unsigned long long)nt,
                     (unsigned long long)kMaxTensors);
    if (nkv > kMaxKv)
        return gfail(NNQ_ERR_INVALID_SHAPE, "GGUF: metadata count %llu exceeds %llu", (unsigned long long)nkv,
                     (unsigned long long)kMaxKv);
    for (uint64_t k = 0; k < nkv; k++) {
        std::string key;
        int rc = read_string(c, &key);
        if (rc) return rc;
        uint32_t type;
        if (!c.get(&type)) return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (metadata type)");
        Meta m;
        rc = read_value(c, type, &m, 0);
        if (rc) return rc;
        g->meta[key] = m;
    }
    g->tensors.resize(nt);
    for (uint64_t k = 0; k < nt; k++) {
        Tensor &t = g->tensors[k];
        int rc = read_string(c, &t.name);
        if (rc) return rc;
        uint32_t nd;
        if (!c.get(&nd)) return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (tensor info)");
        if (nd > kMaxDims) return gfail(NNQ_ERR_INVALID_SHAPE, "GGUF: %u dimensions exceed %u", nd, kMaxDims);
        t.dims.resize(nd);
        for (uint32_t d = 0; d < nd; d++) {
            if (!c.get(&t.dims[d])) return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (tensor dims)");
            if (t.dims[d] == 0)
                return gfail(NNQ_ERR_INVALID_SHAPE, "GGUF: tensor '%s' has a zero dimension at %u", t.name.c_str(), d);
        }
        if (!c.get(&t.dtype) || !c.get(&t.offset))
            return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: unexpected end of file (tensor info)");
        uint64_t bs, ts;
        if (!dtype_sizes(t.dtype, &bs, &ts)) return gfail(NNQ_ERR_WRONG_FORMAT, "GGUF: unknown tensor type %u", t.dtype);
        // checked_num_elements / checked_byte_size (tensor_info.rs:86-138)
        unsigned __int128 ne = 1;
        for (uint64_t d : t.dims) {
            ne *= d;
            if (ne > UINT64_MAX) return gfail(NNQ_ERR_INVALID_SHAPE, "GGUF: element count of '%s' overflows", t.name.c_str());
        }
        const unsigned __int128 bytes = (ne / bs) * ts;
        if (bytes > UINT64_MAX) return gfail(NNQ_ERR_INVALID_SHAPE, "GGUF: byte size of '%s' overflows", t.name.c_str());
        if ((uint64_t)bytes > kMaxTensorBytes)
            return gfail(NNQ_ERR_INVALID_SHAPE, "GGUF: tensor '%s' of %llu bytes exceeds %llu", t.name.c_str(),
                         (unsigned long long)bytes, (unsigned long long)kMaxTensorBytes);
        t.nbytes = (uint64_t)bytes;
        g->index[t.name] = k;
    }
    g->data_offset = (c.pos + kAlign - 1) / kAlign * kAlign;
    for (const Tensor &t : g->tensors) {
        const unsigned __int128 start = (unsigned __int128)g->data_offset + t.offset, end = start + t.nbytes;
        if (end > g->size)
            return gfail(NNQ_ERR_DATA_LENGTH, "GGUF: tensor '%s' data [%llu, %llu) out of bounds (file %llu bytes)",
                         t.name.c_str(), (unsigned long long)start, (unsigned long long)end,
                         (unsigned long long)g->size);
    }
    return NNQ_OK;
}

const Tensor *find(const nnq_gguf *g, const char *name) {
    auto it = g->index.find(name);
    return it == g->index.end() ? nullptr : &g->tensors[it->second];
}

}  // namespace

extern "C" {

int nnq_gguf_open(const char *path, nnq_gguf **out) {
    if (!out || !path) return gfail(NNQ_ERR_INVALID_ARGUMENT, "path or out is null");
    *out = nullptr;
    nnq_gguf *g = new nnq_gguf;
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    if (g->fd < 0) {
        delete g;
        return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF: cannot open '%s': %s", path, strerror(errno));
    }
    struct stat st;
    if (fstat(g->fd, &st) != 0) {
        delete g;
        return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF: cannot stat '%s'", path);
    }
    g->size = (uint64_t)st.st_size;
    if (g->size > 0) {
        void *m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
        if (m == MAP_FAILED) {
            delete g;
            return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF: cannot map '%s': %s", path, strerror(errno));
        }
        g->map = static_cast<const uint8_t *>(m);
    }
    int rc = parse(g);
    if (rc) {
        delete g;
        return rc;
    }
    *out = g;
    return NNQ_OK;
}

int nnq_gguf_close(nnq_gguf *g) {
    delete g;
    return NNQ_OK;
}

int nnq_gguf_info(const nnq_gguf *g, uint32_t *version, int64_t *tensor_count, int64_t *metadata_count,
                  uint64_t *data_offset) {
    if (!g) return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF handle is null");
    if (version) *version = g->version;
    if (tensor_count) *tensor_count = (int64_t)g->tensors.size();
    if (metadata_count) *metadata_count = (int64_t)g->meta.size();
    if (data_offset) *data_offset = g->data_offset;
    return NNQ_OK;
}

int nnq_gguf_tensor_info(const nnq_gguf *g, int64_t i, const char **name, int32_t *n_dims, uint64_t *dims,
                         uint32_t *dtype, uint64_t *offset, uint64_t *nbytes) {
    if (!g) return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF handle is null");
    if (i < 0 || (uint64_t)i >= g->tensors.size())
        return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF: tensor index %lld out of range", (long long)i);
    const Tensor &t = g->tensors[(size_t)i];
    if (name) *name = t.name.c_str();
    if (n_dims) *n_dims = (int32_t)t.dims.size();
    if (dims)
        for (size_t d = 0; d < t.dims.size(); d++) dims[d] = t.dims[d];
    if (dtype) *dtype = t.dtype;
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    return NNQ_OK;
}

int nnq_gguf_tensor_data(const nnq_gguf *g, const char *name, const uint8_t **data, uint64_t *nbytes) {
    if (!g || !name) return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF handle or name is null");
    const Tensor *t = find(g, name);
    if (!t) return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF: tensor not found: %s", name);
    if (data) *data = g->map + g->data_offset + t->offset;
    if (nbytes) *nbytes = t->nbytes;
    return NNQ_OK;
}

int nnq_gguf_metadata(const nnq_gguf *g, const char *key, uint32_t *type, uint64_t *u, int64_t *i, double *f,
                      const char **str, uint32_t *arr_type, uint64_t *arr_count) {
    if (!g || !key) return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF handle or key is null");
    auto it = g->meta.find(key);
    if (it == g->meta.end()) return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF: metadata key not found: %s", key);
    const Meta &m = it->second;
    if (type) *type = m.type;
    if (u) *u = m.u;
    if (i) *i = m.i;
    if (f) *f = m.f;
    if (str) *str = m.s.c_str();
    if (arr_type) *arr_type = m.arr_type;
    if (arr_count) *arr_count = m.arr_count;
    return NNQ_OK;
}

int nnq_gguf_weight_create(const nnq_gguf *g, const char *name, nnq_layout layout, int ggml_order, nnq_weight **out) {
    if (!g || !name || !out) return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF handle, name or out is null");
    *out = nullptr;
    const Tensor *t = find(g, name);
    if (!t) return gfail(NNQ_ERR_INVALID_ARGUMENT, "GGUF: tensor not found: %s", name);
    if (t->dtype != NNQ_FMT_Q8_0 && t->dtype != NNQ_FMT_Q4_K && t->dtype != NNQ_FMT_Q6_K)
        return gfail(NNQ_ERR_WRONG_FORMAT, "GGUF: tensor '%s' has type %u, not Q8_0 / Q4_K / Q6_K", name, t->dtype);
    if (t->dims.size() != 2)
        return gfail(NNQ_ERR_WEIGHT_RANK, "GGUF: tensor '%s' has %zu dimensions, a linear weight has 2", name,
                     t->dims.size());
    // dims as stored: [out, in] (nn-gguf's own writers), or ggml's ne0 = in first
    const int64_t n = (int64_t)(ggml_order ? t->dims[1] : t->dims[0]);
    const int64_t k = (int64_t)(ggml_order ? t->dims[0] : t->dims[1]);
    return nnq_weight_create((nnq_format)t->dtype, layout, g->map + g->data_offset + t->offset, t->nbytes, n, k, out);
}

}  // extern "C"
