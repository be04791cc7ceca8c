// GGUF reader and GGUF -> HBM loader (include/uq_gguf.h).
//
// The header is validated in one pass over the file's bytes (a read-only
// mapping, or a private copy for uq_gguf_parse), in the order of
// gguf::parse (crates/unltd-model-loader/src/gguf.rs:353-520). Nothing is
// copied out of the file except names: metadata values, shapes and tensor
// bytes are served as pointers into the mapping.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/uq_gguf.h"
#include "uq_internal.h"

using uq::set_error;

namespace {

constexpr uint64_t kAlign = 32;  // GGUF_ALIGN, gguf.rs:31

struct Kv {
    std::string key;
    uint32_t type = 0, elem = 0;
    uint64_t count = 1;
    uint64_t data = 0;                                  // file offset of the value(s)
    std::vector<std::pair<uint64_t, uint64_t>> strs;    // (offset, length) per string
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> shape;
    uint32_t type = 0;
    uint64_t offset = 0, nbytes = 0, n_elements = 0;
    bool has_nbytes = false;
};

// ggml_type_blocksize (gguf.rs:193-234): {block bytes, block elements};
// {0, 0} where the table has no entry (unknown, retired).
struct BlockSize {
    uint64_t bytes, elems;
};
BlockSize block_size(uint32_t id) {
    static const BlockSize table[] = {
        {4, 1},     {2, 1},     {18, 32},   {20, 32},  {0, 0},    {0, 0},     {22, 32},   {24, 32},
        {34, 32},   {36, 32},   {84, 256},  {110, 256}, {144, 256}, {176, 256}, {210, 256}, {292, 256},
        {66, 256},  {74, 256},  {98, 256},  {50, 256}, {18, 32},  {110, 256}, {82, 256},  {136, 256},
        {1, 1},     {2, 1},     {4, 1},     {8, 1},    {8, 1},    {56, 256},  {2, 1},     {0, 0},
        {0, 0},     {0, 0},     {54, 256},  {66, 256}, {0, 0},    {0, 0},     {0, 0},     {17, 32},
        {36, 64},   {18, 128},
    };
    return id < sizeof table / sizeof table[0] ? table[id] : BlockSize{0, 0};
}

const char *type_name(uint32_t id) {
    static const char *names[] = {
        "F32",     "F16",    "Q4_0",   "Q4_1",    "retired(Q4_2/Q4_3)", "retired(Q4_2/Q4_3)", "Q5_0",
        "Q5_1",    "Q8_0",   "Q8_1",   "Q2_K",    "Q3_K",               "Q4_K",               "Q5_K",
        "Q6_K",    "Q8_K",   "IQ2_XXS", "IQ2_XS", "IQ3_XXS",            "IQ1_S",              "IQ4_NL",
        "IQ3_S",   "IQ2_S",  "IQ4_XS", "I8",      "I16",                "I32",                "I64",
        "F64",     "IQ1_M",  "BF16",   "retired", "retired",            "retired",            "TQ1_0",
        "TQ2_0",   "retired", "retired", "retired", "MXFP4",            "NVFP4",              "Q1_0",
    };
    return id < sizeof names / sizeof names[0] ? names[id] : nullptr;
}

// Bytes per element for the array cap (GgufValueType::elem_bytes, gguf.rs:76-86).
uint64_t elem_bytes(uint32_t t) {
    switch (t) {
    case UQ_GGUF_U16: case UQ_GGUF_I16: return 2;
    case UQ_GGUF_U32: case UQ_GGUF_I32: case UQ_GGUF_F32: return 4;
    case UQ_GGUF_U64: case UQ_GGUF_I64: case UQ_GGUF_F64: case UQ_GGUF_ARRAY: return 8;
    default: return 1;  // u8, i8, bool, string (strings are capped by their lengths)
    }
}

const char *value_type_name(uint32_t t) {
    static const char *n[] = {"u8", "i8", "u16", "i16", "u32", "i32", "f32", "bool", "string", "array", "u64", "i64", "f64"};
    return t <= 12 ? n[t] : "?";
}

// Bounds-checked little-endian cursor over the file. Every read that would
// cross the end of the file fails the parse with the reference's message.
struct Cursor {
    const uint8_t *base;
    uint64_t size, pos = 0;
    uq_status st = UQ_OK;

    bool take(uint64_t n, const uint8_t **p) {
        if (st) return false;
        if (n > size || pos > size - n) {
            st = set_error(UQ_ERR_FILE, "corrupt file: read of %llu bytes at offset %llu exceeds file size %llu",
                           (unsigned long long)n, (unsigned long long)pos, (unsigned long long)size);
            return false;
        }
        *p = base + pos;
        pos += n;
        return true;
    }
    template <class T>
    T get() {
        const uint8_t *p = nullptr;
        T v{};
        if (take(sizeof(T), &p)) std::memcpy(&v, p, sizeof(T));  // the host is little-endian
        return v;
    }
    // u64 length + bytes (rd_string, gguf.rs:589-600): (offset, length).
    bool str(uint64_t *off, uint64_t *len) {
        const uint64_t at = pos;
        *len = get<uint64_t>();
        if (st) return false;
        if (*len > size) {
            st = set_error(UQ_ERR_FILE, "corrupt file: string length %llu at offset %llu exceeds file size %llu",
                           (unsigned long long)*len, (unsigned long long)at, (unsigned long long)size);
            return false;
        }
        const uint8_t *p = nullptr;
        if (!take(*len, &p)) return false;
        *off = (uint64_t)(p - base);
        return true;
    }
};

}  // namespace

struct uq_gguf_s {
    uint32_t magic = 0x47475546u;
    // file bytes: a read-only mapping (open) or a private copy (parse)
    void *map = nullptr;
    size_t map_len = 0;
    std::vector<uint8_t> copy;
    const uint8_t *base = nullptr;
    uint64_t file_size = 0;

    uint32_t version = 0;
    uint64_t data_start = 0;
    std::vector<Kv> kvs;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, uint64_t> by_name;

    ~uq_gguf_s() {
        if (map) munmap(map, map_len);
    }
};

namespace {

uq_gguf_s *gguf_handle(uq_gguf g) { return g && g->magic == 0x47475546u ? g : nullptr; }

// rd_value (gguf.rs:602-658) into kv, after its key.
bool read_value(Cursor &c, Kv &kv) {
    const uint64_t at = c.pos;
    kv.type = c.get<uint32_t>();
    if (c.st) return false;
    if (kv.type > 12) {
        c.st = set_error(UQ_ERR_FILE, "corrupt file: unknown metadata value type id %u at offset %llu", kv.type,
                         (unsigned long long)at);
        return false;
    }
    kv.elem = kv.type;
    const uint8_t *p = nullptr;
    if (kv.type == UQ_GGUF_STRING) {
        uint64_t off, len;
        if (!c.str(&off, &len)) return false;
        kv.strs.emplace_back(off, len);
        return true;
    }
    if (kv.type != UQ_GGUF_ARRAY) {
        kv.data = c.pos;
        return c.take(elem_bytes(kv.type), &p);
    }
    kv.elem = c.get<uint32_t>();
    if (c.st) return false;
    if (kv.elem > 12) {
        c.st = set_error(UQ_ERR_FILE, "corrupt file: unknown array element type id %u at offset %llu", kv.elem,
                         (unsigned long long)at);
        return false;
    }
    kv.count = c.get<uint64_t>();
    if (c.st) return false;
    const uint64_t eb = elem_bytes(kv.elem);
    if (kv.count > c.size / eb) {  // count * eb > file size, overflow included
        c.st = set_error(UQ_ERR_FILE, "corrupt file: array of %llu %s(s) at offset %llu exceeds file size %llu",
                         (unsigned long long)kv.count, value_type_name(kv.elem), (unsigned long long)at,
                         (unsigned long long)c.size);
        return false;
    }
    if (kv.elem == UQ_GGUF_ARRAY) {
        c.st = set_error(UQ_ERR_FILE, "corrupt file: nested array in GGUF metadata");
        return false;
    }
    if (kv.elem == UQ_GGUF_STRING) {
        for (uint64_t i = 0; i < kv.count; i++) {
            uint64_t off, len;
            if (!c.str(&off, &len)) return false;
            kv.strs.emplace_back(off, len);
        }
        return true;
    }
    kv.data = c.pos;
    return c.take(kv.count * eb, &p);
}

// gguf::parse (gguf.rs:353-520) over g->base[0 .. g->file_size).
uq_status parse(uq_gguf_s *g) {
    Cursor c{g->base, g->file_size};
    const uint8_t *magic = nullptr;
    if (!c.take(4, &magic)) return c.st;
    if (std::memcmp(magic, "GGUF", 4) != 0)
        return set_error(UQ_ERR_MAGIC, "not a GGUF file: bad magic [%02X, %02X, %02X, %02X] (expected 'GGUF')",
                         magic[0], magic[1], magic[2], magic[3]);
    g->version = c.get<uint32_t>();
    if (c.st) return c.st;
    if (g->version != 2 && g->version != 3)
        return set_error(UQ_ERR_VERSION, "unsupported GGUF version %u (supported: 2 and 3)", g->version);

    const uint64_t n_tensors = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    if (c.st) return c.st;
    if (n_kv > c.size / 8)
        return set_error(UQ_ERR_FILE, "corrupt file: n_kv %llu is implausible for a file of %llu bytes",
                         (unsigned long long)n_kv, (unsigned long long)c.size);
    if (n_tensors > c.size / 16)
        return set_error(UQ_ERR_FILE, "corrupt file: n_tensors %llu is implausible for a file of %llu bytes",
                         (unsigned long long)n_tensors, (unsigned long long)c.size);

    // metadata pairs, contiguous
    g->kvs.reserve(n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
        Kv kv;
        uint64_t off, len;
        if (!c.str(&off, &len)) return c.st;
        kv.key.assign((const char *)g->base + off, len);
        if (!read_value(c, kv)) return c.st;
        g->kvs.push_back(std::move(kv));
    }
    // general.alignment: the first pair with that key, when it holds a u32
    for (const Kv &kv : g->kvs) {
        if (kv.key != "general.alignment") continue;
        if (kv.type == UQ_GGUF_U32) {
            uint32_t a;
            std::memcpy(&a, g->base + kv.data, 4);
            if (a != kAlign)
                return set_error(UQ_ERR_FILE, "corrupt file: general.alignment = %u: only %llu is supported", a,
                                 (unsigned long long)kAlign);
        }
        break;
    }

    // tensor infos, contiguous
    g->tensors.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor t;
        uint64_t off, len;
        if (!c.str(&off, &len)) return c.st;
        t.name.assign((const char *)g->base + off, len);
        const uint32_t n_dims = c.get<uint32_t>();
        if (c.st) return c.st;
        if (n_dims == 0) return set_error(UQ_ERR_FILE, "corrupt file: tensor '%s' has n_dims = 0", t.name.c_str());
        if (n_dims > 64)
            return set_error(UQ_ERR_FILE, "corrupt file: tensor '%s' has n_dims %u (sane limit: 64)", t.name.c_str(),
                             n_dims);
        t.shape.resize(n_dims);
        for (uint32_t d = 0; d < n_dims; d++) t.shape[d] = c.get<uint64_t>();
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (c.st) return c.st;
        uint64_t n = 1;
        for (uint64_t d : t.shape) {
            if (d != 0 && n > UINT64_MAX / d)
                return set_error(UQ_ERR_FILE, "corrupt file: tensor '%s': element count overflows u64",
                                 t.name.c_str());
            n *= d;
        }
        if (n == 0) return set_error(UQ_ERR_FILE, "corrupt file: tensor '%s' has zero elements", t.name.c_str());
        t.n_elements = n;
        // ceil(n / block_elems) * block_bytes; unknown type or an overflowing
        // round-up leaves nbytes unknown. The product wraps modulo 2^64 like
        // the reference's release build.
        const BlockSize bs = block_size(t.type);
        if (bs.elems && n <= UINT64_MAX - (bs.elems - 1)) {
            t.nbytes = ((n + bs.elems - 1) / bs.elems) * bs.bytes;
            t.has_nbytes = true;
        }
        g->tensors.push_back(std::move(t));
    }

    // data section: first multiple of 32 after the infos; offsets are relative to it
    g->data_start = (c.pos + kAlign - 1) / kAlign * kAlign;
    for (Tensor &t : g->tensors) {
        if (t.offset > UINT64_MAX - g->data_start)
            return set_error(UQ_ERR_FILE, "corrupt file: tensor '%s': absolute offset overflows u64",
                             t.name.c_str());
        t.offset += g->data_start;
    }

    // range checks in order of absolute offset (a stable sort, as sort_by_key)
    std::vector<const Tensor *> sorted;
    sorted.reserve(g->tensors.size());
    for (const Tensor &t : g->tensors) sorted.push_back(&t);
    std::stable_sort(sorted.begin(), sorted.end(),
                     [](const Tensor *a, const Tensor *b) { return a->offset < b->offset; });
    const Tensor *prev = nullptr;
    for (const Tensor *t : sorted) {
        if (t->offset % kAlign)
            return set_error(UQ_ERR_TENSOR_ALIGN, "tensor '%s' at offset %llu is not aligned to %llu bytes",
                             t->name.c_str(), (unsigned long long)t->offset, (unsigned long long)kAlign);
        if (t->has_nbytes) {
            if (t->nbytes > g->file_size || t->offset > g->file_size - t->nbytes)
                return set_error(UQ_ERR_TENSOR_BOUNDS,
                                 "tensor '%s' claims bytes [%llu, %llu+%llu) beyond file size %llu", t->name.c_str(),
                                 (unsigned long long)t->offset, (unsigned long long)t->offset,
                                 (unsigned long long)t->nbytes, (unsigned long long)g->file_size);
            if (prev && prev->has_nbytes && prev->offset + prev->nbytes > t->offset)
                return set_error(UQ_ERR_TENSOR_OVERLAP, "tensor data overlap: '%s' ends at %llu, '%s' starts at %llu",
                                 prev->name.c_str(), (unsigned long long)(prev->offset + prev->nbytes),
                                 t->name.c_str(), (unsigned long long)t->offset);
        }
        prev = t;
    }

    // name index: a repeated name maps to its last tensor (HashMap::insert)
    for (uint64_t i = 0; i < g->tensors.size(); i++) g->by_name[g->tensors[i].name] = i;
    return UQ_OK;
}

uq_status finish(uq_gguf_s *g, uq_gguf *out) {
    const uq_status st = parse(g);
    if (st) {
        delete g;
        return st;
    }
    *out = g;
    return UQ_OK;
}

const Tensor *find_tensor(const uq_gguf_s *g, const char *name) {
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

// dtype_of (min_forward.rs:39-48).
bool dtype_of(uint32_t id, uq_dtype *d) {
    switch (id) {
    case 0: *d = UQ_F32; return true;
    case 1: *d = UQ_F16; return true;
    case 8: *d = UQ_Q8_0; return true;
    case 12: *d = UQ_Q4_K; return true;
    case 14: *d = UQ_Q6_K; return true;
    default: return false;
    }
}

}  // namespace

extern "C" {

uq_status uq_gguf_open(const char *path, uq_gguf *out) {
    if (!out) return set_error(UQ_ERR_ARG, "gguf_open: null handle pointer");
    *out = nullptr;
    if (!path) return set_error(UQ_ERR_ARG, "gguf_open: null path");
    const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return set_error(UQ_ERR_IO, "i/o error: %s: %s", path, std::strerror(errno));
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        const int e = errno;
        ::close(fd);
        return set_error(UQ_ERR_IO, "i/o error: %s: %s", path, std::strerror(e));
    }
    uq_gguf_s *g = new uq_gguf_s();
    g->file_size = (uint64_t)sb.st_size;
    if (sb.st_size > 0) {
        void *m = mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
        if (m == MAP_FAILED) {
            const int e = errno;
            ::close(fd);
            delete g;
            return set_error(UQ_ERR_IO, "i/o error: mmap %s: %s", path, std::strerror(e));
        }
        g->map = m;
        g->map_len = (size_t)sb.st_size;
        g->base = (const uint8_t *)m;
    } else {
        g->base = g->copy.data();
    }
    ::close(fd);
    return finish(g, out);
}

uq_status uq_gguf_parse(const void *bytes, size_t len, uq_gguf *out) {
    if (!out) return set_error(UQ_ERR_ARG, "gguf_parse: null handle pointer");
    *out = nullptr;
    if (!bytes && len) return set_error(UQ_ERR_ARG, "gguf_parse: null bytes");
    uq_gguf_s *g = new uq_gguf_s();
    g->copy.assign((const uint8_t *)bytes, (const uint8_t *)bytes + len);
    g->base = g->copy.data();
    g->file_size = len;
    return finish(g, out);
}

uq_status uq_gguf_close(uq_gguf gh) {
    uq_gguf_s *g = gguf_handle(gh);
    if (!g) return gh ? set_error(UQ_ERR_ARG, "gguf_close: invalid handle") : UQ_OK;
    g->magic = 0;
    delete g;
    return UQ_OK;
}

uq_status uq_gguf_header(uq_gguf gh, uint32_t *version, uint64_t *file_size, uint64_t *data_start, uint64_t *n_kv,
                         uint64_t *n_tensors) {
    const uq_gguf_s *g = gguf_handle(gh);
    if (!g) return set_error(UQ_ERR_ARG, "gguf_header: invalid handle");
    if (version) *version = g->version;
    if (file_size) *file_size = g->file_size;
    if (data_start) *data_start = g->data_start;
    if (n_kv) *n_kv = g->kvs.size();
    if (n_tensors) *n_tensors = g->tensors.size();
    return UQ_OK;
}

uq_status uq_gguf_tensor_at(uq_gguf gh, uint64_t i, uq_gguf_tensor *out) {
    const uq_gguf_s *g = gguf_handle(gh);
    if (!g || !out) return set_error(UQ_ERR_ARG, "gguf_tensor_at: invalid handle or null output");
    if (i >= g->tensors.size())
        return set_error(UQ_ERR_ARG, "gguf_tensor_at: index %llu >= %zu tensors", (unsigned long long)i,
                         g->tensors.size());
    const Tensor &t = g->tensors[i];
    out->name = t.name.data();
    out->name_len = t.name.size();
    out->offset = t.offset;
    out->nbytes = t.has_nbytes ? t.nbytes : 0;
    out->has_nbytes = t.has_nbytes;
    out->ggml_type = t.type;
    out->n_dims = (uint32_t)t.shape.size();
    out->shape = t.shape.data();
    out->n_elements = t.n_elements;
    return UQ_OK;
}

uq_status uq_gguf_find(uq_gguf gh, const char *name, uint64_t *index) {
    const uq_gguf_s *g = gguf_handle(gh);
    if (!g || !name) return set_error(UQ_ERR_ARG, "gguf_find: invalid handle or null name");
    auto it = g->by_name.find(name);
    if (it == g->by_name.end()) return set_error(UQ_ERR_MISSING_TENSOR, "tensor '%s' not found in the file index", name);
    if (index) *index = it->second;
    return UQ_OK;
}

}  // extern "C"

namespace {

// MappedWeights::tensor / tensor_checked: missing, then (when asked) the
// element count, then an unknown type. The parse has checked that
// offset + nbytes lies inside the file.
uq_status tensor_bytes(uq_gguf gh, const char *name, const uint64_t *n_elements, const uint8_t **bytes,
                       uint64_t *nbytes, const Tensor **tensor) {
    const uq_gguf_s *g = gguf_handle(gh);
    if (!g || !name) return set_error(UQ_ERR_ARG, "gguf_tensor: invalid handle or null name");
    const Tensor *t = find_tensor(g, name);
    if (!t) return set_error(UQ_ERR_MISSING_TENSOR, "tensor '%s' not found in the file index", name);
    if (n_elements && t->n_elements != *n_elements)
        return set_error(UQ_ERR_ELEMENT_COUNT, "tensor '%s' has %llu elements, expected %llu", name,
                         (unsigned long long)t->n_elements, (unsigned long long)*n_elements);
    if (!t->has_nbytes) return set_error(UQ_ERR_GGML_TYPE, "unknown ggml type id %u", t->type);
    if (bytes) *bytes = g->base + t->offset;
    if (nbytes) *nbytes = t->nbytes;
    if (tensor) *tensor = t;
    return UQ_OK;
}

}  // namespace

extern "C" {

uq_status uq_gguf_tensor_checked(uq_gguf g, const char *name, uint64_t n_elements, const uint8_t **bytes,
                                 uint64_t *nbytes) {
    return tensor_bytes(g, name, &n_elements, bytes, nbytes, nullptr);
}

uq_status uq_gguf_tensor_bytes(uq_gguf g, const char *name, const uint8_t **bytes, uint64_t *nbytes) {
    return tensor_bytes(g, name, nullptr, bytes, nbytes, nullptr);
}

uq_status uq_gguf_check(uq_gguf gh, const char *name, uint64_t n_elements, uint64_t allowed, uq_dtype *dtype) {
    const uq_gguf_s *g = gguf_handle(gh);
    if (!g || !name) return set_error(UQ_ERR_ARG, "gguf_check: invalid handle or null name");
    const Tensor *t = find_tensor(g, name);
    if (!t) return set_error(UQ_ERR_MISSING_TENSOR, "tensor '%s' not found in the file index", name);
    if (t->n_elements != n_elements)
        return set_error(UQ_ERR_ELEMENT_COUNT, "tensor '%s' has %llu elements, expected %llu", name,
                         (unsigned long long)t->n_elements, (unsigned long long)n_elements);
    uq_dtype d;
    if (!dtype_of(t->type, &d)) return set_error(UQ_ERR_GGML_TYPE, "unknown ggml type id %u", t->type);
    if (!((allowed >> (unsigned)d) & 1))
        return set_error(UQ_ERR_FILE, "corrupt file: tensor '%s': dtype %s is not among the allowed ones", name,
                         type_name(t->type));
    if (dtype) *dtype = d;
    return UQ_OK;
}

uq_status uq_gguf_upload(uq_gguf gh, const char *name, uq_weights *out) {
    if (!out) return set_error(UQ_ERR_ARG, "gguf_upload: null handle pointer");
    *out = nullptr;
    const uint8_t *bytes = nullptr;
    uint64_t nbytes = 0;
    const Tensor *t = nullptr;
    const uq_status st = tensor_bytes(gh, name, nullptr, &bytes, &nbytes, &t);
    if (st) return st;
    uq_dtype d;
    if (!dtype_of(t->type, &d)) return set_error(UQ_ERR_GGML_TYPE, "unknown ggml type id %u", t->type);
    const uint64_t dim_in = t->shape[0], dim_out = t->n_elements / t->shape[0];
    return uq_weights_upload(out, bytes, (size_t)nbytes, d, (size_t)dim_in, (size_t)dim_out);
}

uq_status uq_gguf_kv_at(uq_gguf gh, uint64_t i, uq_gguf_kv *out) {
    const uq_gguf_s *g = gguf_handle(gh);
    if (!g || !out) return set_error(UQ_ERR_ARG, "gguf_kv_at: invalid handle or null output");
    if (i >= g->kvs.size())
        return set_error(UQ_ERR_ARG, "gguf_kv_at: index %llu >= %zu pairs", (unsigned long long)i, g->kvs.size());
    const Kv &kv = g->kvs[i];
    out->key = kv.key.data();
    out->key_len = kv.key.size();
    out->type = kv.type;
    out->elem_type = kv.elem;
    out->count = kv.count;
    out->data = kv.elem == UQ_GGUF_STRING ? nullptr : g->base + kv.data;
    return UQ_OK;
}

uq_status uq_gguf_kv_find(uq_gguf gh, const char *key, uint64_t *index) {
    const uq_gguf_s *g = gguf_handle(gh);
    if (!g || !key) return set_error(UQ_ERR_ARG, "gguf_kv_find: invalid handle or null key");
    for (uint64_t i = 0; i < g->kvs.size(); i++)
        if (g->kvs[i].key == key) {
            if (index) *index = i;
            return UQ_OK;
        }
    return set_error(UQ_ERR_ARG, "gguf_kv_find: no key '%s'", key);
}

uq_status uq_gguf_kv_string(uq_gguf gh, uint64_t i, uint64_t elem, const char **s, size_t *len) {
    const uq_gguf_s *g = gguf_handle(gh);
    if (!g || !s || !len) return set_error(UQ_ERR_ARG, "gguf_kv_string: invalid handle or null output");
    if (i >= g->kvs.size())
        return set_error(UQ_ERR_ARG, "gguf_kv_string: index %llu >= %zu pairs", (unsigned long long)i, g->kvs.size());
    const Kv &kv = g->kvs[i];
    if (kv.elem != UQ_GGUF_STRING) return set_error(UQ_ERR_ARG, "gguf_kv_string: '%s' holds no string", kv.key.c_str());
    if (kv.type == UQ_GGUF_STRING) elem = 0;
    if (elem >= kv.strs.size())
        return set_error(UQ_ERR_ARG, "gguf_kv_string: element %llu of %zu", (unsigned long long)elem, kv.strs.size());
    *s = (const char *)g->base + kv.strs[elem].first;
    *len = (size_t)kv.strs[elem].second;
    return UQ_OK;
}

uq_status uq_gguf_type_blocksize(uint32_t id, uint64_t *block_bytes, uint64_t *block_elems) {
    const BlockSize bs = block_size(id);
    if (!bs.elems) return set_error(UQ_ERR_GGML_TYPE, "unknown ggml type id %u", id);
    if (block_bytes) *block_bytes = bs.bytes;
    if (block_elems) *block_elems = bs.elems;
    return UQ_OK;
}

uq_status uq_gguf_type_name(uint32_t id, char *buf, size_t len) {
    if (!buf || !len) return set_error(UQ_ERR_ARG, "gguf_type_name: empty buffer");
    const char *n = type_name(id);
    if (n)
        snprintf(buf, len, "%s", n);
    else
        snprintf(buf, len, "unknown(%u)", id);
    return UQ_OK;
}

}  // extern "C"
