// GGUF v2/v3 container reader and the ggml type table (see gguf_file.h for
// the format facts followed, with their reference lines).
#include "gguf_file.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>

namespace xjg {

int scalar_width(uint32_t t) {
    switch (t) {
    case U8: case I8: case BOOL: return 1;
    case U16: case I16: return 2;
    case U32: case I32: case F32: return 4;
    case U64: case I64: case F64: return 8;
    default: return 0;
    }
}

// Integer (or bool) stored at p with type t, truncated to 32 bits the way a C
// cast does; signed types sign-extend first.
static bool load_uint(uint32_t t, const uint8_t *p, uint32_t *out) {
    int64_t s = 0;
    uint64_t u = 0;
    switch (t) {
    case U8: u = p[0]; break;
    case BOOL: u = p[0] != 0; break;
    case I8: s = (int8_t)p[0]; u = (uint64_t)s; break;
    case U16: { uint16_t v; memcpy(&v, p, 2); u = v; break; }
    case I16: { int16_t v; memcpy(&v, p, 2); u = (uint64_t)(int64_t)v; break; }
    case U32: case I32: { uint32_t v; memcpy(&v, p, 4); u = v; break; }
    case U64: case I64: memcpy(&u, p, 8); break;
    default: return false;
    }
    *out = (uint32_t)u;
    return true;
}

bool Value::as_uint(uint32_t *out) const { return load_uint(type, at, out); }

bool Value::as_float(float *out) const {
    if (type == F32) { memcpy(out, at, 4); return true; }
    if (type == F64) { double d; memcpy(&d, at, 8); *out = (float)d; return true; }
    uint32_t u;
    if (!load_uint(type, at, &u)) return false;
    *out = (float)u;
    return true;
}

bool Value::as_string(std::string_view *out) const {
    if (type != STR) return false;
    uint64_t n;
    memcpy(&n, at, 8);
    *out = std::string_view((const char *)at + 8, n);
    return true;
}

bool Value::uint_at(uint64_t i, uint32_t *out) const {
    if (type != ARR || i >= count) return false;
    const int w = scalar_width(elem);
    return w && load_uint(elem, body + i * w, out);
}

namespace {

// Bounds-checked cursor over the header bytes.
struct Cursor {
    const uint8_t *p, *end;
    bool short_read = false;
    bool take(uint64_t n) {
        if ((uint64_t)(end - p) < n) { short_read = true; return false; }
        p += n;
        return true;
    }
    template <class T> bool read(T *v) {
        const uint8_t *at = p;
        if (!take(sizeof(T))) return false;
        memcpy(v, at, sizeof(T));
        return true;
    }
    bool text(std::string_view *s) {
        uint64_t n;
        if (!read(&n)) return false;
        const uint8_t *at = p;
        if (!take(n)) return false;
        *s = std::string_view((const char *)at, n);
        return true;
    }
};

// Steps over one value of type t, filling v's description of it.
bool step_value(Cursor &c, uint32_t t, Value *v) {
    v->type = t;
    v->at = c.p;
    if (t == STR) { std::string_view s; return c.text(&s); }
    if (t != ARR) { const int w = scalar_width(t); return w && c.take(w); }
    if (!c.read(&v->elem) || !c.read(&v->count)) return false;
    v->body = c.p;
    if (v->elem == STR) {
        for (uint64_t i = 0; i < v->count; i++) { std::string_view s; if (!c.text(&s)) return false; }
        return true;
    }
    const int w = scalar_width(v->elem);
    if (!w || v->count > UINT64_MAX / w) return false;
    return c.take(v->count * (uint64_t)w);
}

bool fail(char *err, size_t errlen, const char *msg) {
    snprintf(err, errlen, "%s", msg);
    return false;
}

// Parses the header in buf[0, len) into f; *truncated tells a header that
// runs past len from one that is malformed.
bool parse_header(xj_gguf_file *f, const uint8_t *buf, uint64_t len, char *err, size_t errlen, bool *truncated) {
    Cursor c{buf, buf + len};
    struct Flag { Cursor &c; bool *t; ~Flag() { if (t) *t = c.short_read; } } flag{c, truncated};
    uint32_t magic = 0, version = 0;
    uint64_t n_tensors = 0, n_kv = 0;
    if (!c.read(&magic) || !c.read(&version)) return fail(err, errlen, "GGUF header truncated");
    if (magic != 0x46554747u) return fail(err, errlen, "not a GGUF file");
    if (version < 2 || version > 3) { snprintf(err, errlen, "GGUF version %u not supported", version); return false; }
    if (!c.read(&n_tensors) || !c.read(&n_kv)) return fail(err, errlen, "GGUF header truncated");
    if (n_kv > (1u << 20) || n_tensors > (1u << 20)) return fail(err, errlen, "GGUF header counts out of range");
    f->keys.reserve(n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string_view k;
        uint32_t t = 0;
        Value v;
        if (!c.text(&k) || !c.read(&t)) return fail(err, errlen, "GGUF header truncated");
        if (!step_value(c, t, &v)) {
            if (c.short_read) return fail(err, errlen, "GGUF header truncated");
            snprintf(err, errlen, "GGUF value of type %u unreadable", t);
            return false;
        }
        if (t == U32 && k == "general.alignment") memcpy(&f->alignment, v.at, 4);
        f->keys.emplace(std::string(k), v);   // first occurrence of a key wins
    }
    if (f->alignment == 0 || (f->alignment & (f->alignment - 1))) {
        snprintf(err, errlen, "bad alignment %u", f->alignment);
        return false;
    }
    f->tensors.resize(n_tensors);
    f->by_name.reserve(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        Tensor &t = f->tensors[i];
        std::string_view name;
        if (!c.text(&name) || !c.read(&t.n_dims)) return fail(err, errlen, "GGUF header truncated");
        t.name.assign(name);
        if (t.n_dims > 4) { snprintf(err, errlen, "tensor with %u dims", t.n_dims); return false; }
        for (uint32_t d = 0; d < t.n_dims; d++) {
            uint64_t e;
            if (!c.read(&e)) return fail(err, errlen, "GGUF header truncated");
            t.ne[d] = (int64_t)e;
        }
        if (!c.read(&t.type) || !c.read(&t.offset)) return fail(err, errlen, "GGUF header truncated");
        f->by_name.emplace(t.name, (size_t)i);
        int bb = 0;
        const int bn = xjh_type_block(t.type, &bb);
        if (!bn) continue;                 // unknown type: nbytes 0, refused when bound
        if (t.ne[0] % bn) {
            snprintf(err, errlen, "tensor %s row length %lld not a multiple of the block", t.name.c_str(), (long long)t.ne[0]);
            return false;
        }
        t.nbytes = xjh_row_bytes(t.type, t.ne[0]) * (uint64_t)(t.ne[1] * t.ne[2] * t.ne[3]);
    }
    const uint64_t end = (uint64_t)(c.p - buf);
    f->data_off = (end + f->alignment - 1) / f->alignment * f->alignment;
    return true;
}

int open_file(const char *path, uint64_t *size, char *err, size_t errlen) {
    const int fd = open(path, O_RDONLY);
    if (fd < 0) { snprintf(err, errlen, "cannot open %s", path); return -1; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 16) { close(fd); snprintf(err, errlen, "file too small"); return -1; }
    *size = (uint64_t)st.st_size;
    return fd;
}

}  // namespace

xj_gguf_file *open_mapped(const char *path, char *err, size_t errlen) {
    uint64_t size = 0;
    const int fd = open_file(path, &size, err, errlen);
    if (fd < 0) return nullptr;
    void *m = mmap(nullptr, (size_t)size, PROT_READ, MAP_SHARED, fd, 0);
    if (m == MAP_FAILED) { close(fd); snprintf(err, errlen, "mmap failed"); return nullptr; }
    auto *f = new xj_gguf_file();
    f->fd = fd; f->size = size;
    f->map = (const uint8_t *)m; f->map_off = 0; f->map_len = size;
    if (!parse_header(f, f->map, size, err, errlen, nullptr)) { delete f; return nullptr; }
    for (const Tensor &t : f->tensors)
        if (f->data_off + t.offset + t.nbytes > size) {
            snprintf(err, errlen, "tensor %s runs past the end of the file", t.name.c_str());
            delete f;
            return nullptr;
        }
    return f;
}

xj_gguf_file *open_header(const char *path, char *err, size_t errlen) {
    uint64_t size = 0;
    const int fd = open_file(path, &size, err, errlen);
    if (fd < 0) return nullptr;
    // Read a prefix that doubles from 16 MiB until the header parses or the file ends.
    for (uint64_t want = 16u << 20;; want *= 2) {
        if (want > size) want = size;
        std::vector<uint8_t> buf(want);
        uint64_t got = 0;
        while (got < want) {
            const ssize_t k = pread(fd, buf.data() + got, want - got, (off_t)got);
            if (k <= 0) break;
            got += (uint64_t)k;
        }
        auto *f = new xj_gguf_file();
        f->fd = fd; f->size = size;
        f->header = std::move(buf);        // values point into this storage; it moves with the vector
        bool truncated = false;
        if (parse_header(f, f->header.data(), got, err, errlen, &truncated)) return f;
        f->fd = -1;
        delete f;
        if (!truncated || got < want || want >= size) { close(fd); return nullptr; }
    }
}

bool map_range(xj_gguf_file *f, uint64_t lo, uint64_t hi, char *err, size_t errlen) {
    if (f->map) return fail(err, errlen, "already mapped");
    if (hi > f->size || lo >= hi) return fail(err, errlen, "mapping range runs past the end of the file (incomplete download?)");
    const uint64_t page = (uint64_t)getpagesize(), start = lo / page * page;
    void *m = mmap(nullptr, (size_t)(hi - start), PROT_READ, MAP_SHARED, f->fd, (off_t)start);
    if (m == MAP_FAILED) {
        snprintf(err, errlen, "mapping %llu MB failed", (unsigned long long)((hi - start) >> 20));
        return false;
    }
    f->map = (const uint8_t *)m; f->map_off = start; f->map_len = hi - start;
    return true;
}

}  // namespace xjg

xj_gguf_file::~xj_gguf_file() {
    if (map) munmap((void *)map, map_len);
    if (fd >= 0) close(fd);
}

// ------------------------------------------------------- ggml type table --

namespace {
struct TypeInfo { uint32_t id; int block; int bytes; const char *name; };
constexpr TypeInfo kTypes[] = {
    {XJ_F32, 1, 4, "F32"},       {XJ_F16, 1, 2, "F16"},       {XJ_BF16, 1, 2, "BF16"},
    {XJ_Q4_0, 32, 18, "Q4_0"},   {XJ_Q4_1, 32, 20, "Q4_1"},   {XJ_Q5_0, 32, 22, "Q5_0"},
    {XJ_Q5_1, 32, 24, "Q5_1"},   {XJ_Q8_0, 32, 34, "Q8_0"},   {XJ_Q2_K, 256, 84, "Q2_K"},
    {XJ_Q3_K, 256, 110, "Q3_K"}, {XJ_Q4_K, 256, 144, "Q4_K"}, {XJ_Q5_K, 256, 176, "Q5_K"},
    {XJ_Q6_K, 256, 210, "Q6_K"},
};
const TypeInfo *type_info(uint32_t t) {
    for (const TypeInfo &e : kTypes) if (e.id == t) return &e;
    return nullptr;
}
}  // namespace

extern "C" int xjh_type_block(uint32_t type, int *block_bytes) {
    const TypeInfo *e = type_info(type);
    if (block_bytes) *block_bytes = e ? e->bytes : 0;
    return e ? e->block : 0;
}

extern "C" uint64_t xjh_row_bytes(uint32_t type, int64_t n) {
    const TypeInfo *e = type_info(type);
    return e ? (uint64_t)(n / e->block) * (uint64_t)e->bytes : 0;
}

extern "C" const char *xjh_type_name(uint32_t type) {
    const TypeInfo *e = type_info(type);
    return e ? e->name : "?";
}
