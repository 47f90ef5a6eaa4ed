// GGUF v2/v3 reader (mmap) and qwen35 model table.
//
// Follows the reference's loader so that the xj_model it builds is the one the
// reference would build from the same file:
//   type table / row bytes     src/xiaoju-pipe/core/gguf.c:12-50
//   header + tensor-info parse src/xiaoju-pipe/core/gguf.c:106-186 (alignment key,
//                              data offset = header end rounded up to alignment)
//   hparams, layer pattern,    src/xiaoju-pipe/core/xj_model.c:129-202
//   tied head, fingerprint
//   per-layer tensor names     src/xiaoju-pipe/core/xj_model.c:62-101
//   MTP layer                  src/xiaoju-pipe/core/xj_model.c:104-127 (blk.{block_count-1}
//                              into layers[n_layer], its nextn.* tensors)
//   layer-range load           src/xiaoju-pipe/core/xj_model.c:214-233, 303-328 and
//                              gguf.c:216-262 (header read with pread, one mapping of
//                              the merged byte ranges, pointers outside it left NULL)
#include "xj_hip.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <algorithm>
#include <cstddef>
#include <cstring>
#include <string>
#include <vector>

namespace {

enum { GT_U8 = 0, GT_I8, GT_U16, GT_I16, GT_U32, GT_I32, GT_F32, GT_BOOL, GT_STR, GT_ARR, GT_U64, GT_I64, GT_F64 };

struct KV {
    std::string key;
    uint32_t type = 0, arr_type = 0;
    uint64_t arr_n = 0;
    const uint8_t *val = nullptr;  // points into the mapping
};

struct TInfo {
    std::string name;
    uint32_t n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint32_t type = 0;
    uint64_t offset = 0, nbytes = 0;
};

struct Reader {
    const uint8_t *p, *end;
    bool u32(uint32_t *v) { if (end - p < 4) return false; memcpy(v, p, 4); p += 4; return true; }
    bool u64(uint64_t *v) { if (end - p < 8) return false; memcpy(v, p, 8); p += 8; return true; }
    bool str(std::string *s) {
        uint64_t n;
        if (!u64(&n) || (uint64_t)(end - p) < n) return false;
        s->assign((const char *)p, n); p += n; return true;
    }
};

int scalar_size(uint32_t t) {
    switch (t) {
    case GT_U8: case GT_I8: case GT_BOOL: return 1;
    case GT_U16: case GT_I16: return 2;
    case GT_U32: case GT_I32: case GT_F32: return 4;
    case GT_U64: case GT_I64: case GT_F64: return 8;
    default: return 0;
    }
}

bool skip(Reader &r, uint32_t t, KV *kv) {
    if (t == GT_STR) { std::string s; return r.str(&s); }
    if (t == GT_ARR) {
        uint32_t et; uint64_t n;
        if (!r.u32(&et) || !r.u64(&n)) return false;
        if (kv) { kv->arr_type = et; kv->arr_n = n; }
        if (et == GT_STR) {
            for (uint64_t i = 0; i < n; i++) { std::string s; if (!r.str(&s)) return false; }
            return true;
        }
        int es = scalar_size(et);
        if (!es || n > UINT64_MAX / es || (uint64_t)(r.end - r.p) < n * es) return false;
        r.p += n * es;
        return true;
    }
    int s = scalar_size(t);
    if (!s || r.end - r.p < s) return false;
    r.p += s;
    return true;
}

}  // namespace

struct xj_gguf_file {
    int fd = -1;
    const uint8_t *map = nullptr;      // mapping of file bytes [map_off, map_off + map_len)
    uint64_t map_off = 0, map_len = 0;
    uint64_t size = 0, data_off = 0;
    std::vector<uint8_t> hdr;          // header bytes when only the header was read
    uint32_t alignment = 32;
    std::vector<KV> kv;
    std::vector<TInfo> tensors;

    const KV *find_kv(const char *k) const {
        for (auto &e : kv) if (e.key == k) return &e;
        return nullptr;
    }
    const TInfo *find_tensor(const char *n) const {
        for (auto &t : tensors) if (t.name == n) return &t;
        return nullptr;
    }
    bool get_u32(const char *k, uint32_t *out) const {
        const KV *e = find_kv(k);
        if (!e) return false;
        switch (e->type) {
        case GT_U8: *out = e->val[0]; return true;
        case GT_I8: *out = (uint32_t)(int32_t)(int8_t)e->val[0]; return true;
        case GT_U16: { uint16_t v; memcpy(&v, e->val, 2); *out = v; return true; }
        case GT_I16: { int16_t v; memcpy(&v, e->val, 2); *out = (uint32_t)(int32_t)v; return true; }
        case GT_U32: case GT_I32: memcpy(out, e->val, 4); return true;
        case GT_U64: case GT_I64: { uint64_t v; memcpy(&v, e->val, 8); *out = (uint32_t)v; return true; }
        default: return false;
        }
    }
    bool get_f32(const char *k, float *out) const {
        const KV *e = find_kv(k);
        if (!e) return false;
        if (e->type == GT_F32) { memcpy(out, e->val, 4); return true; }
        if (e->type == GT_F64) { double d; memcpy(&d, e->val, 8); *out = (float)d; return true; }
        return false;
    }
    bool get_str(const char *k, std::string *out) const {
        const KV *e = find_kv(k);
        if (!e || e->type != GT_STR) return false;
        uint64_t n; memcpy(&n, e->val, 8);
        out->assign((const char *)e->val + 8, n);
        return true;
    }
    bool get_arr_u32(const char *k, uint64_t i, uint32_t *out) const {
        const KV *e = find_kv(k);
        if (!e || e->type != GT_ARR || i >= e->arr_n) return false;
        int es = scalar_size(e->arr_type);
        if (!es || e->arr_type == GT_F32 || e->arr_type == GT_F64) return false;
        const uint8_t *p = e->val + 12 + i * es;
        uint64_t v = 0; memcpy(&v, p, es);
        if (e->arr_type == GT_I8) v = (uint64_t)(int64_t)(int8_t)v;
        if (e->arr_type == GT_I16) v = (uint64_t)(int64_t)(int16_t)v;
        *out = (uint32_t)v;
        return true;
    }
    // File offset -> pointer into the mapping, NULL when not mapped (gguf.c:257-260).
    const void *ptr(uint64_t file_off, uint64_t nbytes) const {
        if (!map || file_off < map_off || file_off + nbytes > map_off + map_len) return nullptr;
        return map + (file_off - map_off);
    }
    ~xj_gguf_file() {
        if (map) munmap((void *)map, map_len);
        if (fd >= 0) close(fd);
    }
};

extern "C" int xj_type_block(uint32_t type, int *block_bytes) {
    int n = 0, b = 0;
    switch (type) {
    case XJ_F32: n = 1; b = 4; break;
    case XJ_F16: n = 1; b = 2; break;
    case XJ_BF16: n = 1; b = 2; break;
    case XJ_Q4_0: n = 32; b = 18; break;
    case XJ_Q4_1: n = 32; b = 20; break;
    case XJ_Q5_0: n = 32; b = 22; break;
    case XJ_Q5_1: n = 32; b = 24; break;
    case XJ_Q8_0: n = 32; b = 34; break;
    case XJ_Q2_K: n = 256; b = 84; break;
    case XJ_Q3_K: n = 256; b = 110; break;
    case XJ_Q4_K: n = 256; b = 144; break;
    case XJ_Q5_K: n = 256; b = 176; break;
    case XJ_Q6_K: n = 256; b = 210; break;
    default: break;
    }
    if (block_bytes) *block_bytes = b;
    return n;
}

extern "C" uint64_t xj_row_bytes(uint32_t type, int64_t n) {
    int bb = 0, bn = xj_type_block(type, &bb);
    return bn ? (uint64_t)(n / bn) * (uint64_t)bb : 0;
}

extern "C" const char *xj_type_name(uint32_t type) {
    switch (type) {
    case XJ_F32: return "F32"; case XJ_F16: return "F16"; case XJ_BF16: return "BF16";
    case XJ_Q4_0: return "Q4_0"; case XJ_Q4_1: return "Q4_1"; case XJ_Q5_0: return "Q5_0";
    case XJ_Q5_1: return "Q5_1"; case XJ_Q8_0: return "Q8_0"; case XJ_Q2_K: return "Q2_K";
    case XJ_Q3_K: return "Q3_K"; case XJ_Q4_K: return "Q4_K"; case XJ_Q5_K: return "Q5_K";
    case XJ_Q6_K: return "Q6_K";
    default: return "?";
    }
}

static xj_gguf_file *gguf_parse(const uint8_t *buf, uint64_t len, char *err, size_t errlen) {
    Reader r{buf, buf + len};
    uint32_t magic, version;
    uint64_t n_tensors, n_kv;
    if (!r.u32(&magic) || !r.u32(&version)) { snprintf(err, errlen, "GGUF header truncated"); return nullptr; }
    if (magic != 0x46554747u) { snprintf(err, errlen, "not a GGUF file"); return nullptr; }
    if (version < 2 || version > 3) { snprintf(err, errlen, "GGUF version %u not supported", version); return nullptr; }
    if (!r.u64(&n_tensors) || !r.u64(&n_kv)) { snprintf(err, errlen, "GGUF header truncated"); return nullptr; }
    if (n_kv > (1u << 20) || n_tensors > (1u << 20)) { snprintf(err, errlen, "GGUF header counts out of range"); return nullptr; }
    auto *f = new xj_gguf_file();
    f->kv.resize(n_kv);
    for (uint64_t i = 0; i < n_kv; i++) {
        KV &e = f->kv[i];
        if (!r.str(&e.key) || !r.u32(&e.type)) { snprintf(err, errlen, "GGUF header truncated"); delete f; return nullptr; }
        e.val = r.p;
        if (!skip(r, e.type, &e)) { snprintf(err, errlen, "GGUF value of type %u unreadable", e.type); delete f; return nullptr; }
        if (e.type == GT_U32 && e.key == "general.alignment") memcpy(&f->alignment, e.val, 4);
    }
    if (f->alignment == 0 || (f->alignment & (f->alignment - 1))) {
        snprintf(err, errlen, "bad alignment %u", f->alignment); delete f; return nullptr;
    }
    f->tensors.resize(n_tensors);
    for (uint64_t i = 0; i < n_tensors; i++) {
        TInfo &t = f->tensors[i];
        if (!r.str(&t.name) || !r.u32(&t.n_dims)) { snprintf(err, errlen, "GGUF header truncated"); delete f; return nullptr; }
        if (t.n_dims > 4) { snprintf(err, errlen, "tensor with %u dims", t.n_dims); delete f; return nullptr; }
        for (uint32_t k = 0; k < t.n_dims; k++) {
            uint64_t d;
            if (!r.u64(&d)) { snprintf(err, errlen, "GGUF header truncated"); delete f; return nullptr; }
            t.ne[k] = (int64_t)d;
        }
        if (!r.u32(&t.type) || !r.u64(&t.offset)) { snprintf(err, errlen, "GGUF header truncated"); delete f; return nullptr; }
        int bb = 0, bn = xj_type_block(t.type, &bb);
        if (!bn) { t.nbytes = 0; continue; }
        if (t.ne[0] % bn) { snprintf(err, errlen, "tensor %s row length %lld not a multiple of the block", t.name.c_str(), (long long)t.ne[0]); delete f; return nullptr; }
        t.nbytes = xj_row_bytes(t.type, t.ne[0]) * (uint64_t)(t.ne[1] * t.ne[2] * t.ne[3]);
    }
    uint64_t hdr = (uint64_t)(r.p - buf);
    f->data_off = (hdr + f->alignment - 1) / f->alignment * f->alignment;
    return f;
}

static xj_gguf_file *gguf_open(const char *path, char *err, size_t errlen) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) { snprintf(err, errlen, "cannot open %s", path); return nullptr; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 16) { close(fd); snprintf(err, errlen, "file too small"); return nullptr; }
    void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_SHARED, fd, 0);
    if (m == MAP_FAILED) { close(fd); snprintf(err, errlen, "mmap failed"); return nullptr; }
    xj_gguf_file *f = gguf_parse((const uint8_t *)m, (uint64_t)st.st_size, err, errlen);
    if (!f) { munmap(m, (size_t)st.st_size); close(fd); return nullptr; }
    f->fd = fd; f->map = (const uint8_t *)m; f->size = (uint64_t)st.st_size;
    f->map_off = 0; f->map_len = f->size;
    for (auto &t : f->tensors)
        if (f->data_off + t.offset + t.nbytes > f->size) {
            snprintf(err, errlen, "tensor %s runs past the end of the file", t.name.c_str());
            delete f;
            return nullptr;
        }
    return f;
}

// Reads only the header (pread into a buffer that doubles from 16 MiB until the
// parse succeeds); no tensor bytes are mapped and tensors may lie past the end of
// a partly downloaded file (gguf.c:216-243).
static xj_gguf_file *gguf_open_header(const char *path, char *err, size_t errlen) {
    int fd = open(path, O_RDONLY);
    if (fd < 0) { snprintf(err, errlen, "cannot open %s", path); return nullptr; }
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 16) { close(fd); snprintf(err, errlen, "file too small"); return nullptr; }
    const uint64_t size = (uint64_t)st.st_size;
    for (uint64_t want = 16u << 20;; want *= 2) {
        if (want > size) want = size;
        std::vector<uint8_t> buf(want);
        uint64_t got = 0;
        while (got < want) {
            ssize_t k = pread(fd, buf.data() + got, want - got, (off_t)got);
            if (k <= 0) break;
            got += (uint64_t)k;
        }
        xj_gguf_file *f = gguf_parse(buf.data(), got, err, errlen);
        if (f) {
            f->hdr = std::move(buf);   // the key/value pointers stay valid: the storage moves with it
            f->fd = fd; f->size = size;
            return f;
        }
        if (got < want || want >= size) { close(fd); return nullptr; }
    }
}

// Maps file bytes [lo, hi) once, from the page below lo (gguf.c:245-255).
static bool gguf_map_range(xj_gguf_file *f, uint64_t lo, uint64_t hi, char *err, size_t errlen) {
    if (f->map) { snprintf(err, errlen, "already mapped"); return false; }
    if (hi > f->size || lo >= hi) { snprintf(err, errlen, "mapping range runs past the end of the file (incomplete download?)"); return false; }
    const uint64_t page = (uint64_t)getpagesize(), start = lo / page * page;
    void *m = mmap(nullptr, (size_t)(hi - start), PROT_READ, MAP_SHARED, f->fd, (off_t)start);
    if (m == MAP_FAILED) { snprintf(err, errlen, "mapping %llu MB failed", (unsigned long long)((hi - start) >> 20)); return false; }
    f->map = (const uint8_t *)m; f->map_off = start; f->map_len = hi - start;
    return true;
}

// ------------------------------------------------------------------ model --

static bool get_w(const xj_gguf_file *g, const char *name, xj_w *w, bool required, char *err, size_t errlen) {
    memset(w, 0, sizeof(*w));
    const TInfo *t = g->find_tensor(name);
    if (!t) {
        if (required) snprintf(err, errlen, "model has no tensor %s", name);
        return !required;
    }
    const uint32_t ok[] = {XJ_F32, XJ_F16, XJ_BF16, XJ_Q8_0, XJ_Q4_K, XJ_Q5_K, XJ_Q6_K};
    bool supported = false;
    for (uint32_t o : ok) supported |= t->type == o;
    if (!supported || !xj_type_block(t->type, nullptr)) {
        snprintf(err, errlen, "tensor %s has unsupported type %s", name, xj_type_name(t->type));
        return false;
    }
    w->file_off = g->data_off + t->offset;
    w->data = g->ptr(w->file_off, t->nbytes);
    w->nbytes = t->nbytes;
    w->type = t->type;
    w->ne0 = t->ne[0];
    w->ne1 = t->ne[1] * t->ne[2] * t->ne[3];
    return true;
}

static bool need_u32(const xj_gguf_file *g, const char *key, int *out, char *err, size_t errlen) {
    uint32_t v;
    if (!g->get_u32(key, &v)) { snprintf(err, errlen, "model is missing %s", key); return false; }
    *out = (int)v;
    return true;
}

static uint64_t fnv(uint64_t h, const void *p, size_t n) {
    const uint8_t *b = (const uint8_t *)p;
    for (size_t i = 0; i < n; i++) { h ^= b[i]; h *= 1099511628211ull; }
    return h;
}

static void find_special(const xj_gguf_file *g, xj_hparams *hp) {
    hp->eos = hp->eot = UINT32_MAX;
    uint32_t eos;
    if (g->get_u32("tokenizer.ggml.eos_token_id", &eos)) hp->eos = eos;
    const KV *kv = g->find_kv("tokenizer.ggml.tokens");
    if (!kv || kv->type != GT_ARR || kv->arr_type != GT_STR) return;
    const uint8_t *p = kv->val + 12;
    for (uint64_t i = 0; i < kv->arr_n; i++) {
        uint64_t n; memcpy(&n, p, 8);
        const char *s = (const char *)p + 8;
        if (n == 10 && memcmp(s, "<|im_end|>", 10) == 0) hp->eot = (uint32_t)i;
        if (n == 13 && memcmp(s, "<|endoftext|>", 13) == 0 && hp->eos == UINT32_MAX) hp->eos = (uint32_t)i;
        p += 8 + n;
    }
    hp->n_vocab = (int)kv->arr_n;
}

static bool load_layer(const xj_gguf_file *g, const xj_hparams *hp, int i, xj_layer *L, char *err, size_t errlen) {
    char name[96];
    auto W = [&](xj_w *field, const char *suffix, bool req) {
        snprintf(name, sizeof name, "blk.%d.%s", i, suffix);
        return get_w(g, name, field, req, err, errlen);
    };
    if (!W(&L->attn_norm, "attn_norm.weight", true) || !W(&L->post_norm, "post_attention_norm.weight", true) ||
        !W(&L->ffn_gate, "ffn_gate.weight", true) || !W(&L->ffn_up, "ffn_up.weight", true) ||
        !W(&L->ffn_down, "ffn_down.weight", true))
        return false;
    if (L->recurrent) {
        if (!W(&L->ssm_qkv, "attn_qkv.weight", true) || !W(&L->ssm_gate, "attn_gate.weight", true) ||
            !W(&L->ssm_conv1d, "ssm_conv1d.weight", true) || !W(&L->ssm_dt, "ssm_dt.bias", true) ||
            !W(&L->ssm_a, "ssm_a", true) || !W(&L->ssm_beta, "ssm_beta.weight", true) ||
            !W(&L->ssm_alpha, "ssm_alpha.weight", true) || !W(&L->ssm_norm, "ssm_norm.weight", true) ||
            !W(&L->ssm_out, "ssm_out.weight", true))
            return false;
        if (L->ssm_qkv.ne1 != hp->conv_dim || L->ssm_conv1d.type != XJ_F32 || L->ssm_conv1d.ne0 != hp->conv_k) {
            snprintf(err, errlen, "layer %d: linear-attention tensor shapes are wrong", i); return false;
        }
        if (L->ssm_a.type != XJ_F32 || L->ssm_dt.type != XJ_F32 || L->ssm_norm.type != XJ_F32) {
            snprintf(err, errlen, "layer %d: ssm_a / ssm_dt / ssm_norm must be F32", i); return false;
        }
    } else {
        if (!W(&L->wqkv, "attn_qkv.weight", false)) return false;
        if (!L->wqkv.nbytes) {
            if (!W(&L->wq, "attn_q.weight", true) || !W(&L->wk, "attn_k.weight", true) || !W(&L->wv, "attn_v.weight", true))
                return false;
        }
        if (!W(&L->wo, "attn_output.weight", true) || !W(&L->q_norm, "attn_q_norm.weight", true) ||
            !W(&L->k_norm, "attn_k_norm.weight", true))
            return false;
    }
    if (L->attn_norm.type != XJ_F32 || L->post_norm.type != XJ_F32) {
        snprintf(err, errlen, "layer %d: norms must be F32", i); return false;
    }
    return true;
}

// The MTP layer: blk.{block_count-1} (a full-attention layer) into
// layers[n_layer], with its nextn.* projection and norms (xj_model.c:104-127).
static bool load_mtp(const xj_gguf_file *g, xj_model *m, int block_count, char *err, size_t errlen) {
    const int i = block_count - 1, il = m->hp.n_layer;
    if (il + 1 > XJ_MAX_LAYERS) { snprintf(err, errlen, "too many layers"); return false; }
    xj_layer *L = &m->layers[il];
    memset(L, 0, sizeof(*L));
    L->recurrent = false;
    if (!load_layer(g, &m->hp, i, L, err, errlen)) return false;
    char name[96];
    const struct { xj_w *w; const char *suffix; } t[] = {{&m->mtp_eh, "eh_proj.weight"}, {&m->mtp_enorm, "enorm.weight"},
                                                        {&m->mtp_hnorm, "hnorm.weight"},
                                                        {&m->mtp_head_norm, "shared_head_norm.weight"}};
    for (const auto &e : t) {
        snprintf(name, sizeof name, "blk.%d.nextn.%s", i, e.suffix);
        if (!get_w(g, name, e.w, true, err, errlen)) return false;
    }
    if (m->mtp_eh.ne0 != 2 * m->hp.n_embd || m->mtp_eh.ne1 != m->hp.n_embd) {
        snprintf(err, errlen, "MTP eh_proj shape is wrong"); return false;
    }
    if (m->mtp_enorm.type != XJ_F32 || m->mtp_hnorm.type != XJ_F32 || m->mtp_head_norm.type != XJ_F32) {
        snprintf(err, errlen, "MTP norms must be F32"); return false;
    }
    m->has_mtp = true;
    return true;
}

// The model table from a parsed file; tensors outside its mapping get data = NULL
// (xj_model_from_gguf, xj_model.c:129-202). Takes g; deletes it on failure.
static xj_model *model_from_gguf(xj_gguf_file *g, char *err, size_t errlen) {
    std::string arch;
    if (!g->get_str("general.architecture", &arch) || arch != "qwen35") {
        snprintf(err, errlen, "not a qwen35 model (general.architecture)");
        delete g;
        return nullptr;
    }
    auto *m = (xj_model *)calloc(1, sizeof(xj_model));
    m->gguf = g;
    xj_hparams *hp = &m->hp;
    int block_count = 0, nextn = 0, key_len = 0, val_len = 0;
    auto fail = [&]() -> xj_model * { delete g; free(m); return nullptr; };
    if (!need_u32(g, "qwen35.block_count", &block_count, err, errlen) ||
        !need_u32(g, "qwen35.embedding_length", &hp->n_embd, err, errlen) ||
        !need_u32(g, "qwen35.feed_forward_length", &hp->n_ff, err, errlen) ||
        !need_u32(g, "qwen35.attention.head_count", &hp->n_head, err, errlen) ||
        !need_u32(g, "qwen35.attention.head_count_kv", &hp->n_head_kv, err, errlen) ||
        !need_u32(g, "qwen35.attention.key_length", &key_len, err, errlen) ||
        !need_u32(g, "qwen35.attention.value_length", &val_len, err, errlen) ||
        !need_u32(g, "qwen35.rope.dimension_count", &hp->n_rot, err, errlen) ||
        !need_u32(g, "qwen35.ssm.conv_kernel", &hp->conv_k, err, errlen) ||
        !need_u32(g, "qwen35.ssm.inner_size", &hp->d_inner, err, errlen) ||
        !need_u32(g, "qwen35.ssm.state_size", &hp->s_k, err, errlen) ||
        !need_u32(g, "qwen35.ssm.group_count", &hp->h_k, err, errlen) ||
        !need_u32(g, "qwen35.ssm.time_step_rank", &hp->h_v, err, errlen))
        return fail();
    { uint32_t v; if (g->get_u32("qwen35.nextn_predict_layers", &v)) nextn = (int)v; }
    hp->n_layer = block_count - nextn;
    hp->full_attn_interval = 4;
    { uint32_t v; if (g->get_u32("qwen35.full_attention_interval", &v)) hp->full_attn_interval = (int)v; }
    hp->rope_base = 10000.0f;
    g->get_f32("qwen35.rope.freq_base", &hp->rope_base);
    hp->eps = 1e-6f;
    g->get_f32("qwen35.attention.layer_norm_rms_epsilon", &hp->eps);
    if (key_len != val_len) { snprintf(err, errlen, "key/value head dims differ (%d/%d)", key_len, val_len); return fail(); }
    hp->head_dim = key_len;
    if (hp->h_v <= 0 || hp->h_k <= 0) { snprintf(err, errlen, "bad ssm head counts"); return fail(); }
    hp->s_v = hp->d_inner / hp->h_v;
    if (hp->s_v != hp->s_k) { snprintf(err, errlen, "linear-attention key/value head dims differ"); return fail(); }
    if (hp->h_v % hp->h_k) { snprintf(err, errlen, "value heads not a multiple of key heads"); return fail(); }
    hp->key_dim = hp->s_k * hp->h_k;
    hp->conv_dim = 2 * hp->key_dim + hp->d_inner;
    if (hp->n_layer <= 0 || hp->n_layer > XJ_MAX_LAYERS) { snprintf(err, errlen, "bad layer count %d", hp->n_layer); return fail(); }
    if (hp->n_rot > hp->head_dim || hp->n_rot % 2) { snprintf(err, errlen, "bad rope dims %d", hp->n_rot); return fail(); }
    if (hp->full_attn_interval <= 0) { snprintf(err, errlen, "bad full_attention_interval"); return fail(); }
    find_special(g, hp);
    for (int i = 0; i < hp->n_layer; i++) {
        uint32_t r;
        if (g->get_arr_u32("qwen35.attention.recurrent_layers", i, &r)) m->layers[i].recurrent = r != 0;
        else m->layers[i].recurrent = (i + 1) % hp->full_attn_interval != 0;
    }
    if (!get_w(g, "token_embd.weight", &m->tok_embd, true, err, errlen) ||
        !get_w(g, "output_norm.weight", &m->output_norm, true, err, errlen) ||
        !get_w(g, "output.weight", &m->output, false, err, errlen))
        return fail();
    if (!m->output.nbytes) m->output = m->tok_embd;
    if (!hp->n_vocab) hp->n_vocab = (int)m->tok_embd.ne1;
    for (int i = 0; i < hp->n_layer; i++)
        if (!load_layer(g, hp, i, &m->layers[i], err, errlen)) return fail();
    if (nextn > 0 && !load_mtp(g, m, block_count, err, errlen)) return fail();

    uint64_t h = 1469598103934665603ull;
    h = fnv(h, hp, sizeof(*hp));
    for (auto &t : g->tensors) {
        h = fnv(h, t.name.data(), t.name.size());
        h = fnv(h, &t.type, sizeof t.type);
        h = fnv(h, t.ne, sizeof t.ne);
        h = fnv(h, &t.offset, sizeof t.offset);
    }
    m->fingerprint = h;
    return m;
}

extern "C" xj_model *xj_model_load(const char *path, char *err, size_t errlen) {
    xj_gguf_file *g = gguf_open(path, err, errlen);
    return g ? model_from_gguf(g, err, errlen) : nullptr;
}

// The xj_w fields of a layer, attn_norm to the end (the reference walks them the same way).
static int layer_ws(xj_layer *L, xj_w **ws) {
    *ws = &L->attn_norm;
    return (int)((sizeof(xj_layer) - offsetof(xj_layer, attn_norm)) / sizeof(xj_w));
}

static int add_range(const xj_w *w, uint64_t (*r)[2], int n, int max) {
    if (!w->nbytes || n >= max) return n;
    r[n][0] = w->file_off;
    r[n][1] = w->file_off + w->nbytes;
    return n + 1;
}

extern "C" int xj_model_ranges(const xj_model *m, int l0, int l1, bool include_embd, uint64_t (*r)[2], int max) {
    int n = 0;
    if (include_embd) {
        n = add_range(&m->tok_embd, r, n, max);
        n = add_range(&m->output_norm, r, n, max);
        if (m->output.file_off != m->tok_embd.file_off) n = add_range(&m->output, r, n, max);
    }
    for (int i = l0; i < l1; i++) {
        xj_w *ws;
        const int count = layer_ws(const_cast<xj_layer *>(&m->layers[i]), &ws);
        for (int k = 0; k < count; k++) n = add_range(&ws[k], r, n, max);
    }
    std::vector<std::pair<uint64_t, uint64_t>> v(n);
    for (int i = 0; i < n; i++) v[i] = {r[i][0], r[i][1]};
    std::stable_sort(v.begin(), v.end(), [](const auto &a, const auto &b) { return a.first < b.first; });
    for (int i = 0; i < n; i++) { r[i][0] = v[i].first; r[i][1] = v[i].second; }
    // ranges at most one page apart become one, so a stage maps one span per run of tensors
    int k = 0;
    for (int i = 0; i < n; i++) {
        if (k && r[i][0] <= r[k - 1][1] + 4096) { if (r[i][1] > r[k - 1][1]) r[k - 1][1] = r[i][1]; }
        else { r[k][0] = r[i][0]; r[k][1] = r[i][1]; k++; }
    }
    return k;
}

extern "C" uint64_t xj_model_layer_bytes(const xj_model *m, int l0, int l1) {
    uint64_t s = 0;
    for (int i = l0; i < l1; i++) {
        xj_w *ws;
        const int count = layer_ws(const_cast<xj_layer *>(&m->layers[i]), &ws);
        for (int k = 0; k < count; k++) s += ws[k].nbytes;
    }
    return s;
}

extern "C" xj_model *xj_model_load_layers(const char *path, int l0, int l1, bool with_io, char *err, size_t errlen) {
    xj_gguf_file *g = gguf_open_header(path, err, errlen);
    if (!g) return nullptr;
    xj_model *m = model_from_gguf(g, err, errlen);
    if (!m) return nullptr;
    if (l0 < 0 || l1 > m->hp.n_layer || l0 >= l1) {
        snprintf(err, errlen, "bad layer range [%d,%d)", l0, l1);
        xj_model_free(m);
        return nullptr;
    }
    uint64_t r[512][2];
    const int n = xj_model_ranges(m, l0, l1, with_io, r, 512);
    if (n <= 0 || !gguf_map_range(g, r[0][0], r[n - 1][1], err, errlen)) {
        if (n <= 0) snprintf(err, errlen, "these layers hold no weights");
        xj_model_free(m);
        return nullptr;
    }
    auto fix = [&](xj_w *w) { if (w->nbytes) w->data = g->ptr(w->file_off, w->nbytes); };
    fix(&m->tok_embd); fix(&m->output_norm); fix(&m->output);
    for (int i = 0; i < m->hp.n_layer; i++) {
        xj_w *ws;
        const int count = layer_ws(&m->layers[i], &ws);
        for (int k = 0; k < count; k++) fix(&ws[k]);
    }
    return m;
}

extern "C" void xj_model_free(xj_model *m) {
    if (!m) return;
    delete m->gguf;
    free(m);
}
