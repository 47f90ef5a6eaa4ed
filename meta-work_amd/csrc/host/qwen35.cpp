// The qwen35 model table (xj_model) from a GGUF file, driven by two schemas:
// the hyper-parameter keys and the per-layer tensor slots. What it must
// produce is fixed by the reference loader's observable output, which the
// reference's pipeline, its fingerprint check and its stages consume:
//   keys, defaults and derived sizes        src/xiaoju-pipe/core/xj_model.c:129-170
//   layer pattern (recurrent_layers array,  src/xiaoju-pipe/core/xj_model.c:173-178
//   else every interval-th layer is GQA)
//   tensor names per layer kind, F32-only   src/xiaoju-pipe/core/xj_model.c:62-101
//   tensors, accepted weight types           src/xiaoju-pipe/core/xj_model.c:9-28
//   tied head, vocabulary size, eos / eot    src/xiaoju-pipe/core/xj_model.c:44-60,180-183
//   fingerprint (FNV-1a over hparams and     src/xiaoju-pipe/core/xj_model.c:187-196
//   every tensor's name, type, ne, offset)
//   MTP layer = blk.{block_count-1} + nextn  src/xiaoju-pipe/core/xj_model.c:104-127
//   layer-range load, byte ranges (sorted,   src/xiaoju-pipe/core/xj_model.c:214-233,303-338
//   spans <= 4096 bytes apart merged)
//   MTP layer from a second file             src/xiaoju-pipe/core/xj_model.c:241-300
#include "gguf_file.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

namespace {

using xjg::Value;

// ------------------------------------------------------------ schemas --

// Integer keys under "qwen35." that must be present, and where they go.
struct Dims {
    int block_count, n_embd, n_ff, n_head, n_head_kv, key_len, val_len, n_rot, conv_k, d_inner, s_k, h_k, h_v;
};
struct RequiredKey { const char *key; int Dims::*dst; };
constexpr RequiredKey kRequired[] = {
    {"block_count", &Dims::block_count},           {"embedding_length", &Dims::n_embd},
    {"feed_forward_length", &Dims::n_ff},          {"attention.head_count", &Dims::n_head},
    {"attention.head_count_kv", &Dims::n_head_kv}, {"attention.key_length", &Dims::key_len},
    {"attention.value_length", &Dims::val_len},    {"rope.dimension_count", &Dims::n_rot},
    {"ssm.conv_kernel", &Dims::conv_k},            {"ssm.inner_size", &Dims::d_inner},
    {"ssm.state_size", &Dims::s_k},                {"ssm.group_count", &Dims::h_k},
    {"ssm.time_step_rank", &Dims::h_v},
};

// Which layers carry a tensor slot.
enum Kind : uint8_t { EVERY, DELTANET, GQA };
enum : uint8_t {
    REQUIRED = 1,   // absent -> the load fails
    FLOAT32 = 2,    // must be stored as F32 (read directly, never dequantized)
    UNFUSED = 4,    // required only when the layer has no fused attn_qkv
};
struct Slot { const char *suffix; xj_w xj_layer::*w; Kind kind; uint8_t flags; };
// Every xj_w of xj_layer, in declaration order (the layer walks below rely on
// this table covering the whole struct).
constexpr Slot kSlots[] = {
    {"attn_norm.weight", &xj_layer::attn_norm, EVERY, REQUIRED | FLOAT32},
    {"post_attention_norm.weight", &xj_layer::post_norm, EVERY, REQUIRED | FLOAT32},
    {"attn_qkv.weight", &xj_layer::wqkv, GQA, 0},
    {"attn_q.weight", &xj_layer::wq, GQA, UNFUSED},
    {"attn_k.weight", &xj_layer::wk, GQA, UNFUSED},
    {"attn_v.weight", &xj_layer::wv, GQA, UNFUSED},
    {"attn_output.weight", &xj_layer::wo, GQA, REQUIRED},
    {"attn_q_norm.weight", &xj_layer::q_norm, GQA, REQUIRED},
    {"attn_k_norm.weight", &xj_layer::k_norm, GQA, REQUIRED},
    {"attn_qkv.weight", &xj_layer::ssm_qkv, DELTANET, REQUIRED},
    {"attn_gate.weight", &xj_layer::ssm_gate, DELTANET, REQUIRED},
    {"ssm_conv1d.weight", &xj_layer::ssm_conv1d, DELTANET, REQUIRED | FLOAT32},
    {"ssm_dt.bias", &xj_layer::ssm_dt, DELTANET, REQUIRED | FLOAT32},
    {"ssm_a", &xj_layer::ssm_a, DELTANET, REQUIRED | FLOAT32},
    {"ssm_beta.weight", &xj_layer::ssm_beta, DELTANET, REQUIRED},
    {"ssm_alpha.weight", &xj_layer::ssm_alpha, DELTANET, REQUIRED},
    {"ssm_norm.weight", &xj_layer::ssm_norm, DELTANET, REQUIRED | FLOAT32},
    {"ssm_out.weight", &xj_layer::ssm_out, DELTANET, REQUIRED},
    {"ffn_gate.weight", &xj_layer::ffn_gate, EVERY, REQUIRED},
    {"ffn_up.weight", &xj_layer::ffn_up, EVERY, REQUIRED},
    {"ffn_down.weight", &xj_layer::ffn_down, EVERY, REQUIRED},
};
constexpr int kSlotCount = sizeof(kSlots) / sizeof(kSlots[0]);
static_assert(sizeof(xj_layer) - offsetof(xj_layer, attn_norm) == kSlotCount * sizeof(xj_w),
              "the slot table must list every weight of xj_layer");

// The MTP layer's extra tensors, under blk.{i}.nextn.
struct MtpSlot { const char *suffix; xj_w xj_model::*w; bool float32; };
constexpr MtpSlot kMtpSlots[] = {
    {"eh_proj.weight", &xj_model::mtp_eh, false},
    {"enorm.weight", &xj_model::mtp_enorm, true},
    {"hnorm.weight", &xj_model::mtp_hnorm, true},
    {"shared_head_norm.weight", &xj_model::mtp_head_norm, true},
};

// Weight types a stage can consume.
constexpr uint32_t kUsableTypes[] = {XJ_F32, XJ_F16, XJ_BF16, XJ_Q8_0, XJ_Q4_K, XJ_Q5_K, XJ_Q6_K};

bool usable(uint32_t t) {
    return std::find(std::begin(kUsableTypes), std::end(kUsableTypes), t) != std::end(kUsableTypes);
}

// ------------------------------------------------------------ binding --

// Builds one xj_model from a parsed file. The first failure leaves its
// message in err and makes ok() false; later steps then do nothing.
class Builder {
public:
    Builder(const xj_gguf_file *g, xj_model *m, char *err, size_t errlen) : g_(g), m_(m), err_(err), errlen_(errlen) {}
    bool ok() const { return ok_; }

    bool hparams(int *block_count, int *nextn);
    void layer_kinds();
    void io_tensors();
    void layer(int file_block, int slot_index, bool recurrent);
    void mtp(int block_count);
    void fingerprint();

private:
    template <class... A> void error(const char *fmt, A... a) {
        if (!ok_) return;
        if constexpr (sizeof...(A) == 0) snprintf(err_, errlen_, "%s", fmt);
        else snprintf(err_, errlen_, fmt, a...);
        ok_ = false;
    }
    const Value *key(const std::string &suffix) const { return g_->key(("qwen35." + suffix).c_str()); }
    // Fills w from the named tensor (w zeroed when absent); false when the tensor
    // is absent, or error() when it is present with a type no stage can use.
    bool bind(const std::string &name, xj_w *w, bool required);

    const xj_gguf_file *g_;
    xj_model *m_;
    char *err_;
    size_t errlen_;
    bool ok_ = true;
};

bool Builder::bind(const std::string &name, xj_w *w, bool required) {
    *w = xj_w{};
    const xjg::Tensor *t = g_->tensor(name);
    if (!t) {
        if (required) error("model has no tensor %s", name.c_str());
        return false;
    }
    if (!usable(t->type) || !xjh_type_block(t->type, nullptr)) {
        error("tensor %s has unsupported type %s", name.c_str(), xjh_type_name(t->type));
        return false;
    }
    w->file_off = g_->data_off + t->offset;
    w->nbytes = t->nbytes;
    w->data = g_->ptr(w->file_off, w->nbytes);
    w->type = t->type;
    w->ne0 = t->ne[0];
    w->ne1 = t->ne[1] * t->ne[2] * t->ne[3];
    return true;
}

bool Builder::hparams(int *block_count, int *nextn) {
    std::string_view arch;
    const Value *a = g_->key("general.architecture");
    if (!a || !a->as_string(&arch) || arch != "qwen35") {
        error("not a qwen35 model (general.architecture)");
        return false;
    }
    Dims d{};
    for (const RequiredKey &k : kRequired) {
        const Value *v = key(k.key);
        uint32_t u;
        if (!v || !v->as_uint(&u)) { error("model is missing qwen35.%s", k.key); return false; }
        d.*k.dst = (int)u;
    }
    auto opt_int = [&](const char *suffix, int dflt) {
        const Value *v = key(suffix);
        uint32_t u;
        return v && v->as_uint(&u) ? (int)u : dflt;
    };
    auto opt_float = [&](const char *suffix, float dflt) {
        const Value *v = key(suffix);
        float f;
        return v && v->as_float(&f) ? f : dflt;
    };
    xj_hparams &hp = m_->hp;
    *block_count = d.block_count;
    *nextn = opt_int("nextn_predict_layers", 0);
    hp.n_layer = d.block_count - *nextn;        // the MTP block is not a main layer
    hp.n_embd = d.n_embd;
    hp.n_ff = d.n_ff;
    hp.n_head = d.n_head;
    hp.n_head_kv = d.n_head_kv;
    hp.n_rot = d.n_rot;
    hp.conv_k = d.conv_k;
    hp.d_inner = d.d_inner;
    hp.s_k = d.s_k;
    hp.h_k = d.h_k;
    hp.h_v = d.h_v;
    hp.full_attn_interval = opt_int("full_attention_interval", 4);
    hp.rope_base = opt_float("rope.freq_base", 10000.0f);
    hp.eps = opt_float("attention.layer_norm_rms_epsilon", 1e-6f);
    hp.head_dim = d.key_len;
    if (d.key_len != d.val_len) { error("key/value head dims differ (%d/%d)", d.key_len, d.val_len); return false; }
    if (hp.h_v <= 0 || hp.h_k <= 0) { error("bad ssm head counts"); return false; }
    hp.s_v = hp.d_inner / hp.h_v;
    hp.key_dim = hp.s_k * hp.h_k;
    hp.conv_dim = 2 * hp.key_dim + hp.d_inner;
    const struct { bool bad; const char *what; } checks[] = {
        {hp.s_v != hp.s_k, "linear-attention key/value head dims differ"},
        {hp.h_v % hp.h_k != 0, "value heads not a multiple of key heads"},
        {hp.n_layer <= 0 || hp.n_layer > XJ_MAX_LAYERS, "bad layer count"},
        {hp.n_rot > hp.head_dim || hp.n_rot % 2 != 0, "bad rope dims"},
        {hp.full_attn_interval <= 0, "bad full_attention_interval"},
    };
    for (const auto &c : checks)
        if (c.bad) { error("%s (n_layer %d, n_rot %d)", c.what, hp.n_layer, hp.n_rot); return false; }

    // End tokens: the eos id key if present; otherwise the first "<|endoftext|>"
    // of the vocabulary; eot = the last "<|im_end|>". The vocabulary size is the
    // token list's length when there is one.
    hp.eos = hp.eot = UINT32_MAX;
    if (const Value *v = g_->key("tokenizer.ggml.eos_token_id")) {
        uint32_t u;
        if (v->as_uint(&u)) hp.eos = u;
    }
    if (const Value *toks = g_->key("tokenizer.ggml.tokens")) {
        uint32_t first_eos = UINT32_MAX, last_eot = UINT32_MAX;
        if (toks->each_string([&](uint64_t i, std::string_view s) {
                if (s == "<|im_end|>") last_eot = (uint32_t)i;
                if (s == "<|endoftext|>" && first_eos == UINT32_MAX) first_eos = (uint32_t)i;
            })) {
            hp.eot = last_eot;
            if (hp.eos == UINT32_MAX) hp.eos = first_eos;
            hp.n_vocab = (int)toks->count;
        }
    }
    return true;
}

void Builder::layer_kinds() {
    const xj_hparams &hp = m_->hp;
    const Value *pattern = key("attention.recurrent_layers");
    for (int i = 0; i < hp.n_layer; i++) {
        uint32_t r;
        m_->layers[i].recurrent = pattern && pattern->uint_at((uint64_t)i, &r) ? r != 0
                                                                              : (i + 1) % hp.full_attn_interval != 0;
    }
}

void Builder::io_tensors() {
    if (!ok_) return;
    bind("token_embd.weight", &m_->tok_embd, true);
    bind("output_norm.weight", &m_->output_norm, true);
    if (!bind("output.weight", &m_->output, false) && ok_) m_->output = m_->tok_embd;   // tied head
    if (!m_->hp.n_vocab) m_->hp.n_vocab = (int)m_->tok_embd.ne1;
}

void Builder::layer(int file_block, int slot_index, bool recurrent) {
    if (!ok_) return;
    xj_layer &L = m_->layers[slot_index];
    L = xj_layer{};
    L.recurrent = recurrent;
    const std::string prefix = "blk." + std::to_string(file_block) + ".";
    const Kind mine = recurrent ? DELTANET : GQA;
    bool fused = false;
    for (const Slot &s : kSlots) {
        if (s.kind != EVERY && s.kind != mine) continue;
        if ((s.flags & UNFUSED) && fused) continue;
        const bool present = bind(prefix + s.suffix, &(L.*s.w), (s.flags & (REQUIRED | UNFUSED)) != 0);
        if (!ok_) return;
        if (s.w == &xj_layer::wqkv) fused = present && L.wqkv.nbytes;
        if ((s.flags & FLOAT32) && present && (L.*s.w).type != XJ_F32) {
            error("layer %d: %s must be F32", file_block, s.suffix);
            return;
        }
    }
    if (recurrent && (L.ssm_qkv.ne1 != m_->hp.conv_dim || L.ssm_conv1d.ne0 != m_->hp.conv_k))
        error("layer %d: linear-attention tensor shapes are wrong", file_block);
}

// The MTP block (the file's last) goes to layers[n_layer] as a GQA layer,
// followed by its nextn tensors.
void Builder::mtp(int block_count) {
    if (!ok_) return;
    if (m_->hp.n_layer + 1 > XJ_MAX_LAYERS) { error("too many layers"); return; }
    const int file_block = block_count - 1;
    layer(file_block, m_->hp.n_layer, false);
    if (!ok_) return;
    const std::string prefix = "blk." + std::to_string(file_block) + ".nextn.";
    for (const MtpSlot &s : kMtpSlots) {
        bind(prefix + s.suffix, &(m_->*s.w), true);
        if (!ok_) return;
        if (s.float32 && (m_->*s.w).type != XJ_F32) { error("MTP %s must be F32", s.suffix); return; }
    }
    if (m_->mtp_eh.ne0 != 2 * (int64_t)m_->hp.n_embd || m_->mtp_eh.ne1 != m_->hp.n_embd) {
        error("MTP eh_proj shape is wrong");
        return;
    }
    m_->has_mtp = true;
}

// 64-bit FNV-1a, the fingerprint's hash.
struct Fnv1a {
    uint64_t h = 1469598103934665603ull;
    void add(const void *p, size_t n) {
        for (const uint8_t *b = (const uint8_t *)p, *e = b + n; b != e; ++b) h = (h ^ *b) * 1099511628211ull;
    }
};

void Builder::fingerprint() {
    if (!ok_) return;
    Fnv1a f;
    f.add(&m_->hp, sizeof m_->hp);
    for (const xjg::Tensor &t : g_->tensors) {
        f.add(t.name.c_str(), strlen(t.name.c_str()));
        f.add(&t.type, sizeof t.type);
        f.add(t.ne, sizeof t.ne);
        f.add(&t.offset, sizeof t.offset);
    }
    m_->fingerprint = f.h;
}

// The table of a parsed file; NULL (err set) when it is not a usable qwen35
// model. The model does not own g.
xj_model *build(const xj_gguf_file *g, char *err, size_t errlen) {
    auto *m = (xj_model *)calloc(1, sizeof(xj_model));
    Builder b(g, m, err, errlen);
    int block_count = 0, nextn = 0;
    if (b.hparams(&block_count, &nextn)) {
        b.layer_kinds();
        b.io_tensors();
        for (int i = 0; i < m->hp.n_layer; i++) b.layer(i, i, m->layers[i].recurrent);
        if (nextn > 0) b.mtp(block_count);
        b.fingerprint();
    }
    if (!b.ok()) { free(m); return nullptr; }
    return m;
}

// ------------------------------------------------------ layer walking --

template <class F> void each_weight(const xj_layer &L, F &&f) {
    for (const Slot &s : kSlots) f(L.*s.w);
}
template <class F> void each_weight(xj_layer &L, F &&f) {
    for (const Slot &s : kSlots) f(L.*s.w);
}

// Points every weight at its bytes in g's mapping (NULL outside it).
void remap(const xj_gguf_file *g, xj_w &w) {
    if (w.nbytes) w.data = g->ptr(w.file_off, w.nbytes);
}

// Sorted byte spans, merged where one starts at most `gap` bytes after the
// previous one ends.
std::vector<std::pair<uint64_t, uint64_t>> coalesce(std::vector<std::pair<uint64_t, uint64_t>> v, uint64_t gap) {
    std::sort(v.begin(), v.end(), [](const auto &a, const auto &b) { return a.first < b.first; });
    std::vector<std::pair<uint64_t, uint64_t>> out;
    for (const auto &s : v) {
        if (!out.empty() && s.first <= out.back().second + gap) out.back().second = std::max(out.back().second, s.second);
        else out.push_back(s);
    }
    return out;
}

// Byte span [lo, hi) covering the MTP layer and its nextn tensors.
bool mtp_span(const xj_model *m, uint64_t *lo, uint64_t *hi) {
    if (!m->has_mtp) return false;
    uint64_t a = UINT64_MAX, b = 0;
    auto take = [&](const xj_w &w) {
        if (!w.nbytes) return;
        a = std::min(a, w.file_off);
        b = std::max(b, w.file_off + w.nbytes);
    };
    each_weight(m->layers[m->hp.n_layer], take);
    for (const MtpSlot &s : kMtpSlots) take(m->*s.w);
    *lo = a; *hi = b;
    return b > a;
}

}  // namespace

// ------------------------------------------------------------ exports --

extern "C" xj_model *xjh_model_load(const char *path, char *err, size_t errlen) {
    xj_gguf_file *g = xjg::open_mapped(path, err, errlen);
    if (!g) return nullptr;
    xj_model *m = build(g, err, errlen);
    if (!m) { delete g; return nullptr; }
    m->gguf = g;
    return m;
}

extern "C" void xjh_model_free(xj_model *m) {
    if (!m) return;
    delete m->mtp_gguf;
    delete m->gguf;
    free(m);
}

extern "C" int xjh_model_ranges(const xj_model *m, int l0, int l1, bool include_embd, uint64_t (*ranges)[2], int max) {
    std::vector<std::pair<uint64_t, uint64_t>> spans;
    auto add = [&](const xj_w &w) {
        if (w.nbytes && (int)spans.size() < max) spans.emplace_back(w.file_off, w.file_off + w.nbytes);
    };
    if (include_embd) {
        add(m->tok_embd);
        add(m->output_norm);
        if (m->output.file_off != m->tok_embd.file_off) add(m->output);
    }
    for (int i = l0; i < l1; i++) each_weight(m->layers[i], add);
    const auto merged = coalesce(std::move(spans), 4096);
    for (size_t i = 0; i < merged.size(); i++) { ranges[i][0] = merged[i].first; ranges[i][1] = merged[i].second; }
    return (int)merged.size();
}

extern "C" uint64_t xjh_model_layer_bytes(const xj_model *m, int l0, int l1) {
    uint64_t total = 0;
    for (int i = l0; i < l1; i++) each_weight(m->layers[i], [&](const xj_w &w) { total += w.nbytes; });
    return total;
}

extern "C" xj_model *xjh_model_load_layers(const char *path, int l0, int l1, bool with_io, char *err, size_t errlen) {
    xj_gguf_file *g = xjg::open_header(path, err, errlen);
    if (!g) return nullptr;
    xj_model *m = build(g, err, errlen);
    if (!m) { delete g; return nullptr; }
    m->gguf = g;
    if (l0 < 0 || l1 > m->hp.n_layer || l0 >= l1) {
        snprintf(err, errlen, "bad layer range [%d,%d)", l0, l1);
        xjh_model_free(m);
        return nullptr;
    }
    static constexpr int kMaxSpans = 512;
    std::vector<uint64_t> r(2 * kMaxSpans);
    const int n = xjh_model_ranges(m, l0, l1, with_io, (uint64_t(*)[2])r.data(), kMaxSpans);
    if (n <= 0) {
        snprintf(err, errlen, "these layers hold no weights");
        xjh_model_free(m);
        return nullptr;
    }
    if (!xjg::map_range(g, r[0], r[2 * (n - 1) + 1], err, errlen)) { xjh_model_free(m); return nullptr; }
    remap(g, m->tok_embd);
    remap(g, m->output_norm);
    remap(g, m->output);
    for (int i = 0; i < m->hp.n_layer; i++) each_weight(m->layers[i], [&](xj_w &w) { remap(g, w); });
    return m;
}

extern "C" int xjh_model_mtp_range(const char *path, uint64_t *lo, uint64_t *hi, char *err, size_t errlen) {
    xj_gguf_file *g = xjg::open_header(path, err, errlen);
    if (!g) return -1;
    xj_model *t = build(g, err, errlen);
    int rc = -1;
    if (t) {
        if (mtp_span(t, lo, hi)) rc = 0;
        else snprintf(err, errlen, "the file has no MTP layer");
        free(t);
    }
    delete g;
    return rc;
}

extern "C" int xjh_model_attach_mtp(xj_model *m, const char *path, char *err, size_t errlen) {
    if (m->has_mtp) return 0;
    xj_gguf_file *g = xjg::open_header(path, err, errlen);
    if (!g) return -1;
    xj_model *t = build(g, err, errlen);
    if (!t) { delete g; return -1; }
    auto drop = [&](int rc) { free(t); delete g; return rc; };
    const xj_hparams &a = m->hp, &b = t->hp;
    const bool same = a.n_layer == b.n_layer && a.n_embd == b.n_embd && a.n_ff == b.n_ff && a.n_head == b.n_head &&
                      a.n_head_kv == b.n_head_kv && a.head_dim == b.head_dim && a.n_vocab == b.n_vocab;
    if (!same) { snprintf(err, errlen, "the MTP file is not of this model (shapes differ)"); return drop(-1); }
    uint64_t lo = 0, hi = 0;
    if (!mtp_span(t, &lo, &hi)) { snprintf(err, errlen, "the file has no MTP layer"); return drop(-1); }
    if (!xjg::map_range(g, lo, hi, err, errlen)) return drop(-1);
    xj_layer &L = m->layers[m->hp.n_layer];
    L = t->layers[t->hp.n_layer];
    each_weight(L, [&](xj_w &w) { remap(g, w); });
    for (const MtpSlot &s : kMtpSlots) {
        m->*s.w = t->*s.w;
        remap(g, m->*s.w);
    }
    free(t);
    m->mtp_gguf = g;
    m->has_mtp = true;
    return 0;
}
