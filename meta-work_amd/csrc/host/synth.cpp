// Random-weight qwen35 models: generator, K-quant quantizers, GGUF v3 writer.
//
// The reference has no Q4_K/Q6_K quantizer (its only one is the Python Q8_0
// of src/xiaoju-pipe/tests/make_tiny_model.py:61-72), so the three quantizers
// here are written from the block formats that
// src/xiaoju-pipe/core/xj_quant.h:55-118 decodes:
//   Q8_0  34 B / 32: fp16 d | int8 q[32]                      y = d*q
//   Q4_K 144 B / 256: fp16 d | fp16 dmin | 12 B packed 6-bit (scale, min) x 8
//                     | 128 B nibbles                          y = d*sc*q - dmin*m
//   Q6_K 210 B / 256: ql[128] | qh[64] | int8 sc[16] | fp16 d  y = d*sc*(q-32)
// Their quality only matters as much as any quantizer's; every parity check
// compares decodes of the bytes they produce.
//
// The tensor set, names and F32-only tensors follow what the loader requires
// (src/xiaoju-pipe/core/xj_model.c:62-101) and the initialisation recipe of
// the reference's tiny-model generator (make_tiny_model.py:81-82, 97-99).
#include "xj_hip.h"

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

namespace {

// ---- fp16 (round to nearest even), same rule as xj_to_f16 (xj_quant.h:25-43)
uint16_t to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000;
    int32_t e = (int32_t)((x >> 23) & 0xff) - 127 + 15;
    uint32_t man = x & 0x7fffff;
    if (((x >> 23) & 0xff) == 0xff) return (uint16_t)(sign | 0x7c00 | (man ? 0x200 : 0));
    if (e >= 31) return (uint16_t)(sign | 0x7c00);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t h = man >> shift, rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fff;
    if (rem > 0x1000 || (rem == 0x1000 && (h & 1))) h++;
    return (uint16_t)h;
}

float from_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16, e = (h >> 10) & 0x1f, man = h & 0x3ff, bits;
    if (e == 0) {
        if (!man) bits = sign;
        else {
            e = 127 - 15 + 1;
            while (!(man & 0x400)) { man <<= 1; e--; }
            bits = sign | (e << 23) | ((man & 0x3ff) << 13);
        }
    } else if (e == 31) bits = sign | 0x7f800000u | (man << 13);
    else bits = sign | ((e + 127 - 15) << 23) | (man << 13);
    float f; memcpy(&f, &bits, 4); return f;
}

// ---- generator: splitmix64 -> uniform (0,1] doubles -> Box-Muller
struct Rng {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    double uniform() { return ((next() >> 11) + 1) * (1.0 / 9007199254740992.0); }  // (0, 1]
};

void fill_normal_row(float *out, int64_t n, uint64_t seed, float sd) {
    Rng r{seed};
    for (int64_t i = 0; i < n; i += 2) {
        double u1 = r.uniform(), u2 = r.uniform();
        double rad = std::sqrt(-2.0 * std::log(u1)), th = 6.283185307179586 * u2;
        out[i] = (float)(rad * std::cos(th) * sd);
        if (i + 1 < n) out[i + 1] = (float)(rad * std::sin(th) * sd);
    }
}

uint64_t row_seed(uint64_t tseed, int64_t row) {
    Rng r{tseed ^ ((uint64_t)(row + 1) * 0xD1B54A32D192ED03ull)};
    return r.next();
}

template <class F>
void parallel_rows(int64_t n, F f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 4;
    if (nt > 16) nt = 16;
    if (n < 64) nt = 1;
    std::vector<std::thread> th;
    for (unsigned t = 0; t < nt; t++)
        th.emplace_back([=]() { for (int64_t r = t; r < n; r += nt) f(r); });
    for (auto &x : th) x.join();
}

// ---- Q8_0
void quant_q8_0(const float *x, int64_t k, uint8_t *out) {
    for (int64_t b = 0; b < k / 32; b++, x += 32, out += 34) {
        float amax = 0;
        for (int i = 0; i < 32; i++) amax = std::fmax(amax, std::fabs(x[i]));
        float d = amax / 127.0f;
        uint16_t dh = to_f16(d);
        memcpy(out, &dh, 2);
        float df = from_f16(dh), id = df != 0 ? 1.0f / df : 0.0f;
        for (int i = 0; i < 32; i++) {
            float v = std::nearbyint(x[i] * id);
            v = std::fmin(127.0f, std::fmax(-127.0f, v));
            out[2 + i] = (uint8_t)(int8_t)v;
        }
    }
}

// least-squares fit of x ~= s*q - m over one sub-block for fixed q (m >= 0)
void fit_affine(const float *x, const int *q, int n, float *s, float *m) {
    double sq = 0, sqq = 0, sx = 0, sqx = 0;
    for (int i = 0; i < n; i++) { sq += q[i]; sqq += (double)q[i] * q[i]; sx += x[i]; sqx += (double)q[i] * x[i]; }
    double det = n * sqq - sq * sq;
    if (det <= 0) return;
    double a = (n * sqx - sq * sx) / det, b = (sqq * sx - sq * sqx) / det;  // x ~= a q + b
    if (a <= 0) return;
    if (b > 0) { b = 0; a = sqq > 0 ? sqx / sqq : a; }  // min must be >= 0
    *s = (float)a; *m = (float)-b;
}

// ---- Q4_K
void quant_q4_K(const float *x, int64_t k, uint8_t *out) {
    for (int64_t b = 0; b < k / 256; b++, x += 256, out += 144) {
        float sc[8], mn[8];
        int q[256];
        for (int j = 0; j < 8; j++) {
            const float *v = x + 32 * j;
            float lo = v[0], hi = v[0];
            for (int i = 1; i < 32; i++) { lo = std::fmin(lo, v[i]); hi = std::fmax(hi, v[i]); }
            if (lo > 0) lo = 0;
            float s = (hi - lo) / 15.0f, m = -lo;
            for (int it = 0; it < 2 && s > 0; it++) {
                for (int i = 0; i < 32; i++) {
                    int qi = (int)std::nearbyint((v[i] + m) / s);
                    q[32 * j + i] = qi < 0 ? 0 : qi > 15 ? 15 : qi;
                }
                fit_affine(v, q + 32 * j, 32, &s, &m);
            }
            sc[j] = s; mn[j] = m;
        }
        float smax = 0, mmax = 0;
        for (int j = 0; j < 8; j++) { smax = std::fmax(smax, sc[j]); mmax = std::fmax(mmax, mn[j]); }
        uint16_t dh = to_f16(smax / 63.0f), mh = to_f16(mmax / 63.0f);
        float d = from_f16(dh), dmin = from_f16(mh);
        uint8_t is[8], im[8];
        for (int j = 0; j < 8; j++) {
            int a = d > 0 ? (int)std::nearbyint(sc[j] / d) : 0, c = dmin > 0 ? (int)std::nearbyint(mn[j] / dmin) : 0;
            is[j] = (uint8_t)(a < 0 ? 0 : a > 63 ? 63 : a);
            im[j] = (uint8_t)(c < 0 ? 0 : c > 63 ? 63 : c);
        }
        memcpy(out, &dh, 2);
        memcpy(out + 2, &mh, 2);
        uint8_t *s12 = out + 4;
        for (int j = 0; j < 4; j++) {
            s12[j] = (uint8_t)((is[j] & 63) | ((is[j + 4] >> 4) << 6));
            s12[j + 4] = (uint8_t)((im[j] & 63) | ((im[j + 4] >> 4) << 6));
            s12[j + 8] = (uint8_t)((is[j + 4] & 0xF) | ((im[j + 4] & 0xF) << 4));
        }
        for (int j = 0; j < 8; j++) {
            float ds = d * is[j], dm = dmin * im[j];
            for (int i = 0; i < 32; i++) {
                int qi = ds > 0 ? (int)std::nearbyint((x[32 * j + i] + dm) / ds) : 0;
                q[32 * j + i] = qi < 0 ? 0 : qi > 15 ? 15 : qi;
            }
        }
        uint8_t *qs = out + 16;
        for (int p = 0; p < 4; p++)
            for (int l = 0; l < 32; l++)
                qs[32 * p + l] = (uint8_t)(q[64 * p + l] | (q[64 * p + 32 + l] << 4));
    }
}

// ---- Q6_K
void quant_q6_K(const float *x, int64_t k, uint8_t *out) {
    for (int64_t b = 0; b < k / 256; b++, x += 256, out += 210) {
        float sc[16];
        for (int i = 0; i < 16; i++) {
            const float *v = x + 16 * i;
            float big = 0;
            for (int l = 0; l < 16; l++) if (std::fabs(v[l]) > std::fabs(big)) big = v[l];
            sc[i] = big / -32.0f;  // the largest magnitude maps to -32
        }
        float amax = 0;
        for (int i = 0; i < 16; i++) amax = std::fmax(amax, std::fabs(sc[i]));
        uint16_t dh = to_f16(amax / 127.0f);
        float d = from_f16(dh);
        int8_t isc[16];
        int q[256];
        for (int i = 0; i < 16; i++) {
            int a = d > 0 ? (int)std::nearbyint(sc[i] / d) : 0;
            isc[i] = (int8_t)(a < -128 ? -128 : a > 127 ? 127 : a);
            float s = d * isc[i];
            for (int l = 0; l < 16; l++) {
                int qi = s != 0 ? (int)std::nearbyint(x[16 * i + l] / s) : 0;
                q[16 * i + l] = (qi < -32 ? -32 : qi > 31 ? 31 : qi) + 32;
            }
        }
        uint8_t *ql = out, *qh = out + 128;
        for (int h = 0; h < 2; h++)
            for (int l = 0; l < 32; l++) {
                int q1 = q[128 * h + l], q2 = q[128 * h + 32 + l], q3 = q[128 * h + 64 + l], q4 = q[128 * h + 96 + l];
                ql[64 * h + l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
                ql[64 * h + 32 + l] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
                qh[32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        memcpy(out + 192, isc, 16);
        memcpy(out + 208, &dh, 2);
    }
}

// ---- GGUF v3 writer
struct Writer {
    std::vector<uint8_t> hdr;
    void u32(uint32_t v) { const uint8_t *p = (const uint8_t *)&v; hdr.insert(hdr.end(), p, p + 4); }
    void u64(uint64_t v) { const uint8_t *p = (const uint8_t *)&v; hdr.insert(hdr.end(), p, p + 8); }
    void str(const std::string &s) { u64(s.size()); hdr.insert(hdr.end(), s.begin(), s.end()); }
    void kv_u32(const char *k, uint32_t v) { str(k); u32(4 /*U32*/); u32(v); }
    void kv_f32(const char *k, float v) { str(k); u32(6 /*F32*/); uint32_t b; memcpy(&b, &v, 4); u32(b); }
    void kv_str(const char *k, const char *v) { str(k); u32(8 /*STR*/); str(v); }
    void kv_strs(const char *k, const std::vector<std::string> &v) {
        str(k); u32(9 /*ARR*/); u32(8 /*STR*/); u64(v.size());
        for (const auto &e : v) str(e);
    }
};

struct TensorSpec {
    std::string name;
    int64_t ne0, ne1;      // ne1 == 0: 1-D tensor
    uint32_t type;
    int kind;              // 0 matrix N(0,w_std); 1 norm 1+0.1N; 2 ssm_a; 3 0.5 N
    uint64_t offset, nbytes;
};

}  // namespace

extern "C" void xjs_fill_normal(float *out, int64_t n, uint64_t seed, float sd) {
    // rows of 4096 values, each from its own stream, so large fills run in parallel
    const int64_t R = 4096, rows = (n + R - 1) / R;
    parallel_rows(rows, [&](int64_t r) {
        int64_t len = (r + 1) * R <= n ? R : n - r * R;
        fill_normal_row(out + r * R, len, row_seed(seed, r), sd);
    });
}

extern "C" uint64_t xjs_tensor_seed(uint64_t seed, const char *name) {
    uint64_t h = 1469598103934665603ull;
    for (const char *p = name; *p; p++) { h ^= (uint8_t)*p; h *= 1099511628211ull; }
    return seed ^ h;
}

extern "C" int xjs_quantize(uint32_t type, const float *x, int64_t n_rows, int64_t k, void *out,
                            char *err, size_t errlen) {
    int bb = 0, bn = xjh_type_block(type, &bb);
    if (!bn || k % bn) { snprintf(err, errlen, "cannot quantize %lld columns to %s", (long long)k, xjh_type_name(type)); return -1; }
    if (type != XJ_F32 && type != XJ_Q8_0 && type != XJ_Q4_K && type != XJ_Q6_K) {
        snprintf(err, errlen, "no quantizer for %s", xjh_type_name(type)); return -1;
    }
    const uint64_t rb = xjh_row_bytes(type, k);
    parallel_rows(n_rows, [&](int64_t r) {
        const float *src = x + r * k;
        uint8_t *dst = (uint8_t *)out + r * rb;
        switch (type) {
        case XJ_F32: memcpy(dst, src, k * 4); break;
        case XJ_Q8_0: quant_q8_0(src, k, dst); break;
        case XJ_Q4_K: quant_q4_K(src, k, dst); break;
        case XJ_Q6_K: quant_q6_K(src, k, dst); break;
        }
    });
    return 0;
}

extern "C" int64_t xjs_write_model(const char *path, const xjs_config *c, char *err, size_t errlen) {
    const int E = c->n_embd, FF = c->n_ff, V = c->n_vocab, H = c->n_head, HKV = c->n_head_kv, D = c->head_dim;
    const int SK = c->s_k, HK = c->h_k, HV = c->h_v, DI = HV * SK, CD = 2 * SK * HK + DI, KC = c->conv_k;
    if (c->full_attn_interval <= 0 || HV % HK || c->n_rot > D) { snprintf(err, errlen, "bad config"); return -1; }
    std::vector<TensorSpec> ts;
    auto mat = [&](std::string n, int64_t k, int64_t rows, uint32_t t) { ts.push_back({n, k, rows, t, 0, 0, 0}); };
    auto vec = [&](std::string n, int64_t len, int kind) { ts.push_back({n, len, 0, XJ_F32, kind, 0, 0}); };
    mat("token_embd.weight", E, V, c->type_embd);
    vec("output_norm.weight", E, 1);
    mat("output.weight", E, V, c->type_out);
    for (int i = 0; i < c->n_layer; i++) {
        std::string p = "blk." + std::to_string(i) + ".";
        vec(p + "attn_norm.weight", E, 1);
        vec(p + "post_attention_norm.weight", E, 1);
        mat(p + "ffn_gate.weight", E, FF, c->type_default);
        mat(p + "ffn_up.weight", E, FF, c->type_default);
        mat(p + "ffn_down.weight", FF, E, c->type_down);
        if ((i + 1) % c->full_attn_interval) {
            mat(p + "attn_qkv.weight", E, CD, c->type_default);
            mat(p + "attn_gate.weight", E, DI, c->type_default);
            ts.push_back({p + "ssm_conv1d.weight", KC, CD, XJ_F32, 3, 0, 0});
            vec(p + "ssm_dt.bias", HV, 3);
            vec(p + "ssm_a", HV, 2);
            mat(p + "ssm_beta.weight", E, HV, c->type_default);
            mat(p + "ssm_alpha.weight", E, HV, c->type_default);
            vec(p + "ssm_norm.weight", SK, 1);
            mat(p + "ssm_out.weight", DI, E, c->type_default);
        } else {
            mat(p + "attn_q.weight", E, 2 * H * D, c->type_default);
            mat(p + "attn_k.weight", E, HKV * D, c->type_default);
            mat(p + "attn_v.weight", E, HKV * D, c->type_v);
            mat(p + "attn_output.weight", H * D, E, c->type_default);
            vec(p + "attn_q_norm.weight", D, 1);
            vec(p + "attn_k_norm.weight", D, 1);
        }
    }
    if (c->nextn) {   // the MTP layer: blk.{n_layer}, a full-attention layer + nextn.*
        std::string p = "blk." + std::to_string(c->n_layer) + ".";
        vec(p + "attn_norm.weight", E, 1);
        vec(p + "post_attention_norm.weight", E, 1);
        mat(p + "ffn_gate.weight", E, FF, c->type_default);
        mat(p + "ffn_up.weight", E, FF, c->type_default);
        mat(p + "ffn_down.weight", FF, E, c->type_down);
        mat(p + "attn_q.weight", E, 2 * H * D, c->type_default);
        mat(p + "attn_k.weight", E, HKV * D, c->type_default);
        mat(p + "attn_v.weight", E, HKV * D, c->type_v);
        mat(p + "attn_output.weight", H * D, E, c->type_default);
        vec(p + "attn_q_norm.weight", D, 1);
        vec(p + "attn_k_norm.weight", D, 1);
        mat(p + "nextn.eh_proj.weight", 2 * E, E, c->type_default);
        vec(p + "nextn.enorm.weight", E, 1);
        vec(p + "nextn.hnorm.weight", E, 1);
        vec(p + "nextn.shared_head_norm.weight", E, 1);
    }
    const uint64_t ALIGN = 32;
    uint64_t off = 0;
    for (auto &t : ts) {
        int bn = xjh_type_block(t.type, nullptr);
        if (!bn || t.ne0 % bn) { snprintf(err, errlen, "tensor %s: %lld columns do not fit %s", t.name.c_str(), (long long)t.ne0, xjh_type_name(t.type)); return -1; }
        t.offset = off;
        t.nbytes = xjh_row_bytes(t.type, t.ne0) * (uint64_t)(t.ne1 ? t.ne1 : 1);
        off = (off + t.nbytes + ALIGN - 1) / ALIGN * ALIGN;
    }
    if (c->eos_id >= V || c->eot_id >= V) { snprintf(err, errlen, "end token id outside the vocabulary"); return -1; }
    Writer w;
    w.u32(0x46554747u); w.u32(3); w.u64(ts.size());
    w.u64(20 + (c->nextn ? 1 : 0) + (c->eos_id >= 0) + (c->eot_id >= 0));  // number of key/values below
    w.kv_str("general.architecture", "qwen35");
    w.kv_str("general.name", "synthetic-qwen35");
    w.kv_u32("general.alignment", (uint32_t)ALIGN);
    w.kv_u32("qwen35.block_count", c->n_layer + (c->nextn ? 1 : 0));
    if (c->nextn) w.kv_u32("qwen35.nextn_predict_layers", 1);
    w.kv_u32("qwen35.context_length", 262144);
    w.kv_u32("qwen35.embedding_length", E);
    w.kv_u32("qwen35.feed_forward_length", FF);
    w.kv_u32("qwen35.attention.head_count", H);
    w.kv_u32("qwen35.attention.head_count_kv", HKV);
    w.kv_u32("qwen35.attention.key_length", D);
    w.kv_u32("qwen35.attention.value_length", D);
    w.kv_u32("qwen35.rope.dimension_count", c->n_rot);
    w.kv_f32("qwen35.rope.freq_base", c->rope_base);
    w.kv_f32("qwen35.attention.layer_norm_rms_epsilon", c->eps);
    w.kv_u32("qwen35.ssm.conv_kernel", KC);
    w.kv_u32("qwen35.ssm.inner_size", DI);
    w.kv_u32("qwen35.ssm.state_size", SK);
    w.kv_u32("qwen35.ssm.group_count", HK);
    w.kv_u32("qwen35.ssm.time_step_rank", HV);
    w.kv_u32("qwen35.full_attention_interval", c->full_attn_interval);
    if (c->eos_id >= 0) w.kv_u32("tokenizer.ggml.eos_token_id", (uint32_t)c->eos_id);
    if (c->eot_id >= 0) {   // a vocabulary of placeholder pieces with <|im_end|> at eot_id
        std::vector<std::string> toks((size_t)V);
        for (int i = 0; i < V; i++) toks[i] = "<t" + std::to_string(i) + ">";
        toks[(size_t)c->eot_id] = "<|im_end|>";
        w.kv_strs("tokenizer.ggml.tokens", toks);
    }
    for (auto &t : ts) {
        w.str(t.name);
        w.u32(t.ne1 ? 2 : 1);
        w.u64((uint64_t)t.ne0);
        if (t.ne1) w.u64((uint64_t)t.ne1);
        w.u32(t.type);
        w.u64(t.offset);
    }
    while (w.hdr.size() % ALIGN) w.hdr.push_back(0);
    FILE *f = fopen(path, "wb");
    if (!f) { snprintf(err, errlen, "cannot write %s", path); return -1; }
    bool ok = fwrite(w.hdr.data(), 1, w.hdr.size(), f) == w.hdr.size();
    uint64_t pos = 0;
    std::vector<float> vals;
    std::vector<uint8_t> q;
    for (auto &t : ts) {
        if (!ok) break;
        while (pos < t.offset) { fputc(0, f); pos++; }
        const int64_t rows = t.ne1 ? t.ne1 : 1;
        vals.resize((size_t)rows * t.ne0);
        const uint64_t tseed = xjs_tensor_seed(c->seed, t.name.c_str());
        float sd = t.kind == 0 ? c->w_std : t.kind == 1 ? 0.1f : 0.5f;
        parallel_rows(rows, [&](int64_t r) { fill_normal_row(vals.data() + r * t.ne0, t.ne0, row_seed(tseed, r), sd); });
        if (t.kind == 1) for (auto &v : vals) v = 1.0f + v;
        if (t.kind == 2) for (auto &v : vals) v = -std::exp(v);
        q.resize(t.nbytes);
        if (xjs_quantize(t.type, vals.data(), rows, t.ne0, q.data(), err, errlen)) { fclose(f); return -1; }
        ok = fwrite(q.data(), 1, q.size(), f) == q.size();
        pos += q.size();
    }
    if (fclose(f) != 0) ok = false;
    if (!ok) { snprintf(err, errlen, "write to %s failed", path); return -1; }
    return (int64_t)(w.hdr.size() + pos);
}
