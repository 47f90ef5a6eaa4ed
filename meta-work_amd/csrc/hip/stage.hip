// The HIP stage: drop-in replacement for the Metal stage of the xiaoju-pipe
// token loop, plus the device-resident chain and the speculative driver.
//
// Contract followed (behaviour, not code):
//   constructor      xj_metal_stage_new  src/xiaoju-pipe/metal/xj_metal.m:554-663
//   forward          metal_forward       xj_metal.m:422-475 (T and context checks,
//                    keep only for T > 1, ck_start/ck_T, n_past += T, keep cleared)
//   logits           metal_logits        xj_metal.m:477-497
//   rollback         metal_rollback      xj_metal.m:500-534 (recurrent stages restore
//                    checkpoint n_past-ck_start-1; attention-only stages truncate)
//   reset            metal_reset         xj_metal.m:536-541 (state zeroed, KV kept)
//   chain eval       eval_once, no-remote branch, src/xiaoju-pipe/core/xj_net.c:532-559
//   spec accept      xj_spec_next        src/xiaoju-pipe/core/xj_spec.c:179-207
//
// Per layer the stage issues five kernels (plus one for attention's KV store):
//   DeltaNet: GEMV[qkv(conv epilogue)|z|beta|alpha] -> delta -> GEMV ssm_out(+x)
//   GQA:      GEMV[q|k|v] -> kv store -> attention -> GEMV wo(+x)
//   both:     GEMV[gate|up] -> GEMV down(+x, SwiGLU prologue)
// The hidden state, KV cache, recurrent state and checkpoints live in HBM.
#include "common.h"
#include "dequant.h"
#include "kernels.h"
#include "xj_hip.h"

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

using namespace xjk;

namespace {

constexpr int kSnapSlots = 9;       // 0..7 for callers, kDecodeSlot for xjh_chain_decode
constexpr int kDecodeSlot = kSnapSlots - 1;

struct HLayer {
    bool rec = false;
    const float *attn_norm = nullptr, *post_norm = nullptr;
    DevW wq, wk, wv, wqkv, wo;
    const float *q_norm = nullptr, *k_norm = nullptr;
    DevW ssm_qkv, ssm_gate, ssm_beta, ssm_alpha, ssm_out;
    const float *conv_w = nullptr, *dt = nullptr, *A = nullptr, *ssm_norm = nullptr;
    DevW ffn_gate, ffn_up, ffn_down;
    uint16_t *kc = nullptr, *vc = nullptr;
    float *conv = nullptr, *ssm = nullptr;
    float *ck_conv = nullptr, *ck_ssm = nullptr;
    float *snap_conv[kSnapSlots] = {}, *snap_ssm[kSnapSlots] = {};
};

struct HStage {
    xj_stage s;                      // first member: the vtable the callers see
    hipStream_t st = nullptr;
    std::vector<void *> allocs;
    std::map<const void *, DevW> wcache;
    std::vector<HLayer> L;
    DevW output, tok_embd;
    const float *out_norm = nullptr;
    // MTP stage: [embedding | hidden] rows in mx, each half normalised into mh,
    // eh_proj back to n_embd (activations in xq_2e)
    DevW mtp_eh;
    const float *mtp_enorm = nullptr, *mtp_hnorm = nullptr;
    float *mx = nullptr, *mh = nullptr;
    uint8_t *xq_2e = nullptr;
    float *x = nullptr, *qkv = nullptr, *kb = nullptr, *vb = nullptr, *z = nullptr, *beta = nullptr,
          *alpha = nullptr, *o = nullptr, *g = nullptr, *u = nullptr, *qr = nullptr, *scores = nullptr,
          *logits = nullptr;
    unsigned long long *amax = nullptr;
    int head_nwg = 0, head_rows = 0;   // argmax partials per logits row, rows per partial
    int32_t *npast = nullptr;
    // prepared GEMV activations, max_batch tokens each: inputs of K = n_embd
    // (attention/DeltaNet in-projections, gate|up, head), d_inner (ssm_out),
    // n_head*head_dim (wo) and n_ff (down)
    uint8_t *xq_e = nullptr, *xq_di = nullptr, *xq_att = nullptr, *xq_ff = nullptr;
    // arrival counters of the producer tails (zero between launches)
    int32_t *cnt_grp = nullptr;
    // prefill on the matrix cores: per-token RMSNorm scales, the GEMM's K-split
    // partials and the chunked delta rule's work area
    float *tsc = nullptr, *gpart = nullptr, *dwork = nullptr;
    uint8_t *hq = nullptr;     // the GEMM's activations, max_batch tokens of the largest input
    int64_t gpart_floats = 0;
    int32_t *gcnt = nullptr;   // the GEMM's arrival counters (zero between launches)
    int32_t n_gcnt = 0;
    float2 *rope = nullptr;
    float *h_x = nullptr;            // pinned staging [max_batch][n_embd]
    int32_t *h_i = nullptr;          // pinned scalar
    int n_ck = 0;
    size_t conv_n = 0, ssm_n = 0;    // floats per layer
    size_t weight_bytes = 0;
    // a reset whose clearing failed: the recurrent state is not known to be
    // zero, so every forward and logits call reports this until a reset succeeds
    std::string reset_err;
};

std::string g_name, g_note;
thread_local char g_lasterr[512];

int env_int(const char *k, int def) {
    const char *v = getenv(k);
    return v ? atoi(v) : def;
}

HStage *H(xj_stage *s) { return reinterpret_cast<HStage *>(s); }

template <class T>
T *dalloc(HStage *S, size_t n, char *err, size_t errlen) {
    void *p = nullptr;
    if (n == 0) n = 1;
    if (hipMalloc(&p, n * sizeof(T)) != hipSuccess) {
        snprintf(err, errlen, "HBM allocation of %zu bytes failed", n * sizeof(T));
        return nullptr;
    }
    S->allocs.push_back(p);
    return (T *)p;
}

bool gemv_type_ok(uint32_t t) {
    return t == XJ_F32 || t == XJ_F16 || t == XJ_BF16 || t == XJ_Q4_K || t == XJ_Q5_K || t == XJ_Q6_K || t == XJ_Q8_0;
}

bool upload(HStage *S, const xj_w &w, DevW *out, char *err, size_t errlen) {
    *out = DevW();
    if (!w.nbytes) return true;
    // a layer-range load leaves tensors outside its mapping with data == NULL
    if (!w.data) { snprintf(err, errlen, "tensor not mapped (%lld x %lld)", (long long)w.ne1, (long long)w.ne0); return false; }
    auto it = S->wcache.find(w.data);
    if (it != S->wcache.end()) { *out = it->second; return true; }
    if (!gemv_type_ok(w.type)) {
        snprintf(err, errlen, "tensor type %s is not supported by the HIP backend", xjh_type_name(w.type));
        return false;
    }
    uint8_t *p = dalloc<uint8_t>(S, w.nbytes + kWeightPad, err, errlen);
    if (!p || upload_repack(w.type, w.data, w.ne1, w.ne0, p, S->st, err, errlen)) return false;
    out->p = p; out->type = w.type; out->n_rows = w.ne1; out->k = w.ne0; out->bytes = w.nbytes;
    S->wcache[w.data] = *out;
    S->weight_bytes += w.nbytes;
    return true;
}

bool upload_f32(HStage *S, const xj_w &w, const float **out, char *err, size_t errlen) {
    *out = nullptr;
    if (!w.nbytes) return true;
    if (w.type != XJ_F32) { snprintf(err, errlen, "norm/conv tensors must be F32"); return false; }
    DevW d;
    if (!upload(S, w, &d, err, errlen)) return false;
    *out = (const float *)d.p;
    return true;
}

// ------------------------------------------------------------- GEMV helper --

// Algorithmic HBM bytes of one GEMV launch over T tokens: every weight byte,
// the activations read (x, and x2 for SwiGLU / gated RMSNorm), the outputs
// written, and the outputs read back for a residual add.
double gemv_algo_bytes(const GArgs &a, int T) {
    double b = (double)T * xq_off(a.K).v_off;
    for (int i = 0; i < a.nseg; i++) {
        const GSeg &s = a.seg[i];
        b += (double)s.n_rows * xjh_row_bytes(s.type, a.K) + (double)T * s.n_rows * 4 * (s.epi == EPI_ADD ? 2 : 1);
    }
    return b;
}

// Profiling mode: the GEMV launches of a decode step only (prep, attention
// and DeltaNet launches are left out), with every epilogue turned into a
// plain store into scratch so no model state changes; the GEMVs' own
// activation tails still run (into the xq buffers, which the next real step
// rewrites before reading).
struct Profile {
    float *sink = nullptr;
    double bytes = 0;
    int launches = 0;
};

// One fused GEMV: segments sharing the input, its prepared activations
// (built by a prep launch unless `prepared`, or, for an RMSNorm prologue over
// quantized rows, by the GEMV's own work-groups), an optional tail that leaves
// the next GEMV's activations behind, tiled over T. Token t of the tile that starts at
// t0 uses xq + (t0 + t) * stride, so every buffer holds max_batch tokens.
struct Gemv {
    GArgs a{};
    Profile *prof = nullptr;
    bool prepared = false;
    explicit Gemv(uint8_t *xq, Profile *p = nullptr) : prof(p) { a.xq = xq; }
    Gemv(uint8_t *xq, Profile *p, float *tsc_, float *part_, int64_t part_floats_, int32_t *cnt_, int32_t n_cnt_,
         uint8_t *hq_)
        : prof(p), tsc(tsc_), part(part_), part_floats(part_floats_), cnt(cnt_), n_cnt(n_cnt_), hq(hq_) {
        a.xq = xq;
    }
    Gemv &seg(const DevW &w, float *y, int ys, int epi) {
        GSeg &s = a.seg[a.nseg];
        s = GSeg{};
        s.w = w.p; s.type = w.type; s.n_rows = (int32_t)w.n_rows;
        s.nblk = xjd::dev_nblk(w.type, w.n_rows, w.k);
        s.y = y; s.ys = ys; s.epi = epi;
        a.K = (int32_t)w.k;
        a.nseg++;
        return *this;
    }
    Gemv &post(int mode, uint8_t *xq, int32_t *cnt) {
        a.post = PostPrep{mode, xq, cnt, nullptr};
        return *this;
    }
    // RMSNorm prologues run inside the GEMV's work-groups (F32 rows read a prep launch's xq)
    bool inwg() const {
        bool ok = a.pro == PRO_RMSU && !prepared && !((uintptr_t)a.x & 15) && !(a.xs & 3) && !((uintptr_t)a.pro_w & 15);
        for (int i = 0; i < a.nseg; i++)
            ok = ok && a.seg[i].type != XJ_F32 && a.seg[i].type != XJ_F16 && a.seg[i].type != XJ_BF16;
        return ok;
    }
    // One token of gate|up: POST_SWIGLU_H into h when the per-CU launch serves it.
    bool swiglu_h(float *h) {
        GArgs b = a;
        b.T = 1;
        b.post = PostPrep{POST_SWIGLU_H, nullptr, nullptr, h};
        if (inwg()) b.pro = PRO_RMSU_X;
        if (!gemv_swiglu_h_ok(b)) return false;
        a.post = b.post;
        return true;
    }
    // work-group ranges of the segments under the launch plan for (K, all rows)
    void place() {
        int64_t total = 0;
        for (int i = 0; i < a.nseg; i++) total += a.seg[i].n_rows;
        const int rows = gemv_plan(a.K, total).rows_per_group;
        for (int i = 0; i < a.nseg; i++) {
            a.seg[i].wg0 = i ? a.seg[i - 1].wg0 + a.seg[i - 1].nwg : 0;
            a.seg[i].nwg = (int32_t)((a.seg[i].n_rows + rows - 1) / rows);
        }
    }
    // Prefill buffers of the stage (set by the stage for its GEMVs; without
    // them every launch takes the GEMV form).
    float *tsc = nullptr, *part = nullptr;
    int64_t part_floats = 0;
    int32_t *cnt = nullptr;
    int32_t n_cnt = 0;
    // the GEMM's activations (hq records, xq.h): built by the prep launch; for
    // a prepared input, already built by the previous GEMM's SwiGLU prep
    // (hq_ready) or else from the prepared values
    uint8_t *hq = nullptr;
    bool hq_ready = false;
    bool hq_out = false;   // set by a GEMM run whose SwiGLU prep built the next input's hq
    // Chunks of at least kGemmMinT tokens take the matrix-core GEMM
    // (gemm.hip): the prep launch builds the T tokens' activations once, the
    // RMSNorm scale is applied per token after the dot products (as the GEMV
    // applies it), the conv + SiLU runs as its own launch and the SwiGLU tail
    // as the down projection's prep. Segments the GEMM does not take (float
    // rows) and every other case keep the GEMV.
    static constexpr int kGemmMinT = 16;
    bool gemm_ok(int T) const {
        static const bool on = env_int("XJ_PREFILL_GEMM", 1) != 0;
        if (!on || T < kGemmMinT || prof || !tsc || !part || !cnt || !a.xq || !hq) return false;
        if (a.pro != PRO_NONE && a.pro != PRO_RMSU && a.pro != PRO_SWIGLU && a.pro != PRO_GATED_RMS) return false;
        if (a.post.mode != POST_NONE && a.post.mode != POST_SWIGLU) return false;
        if (a.K % 256) return false;
        bool any = false;
        for (int i = 0; i < a.nseg; i++) any = any || a.seg[i].type == XJ_Q4_K || a.seg[i].type == XJ_Q6_K;
        return any;
    }
    int run_gemm(int T, hipStream_t st) {
        const int64_t xs = xq_off(a.K).stride, hs = hq_stride(a.K);
        if (!prepared) {   // the T tokens' activations, once (no digits when no segment takes the GEMV)
            GArgs b = a;
            b.T = T;
            b.hq = hq;
            b.hq_only = 1;
            for (int i = 0; i < a.nseg; i++)
                if (a.seg[i].type != XJ_Q4_K && a.seg[i].type != XJ_Q6_K) b.hq_only = 0;
            if (prep_launch(b, st)) return -1;
        } else if (!hq_ready && hq_from_v_launch(a.xq, a.K, T, hq, st)) {
            return -1;
        }
        const bool rms = a.pro == PRO_RMSU;
        if (rms && rms_scale_launch(a.xq, xs, a.K, T, a.eps, tsc, st)) return -1;
        const int mt = gemm_max_tokens(), tile = gemv_max_tile(a.K);
        // the Q4_K and Q6_K segments in one launch sharing the activations,
        // each type on its own share of the work-groups (an attention
        // layer's q|k and v: 20 us less per chunk than a launch of its own
        // for v); XJ_GEMM_MIXED=0: one launch per type
        static const bool mixed_on = env_int("XJ_GEMM_MIXED", 1) != 0;
        auto launch_tokens = [&](const GemmArgs &g) {
            for (int t0 = 0; t0 < T; t0 += mt) {
                GemmArgs b = g;
                b.T = T - t0 < mt ? T - t0 : mt;
                b.hq = hq + t0 * hs;
                for (int i = 0; i < b.nseg; i++) b.seg[i].y = g.seg[i].y + (int64_t)t0 * g.seg[i].ys;
                b.tsc = rms ? tsc + t0 : nullptr;
                if (gemm_launch(b, part_floats, n_cnt, st)) return -1;
            }
            return 0;
        };
        GemmArgs gk[2]{};
        for (int k = 0; k < 2; k++) {
            const uint32_t ty = k ? XJ_Q6_K : XJ_Q4_K;
            GemmArgs &g = gk[k];
            g.type = ty; g.K = a.K; g.hs = hs; g.part = part; g.cnt = cnt;
            for (int i = 0; i < a.nseg; i++) {
                const GSeg &s = a.seg[i];
                if (s.type == ty) g.seg[g.nseg++] = GemmSeg{s.w, s.n_rows, s.y, s.ys, s.epi == EPI_ADD};
            }
        }
        if (mixed_on && gk[0].nseg && gk[1].nseg) {
            GemmArgs g = gk[0];
            for (int i = 0; i < gk[1].nseg; i++) g.seg[g.nseg++] = gk[1].seg[i];
            g.n6 = gk[1].nseg;
            if (launch_tokens(g)) return -1;
        } else {
            for (int k = 0; k < 2; k++)
                if (gk[k].nseg && launch_tokens(gk[k])) return -1;
        }
        for (int i = 0; i < a.nseg; i++) {
            const GSeg &s = a.seg[i];
            if (s.type != XJ_Q4_K && s.type != XJ_Q6_K) {   // this segment alone on the GEMV, reading the prepared activations
                if (tile < 1) return -1;
                GArgs one = a;
                one.nseg = 1;
                one.seg[0] = s;
                one.seg[0].epi = s.epi == EPI_CONV ? EPI_STORE : s.epi;
                one.post = PostPrep{};
                one.inc_ptr = nullptr;
                one.pro = rms ? PRO_RMSU : PRO_NONE;
                one.seg[0].wg0 = 0;
                one.seg[0].nwg = (int32_t)((s.n_rows + gemv_plan(a.K, s.n_rows).rows_per_group - 1) /
                                           gemv_plan(a.K, s.n_rows).rows_per_group);
                for (int t0 = 0; t0 < T; t0 += tile) {
                    GArgs b = one;
                    b.T = T - t0 < tile ? T - t0 : tile;
                    b.xq = a.xq + t0 * xs;
                    b.x = nullptr; b.x2 = nullptr;
                    b.seg[0].y = s.y + (int64_t)t0 * s.ys;
                    if (gemv_launch(b, st)) return -1;
                }
            }
            // depthwise causal conv + SiLU over the T tokens, with its state and checkpoints
            if (s.epi == EPI_CONV &&
                conv_silu_launch(s.y, s.conv_state, s.conv_w, s.n_rows, s.conv_k, T, s.conv_ck, a.keep_n, st))
                return -1;
        }
        if (a.post.mode == POST_SWIGLU) {   // silu(gate) * up as the next GEMV's activations
            GArgs b{};
            b.x = a.seg[0].y; b.xs = a.seg[0].ys; b.x2 = a.seg[1].y; b.x2s = a.seg[1].ys;
            b.pro = PRO_SWIGLU; b.K = a.seg[0].n_rows; b.T = T; b.xq = a.post.xq;
            if (b.K % 256 == 0) b.hq = hq;   // the down projection's GEMM input as well
            if (prep_launch(b, st)) return -1;
            hq_out = b.hq != nullptr;
        }
        if (a.inc_ptr && inc_launch(a.inc_ptr, a.inc_by, st)) return -1;
        return 0;
    }
    // Run over T tokens in tiles that fit LDS; row results do not depend on the tiling.
    int run(int T, hipStream_t st) {
        if (gemm_ok(T)) return run_gemm(T, st);
        const int tile = gemv_max_tile(a.K);
        if (tile < 1 || !a.xq) return -1;
        place();
        if (prof) {
            prof->bytes += gemv_algo_bytes(a, T);
            prof->launches += (T + tile - 1) / tile;
            for (int i = 0; i < a.nseg; i++) {
                a.seg[i].epi = EPI_STORE;
                a.seg[i].y = prof->sink;
                a.seg[i].amax = nullptr;
            }
            a.inc_ptr = nullptr;
        }
        const bool in_wg = inwg();
        const int64_t xs_in = xq_off(a.K).stride;
        const int64_t xs_out = a.post.mode == POST_SWIGLU ? xq_off(a.seg[0].n_rows).stride : 0;
        if (a.post.mode == POST_SWIGLU_H && T != 1) return -1;
        for (int t0 = 0; t0 < T; t0 += tile) {
            GArgs b = a;
            b.T = T - t0 < tile ? T - t0 : tile;
            b.t0 = a.t0 + t0;
            b.x = a.x ? a.x + (int64_t)t0 * a.xs : nullptr;
            if (a.x2) b.x2 = a.x2 + (int64_t)t0 * a.x2s;
            b.xq = a.xq + t0 * xs_in;
            if (a.post.mode == POST_SWIGLU) b.post.xq = a.post.xq + t0 * xs_out;
            for (int i = 0; i < a.nseg; i++) {
                b.seg[i].y = a.seg[i].y + (int64_t)t0 * a.seg[i].ys;
                if (a.seg[i].amax) b.seg[i].amax = a.seg[i].amax + (int64_t)t0 * a.seg[i].nwg;
            }
            if (t0 + b.T < T) b.inc_ptr = nullptr;
            if (in_wg) {
                b.pro = PRO_RMSU_X;
            } else if (a.pro != PRO_X) {   // PRO_X: built from x inside the GEMV
                if (!prof && !prepared && prep_launch(b, st)) return -1;
                if (b.pro != PRO_RMSU && b.pro != PRO_HEADRMS) b.pro = PRO_NONE;   // the GEMV reads xq
            }
            if (gemv_launch(b, st)) return -1;
        }
        return 0;
    }
};

// --------------------------------------------------------------- layers --

// Layer il on T tokens of x. The GEMVs that read the residual stream build
// their RMSNorm activations inside their own work-groups; every other
// prologue is produced by the kernel before its GEMV: the down input by
// gate|up, the ssm_out input by the DeltaNet kernel, the wo input by attention.
int enqueue_layer(HStage *S, int il, float *x, int T, int keep_n, int32_t *inc, hipStream_t st, Profile *pf = nullptr) {
    const xj_hparams &hp = S->s.m->hp;
    HLayer &L = S->L[il - S->s.l0];
    const int E = hp.n_embd, FF = hp.n_ff;
    // every GEMV of the layer with the stage's prefill buffers
    auto gemv = [&](uint8_t *xq) { return Gemv(xq, pf, S->tsc, S->gpart, S->gpart_floats, S->gcnt, S->n_gcnt, S->hq); };
    auto rms_in = [&](Gemv &g, const float *w) {
        g.a.x = x; g.a.xs = E; g.a.pro = PRO_RMSU; g.a.pro_w = w; g.a.eps = hp.eps;
    };
    if (L.rec) {
        const int CD = hp.conv_dim, DI = hp.d_inner, Hv = hp.h_v;
        Gemv p = gemv(S->xq_e);
        rms_in(p, L.attn_norm);
        p.a.keep_n = keep_n;
        p.seg(L.ssm_qkv, S->qkv, CD, EPI_CONV).seg(L.ssm_gate, S->z, DI, EPI_STORE)
         .seg(L.ssm_beta, S->beta, Hv, EPI_STORE).seg(L.ssm_alpha, S->alpha, Hv, EPI_STORE);
        GSeg &cs = p.a.seg[0];
        cs.conv_state = L.conv; cs.conv_w = L.conv_w; cs.conv_ck = L.ck_conv; cs.conv_k = hp.conv_k;
        if (p.run(T, st)) return -1;
        // a prefill chunk without checkpoints: the chunked rule on the matrix
        // cores (delta_chunk.hip) over inputs prepared from the projections,
        // then the gated RMSNorm (xj_cpu.c:215-217) as ssm_out's prep launch
        static const bool chunked_on = env_int("XJ_PREFILL_CHUNKED", 1) != 0;
        const int Sd = hp.s_k;
        if (chunked_on && !pf && keep_n == 0 && T >= Gemv::kGemmMinT && S->dwork && (Sd == 64 || Sd == 128) &&
            hp.s_v == Sd && T <= S->s.max_batch) {
            DeltaPrepArgs dp{};
            dp.qkv = S->qkv; dp.qkv_s = CD; dp.k_off = hp.key_dim; dp.v_off = 2 * hp.key_dim;
            dp.beta = S->beta; dp.beta_s = Hv; dp.alpha = S->alpha; dp.alpha_s = Hv; dp.dt = L.dt; dp.A = L.A;
            // kb / vb / u / g are free until the FFN: q, k, v [T][Hv][S], decay and beta [T][Hv]
            dp.q = S->kb; dp.k = S->vb; dp.v = S->u; dp.decay = S->g; dp.bt = S->g + (size_t)T * Hv;
            dp.T = T; dp.Hk = hp.h_k; dp.Hv = Hv; dp.S = Sd; dp.eps = hp.eps;
            if (delta_prefill_prep_launch(dp, st) ||
                delta_chunked_launch(Hv, Sd, T, 64, dp.q, dp.k, dp.v, dp.decay, dp.bt, 1.0f / sqrtf((float)Sd), L.ssm,
                                     S->o, S->dwork, st))
                return -1;
            Gemv q = gemv(S->xq_di);
            q.a.x = S->o; q.a.xs = DI; q.a.x2 = S->z; q.a.x2s = DI;
            q.a.pro = PRO_GATED_RMS; q.a.pro_w = L.ssm_norm; q.a.group = Sd; q.a.eps = hp.eps;
            q.seg(L.ssm_out, x, E, EPI_ADD);
            if (q.run(T, st)) return -1;
        } else {
        DeltaArgs d{};
        d.qkv = S->qkv; d.qkv_s = CD; d.k_off = hp.key_dim; d.v_off = 2 * hp.key_dim;
        d.beta = S->beta; d.beta_s = Hv; d.alpha = S->alpha; d.alpha_s = Hv; d.dt = L.dt; d.A = L.A;
        d.state = L.ssm; d.ck = L.ck_ssm; d.out = S->o; d.out_s = DI;
        d.T = T; d.Hk = hp.h_k; d.Hv = Hv; d.S = hp.s_k; d.keep_n = keep_n; d.eps = hp.eps;
        d.qscale = 1.0f / sqrtf((float)hp.s_k);
        d.xq = S->xq_di; d.z = S->z; d.z_s = DI; d.norm_w = L.ssm_norm;
        // one work-group per 32 value rows, the norm's per-head scale applied
        // by the ssm_out GEMV (its float rows read v, which must be final)
        const uint32_t ot = L.ssm_out.type;
        static const bool split_on = env_int("XJ_DELTA_SPLIT", 1) != 0;
        d.split = split_on && ot != XJ_F32 && ot != XJ_F16 && ot != XJ_BF16 && hp.s_k % 32 == 0;
        if (!pf && delta_launch(d, st)) return -1;
        Gemv q = gemv(S->xq_di);
        q.prepared = true;
        if (d.split) {
            q.a.pro = PRO_HEADRMS; q.a.group = hp.s_k; q.a.eps = hp.eps;
        }
        q.seg(L.ssm_out, x, E, EPI_ADD);
        if (q.run(T, st)) return -1;
        }
    } else {
        const int D = hp.head_dim, Hq = hp.n_head, Hkv = hp.n_head_kv, nq = 2 * Hq * D, nk = Hkv * D;
        Gemv p = gemv(S->xq_e);
        rms_in(p, L.attn_norm);
        AttnArgs at{};
        if (L.wqkv.p) {
            p.seg(L.wqkv, S->qkv, nq + 2 * nk, EPI_STORE);
            at.qg = S->qkv; at.qg_s = nq + 2 * nk;
            at.kn = S->qkv + nq; at.kn_s = nq + 2 * nk;
            at.vn = S->qkv + nq + nk; at.vn_s = nq + 2 * nk;
        } else {
            p.seg(L.wq, S->qkv, nq, EPI_STORE).seg(L.wk, S->kb, nk, EPI_STORE).seg(L.wv, S->vb, nk, EPI_STORE);
            at.qg = S->qkv; at.qg_s = nq; at.kn = S->kb; at.kn_s = nk; at.vn = S->vb; at.vn_s = nk;
        }
        if (p.run(T, st)) return -1;
        at.kc = L.kc; at.vc = L.vc; at.qnorm_w = L.q_norm; at.knorm_w = L.k_norm; at.rope = S->rope;
        at.npast = S->npast; at.qr = S->qr; at.scores = S->scores; at.out = S->o;
        at.T = T; at.H = Hq; at.Hkv = Hkv; at.D = D; at.n_rot = hp.n_rot; at.n_ctx = S->s.n_ctx;
        at.n_split = attn_splits(S->s.n_ctx);
        at.eps = hp.eps; at.scale = 1.0f / sqrtf((float)D);
        at.xq = S->xq_att;
        if (!pf && attn_launch(at, st)) return -1;
        Gemv q = gemv(S->xq_att);
        q.prepared = true;
        q.seg(L.wo, x, E, EPI_ADD);
        if (q.run(T, st)) return -1;
    }
    Gemv f = gemv(S->xq_e);
    rms_in(f, L.post_norm);
    f.seg(L.ffn_gate, S->g, FF, EPI_STORE).seg(L.ffn_up, S->u, FF, EPI_STORE);
    // one token: every work-group of gate|up leaves silu(gate) * up of its
    // rows in g, and down builds its activations from them (float rows of
    // down read a prepared xq instead)
    const uint32_t dt = L.ffn_down.type;
    const bool h = T == 1 && dt != XJ_F32 && dt != XJ_F16 && dt != XJ_BF16 && f.swiglu_h(S->g);
    if (!h) f.post(POST_SWIGLU, S->xq_ff, S->cnt_grp);
    if (f.run(T, st)) return -1;
    Gemv dn = gemv(S->xq_ff);
    if (h) {
        dn.a.x = S->g; dn.a.xs = FF; dn.a.pro = PRO_X;
    } else {
        dn.prepared = true;
        dn.hq_ready = f.hq_out;
    }
    dn.a.inc_ptr = inc; dn.a.inc_by = T;
    dn.seg(L.ffn_down, x, E, EPI_ADD);
    return dn.run(T, st);
}

// Layers [lo, hi) of the stage; inc: the stage's position counter advances
// by T after the last of them.
int enqueue_layer_range(HStage *S, int lo, int hi, float *x, int T, int keep_n, bool inc, hipStream_t st,
                        Profile *pf = nullptr) {
    for (int il = lo; il < hi; il++)
        if (enqueue_layer(S, il, x, T, keep_n, inc && il + 1 == hi ? S->npast : nullptr, st, pf)) return -1;
    return 0;
}
int enqueue_layers(HStage *S, float *x, int T, int keep_n, bool inc, hipStream_t st, Profile *pf = nullptr) {
    return enqueue_layer_range(S, S->s.l0, S->s.l1, x, T, keep_n, inc, st, pf);
}

// logits[t] = output . rmsnorm(x[t]) * output_norm; greedy partial keys into S->amax
int enqueue_head(HStage *S, const float *x, int T, float *logits, hipStream_t st, Profile *pf = nullptr) {
    const xj_hparams &hp = S->s.m->hp;
    Gemv h(S->xq_e, pf);
    h.a.x = x; h.a.xs = hp.n_embd; h.a.pro = PRO_RMSU; h.a.pro_w = S->out_norm; h.a.eps = hp.eps;
    h.seg(S->output, logits, (int)S->output.n_rows, EPI_STORE);
    h.a.seg[0].amax = S->amax;
    return h.run(T, st);
}

int sync_check(HStage *S, char *err, size_t errlen) {
    hipError_t e = hipStreamSynchronize(S->st);
    if (e == hipSuccess) e = hipGetLastError();
    if (e != hipSuccess) { snprintf(err, errlen, "GPU error: %s", hipGetErrorString(e)); return -1; }
    return 0;
}

int ensure_ck(HStage *S, int n, char *err, size_t errlen) {
    if (n <= S->n_ck) return 0;
    for (auto &L : S->L) {
        if (!L.rec) continue;
        if (L.ck_conv) { (void)hipFree(L.ck_conv); (void)hipFree(L.ck_ssm); }
        L.ck_conv = L.ck_ssm = nullptr;
        if (hipMalloc(&L.ck_conv, n * S->conv_n * 4) != hipSuccess || hipMalloc(&L.ck_ssm, n * S->ssm_n * 4) != hipSuccess) {
            S->n_ck = 0;
            snprintf(err, errlen, "out of HBM for speculative checkpoints");
            return -1;
        }
    }
    S->n_ck = n;
    return 0;
}

int set_npast(HStage *S, hipStream_t st) {
    *S->h_i = S->s.n_past;
    return hipMemcpyAsync(S->npast, S->h_i, 4, hipMemcpyHostToDevice, st) == hipSuccess ? 0 : -1;
}

// the sticky error of a failed reset, if any
int reset_check(HStage *S, char *err, size_t errlen) {
    if (S->reset_err.empty()) return 0;
    snprintf(err, errlen, "%s", S->reset_err.c_str());
    return -1;
}

// forward-call bookkeeping shared by the vtable and the chain (xj_metal.m:426-431)
int begin_forward(HStage *S, int T, int *keep_n, char *err, size_t errlen) {
    xj_stage *s = &S->s;
    if (reset_check(S, err, errlen)) { s->keep = 0; return -1; }
    if (T <= 0 || T > s->max_batch) { snprintf(err, errlen, "%d tokens exceed max_batch %d", T, s->max_batch); s->keep = 0; return -1; }
    if (s->n_past + T > s->n_ctx) { snprintf(err, errlen, "context full (%d)", s->n_ctx); s->keep = 0; return -1; }
    if (s->keep && T > 1 && ensure_ck(S, T - 1, err, errlen)) { s->keep = 0; return -1; }
    if (T == 1) s->keep = 0;
    s->ck_start = s->n_past;
    s->ck_T = s->keep ? T : 0;
    *keep_n = s->keep ? T - 1 : 0;
    return 0;
}

// MTP stage (xj_cpu.c:253-261): x holds T rows of [embedding | hidden] (2 n_embd
// floats); each half is RMS-normalised with its own weights and eh_proj maps
// the pair back to n_embd, into S->x.
int enqueue_mtp_prologue(HStage *S, const float *x, int T) {
    const xj_hparams &hp = S->s.m->hp;
    const int E = hp.n_embd;
    memcpy(S->h_x, x, sizeof(float) * T * 2 * E);
    if (hipMemcpyAsync(S->mx, S->h_x, sizeof(float) * T * 2 * E, hipMemcpyHostToDevice, S->st) != hipSuccess ||
        norm_rows_launch(0, S->mx, 2 * E, S->mtp_enorm, E, T, hp.eps, S->mh, 2 * E, S->st) ||
        norm_rows_launch(0, S->mx + E, 2 * E, S->mtp_hnorm, E, T, hp.eps, S->mh + E, 2 * E, S->st))
        return -1;
    Gemv g(S->xq_2e);
    g.a.x = S->mh; g.a.xs = 2 * E; g.a.pro = PRO_NONE;
    g.seg(S->mtp_eh, S->x, E, EPI_STORE);
    return g.run(T, S->st);
}

int hip_forward(xj_stage *s, float *x, int T, char *err, size_t errlen) {
    HStage *S = H(s);
    const int E = s->m->hp.n_embd;
    int keep_n = 0;
    if (begin_forward(S, T, &keep_n, err, errlen)) return -1;
    if (s->mtp && enqueue_mtp_prologue(S, x, T)) {
        snprintf(err, errlen, "kernel launch failed");
        s->keep = 0;
        return -1;
    }
    if (!s->mtp) memcpy(S->h_x, x, sizeof(float) * T * E);
    if ((!s->mtp && hipMemcpyAsync(S->x, S->h_x, sizeof(float) * T * E, hipMemcpyHostToDevice, S->st) != hipSuccess) ||
        set_npast(S, S->st) || enqueue_layers(S, S->x, T, keep_n, false, S->st) ||
        hipMemcpyAsync(S->h_x, S->x, sizeof(float) * T * E, hipMemcpyDeviceToHost, S->st) != hipSuccess) {
        snprintf(err, errlen, "kernel launch failed");
        s->keep = 0;
        return -1;
    }
    if (sync_check(S, err, errlen)) { s->keep = 0; return -1; }
    memcpy(x, S->h_x, sizeof(float) * T * E);
    s->n_past += T;
    s->keep = 0;
    return 0;
}

int hip_logits(xj_stage *s, const float *x, int T, float *logits, char *err, size_t errlen) {
    HStage *S = H(s);
    const int E = s->m->hp.n_embd;
    if (!s->has_head) { snprintf(err, errlen, "this stage has no output head"); return -1; }
    if (T < 1 || T > s->max_batch) { snprintf(err, errlen, "head called with %d tokens", T); return -1; }
    if (reset_check(S, err, errlen)) return -1;
    memcpy(S->h_x, x, sizeof(float) * T * E);
    if (hipMemcpyAsync(S->x, S->h_x, sizeof(float) * T * E, hipMemcpyHostToDevice, S->st) != hipSuccess ||
        enqueue_head(S, S->x, T, S->logits, S->st)) {
        snprintf(err, errlen, "kernel launch failed");
        return -1;
    }
    if (sync_check(S, err, errlen)) return -1;
    const size_t V = (size_t)S->output.n_rows;
    if (hipMemcpy(logits, S->logits, sizeof(float) * V * T, hipMemcpyDeviceToHost) != hipSuccess) {
        snprintf(err, errlen, "logits copy failed");
        return -1;
    }
    return 0;
}

// The conv and recurrent states of every DeltaNet layer copied in one launch
// (per-layer copies cost a launch each): pick(L, conv_src, conv_dst,
// ssm_src, ssm_dst) names each layer's ends.
template <class F>
static int states_copy(HStage *S, hipStream_t st, F pick) {
    CopyList c{};
    for (auto &L : S->L) {
        if (!L.rec) continue;
        const float *cs = nullptr, *ss = nullptr;
        float *cd = nullptr, *sd = nullptr;
        pick(L, cs, cd, ss, sd);
        if (c.cnt + 2 > kCopyMax) {
            if (copy_list_launch(c, st)) return -1;
            c.cnt = 0;
        }
        c.src[c.cnt] = cs; c.dst[c.cnt] = cd; c.n[c.cnt++] = (int64_t)S->conv_n;
        c.src[c.cnt] = ss; c.dst[c.cnt] = sd; c.n[c.cnt++] = (int64_t)S->ssm_n;
    }
    return copy_list_launch(c, st);
}

int hip_rollback(xj_stage *s, int n_past, char *err, size_t errlen) {
    HStage *S = H(s);
    if (n_past == s->n_past) { s->ck_T = 0; return 0; }
    bool rec = false;
    for (auto &L : S->L) rec |= L.rec;
    if (!rec) {
        if (n_past < 0 || n_past > s->n_past) { snprintf(err, errlen, "cannot roll back to %d", n_past); return -1; }
        s->n_past = n_past;
        return 0;
    }
    const int j = n_past - s->ck_start - 1;
    if (!s->ck_T || s->n_past != s->ck_start + s->ck_T || j < 0 || j >= s->ck_T - 1) {
        snprintf(err, errlen, "cannot roll back to %d (checkpoints %d+%d, now %d)", n_past, s->ck_start, s->ck_T, s->n_past);
        return -1;
    }
    if (states_copy(S, S->st, [&](HLayer &L, const float *&cs, float *&cd, const float *&ss, float *&sd) {
            cs = L.ck_conv + j * S->conv_n; cd = L.conv;
            ss = L.ck_ssm + j * S->ssm_n; sd = L.ssm;
        })) {
        snprintf(err, errlen, "checkpoint copy failed");
        return -1;
    }
    if (sync_check(S, err, errlen)) return -1;
    s->n_past = n_past;
    s->ck_T = 0;
    return 0;
}

// The vtable's reset returns nothing (xj_stage.h): a failure to clear the
// state is kept and reported by every later forward / logits call until a
// reset succeeds.
void hip_reset(xj_stage *s) {
    HStage *S = H(s);
    hipError_t e = hipSuccess;
    for (auto &L : S->L) {
        if (!L.rec) continue;
        if (e == hipSuccess) e = hipMemsetAsync(L.conv, 0, S->conv_n * 4, S->st);
        if (e == hipSuccess) e = hipMemsetAsync(L.ssm, 0, S->ssm_n * 4, S->st);
    }
    const hipError_t e2 = hipStreamSynchronize(S->st);
    if (e == hipSuccess) e = e2;
    if (e == hipSuccess) e = hipGetLastError();
    if (e != hipSuccess) S->reset_err = std::string("stage reset failed, recurrent state not cleared: ") + hipGetErrorString(e);
    else S->reset_err.clear();
    s->n_past = 0;
}

static size_t scratch_floats(const xj_hparams &hp) {
    size_t n = (size_t)hp.n_ff;
    const size_t qkv = 2 * (size_t)hp.n_head * hp.head_dim + 2 * (size_t)hp.n_head_kv * hp.head_dim;
    if (qkv > n) n = qkv;
    if ((size_t)hp.conv_dim > n) n = hp.conv_dim;
    if ((size_t)hp.n_embd * 2 > n) n = 2 * (size_t)hp.n_embd;
    return n;
}

// The scratch of a stage's forward passes (max_batch tokens): hidden rows,
// projections, attention partials, prepared activations, the prefill
// GEMM's buffers and the chunked rule's work area, and its position counter.
static bool alloc_scratch(HStage *S, char *err, size_t errlen) {
    const xj_hparams &hp = S->s.m->hp;
    const size_t mb = S->s.max_batch, E = hp.n_embd;
    const int n_ctx = S->s.n_ctx;
    const size_t sf = scratch_floats(hp);
    S->x = dalloc<float>(S, mb * E, err, errlen);
    S->qkv = dalloc<float>(S, mb * sf, err, errlen);
    S->kb = dalloc<float>(S, mb * sf, err, errlen);
    S->vb = dalloc<float>(S, mb * sf, err, errlen);
    S->z = dalloc<float>(S, mb * sf, err, errlen);
    S->beta = dalloc<float>(S, mb * (hp.h_v + 1), err, errlen);
    S->alpha = dalloc<float>(S, mb * (hp.h_v + 1), err, errlen);
    S->o = dalloc<float>(S, mb * sf, err, errlen);
    S->g = dalloc<float>(S, mb * sf, err, errlen);
    S->u = dalloc<float>(S, mb * sf, err, errlen);
    S->qr = dalloc<float>(S, mb * hp.n_head * (size_t)hp.head_dim, err, errlen);
    S->scores = dalloc<float>(S, mb * hp.n_head * (size_t)attn_splits(n_ctx) * (hp.head_dim + 2), err, errlen);
    S->npast = dalloc<int32_t>(S, 1, err, errlen);
    // prefill on the matrix cores (chunks of at least 16 tokens)
    S->tsc = dalloc<float>(S, mb, err, errlen);
    // every GEMM launch covers at most 2 sf + 2 h_v rows (gate|up, the DeltaNet in-projection)
    const int64_t grows = 2 * (int64_t)sf + 2 * (int64_t)hp.h_v;
    S->gpart_floats = gemm_part_floats(grows, (int)(mb < gemm_max_tokens() ? mb : gemm_max_tokens()));
    S->gpart = dalloc<float>(S, (size_t)S->gpart_floats, err, errlen);
    S->n_gcnt = gemm_counters(grows);
    S->gcnt = dalloc<int32_t>(S, (size_t)S->n_gcnt, err, errlen);
    S->hq = dalloc<uint8_t>(S, mb * (size_t)hq_stride((int)sf), err, errlen);
    if (!S->tsc || !S->gpart || !S->gcnt || !S->hq) return false;
    XJ_CHECK(hipMemset(S->gcnt, 0, (size_t)S->n_gcnt * 4), err, errlen, false);
    {
        bool rec = false;
        for (int il = S->s.l0; il < S->s.l1 && il < hp.n_layer; il++) rec = rec || S->s.m->layers[il].recurrent;
        const size_t wb = rec ? delta_chunked_work_bytes(hp.h_v, hp.s_k, (int)mb, 64) : 0;
        if (wb) {
            S->dwork = (float *)dalloc<uint8_t>(S, wb, err, errlen);
            if (!S->dwork) return false;
        }
    }
    {
        auto xqb = [&](int K) { return K >= 32 ? mb * (size_t)xq_off(K).stride : 256; };
        S->xq_e = dalloc<uint8_t>(S, xqb(hp.n_embd), err, errlen);
        S->xq_di = dalloc<uint8_t>(S, xqb(hp.d_inner), err, errlen);
        S->xq_att = dalloc<uint8_t>(S, xqb(hp.n_head * hp.head_dim), err, errlen);
        S->xq_ff = dalloc<uint8_t>(S, xqb(hp.n_ff), err, errlen);
        const size_t nc = (size_t)(hp.n_ff / 32) + 1;
        int32_t *cnt = dalloc<int32_t>(S, nc, err, errlen);
        if (!S->xq_e || !S->xq_di || !S->xq_att || !S->xq_ff || !cnt) return false;
        XJ_CHECK(hipMemset(cnt, 0, nc * 4), err, errlen, false);
        S->cnt_grp = cnt;
    }
    if (!S->x || !S->qkv || !S->kb || !S->vb || !S->z || !S->beta || !S->alpha || !S->o || !S->g || !S->u ||
        !S->qr || !S->scores || !S->npast)
        return false;
    return true;
}

// A second set of scratch for a stage whose prompt chunks run as two
// pipelined halves (chain_eval): the stage's weights, layer states and head
// buffers shared, its own scratch, stream and position counter.
static HStage *twin_new(HStage *S, char *err, size_t errlen) {
    HStage *T = new HStage();
    T->s = S->s;
    T->L = S->L;
    T->output = S->output; T->tok_embd = S->tok_embd; T->out_norm = S->out_norm;
    T->rope = S->rope; T->logits = S->logits; T->amax = S->amax;
    T->head_nwg = S->head_nwg; T->head_rows = S->head_rows;
    T->conv_n = S->conv_n; T->ssm_n = S->ssm_n; T->n_ck = S->n_ck;
    if (hipStreamCreateWithFlags(&T->st, hipStreamNonBlocking) != hipSuccess) {
        snprintf(err, errlen, "stream creation failed");
        T->st = nullptr;
    } else if (hipHostMalloc((void **)&T->h_i, 64, hipHostMallocDefault) != hipSuccess) {
        snprintf(err, errlen, "pinned allocation failed");
        T->h_i = nullptr;
    } else if (alloc_scratch(T, err, errlen)) {
        return T;
    }
    for (void *p : T->allocs) (void)hipFree(p);
    if (T->h_i) (void)hipHostFree(T->h_i);
    if (T->st) (void)hipStreamDestroy(T->st);
    delete T;
    return nullptr;
}
static void twin_free(HStage *T) {
    if (!T) return;
    if (T->st) (void)hipStreamSynchronize(T->st);
    for (void *p : T->allocs) (void)hipFree(p);
    if (T->h_i) (void)hipHostFree(T->h_i);
    if (T->st) (void)hipStreamDestroy(T->st);
    delete T;
}

void hip_destroy(xj_stage *s) {
    if (!s) return;
    HStage *S = H(s);
    if (S->st) (void)hipStreamSynchronize(S->st);
    for (auto &L : S->L) {
        if (L.ck_conv) (void)hipFree(L.ck_conv);
        if (L.ck_ssm) (void)hipFree(L.ck_ssm);
        for (int i = 0; i < kSnapSlots; i++) {
            if (L.snap_conv[i]) (void)hipFree(L.snap_conv[i]);
            if (L.snap_ssm[i]) (void)hipFree(L.snap_ssm[i]);
        }
    }
    for (void *p : S->allocs) (void)hipFree(p);
    if (S->h_x) (void)hipHostFree(S->h_x);
    if (S->h_i) (void)hipHostFree(S->h_i);
    if (S->st) (void)hipStreamDestroy(S->st);
    delete S;
}

void init_names() {
    if (!g_name.empty()) return;
    hipDeviceProp_t p;
    int dev = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipGetDeviceProperties(&p, dev) == hipSuccess)
        g_name = std::string(p.name) + " (" + p.gcnArchName + ", " + std::to_string(p.multiProcessorCount) + " CUs)";
    else
        g_name = "hip";
}

}  // namespace

// ================================================================= stage ==

extern "C" const char *xj_hip_device_name(void) { init_names(); return g_name.c_str(); }
extern "C" const char *xj_hip_tune_note(void) { return g_note.c_str(); }


extern "C" uint64_t xj_hip_stage_state_bytes(const xj_model *m, int l0, int l1, int n_ctx, int max_batch) {
    const xj_hparams &hp = m->hp;
    uint64_t b = 0;
    for (int il = l0; il < l1; il++) {
        if (m->layers[il].recurrent)
            b += 4ull * ((uint64_t)hp.conv_dim * (hp.conv_k - 1) + (uint64_t)hp.h_v * hp.s_v * hp.s_k);
        else
            b += 2ull * 2 * n_ctx * hp.n_head_kv * hp.head_dim;
    }
    b += 10ull * 4 * max_batch * scratch_floats(hp) +
         4ull * max_batch * hp.n_head * ((n_ctx + 63) / 64) * (hp.head_dim + 2);
    // prefill on the matrix cores: RMSNorm scales, K-split partials and counters, chunked-rule work
    const int64_t grows = 2 * (int64_t)scratch_floats(hp) + 2 * (int64_t)hp.h_v;
    b += 4ull * max_batch + 4ull * gemm_part_floats(grows, max_batch < gemm_max_tokens() ? max_batch : gemm_max_tokens()) +
         4ull * gemm_counters(grows) + (uint64_t)max_batch * hq_stride((int)scratch_floats(hp));
    bool rec = false;
    for (int il = l0; il < l1 && il < (int)hp.n_layer; il++) rec = rec || m->layers[il].recurrent;
    if (rec) b += delta_chunked_work_bytes(hp.h_v, hp.s_k, max_batch, 64);
    return b;
}

extern "C" xj_stage *xj_hip_stage_new(const xj_model *m, int l0, int l1, int n_ctx, int max_batch, bool has_head,
                                      char *err, size_t errlen) {
    const xj_hparams &hp = m->hp;
    // the MTP stage is the range [n_layer, n_layer + 1) of a model with an MTP layer (xj_cpu.c:378-379)
    const bool mtp = m->has_mtp && l0 == hp.n_layer && l1 == hp.n_layer + 1;
    if (l0 < 0 || (l1 > hp.n_layer && !mtp) || l0 > l1) { snprintf(err, errlen, "bad layer range [%d,%d)", l0, l1); return nullptr; }
    for (int il = l0; il < l1; il++)
        if (!m->layers[il].ffn_down.data) { snprintf(err, errlen, "layer %d weights are not mapped", il); return nullptr; }
    if (has_head && !m->output.data) { snprintf(err, errlen, "output head is not mapped"); return nullptr; }
    if (max_batch < 1 || n_ctx < 1) { snprintf(err, errlen, "bad n_ctx/max_batch"); return nullptr; }
    bool any_attn = false, any_rec = false;
    for (int il = l0; il < l1; il++) (m->layers[il].recurrent ? any_rec : any_attn) = true;
    if (any_attn && hp.head_dim != 64 && hp.head_dim != 128 && hp.head_dim != 256) {
        snprintf(err, errlen, "head_dim %d not supported (64/128/256)", hp.head_dim); return nullptr;
    }
    if (any_rec && hp.s_k != 64 && hp.s_k != 128) { snprintf(err, errlen, "ssm state_size %d not supported (64/128)", hp.s_k); return nullptr; }
    if (any_rec && (hp.conv_k < 2 || hp.conv_k > 8)) { snprintf(err, errlen, "conv kernel %d not supported", hp.conv_k); return nullptr; }
    if (hp.n_embd % 256 || hp.n_ff % 32) { snprintf(err, errlen, "n_embd must be a multiple of 256"); return nullptr; }
    if (hp.n_head_kv < 1 || hp.n_head % hp.n_head_kv) { snprintf(err, errlen, "n_head must be a multiple of n_head_kv"); return nullptr; }
    if (hp.n_head / hp.n_head_kv > 8) { snprintf(err, errlen, "at most 8 query heads per kv head are supported"); return nullptr; }
    {   // every tensor a kernel reads must have the shape the kernel assumes
        const int64_t E = hp.n_embd, FF = hp.n_ff, D = hp.head_dim, nq = 2 * (int64_t)hp.n_head * D, nk = (int64_t)hp.n_head_kv * D;
        auto bad = [&](const xj_w &w, int64_t ne0, int64_t ne1, const char *what, int il) {
            if (w.ne0 == ne0 && w.ne1 == ne1) return false;
            snprintf(err, errlen, "layer %d: %s has shape %lldx%lld, expected %lldx%lld", il, what, (long long)w.ne0,
                     (long long)w.ne1, (long long)ne0, (long long)ne1);
            return true;
        };
        for (int il = l0; il < l1; il++) {
            const xj_layer &w = m->layers[il];
            if (bad(w.attn_norm, E, 1, "attn_norm", il) || bad(w.post_norm, E, 1, "post_norm", il) ||
                bad(w.ffn_gate, E, FF, "ffn_gate", il) || bad(w.ffn_up, E, FF, "ffn_up", il) || bad(w.ffn_down, FF, E, "ffn_down", il))
                return nullptr;
            if (w.recurrent) {
                if (bad(w.ssm_qkv, E, hp.conv_dim, "attn_qkv", il) || bad(w.ssm_gate, E, hp.d_inner, "attn_gate", il) ||
                    bad(w.ssm_beta, E, hp.h_v, "ssm_beta", il) || bad(w.ssm_alpha, E, hp.h_v, "ssm_alpha", il) ||
                    bad(w.ssm_out, hp.d_inner, E, "ssm_out", il) || bad(w.ssm_conv1d, hp.conv_k, hp.conv_dim, "ssm_conv1d", il) ||
                    bad(w.ssm_dt, hp.h_v, 1, "ssm_dt", il) || bad(w.ssm_a, hp.h_v, 1, "ssm_a", il) || bad(w.ssm_norm, hp.s_k, 1, "ssm_norm", il))
                    return nullptr;
            } else {
                if (w.wqkv.nbytes ? bad(w.wqkv, E, nq + 2 * nk, "attn_qkv", il)
                                  : (bad(w.wq, E, nq, "attn_q", il) || bad(w.wk, E, nk, "attn_k", il) || bad(w.wv, E, nk, "attn_v", il)))
                    return nullptr;
                if (bad(w.wo, (int64_t)hp.n_head * D, E, "attn_output", il) || bad(w.q_norm, D, 1, "q_norm", il) ||
                    bad(w.k_norm, D, 1, "k_norm", il))
                    return nullptr;
            }
        }
        if (has_head && (bad(m->output, E, m->output.ne1, "output", -1) || bad(m->output_norm, E, 1, "output_norm", -1))) return nullptr;
        if (mtp && (bad(m->mtp_eh, 2 * E, E, "nextn.eh_proj", l0) || bad(m->mtp_enorm, E, 1, "nextn.enorm", l0) ||
                    bad(m->mtp_hnorm, E, 1, "nextn.hnorm", l0) || bad(m->mtp_head_norm, E, 1, "nextn.shared_head_norm", l0)))
            return nullptr;
        if (bad(m->tok_embd, E, m->tok_embd.ne1, "token_embd", -1)) return nullptr;
    }
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) { snprintf(err, errlen, "no HIP device"); return nullptr; }
    if (gemv_init(err, errlen)) return nullptr;
    init_names();

    HStage *S = new HStage();
    xj_stage *s = &S->s;
    memset(s, 0, sizeof(*s));
    s->m = m; s->l0 = l0; s->l1 = l1; s->n_ctx = n_ctx; s->max_batch = max_batch; s->has_head = has_head;
    s->mtp = mtp; s->backend = "hip";
    s->forward = hip_forward; s->logits = hip_logits; s->rollback = hip_rollback; s->reset = hip_reset;
    s->destroy = hip_destroy; s->impl = S;
    auto fail = [&]() -> xj_stage * { hip_destroy(s); return nullptr; };
    if (hipStreamCreateWithFlags(&S->st, hipStreamNonBlocking) != hipSuccess) { snprintf(err, errlen, "stream creation failed"); return fail(); }

    S->conv_n = (size_t)hp.conv_dim * (hp.conv_k - 1);
    S->ssm_n = (size_t)hp.h_v * hp.s_v * hp.s_k;
    S->L.resize(l1 - l0);
    for (int il = l0; il < l1; il++) {
        const xj_layer &w = m->layers[il];
        HLayer &L = S->L[il - l0];
        L.rec = w.recurrent;
        bool ok = upload_f32(S, w.attn_norm, &L.attn_norm, err, errlen) && upload_f32(S, w.post_norm, &L.post_norm, err, errlen) &&
                  upload(S, w.ffn_gate, &L.ffn_gate, err, errlen) && upload(S, w.ffn_up, &L.ffn_up, err, errlen) &&
                  upload(S, w.ffn_down, &L.ffn_down, err, errlen);
        if (ok && L.rec) {
            ok = upload(S, w.ssm_qkv, &L.ssm_qkv, err, errlen) && upload(S, w.ssm_gate, &L.ssm_gate, err, errlen) &&
                 upload(S, w.ssm_beta, &L.ssm_beta, err, errlen) && upload(S, w.ssm_alpha, &L.ssm_alpha, err, errlen) &&
                 upload(S, w.ssm_out, &L.ssm_out, err, errlen) && upload_f32(S, w.ssm_conv1d, &L.conv_w, err, errlen) &&
                 upload_f32(S, w.ssm_dt, &L.dt, err, errlen) && upload_f32(S, w.ssm_a, &L.A, err, errlen) &&
                 upload_f32(S, w.ssm_norm, &L.ssm_norm, err, errlen);
            if (ok) {
                L.conv = dalloc<float>(S, S->conv_n, err, errlen);
                L.ssm = dalloc<float>(S, S->ssm_n, err, errlen);
                ok = L.conv && L.ssm;
            }
        } else if (ok) {
            ok = upload(S, w.wqkv, &L.wqkv, err, errlen) && upload(S, w.wq, &L.wq, err, errlen) &&
                 upload(S, w.wk, &L.wk, err, errlen) && upload(S, w.wv, &L.wv, err, errlen) &&
                 upload(S, w.wo, &L.wo, err, errlen) && upload_f32(S, w.q_norm, &L.q_norm, err, errlen) &&
                 upload_f32(S, w.k_norm, &L.k_norm, err, errlen);
            if (ok) {
                const size_t kvn = (size_t)n_ctx * hp.n_head_kv * hp.head_dim;
                L.kc = dalloc<uint16_t>(S, kvn, err, errlen);
                L.vc = dalloc<uint16_t>(S, kvn, err, errlen);
                ok = L.kc && L.vc;
            }
        }
        if (!ok) return fail();
    }
    if (has_head) {
        // the MTP stage's head normalises with shared_head_norm (xj_cpu.c:287)
        if (!upload(S, m->output, &S->output, err, errlen) ||
            !upload_f32(S, mtp ? m->mtp_head_norm : m->output_norm, &S->out_norm, err, errlen))
            return fail();
        if (S->output.k != hp.n_embd) { snprintf(err, errlen, "output head shape mismatch"); return fail(); }
    }
    const size_t mb = max_batch, E = hp.n_embd;
    if (!alloc_scratch(S, err, errlen)) return fail();
    const int half = hp.n_rot / 2 > 0 ? hp.n_rot / 2 : 1;
    S->rope = dalloc<float2>(S, (size_t)n_ctx * half, err, errlen);
    if (!S->x || !S->qkv || !S->kb || !S->vb || !S->z || !S->beta || !S->alpha || !S->o || !S->g || !S->u ||
        !S->qr || !S->scores || !S->npast || !S->rope)
        return fail();
    if (has_head) {
        S->logits = dalloc<float>(S, mb * (size_t)S->output.n_rows, err, errlen);
        const int rows = gemv_plan((int)S->output.k, S->output.n_rows).rows_per_group;
        S->head_nwg = (int)((S->output.n_rows + rows - 1) / rows);
        S->head_rows = rows;
        S->amax = dalloc<unsigned long long>(S, mb * (size_t)S->head_nwg, err, errlen);
        if (!S->logits || !S->amax) return fail();
    }
    {   // cos and sin of theta = pos * base^(-2i/n_rot) for every position, in float as the
        // reference's rope evaluates them (xj_cpu.c:68-77)
        std::vector<float2> cs((size_t)n_ctx * half, float2{1.f, 0.f});
        rope_table(0, n_ctx, hp.n_rot, hp.rope_base, cs.data());
        XJ_CHECK(hipMemcpy(S->rope, cs.data(), cs.size() * sizeof(float2), hipMemcpyHostToDevice), err, errlen, fail());
    }
    if (mtp) {
        if (!upload(S, m->mtp_eh, &S->mtp_eh, err, errlen) || !upload_f32(S, m->mtp_enorm, &S->mtp_enorm, err, errlen) ||
            !upload_f32(S, m->mtp_hnorm, &S->mtp_hnorm, err, errlen))
            return fail();
        S->mx = dalloc<float>(S, mb * 2 * E, err, errlen);
        S->mh = dalloc<float>(S, mb * 2 * E, err, errlen);
        S->xq_2e = dalloc<uint8_t>(S, mb * (size_t)xq_off(2 * (int)E).stride, err, errlen);
        if (!S->mx || !S->mh || !S->xq_2e) return fail();
    }
    XJ_CHECK(hipHostMalloc((void **)&S->h_x, sizeof(float) * mb * E * (mtp ? 2 : 1), hipHostMallocDefault), err, errlen, fail());
    XJ_CHECK(hipHostMalloc((void **)&S->h_i, 64, hipHostMallocDefault), err, errlen, fail());
    hip_reset(s);
    char note[160];
    const GemvPlan pe = gemv_plan(hp.n_embd, hp.n_ff);
    snprintf(note, sizeof note, "gemv K=n_embd: %d lanes x %d rows per team, %.0f MB weights in HBM", pe.lanes, pe.rpt,
             S->weight_bytes / 1048576.0);
    g_note = note;
    return s;
}

// The recurrent state of every DeltaNet layer into snapshot slot `slot`,
// enqueued on `st` (allocated on first use).
static int snapshot_enqueue(HStage *S, int slot, hipStream_t st, char *err, size_t errlen) {
    if (slot < 0 || slot >= kSnapSlots) { snprintf(err, errlen, "snapshot slot %d out of range", slot); return -1; }
    for (auto &L : S->L) {
        if (!L.rec || L.snap_conv[slot]) continue;
        if (hipMalloc(&L.snap_conv[slot], S->conv_n * 4) != hipSuccess || hipMalloc(&L.snap_ssm[slot], S->ssm_n * 4) != hipSuccess) {
            snprintf(err, errlen, "out of HBM for snapshots");
            return -1;
        }
    }
    if (states_copy(S, st, [&](HLayer &L, const float *&cs, float *&cd, const float *&ss, float *&sd) {
            cs = L.conv; cd = L.snap_conv[slot];
            ss = L.ssm; sd = L.snap_ssm[slot];
        })) {
        snprintf(err, errlen, "snapshot copy failed");
        return -1;
    }
    return 0;
}

extern "C" int xj_hip_stage_snapshot(xj_stage *s, int slot, char *err, size_t errlen) {
    if (slot < 0 || slot >= kDecodeSlot) { snprintf(err, errlen, "snapshot slot %d out of range", slot); return -1; }
    return snapshot_enqueue(H(s), slot, H(s)->st, err, errlen);
}

extern "C" int xj_hip_stage_fill_kv(xj_stage *s, int pos0, uint16_t bits, char *err, size_t errlen) {
    HStage *S = H(s);
    if (pos0 < 0 || pos0 > s->n_ctx) { snprintf(err, errlen, "bad position %d", pos0); return -1; }
    const xj_hparams &hp = S->s.m->hp;
    const size_t nk = (size_t)hp.n_head_kv * hp.head_dim, n = (size_t)(s->n_ctx - pos0) * nk;
    for (auto &L : S->L) {
        if (L.rec || !L.kc || !n) continue;
        if (hipMemsetD16Async((hipDeviceptr_t)(L.kc + pos0 * nk), bits, n, S->st) != hipSuccess ||
            hipMemsetD16Async((hipDeviceptr_t)(L.vc + pos0 * nk), bits, n, S->st) != hipSuccess) {
            snprintf(err, errlen, "cache fill failed");
            return -1;
        }
    }
    return sync_check(S, err, errlen);
}

// Restores slot `slot` on `st` (enqueued only) and sets n_past.
static int restore_enqueue(HStage *S, int slot, int n_past, hipStream_t st, char *err, size_t errlen) {
    xj_stage *s = &S->s;
    if (n_past < 0 || n_past > s->n_ctx) { snprintf(err, errlen, "bad n_past %d", n_past); return -1; }
    for (auto &L : S->L)
        if (L.rec && !L.snap_conv[slot]) { snprintf(err, errlen, "snapshot slot %d is empty", slot); return -1; }
    if (states_copy(S, st, [&](HLayer &L, const float *&cs, float *&cd, const float *&ss, float *&sd) {
            cs = L.snap_conv[slot]; cd = L.conv;
            ss = L.snap_ssm[slot]; sd = L.ssm;
        })) {
        snprintf(err, errlen, "restore copy failed");
        return -1;
    }
    s->n_past = n_past;
    s->ck_T = 0;
    return 0;
}

extern "C" int xj_hip_stage_restore(xj_stage *s, int slot, int n_past, char *err, size_t errlen) {
    HStage *S = H(s);
    if (slot < 0 || slot >= kDecodeSlot) { snprintf(err, errlen, "snapshot slot %d out of range", slot); return -1; }
    if (restore_enqueue(S, slot, n_past, S->st, err, errlen)) return -1;
    return sync_check(S, err, errlen);
}

// ================================================================= chain ==

constexpr int kMaxParts = 4;   // parts of a single stage's layers in a pipelined prefill
struct xjh_chain {
    std::vector<HStage *> st;
    std::vector<HStage *> twins;   // a single stage's later parts of the layers in prefill (twin_new)
    hipStream_t stream = nullptr;
    float *x = nullptr;
    int mb = 0, hist_cap = 0;
    int32_t *d_tokens = nullptr, *d_argmax = nullptr, *d_tok = nullptr, *d_hist = nullptr, *d_step = nullptr;
    int32_t *h_buf = nullptr;   // pinned
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    double last_ms = 0;
    int last_tok = -1;
    // prefill: the whole prompt's ids on the device, and per stage the events
    // of the chunk hand-off (this stage's layers done; its copy of the
    // upstream stage's output done)
    int32_t *d_prompt = nullptr;
    int prompt_cap = 0;
    std::vector<hipEvent_t> ev_done, ev_taken;
    // the app's sampler (xjh_chain_set_sampler): temperature, the uniform
    // numbers on the device, how many are drawn; the sampled decode graph
    float temp = 0.f;
    uint32_t *d_rnd = nullptr;
    int n_rnd = 0, rnd_cap = 0, used = 0;
    float *d_temp = nullptr;
    int32_t *d_rbase = nullptr, *d_pick = nullptr;
    hipGraphExec_t exec_s = nullptr;
    hipGraph_t graph_s = nullptr;
};

// Parts of a single stage's layers in a prompt of several chunks
// (XJ_STAGE_SPLIT, with chunks overlapped on the parts' streams), else 1.
static int stage_parts(const xjh_chain *c) {
    static const bool overlap = env_int("XJ_CHAIN_OVERLAP", 1) != 0;
    static const int split_env = env_int("XJ_STAGE_SPLIT", 3);
    if (c->st.size() != 1 || !overlap) return 1;
    const int nl = c->st[0]->s.l1 - c->st[0]->s.l0;
    return split_env < 1 ? 1 : split_env > kMaxParts ? kMaxParts : split_env > nl ? nl : split_env;
}
// the later parts' scratch sets (twin_new), created once
static int chain_twins(xjh_chain *c, int npart, char *err, size_t errlen) {
    while ((int)c->twins.size() < npart - 1) {
        HStage *T = twin_new(c->st[0], err, errlen);
        if (!T) return -1;
        c->twins.push_back(T);
    }
    return 0;
}
extern "C" void xjh_chain_free(xjh_chain *c) {
    if (!c) return;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->exec) (void)hipGraphExecDestroy(c->exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    if (c->exec_s) (void)hipGraphExecDestroy(c->exec_s);
    if (c->graph_s) (void)hipGraphDestroy(c->graph_s);
    if (c->d_rnd) (void)hipFree(c->d_rnd);
    if (c->d_temp) (void)hipFree(c->d_temp);
    for (auto *S : c->st) if (S->st) (void)hipStreamSynchronize(S->st);
    if (c->ev0) (void)hipEventDestroy(c->ev0);
    if (c->ev1) (void)hipEventDestroy(c->ev1);
    for (hipEvent_t e : c->ev_done) if (e) (void)hipEventDestroy(e);
    for (hipEvent_t e : c->ev_taken) if (e) (void)hipEventDestroy(e);
    if (c->d_prompt) (void)hipFree(c->d_prompt);
    for (HStage *T : c->twins) twin_free(T);
    for (int32_t *p : {c->d_tokens, c->d_argmax, c->d_tok, c->d_hist, c->d_step, c->d_rbase, c->d_pick}) if (p) (void)hipFree(p);
    if (c->h_buf) (void)hipHostFree(c->h_buf);
    delete c;
}

extern "C" xjh_chain *xjh_chain_new(xj_stage **stages, int n, char *err, size_t errlen) {
    if (n < 1) { snprintf(err, errlen, "empty chain"); return nullptr; }
    auto *c = new xjh_chain();
    for (int i = 0; i < n; i++) {
        if (!stages[i] || strcmp(stages[i]->backend, "hip") != 0) { snprintf(err, errlen, "chain stage %d is not a HIP stage", i); xjh_chain_free(c); return nullptr; }
        if (stages[i]->m != stages[0]->m) { snprintf(err, errlen, "chain stages use different models"); xjh_chain_free(c); return nullptr; }
        if (i > 0 && stages[i]->l0 != stages[i - 1]->l1) { snprintf(err, errlen, "chain stages are not contiguous"); xjh_chain_free(c); return nullptr; }
        c->st.push_back(H(stages[i]));
    }
    if (c->st[0]->s.l0 != 0 || !c->st.back()->s.has_head || c->st.back()->s.l1 != c->st[0]->s.m->hp.n_layer) {
        snprintf(err, errlen, "a chain must cover all layers and end with the head");
        xjh_chain_free(c);
        return nullptr;
    }
    HStage *S0 = c->st[0];
    const xj_model *m = S0->s.m;
    if (!S0->tok_embd.p && !upload(S0, m->tok_embd, &S0->tok_embd, err, errlen)) { xjh_chain_free(c); return nullptr; }
    c->stream = S0->st;
    c->x = S0->x;
    c->mb = S0->s.max_batch;
    for (auto *S : c->st) if (S->s.max_batch < c->mb) c->mb = S->s.max_batch;
    c->hist_cap = 1 << 16;
    if (hipMalloc(&c->d_tokens, 4 * c->mb) != hipSuccess || hipMalloc(&c->d_argmax, 4 * c->mb) != hipSuccess ||
        hipMalloc(&c->d_tok, 4) != hipSuccess || hipMalloc(&c->d_hist, 4 * c->hist_cap) != hipSuccess ||
        hipMalloc(&c->d_step, 4) != hipSuccess || hipMalloc(&c->d_rbase, 4) != hipSuccess ||
        hipMalloc(&c->d_pick, 4 * c->mb) != hipSuccess || hipMalloc(&c->d_temp, 4) != hipSuccess ||
        hipHostMalloc((void **)&c->h_buf, 4 * (c->mb + 16), hipHostMallocDefault) != hipSuccess ||
        hipEventCreate(&c->ev0) != hipSuccess || hipEventCreate(&c->ev1) != hipSuccess) {
        snprintf(err, errlen, "chain allocation failed");
        xjh_chain_free(c);
        return nullptr;
    }
    const size_t nev = c->st.size() < kMaxParts ? kMaxParts : c->st.size();   // a single stage may run in parts
    c->ev_done.assign(nev, nullptr);
    c->ev_taken.assign(nev, nullptr);
    for (size_t i = 0; i < nev; i++)
        if (hipEventCreateWithFlags(&c->ev_done[i], hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&c->ev_taken[i], hipEventDisableTiming) != hipSuccess) {
            snprintf(err, errlen, "chain allocation failed");
            xjh_chain_free(c);
            return nullptr;
        }
    // a stage whose chunks take the prefill GEMM gets its parts' scratch now,
    // so that its first long prompt does not pay for the allocations
    // (a 4B 1024-token prefill: 0.083 s on the first call, 0.073 s after)
    if (c->mb >= Gemv::kGemmMinT && stage_parts(c) > 1 && chain_twins(c, stage_parts(c), err, errlen)) {
        xjh_chain_free(c);
        return nullptr;
    }
    return c;
}

static int chain_sync(xjh_chain *c, char *err, size_t errlen) {
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e == hipSuccess) e = hipGetLastError();
    if (e != hipSuccess) { snprintf(err, errlen, "GPU error: %s", hipGetErrorString(e)); return -1; }
    return 0;
}

// The prompt in chunks of max_batch, the stages pipelined (pipe/core/xj_net.c:561-604
// pipelines a remote worker's half against the host's): each stage runs on its
// own stream from its own hidden-state buffer, so stage i works on chunk k + 1
// while stage i + 1 works on chunk k. A single stage's layers run the same
// way in XJ_STAGE_SPLIT parts (3: a 4B 1024-token prefill 0.118 -> 0.083 s;
// 2 parts 0.091 s, 4 parts 0.093 s). Stage i + 1 takes chunk k by a device
// copy once stage i has finished it (event done[i]); stage i overwrites its
// buffer with chunk k + 1 only after that copy (event taken[i + 1]). Every
// stage's n_past advances on the device at the end of each chunk, so no host
// round trip separates the chunks; XJ_CHAIN_OVERLAP=0 runs all stages on one
// stream.
static int chain_finish(xjh_chain *c, int nl, int32_t *argmax, char *err, size_t errlen);
// wait = false: returns once everything is enqueued (nlog > 0, no logits);
// chain_finish collects the argmax of the nlog rows.
static int chain_eval(xjh_chain *c, const int32_t *tokens, int n, int nlog, int keep, float *logits, int32_t *argmax,
                      char *err, size_t errlen, bool wait = true) {
    const int B = c->mb, E = c->st[0]->s.m->hp.n_embd, ns = (int)c->st.size();
    if (!wait && (nlog < 1 || logits || n > B)) { snprintf(err, errlen, "asynchronous eval of one chunk with argmax only"); return -1; }
    if (n <= 0) { snprintf(err, errlen, "no tokens"); return -1; }
    if (keep && n > B) { snprintf(err, errlen, "verify batch %d exceeds max_batch %d", n, B); return -1; }
    static const bool overlap = env_int("XJ_CHAIN_OVERLAP", 1) != 0;
    // the pipeline's parts: every stage, or a single stage's layers in
    // XJ_STAGE_SPLIT contiguous parts (the later ones on twins' scratch and
    // streams) when the prompt spans several chunks
    struct Part { HStage *S; int lo, hi; bool twin; };
    std::vector<Part> parts;
    HStage *S0 = c->st[0];
    const int nl = S0->s.l1 - S0->s.l0;
    const int npart = stage_parts(c);
    if (npart > 1 && n > B && !keep) {
        if (chain_twins(c, npart, err, errlen)) return -1;
        for (int p = 0; p < npart; p++) {
            HStage *S = p ? c->twins[p - 1] : S0;
            if (p) {
                S->L = S0->L;   // checkpoint and snapshot buffers allocated since
                S->n_ck = S0->n_ck;
            }
            parts.push_back(Part{S, S0->s.l0 + nl * p / npart, S0->s.l0 + nl * (p + 1) / npart, p > 0});
        }
    } else {
        for (auto *S : c->st) parts.push_back(Part{S, S->s.l0, S->s.l1, false});
    }
    const int np = (int)parts.size();
    HStage *head = parts.back().S;
    auto stream_of = [&](int i) { return overlap ? parts[i].S->st : c->stream; };
    auto fail_sync = [&]() {
        for (int i = 0; i < np; i++) (void)hipStreamSynchronize(parts[i].S->st);
        for (auto *S : c->st) S->s.keep = 0;
        return -1;
    };
    for (auto *S : c->st)
        if (S->s.n_past + n > S->s.n_ctx) { snprintf(err, errlen, "context full (%d)", S->s.n_ctx); return -1; }
    if (n > c->prompt_cap) {
        if (c->d_prompt) (void)hipFree(c->d_prompt);
        c->d_prompt = nullptr, c->prompt_cap = 0;
        if (hipMalloc(&c->d_prompt, 4 * (size_t)n) != hipSuccess) { snprintf(err, errlen, "prompt allocation failed"); return -1; }
        c->prompt_cap = n;
    }
    // the ids (synchronous copy from the caller's memory) and every part's
    // starting position (a twin starts where its stage is)
    if (hipMemcpy(c->d_prompt, tokens, 4 * (size_t)n, hipMemcpyHostToDevice) != hipSuccess) {
        snprintf(err, errlen, "token upload failed"); return -1;
    }
    for (int i = 0; i < np; i++) {
        HStage *S = parts[i].S;
        *S->h_i = parts[i].twin ? S0->s.n_past : S->s.n_past;
        if (hipMemcpyAsync(S->npast, S->h_i, 4, hipMemcpyHostToDevice, stream_of(i)) != hipSuccess ||
            hipStreamSynchronize(stream_of(i)) != hipSuccess) {   // h_i is reused by later calls
            snprintf(err, errlen, "position upload failed"); return -1;
        }
    }
    for (int k0 = 0; k0 < n; k0 += B) {
        const int T = n - k0 < B ? n - k0 : B;
        for (int i = 0; i < np; i++) {
            HStage *S = parts[i].S;
            hipStream_t st = stream_of(i);
            if (i == 0) {
                // chunk k0 into part 0's buffer, once part 1 has taken the previous chunk
                if (np > 1 && k0 > 0 && hipStreamWaitEvent(st, c->ev_taken[1], 0) != hipSuccess) return fail_sync();
                EmbedArgs ea{c->d_prompt + k0, S->tok_embd, S->x, T};
                if (embed_launch(ea, st)) { snprintf(err, errlen, "embed launch failed"); return fail_sync(); }
            } else {
                // this part's previous chunk is done with its buffer (same stream); the
                // upstream part's output of this chunk is final
                if (i + 1 < np && k0 > 0 && hipStreamWaitEvent(st, c->ev_taken[i + 1], 0) != hipSuccess) return fail_sync();
                if (hipStreamWaitEvent(st, c->ev_done[i - 1], 0) != hipSuccess ||
                    hipMemcpyAsync(S->x, parts[i - 1].S->x, sizeof(float) * (size_t)T * E, hipMemcpyDeviceToDevice, st) != hipSuccess ||
                    hipEventRecord(c->ev_taken[i], st) != hipSuccess) {
                    snprintf(err, errlen, "chunk hand-off failed"); return fail_sync();
                }
            }
            int keep_n = 0;
            if (!parts[i].twin) {
                if (keep) S->s.keep = T;
                if (begin_forward(S, T, &keep_n, err, errlen)) return fail_sync();
            }
            if (enqueue_layer_range(S, parts[i].lo, parts[i].hi, S->x, T, keep_n, true, st) ||
                hipEventRecord(c->ev_done[i], st) != hipSuccess) {
                snprintf(err, errlen, "layer launch failed"); return fail_sync();
            }
            if (!parts[i].twin) {
                S->s.n_past += T;
                if (k0 + T < n) S->s.keep = 0;
            }
        }
    }
    const int T = n - (n - 1) / B * B;   // tokens of the last chunk
    hipStream_t hs = stream_of(np - 1);
    if (nlog > 0) {
        const int nl = nlog < T ? nlog : T;
        if (enqueue_head(head, head->x + (int64_t)(T - nl) * E, nl, head->logits, hs) ||
            argmax_finalize_launch(head->amax, head->head_nwg, nl, c->d_argmax, c->d_tok, nullptr, nullptr, hs)) {
            snprintf(err, errlen, "head launch failed"); return fail_sync();
        }
    }
    // the last chunk's hidden rows where the decode step and the drivers read
    // them (the chain's buffer, stage 0's); the head stream is ordered after
    // every part's last chunk through the hand-off events
    if (np > 1 && hipMemcpyAsync(c->x, head->x, sizeof(float) * (size_t)T * E, hipMemcpyDeviceToDevice, hs) != hipSuccess) {
        snprintf(err, errlen, "hidden copy failed"); return fail_sync();
    }
    if (!wait) {   // a single part: the head stream is the chain's
        const int nl = nlog < T ? nlog : T;
        if (hipMemcpyAsync(c->h_buf, c->d_argmax, 4 * nl, hipMemcpyDeviceToHost, hs) != hipSuccess) {
            snprintf(err, errlen, "argmax copy failed"); return fail_sync();
        }
        return 0;
    }
    for (int i = 0; i < np; i++) {
        hipError_t e = hipStreamSynchronize(stream_of(i));
        if (e == hipSuccess) e = hipGetLastError();
        if (e != hipSuccess) { snprintf(err, errlen, "GPU error: %s", hipGetErrorString(e)); return fail_sync(); }
    }
    if (nlog > 0) {
        const int nl = nlog < T ? nlog : T;
        if (logits && hipMemcpy(logits, head->logits, sizeof(float) * nl * head->output.n_rows, hipMemcpyDeviceToHost) != hipSuccess) {
            snprintf(err, errlen, "logits copy failed"); return -1;
        }
        if (hipMemcpy(c->h_buf, c->d_argmax, 4 * nl, hipMemcpyDeviceToHost) != hipSuccess) { snprintf(err, errlen, "argmax copy failed"); return -1; }
        if (argmax) memcpy(argmax, c->h_buf, 4 * nl);
        c->last_tok = c->h_buf[nl - 1];
    }
    for (auto *S : c->st) S->s.keep = 0;
    return 0;
}

// The end of an asynchronous chain_eval of a single chunk: every stage's
// stream synchronised, the argmax of its nl rows.
static int chain_finish(xjh_chain *c, int nl, int32_t *argmax, char *err, size_t errlen) {
    int rc = 0;
    for (auto *S : c->st) {
        hipError_t e = hipStreamSynchronize(S->st);
        if (e == hipSuccess) e = hipGetLastError();
        if (e != hipSuccess && !rc) { snprintf(err, errlen, "GPU error: %s", hipGetErrorString(e)); rc = -1; }
    }
    if (c->stream) {
        hipError_t e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess && !rc) { snprintf(err, errlen, "GPU error: %s", hipGetErrorString(e)); rc = -1; }
    }
    for (auto *S : c->st) S->s.keep = 0;
    if (rc) return rc;
    memcpy(argmax, c->h_buf, 4 * (size_t)nl);
    c->last_tok = c->h_buf[nl - 1];
    return 0;
}

static bool sampling(const xjh_chain *c) { return !(c->temp <= 0.f); }

// The sampler's tokens after rows [row0, row0 + n) of the head's last logits,
// row row0 + i drawn with number used + i (the caller counts what it
// consumes); the argmax of those rows when the sampler is off.
static int chain_draw(xjh_chain *c, int row0, int n, int32_t *out, char *err, size_t errlen) {
    HStage *head = c->st.back();
    if (n < 1 || n > c->mb) { snprintf(err, errlen, "draw of %d rows", n); return -1; }
    if (sampling(c) && c->used + n > c->n_rnd) {
        snprintf(err, errlen, "sampler: %d random numbers left, %d needed", c->n_rnd - c->used, n); return -1;
    }
    SampleArgs sa{};
    sa.lg = head->logits + (int64_t)row0 * head->output.n_rows;
    sa.V = (int32_t)head->output.n_rows;
    sa.T = n;
    sa.temp = c->temp;
    sa.rnd = c->d_rnd ? c->d_rnd + c->used : nullptr;
    sa.out = c->d_pick;
    sa.part = head->amax + (int64_t)row0 * head->head_nwg;
    sa.n_part = head->head_nwg;
    sa.part_rows = head->head_rows;
    if (sample_launch(sa, c->stream) ||
        hipMemcpyAsync(c->h_buf, c->d_pick, 4 * (size_t)n, hipMemcpyDeviceToHost, c->stream) != hipSuccess) {
        snprintf(err, errlen, "sample launch failed"); return -1;
    }
    if (chain_sync(c, err, errlen)) return -1;
    memcpy(out, c->h_buf, 4 * (size_t)n);
    return 0;
}

// The public eval: with the sampler on, the token after the last row is drawn
// (one number) and becomes the token the next step feeds.
extern "C" int xjh_chain_eval(xjh_chain *c, const int32_t *tokens, int n, int nlog, int keep, float *logits,
                              int32_t *argmax, char *err, size_t errlen) {
    const bool draw = nlog > 0 && sampling(c);
    if (draw && c->used + 1 > c->n_rnd) { snprintf(err, errlen, "sampler: no random numbers left"); return -1; }
    if (chain_eval(c, tokens, n, nlog, keep, logits, argmax, err, errlen)) return -1;
    if (draw) {
        const int T = keep ? n : n - (n - 1) / c->mb * c->mb;   // rows of the last chunk
        const int nl = nlog < T ? nlog : T;
        int32_t t;
        if (chain_draw(c, nl - 1, 1, &t, err, errlen)) return -1;
        c->last_tok = t;
        c->used += 1;
    }
    return 0;
}

extern "C" int xjh_chain_set_sampler(xjh_chain *c, float temperature, const uint32_t *rand30, int n, char *err,
                                     size_t errlen) {
    if (n < 0 || (n > 0 && !rand30)) { snprintf(err, errlen, "sampler: bad random numbers"); return -1; }
    for (int i = 0; i < n; i++)
        if (rand30[i] >= (1u << 30)) { snprintf(err, errlen, "sampler: number %d (%u) not below 2^30", i, rand30[i]); return -1; }
    if (n > c->rnd_cap) {   // the sampled graph holds the array's address: rebuilt on its next use
        if (c->exec_s) (void)hipGraphExecDestroy(c->exec_s);
        if (c->graph_s) (void)hipGraphDestroy(c->graph_s);
        c->exec_s = nullptr;
        c->graph_s = nullptr;
        if (c->d_rnd) (void)hipFree(c->d_rnd);
        c->d_rnd = nullptr;
        c->rnd_cap = 0;
        if (hipMalloc(&c->d_rnd, 4 * (size_t)n) != hipSuccess) { snprintf(err, errlen, "sampler: hipMalloc failed"); return -1; }
        c->rnd_cap = n;
    }
    if ((n > 0 && hipMemcpy(c->d_rnd, rand30, 4 * (size_t)n, hipMemcpyHostToDevice) != hipSuccess) ||
        hipMemcpy(c->d_temp, &temperature, 4, hipMemcpyHostToDevice) != hipSuccess) {
        snprintf(err, errlen, "sampler: upload failed"); return -1;
    }
    c->temp = temperature;
    c->n_rnd = n;
    c->used = 0;
    return 0;
}

extern "C" int xjh_chain_sampler_used(xjh_chain *c) { return c->used; }

// One greedy decode step, entirely on the device: embedding of d_tok, every
// stage (the last GEMV of each advances its n_past), the head, and the argmax
// that writes d_tok and appends it to the history.
// One decode step from the embedding already in c->x: the layers, the head,
// and the argmax launch, which records the token and writes its embedding
// into c->x for the next step (embed_first: the set-up's embedding of d_tok).
static int embed_first(xjh_chain *c) {
    EmbedArgs ea{c->d_tok, c->st[0]->tok_embd, c->x, 1};
    return embed_launch(ea, c->stream);
}

// sampled: the app's draw (temperature and numbers read from the device,
// number d_rbase + step) in place of the argmax launch.
static int enqueue_decode_step(xjh_chain *c, bool sampled) {
    HStage *head = c->st.back();
    int rc = 0;
    for (auto *S : c->st) rc = rc ? rc : enqueue_layers(S, c->x, 1, 0, true, c->stream);
    if (!rc) rc = enqueue_head(head, c->x, 1, head->logits, c->stream);
    const EmbedArgs next{nullptr, c->st[0]->tok_embd, c->x, 1};
    if (rc) return rc;
    if (!sampled)
        return argmax_finalize_launch(head->amax, head->head_nwg, 1, nullptr, c->d_tok, c->d_hist, c->d_step, c->stream,
                                      &next);
    SampleArgs sa{};
    sa.lg = head->logits;
    sa.V = (int32_t)head->output.n_rows;
    sa.T = 1;
    sa.part = head->amax;
    sa.n_part = head->head_nwg;
    sa.part_rows = head->head_rows;
    sa.temp_dev = c->d_temp;
    sa.rnd = c->d_rnd;
    sa.rbase = c->d_rbase;
    sa.tok_out = c->d_tok;
    sa.hist = c->d_hist;
    sa.step = c->d_step;
    sa.embed = next;
    return sample_launch(sa, c->stream);
}

static int build_decode_graph(xjh_chain *c, bool sampled, char *err, size_t errlen) {
    if (hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        snprintf(err, errlen, "graph capture failed to start"); return -1;
    }
    const int rc = enqueue_decode_step(c, sampled);
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &g);
    if (rc || e != hipSuccess) { snprintf(err, errlen, "graph capture failed"); if (g) (void)hipGraphDestroy(g); return -1; }
    hipGraphExec_t &ex = sampled ? c->exec_s : c->exec;
    if (hipGraphInstantiate(&ex, g, nullptr, nullptr, 0) != hipSuccess) {
        snprintf(err, errlen, "graph instantiation failed"); (void)hipGraphDestroy(g); ex = nullptr; return -1;
    }
    (sampled ? c->graph_s : c->graph) = g;
    return 0;
}

// End tokens of the model (xj_spec.c:29): greedy generation stops at either.
static bool is_end(const xj_hparams &hp, int32_t t) { return (uint32_t)t == hp.eot || (uint32_t)t == hp.eos; }
static bool has_end(const xj_hparams &hp) { return hp.eos != UINT32_MAX || hp.eot != UINT32_MAX; }

// n replays of the decode step from token `tok` at the stages' current n_past
// (enqueued, not synchronised); the tokens land in d_hist[0, n).
static int decode_enqueue(xjh_chain *c, int tok, int n, bool direct, bool sampled, char *err, size_t errlen) {
    c->h_buf[0] = 0;
    c->h_buf[1] = tok;
    c->h_buf[3] = c->used;   // sampled: step i draws number used + i
    if (hipMemcpyAsync(c->d_step, &c->h_buf[0], 4, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
        hipMemcpyAsync(c->d_tok, &c->h_buf[1], 4, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
        (sampled && hipMemcpyAsync(c->d_rbase, &c->h_buf[3], 4, hipMemcpyHostToDevice, c->stream) != hipSuccess)) {
        snprintf(err, errlen, "decode setup failed"); return -1;
    }
    for (auto *S : c->st) if (set_npast(S, c->stream)) { snprintf(err, errlen, "decode setup failed"); return -1; }
    if (embed_first(c)) { snprintf(err, errlen, "decode setup failed"); return -1; }
    if (chain_sync(c, err, errlen)) return -1;   // the pinned set-up words are reused below
    (void)hipEventRecord(c->ev0, c->stream);
    for (int i = 0; i < n; i++)
        if (direct ? enqueue_decode_step(c, sampled) != 0
                   : hipGraphLaunch(sampled ? c->exec_s : c->exec, c->stream) != hipSuccess) {
            snprintf(err, errlen, "decode step launch failed"); return -1;
        }
    (void)hipEventRecord(c->ev1, c->stream);
    return 0;
}

extern "C" int xjh_chain_decode(xjh_chain *c, int n_steps, int32_t *out, char *err, size_t errlen) {
    if (n_steps <= 0) return 0;
    if (c->last_tok < 0) { snprintf(err, errlen, "decode needs a previous eval with logits"); return -1; }
    const xj_hparams &hp = c->st[0]->s.m->hp;
    if (is_end(hp, c->last_tok)) return 0;   // an end token is never fed (xj_spec.c:139)
    for (auto *S : c->st) if (reset_check(S, err, errlen)) return -1;
    for (auto *S : c->st)
        if (S->s.n_past + n_steps > S->s.n_ctx) { snprintf(err, errlen, "context full (%d)", S->s.n_ctx); return -1; }
    // with the sampler on, step i draws number used + i
    const bool smp = sampling(c);
    if (smp && c->used + n_steps > c->n_rnd) {
        snprintf(err, errlen, "sampler: %d random numbers left, %d steps asked", c->n_rnd - c->used, n_steps); return -1;
    }
    // XJ_DECODE_GRAPH=0 enqueues the same kernels step by step instead of
    // replaying the captured graph (for tracing tools that do not follow graphs)
    const bool direct = env_int("XJ_DECODE_GRAPH", 1) == 0;
    if (!direct && !(smp ? c->exec_s : c->exec) && build_decode_graph(c, smp, err, errlen)) return -1;
    // With end tokens the steps run in windows, the recurrent state saved at
    // the start of each: when step j of a window yields an end token, the
    // window is replayed from the saved state for j + 1 steps only, so the
    // state is that of feeding exactly the tokens before the end token.
    const int window = has_end(hp) ? 32 : c->hist_cap;
    double total_ms = 0;
    int done = 0;
    while (done < n_steps) {
        const int n = n_steps - done < window ? n_steps - done : window;
        std::vector<int> past0;
        if (has_end(hp))
            for (auto *S : c->st) {
                past0.push_back(S->s.n_past);
                if (snapshot_enqueue(S, kDecodeSlot, c->stream, err, errlen)) return -1;
            }
        const int tok0 = c->last_tok;
        if (decode_enqueue(c, tok0, n, direct, smp, err, errlen) || chain_sync(c, err, errlen)) return -1;
        float ms = 0;
        (void)hipEventElapsedTime(&ms, c->ev0, c->ev1);
        total_ms += ms;
        if (hipMemcpy(out + done, c->d_hist, 4 * n, hipMemcpyDeviceToHost) != hipSuccess) { snprintf(err, errlen, "history copy failed"); return -1; }
        int ran = n;
        if (has_end(hp))
            for (int j = 0; j < n; j++)
                if (is_end(hp, out[done + j])) { ran = j + 1; break; }
        if (ran < n) {
            for (size_t i = 0; i < c->st.size(); i++)
                if (restore_enqueue(c->st[i], kDecodeSlot, past0[i], c->stream, err, errlen)) return -1;
            if (decode_enqueue(c, tok0, ran, direct, smp, err, errlen) || chain_sync(c, err, errlen)) return -1;
        }
        for (auto *S : c->st) S->s.n_past += ran;
        if (smp) c->used += ran;
        c->last_tok = out[done + ran - 1];
        done += ran;
        if (ran < n) break;
    }
    c->last_ms = total_ms / done;
    return done;
}

extern "C" int xjh_chain_last_token(xjh_chain *c) { return c->last_tok; }
extern "C" double xjh_chain_last_decode_ms(xjh_chain *c) { return c->last_ms; }
extern "C" int xjh_chain_n_past(xjh_chain *c) { return c->st[0]->s.n_past; }

extern "C" int xjh_chain_rollback(xjh_chain *c, int n_past, char *err, size_t errlen) {
    for (auto *S : c->st)
        if (S->s.rollback(&S->s, n_past, err, errlen)) return -1;
    return 0;
}

extern "C" void xjh_chain_reset(xjh_chain *c) {
    for (auto *S : c->st) S->s.reset(&S->s);
    c->last_tok = -1;
}

// one greedy step of the draft fed with token t; returns its argmax
static int draft_step(xjh_chain *d, int t, int *next, char *err, size_t errlen) {
    for (auto *S : d->st) {
        if (S->s.n_past + 1 > S->s.n_ctx) { snprintf(err, errlen, "context full (%d)", S->s.n_ctx); return -1; }
        if (reset_check(S, err, errlen)) return -1;
    }
    const bool direct = env_int("XJ_DECODE_GRAPH", 1) == 0;
    if (!direct && !d->exec && build_decode_graph(d, false, err, errlen)) return -1;
    if (decode_enqueue(d, t, 1, direct, false, err, errlen) ||
        hipMemcpyAsync(&d->h_buf[2], d->d_hist, 4, hipMemcpyDeviceToHost, d->stream) != hipSuccess ||
        chain_sync(d, err, errlen))
        return -1;
    for (auto *S : d->st) S->s.n_past += 1;
    *next = d->last_tok = d->h_buf[2];
    return 0;
}

// n greedy steps of the draft fed with token t, enqueued on its stream: one
// set-up, the decode graph replayed n times, after step j the recurrent state
// copied into snapshot slot slots[j] (< 0: none), the n argmax tokens copied
// to the host buffer; draft_collect waits for them.
static int draft_enqueue(xjh_chain *d, int t, int n, const int *slots, char *err, size_t errlen) {
    for (auto *S : d->st) {
        if (S->s.n_past + n > S->s.n_ctx) { snprintf(err, errlen, "context full (%d)", S->s.n_ctx); return -1; }
        if (reset_check(S, err, errlen)) return -1;
    }
    const bool direct = env_int("XJ_DECODE_GRAPH", 1) == 0;
    if (!direct && !d->exec && build_decode_graph(d, false, err, errlen)) return -1;
    d->h_buf[0] = 0;
    d->h_buf[1] = t;
    if (hipMemcpyAsync(d->d_step, &d->h_buf[0], 4, hipMemcpyHostToDevice, d->stream) != hipSuccess ||
        hipMemcpyAsync(d->d_tok, &d->h_buf[1], 4, hipMemcpyHostToDevice, d->stream) != hipSuccess) {
        snprintf(err, errlen, "draft setup failed"); return -1;
    }
    for (auto *S : d->st) if (set_npast(S, d->stream)) { snprintf(err, errlen, "draft setup failed"); return -1; }
    if (embed_first(d)) { snprintf(err, errlen, "draft setup failed"); return -1; }
    for (int j = 0; j < n; j++) {
        if (direct ? enqueue_decode_step(d, false) != 0 : hipGraphLaunch(d->exec, d->stream) != hipSuccess) {
            snprintf(err, errlen, "draft step launch failed"); return -1;
        }
        if (slots[j] >= 0)
            for (auto *S : d->st)
                if (snapshot_enqueue(S, slots[j], d->stream, err, errlen)) return -1;
    }
    if (hipMemcpyAsync(&d->h_buf[2], d->d_hist, 4 * n, hipMemcpyDeviceToHost, d->stream) != hipSuccess) {
        snprintf(err, errlen, "draft history copy failed"); return -1;
    }
    return 0;
}
static int draft_collect(xjh_chain *d, int n, int32_t *toks, char *err, size_t errlen) {
    if (chain_sync(d, err, errlen)) return -1;
    for (int j = 0; j < n; j++) toks[j] = d->h_buf[2 + j];
    for (auto *S : d->st) S->s.n_past += n;
    d->last_tok = toks[n - 1];
    return 0;
}

// kk greedy steps of the draft fed with token t, the state after step j in
// snapshot slot base + j (j < kk - 1; the last state is the draft's own), one
// synchronisation; toks receives the kk argmax tokens. catch_tok >= 0: a
// token the draft has not been fed yet, before t (the last draft of a fully
// accepted round): it and t go in as one two-token pass, whose rows are
// those of two steps bit for bit, instead of a step of their own.
static int draft_run(xjh_chain *d, int catch_tok, int t, int kk, int32_t *toks, int base, char *err, size_t errlen) {
    if (catch_tok >= 0 && d->mb < 2) {
        int nx;
        if (draft_step(d, catch_tok, &nx, err, errlen)) return -1;
        catch_tok = -1;
    }
    int done = 0;
    if (catch_tok >= 0) {
        const int32_t in2[2] = {catch_tok, t};
        int32_t am = -1;
        if (chain_eval(d, in2, 2, 1, 0, nullptr, &am, err, errlen)) return -1;
        if (kk > 1)
            for (auto *S : d->st)
                if (snapshot_enqueue(S, base, d->stream, err, errlen)) return -1;
        toks[0] = am;
        t = am;
        done = 1;
        if (kk == 1) {
            d->last_tok = am;
            return chain_sync(d, err, errlen);
        }
    }
    const int n = kk - done;
    int slots[8];
    for (int j = 0; j < n; j++) slots[j] = done + j < kk - 1 ? base + done + j : -1;   // the last state stays in place
    if (draft_enqueue(d, t, n, slots, err, errlen)) return -1;
    return draft_collect(d, n, toks + done, err, errlen);
}

extern "C" int xjh_spec_generate(xjh_chain *tgt, xjh_chain *dft, int k, int n_gen, const int32_t *oracle, int n_oracle,
                                 int oracle_miss, int32_t *out, xjh_spec_stats *stats, char *err, size_t errlen) {
    xjh_spec_stats st{};
    const xj_hparams &hp = tgt->st[0]->s.m->hp;
    const int V = (int)tgt->st.back()->output.n_rows;
    if (k < 1) k = 1;
    if (k > 4) k = 4;
    if (k + 1 > tgt->mb) k = tgt->mb - 1;
    if (tgt->last_tok < 0 || dft->st[0]->s.n_past != tgt->st[0]->s.n_past) {
        snprintf(err, errlen, "target and draft must have been fed the same prompt"); return -1;
    }
    (void)hipEventRecord(tgt->ev0, tgt->stream);
    auto now_ms = []() { timespec t; clock_gettime(CLOCK_MONOTONIC, &t); return t.tv_sec * 1e3 + t.tv_nsec * 1e-6; };
    const double t_start = now_ms();
    int produced = 0;
    long n_gen_tok = 0;
    int pending = tgt->last_tok;
    const bool smp = sampling(tgt);
    // Greedy rounds overlap after `need` rounds in a row whose drafts were all
    // accepted (2, doubled after each overlap that failed, back to 2 after one
    // that held): while
    // the target verifies round r, the draft goes on from round r's last
    // draft, one step for the target's next token and k for round r + 1
    // (XJ_SPEC_PIPE=0: never; the two models' launches share the CUs, so the
    // ahead steps slow a verification whose drafts then fail). When the target accepts
    // every draft and its next token is the draft's, round r + 1's drafts are
    // those and its verification starts at once; otherwise the draft returns
    // to a snapshot, as after a sequential round. Snapshot slots come in two
    // banks of four: slot base + j holds the state after the round's token j
    // (j = 3: taken before the draft runs ahead), and slot 3 of the other
    // bank the state after the round's last draft.
    static const bool pipe_env = env_int("XJ_SPEC_PIPE", 1) != 0;
    const bool pipe = pipe_env && !smp && k == 4;
    int base = 0;
    int catch_tok = -1;   // the last draft of a fully accepted round, not fed to the draft yet
    bool have_next = false;
    int full = 0, need = 2;   // rounds in a row whose drafts were all accepted
    int32_t next_toks[5];
    auto oracle_fill = [&](int32_t *toks, int kk) {   // oracle drafts stand in for the draft's
        for (int j = 1; j <= kk && oracle; j++) {
            const long gi = n_gen_tok + j;   // index of the generated token this draft stands for
            if (gi < n_oracle) toks[j] = oracle[gi];
            if (oracle_miss && (gi * 7 + j) % oracle_miss == 0) toks[j] = (toks[j] + 1) % V;
        }
    };
    while (produced < n_gen) {
        if (is_end(hp, pending)) { out[produced++] = pending; break; }   // returned, never fed (xj_spec.c:139)
        const int P = tgt->st[0]->s.n_past;
        int kk = k;
        if (kk > n_gen - produced - 1) kk = n_gen - produced - 1;
        for (auto *S : tgt->st) if (kk > S->s.n_ctx - P - 1) kk = S->s.n_ctx - P - 1;
        if (smp && kk > tgt->n_rnd - tgt->used - 1) kk = tgt->n_rnd - tgt->used - 1;   // numbers for kk + 1 draws
        if (have_next && kk != k) {   // cannot happen: the ahead drafts were only made with room for a full round
            snprintf(err, errlen, "speculation pipeline out of step"); return -1;
        }
        if (kk <= 0) {   // no room to speculate: plain step on both models (the target's token drawn)
            out[produced++] = pending;
            int32_t nt, dn;
            if (catch_tok >= 0 && xjh_chain_eval(dft, &catch_tok, 1, 1, 0, nullptr, &dn, err, errlen)) return -1;
            catch_tok = -1;
            if (xjh_chain_eval(tgt, &pending, 1, 1, 0, nullptr, &nt, err, errlen) ||
                xjh_chain_eval(dft, &pending, 1, 1, 0, nullptr, &dn, err, errlen)) return -1;
            pending = tgt->last_tok;
            n_gen_tok++;
            continue;
        }
        // 1) draft proposes kk tokens by greedy T=1 steps, snapshot after each
        //    (or they were made while the previous round was verified)
        const double t0 = now_ms();
        int32_t toks[5];
        toks[0] = pending;
        if (have_next) {
            for (int j = 1; j <= kk; j++) toks[j] = next_toks[j];
            have_next = false;
        } else {
            if (draft_run(dft, catch_tok, pending, kk, toks + 1, base, err, errlen)) return -1;
            catch_tok = -1;
        }
        st.t_draft_ms += now_ms() - t0;
        oracle_fill(toks, kk);
        // 2) verify [t, d1..dk] on the target in one batch with checkpoints;
        //    the target's token after each row: its argmax, or with the
        //    sampler on its draw (row i with number used + i, xj_spec.c:185)
        int32_t am[5];
        const int nb = base ^ 4;   // the other bank
        const long rest = (long)n_gen - produced - (kk + 1);
        bool ahead = pipe && full >= need && kk == k && rest - 1 >= k;
        for (auto *S : tgt->st) ahead = ahead && S->s.n_ctx - (P + kk + 1) - 1 >= k;
        for (auto *S : dft->st) ahead = ahead && S->s.n_past + 1 + k <= S->s.n_ctx;
        int32_t at[5];
        if (ahead) {
            if (chain_eval(tgt, toks, kk + 1, kk + 1, 1, nullptr, nullptr, err, errlen, false)) return -1;
            // the draft's state after toks[0..kk-1], then the draft fed round
            // r's last draft and its own tokens: the target's next token, then
            // round r + 1's drafts
            for (auto *S : dft->st)
                if (snapshot_enqueue(S, base + kk - 1, dft->stream, err, errlen)) return -1;
            const int slots[5] = {nb + 3, nb, nb + 1, nb + 2, -1};
            if (draft_enqueue(dft, toks[kk], k + 1, slots, err, errlen) ||
                chain_finish(tgt, kk + 1, am, err, errlen) || draft_collect(dft, k + 1, at, err, errlen))
                return -1;
        } else if (chain_eval(tgt, toks, kk + 1, kk + 1, 1, nullptr, am, err, errlen) ||
                   (smp && chain_draw(tgt, 0, kk + 1, am, err, errlen))) {
            return -1;
        }
        // 3) accept the longest agreeing prefix (xj_spec.c:184-191); an accepted
        //    end token is returned but neither it nor what follows is fed (:193-194)
        int a = 0;
        while (a < kk && am[a] == toks[a + 1]) { st.acc_at[a]++; a++; }
        full = a == kk ? full + 1 : 0;
        int fed = a + 1, n_out = a + 1;
        for (int i = 1; i <= a; i++)
            if (is_end(hp, toks[i])) { fed = i; n_out = i + 1; break; }
        if (smp) tgt->used += n_out > fed ? fed : a + 1;   // one number per token produced
        for (int i = 0; i < n_out && produced < n_gen; i++) out[produced++] = toks[i];
        const long gi_next = n_gen_tok + kk + 1;   // index of the target's token after a full round
        n_gen_tok += fed;
        st.n_steps++; st.n_drafted += kk; st.n_accepted += fed - 1 < a ? fed - 1 : a;
        if (fed < kk + 1 && xjh_chain_rollback(tgt, P + fed, err, errlen)) return -1;
        // 4) bring the draft to the same prefix [.., t, d1..d(fed-1)]: slot base + j
        //    holds its state after feeding toks[0..j]
        if (ahead) {
            // the guess of the target's next token (with oracle drafts the
            // oracle's, as the draft's own stand in for nothing)
            const int32_t guess = oracle && gi_next < n_oracle ? oracle[gi_next] : at[0];
            need = fed == kk + 1 && am[kk] == guess ? 2 : (need < 64 ? 2 * need : need);
            st.n_overlap++;
            if (fed == kk + 1 && n_out == fed && am[kk] == guess) {
                for (int j = 1; j <= k; j++) next_toks[j] = at[j];
                have_next = true;
                base = nb;
                st.n_overlap_held++;
            } else if (fed == kk + 1) {
                // every draft accepted, the next token not the guess: the draft
                // back to its state after round r's last draft
                for (auto *S : dft->st)
                    if (xj_hip_stage_restore(&S->s, nb + 3, P + kk + 1, err, errlen)) return -1;
            } else {
                for (auto *S : dft->st)
                    if (xj_hip_stage_restore(&S->s, base + fed - 1, P + fed, err, errlen)) return -1;
            }
        } else if (fed < kk) {
            for (auto *S : dft->st)
                if (xj_hip_stage_restore(&S->s, base + fed - 1, P + fed, err, errlen)) return -1;
        } else if (fed == kk) {
            // the draft already holds the state after toks[0..kk-1] at n_past P + kk
        } else {
            catch_tok = toks[kk];   // fed with the next round's first token
        }
        if (n_out > fed) { pending = toks[fed]; break; }   // stopped at an accepted end token
        pending = am[a];
        tgt->last_tok = pending;
    }
    if (have_next) {   // the draft ran ahead of the last round: back to the target's prefix
        const int P = tgt->st[0]->s.n_past;
        for (auto *S : dft->st)
            if (xj_hip_stage_restore(&S->s, base + 3, P, err, errlen)) return -1;
    }
    if (catch_tok >= 0) {   // the draft ends fed with the target's prefix, as each round leaves it
        int nx;
        if (draft_step(dft, catch_tok, &nx, err, errlen)) return -1;
    }
    (void)hipEventRecord(tgt->ev1, tgt->stream);
    st.t_total_ms = now_ms() - t_start;
    if (stats) *stats = st;
    tgt->last_tok = pending;
    return produced;
}

// ------------------------------------------------------------ MTP drafting --

namespace {
struct MtpRun {
    HStage *S;                 // the MTP stage
    xjh_chain *c;              // the target chain (its embedding table)
    int32_t *d_ids = nullptr;  // token ids of the rows being built
    int32_t *d_am = nullptr;   // argmax of the MTP head
    float *d_hn = nullptr;     // output_norm of the target's hidden rows [mb][E]
    bool main_post = true;     // hidden rows pass the target's output_norm (XJ_MTP_MAIN_POST)
    bool chain_post = true;    // an MTP output passes shared_head_norm before it is fed back (XJ_MTP_CHAIN_POST)
    int last_row = 0;          // row of S->x holding the last MTP output
    std::vector<float> ph;     // pending positions: main-model hidden rows [n][E]
    std::vector<int32_t> pt;   // and the token after each (-1: not known yet)
};

// rows [embedding(ids[t]) | hid row t] into S->mx (hid may be null: the
// caller fills the second half)
int mtp_rows(MtpRun &R, const int32_t *ids, const float *hid, int T, char *err, size_t errlen) {
    HStage *S = R.S;
    const int E = S->s.m->hp.n_embd;
    EmbedArgs ea{R.d_ids, R.c->st[0]->tok_embd, S->mh, T};
    if (hipMemcpy(R.d_ids, ids, 4 * T, hipMemcpyHostToDevice) != hipSuccess || embed_launch(ea, S->st) ||
        hipMemcpy2DAsync(S->mx, 8 * E, S->mh, 4 * E, 4 * E, T, hipMemcpyDeviceToDevice, S->st) != hipSuccess ||
        (hid && hipMemcpy2DAsync(S->mx + E, 8 * E, hid, 4 * E, 4 * E, T, hipMemcpyHostToDevice, S->st) != hipSuccess) ||
        sync_check(S, err, errlen)) {
        if (!err[0]) snprintf(err, errlen, "MTP row setup failed");
        return -1;
    }
    return 0;
}

// MTP forward over the T rows in S->mx (xj_cpu.c:253-261, then the layer);
// want: the greedy token after the last row through the shared head
int mtp_forward(MtpRun &R, int T, bool want, int32_t *tok, char *err, size_t errlen) {
    HStage *S = R.S;
    const xj_hparams &hp = S->s.m->hp;
    const int E = hp.n_embd;
    int keep_n = 0;
    if (begin_forward(S, T, &keep_n, err, errlen)) return -1;
    Gemv g(S->xq_2e);
    g.a.x = S->mh; g.a.xs = 2 * E; g.a.pro = PRO_NONE;
    g.seg(S->mtp_eh, S->x, E, EPI_STORE);
    if (norm_rows_launch(0, S->mx, 2 * E, S->mtp_enorm, E, T, hp.eps, S->mh, 2 * E, S->st) ||
        norm_rows_launch(0, S->mx + E, 2 * E, S->mtp_hnorm, E, T, hp.eps, S->mh + E, 2 * E, S->st) ||
        g.run(T, S->st) || set_npast(S, S->st) || enqueue_layers(S, S->x, T, keep_n, false, S->st) ||
        (want && (enqueue_head(S, S->x + (int64_t)(T - 1) * E, 1, S->logits, S->st) ||
                  argmax_finalize_launch(S->amax, S->head_nwg, 1, R.d_am, nullptr, nullptr, nullptr, S->st)))) {
        snprintf(err, errlen, "MTP launch failed");
        return -1;
    }
    if (sync_check(S, err, errlen)) return -1;
    if (want && hipMemcpy(tok, R.d_am, 4, hipMemcpyDeviceToHost) != hipSuccess) { snprintf(err, errlen, "MTP argmax copy failed"); return -1; }
    S->s.n_past += T;
    R.last_row = T - 1;
    return 0;
}

// the MTP stage takes the first n pending positions (their next tokens known)
// in batches; want: the greedy token after the last (xj_spec.c:97-116)
int mtp_flush(MtpRun &R, int n, bool want, int32_t *tok, char *err, size_t errlen) {
    const int E = R.S->s.m->hp.n_embd, B = R.S->s.max_batch;
    for (int i = 0; i < n; i += B) {
        const int T = n - i < B ? n - i : B;
        if (mtp_rows(R, R.pt.data() + i, R.ph.data() + (size_t)i * E, T, err, errlen) ||
            mtp_forward(R, T, want && i + T == n, tok, err, errlen))
            return -1;
    }
    R.ph.erase(R.ph.begin(), R.ph.begin() + (size_t)n * E);
    R.pt.erase(R.pt.begin(), R.pt.begin() + n);
    return 0;
}

// the first `rows` hidden rows of the target's last evaluation become
// pending, normalised with the target's output_norm as the reference driver
// does by default (push_ph, xj_spec.c:50-58)
int push_hidden(MtpRun &R, int rows, char *err, size_t errlen) {
    const xj_hparams &hp = R.S->s.m->hp;
    const int E = hp.n_embd;
    const size_t n0 = R.ph.size();
    R.ph.resize(n0 + (size_t)rows * E);
    hipStream_t st = R.c->stream;
    const float *src = R.c->x;
    if (R.main_post) {
        if (norm_rows_launch(2, R.c->x, E, R.c->st.back()->out_norm, E, rows, hp.eps, R.d_hn, E, st)) {
            snprintf(err, errlen, "hidden norm launch failed"); return -1;
        }
        src = R.d_hn;
    }
    if (hipMemcpyAsync(R.ph.data() + n0, src, sizeof(float) * rows * E, hipMemcpyDeviceToHost, st) != hipSuccess ||
        chain_sync(R.c, err, errlen)) {
        if (!err[0]) snprintf(err, errlen, "hidden copy failed");
        return -1;
    }
    return 0;
}
}  // namespace

extern "C" int xjh_spec_generate_mtp(xjh_chain *tgt, xj_stage *mtp, int k, const int32_t *prompt, int n_prompt, int n_gen,
                                     const int32_t *oracle, int n_oracle, int oracle_miss, int32_t *out,
                                     xjh_spec_stats *stats, int32_t *draft_log, int draft_cap, char *err, size_t errlen) {
    err[0] = 0;
    if (!mtp || !mtp->mtp || strcmp(mtp->backend, "hip") != 0 || mtp->m != tgt->st[0]->s.m || !mtp->has_head) {
        snprintf(err, errlen, "an MTP stage of the target's model (HIP, with its head) is required"); return -1;
    }
    if (n_prompt < 1 || n_gen < 1) { snprintf(err, errlen, "empty prompt or generation"); return -1; }
    MtpRun R;
    R.S = H(mtp);
    R.c = tgt;
    const xj_hparams &hp = R.S->s.m->hp;
    const int E = hp.n_embd, V = (int)tgt->st.back()->output.n_rows, B = tgt->mb;
    R.main_post = env_int("XJ_MTP_MAIN_POST", 1) != 0;
    R.chain_post = env_int("XJ_MTP_CHAIN_POST", 1) != 0;
    if (k < 1) k = 1;
    if (k > 4) k = 4;
    if (k + 1 > B) k = B - 1;
    if (k > R.S->s.max_batch) k = R.S->s.max_batch;
    if (hipMalloc(&R.d_ids, 4 * (size_t)R.S->s.max_batch) != hipSuccess || hipMalloc(&R.d_am, 4) != hipSuccess ||
        hipMalloc(&R.d_hn, sizeof(float) * (size_t)B * E) != hipSuccess) {
        snprintf(err, errlen, "hipMalloc failed");
        (void)hipFree(R.d_ids); (void)hipFree(R.d_am);
        return -1;
    }
    auto done = [&](int rc) { (void)hipFree(R.d_ids); (void)hipFree(R.d_am); (void)hipFree(R.d_hn); return rc; };
    int n_log = 0;
    auto log_draft = [&](int32_t d) { if (draft_log && n_log < draft_cap) draft_log[n_log++] = d; };
    xjh_spec_stats st{};
    auto now_ms = []() { timespec ts; clock_gettime(CLOCK_MONOTONIC, &ts); return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6; };
    xjh_chain_reset(tgt);
    mtp->reset(mtp);
    // the prompt (xj_spec.c:117-129): the target in batches, every position
    // pending for the MTP stage with the token after it, all but the last taken now
    int32_t t = -1;
    for (int i = 0; i < n_prompt; i += B) {
        const int T = n_prompt - i < B ? n_prompt - i : B;
        int32_t am = -1;
        if (xjh_chain_eval(tgt, prompt + i, T, i + T == n_prompt ? 1 : 0, 0, nullptr, &am, err, errlen) ||
            push_hidden(R, T, err, errlen))
            return done(-1);
        for (int j = 0; j < T; j++) R.pt.push_back(i + j + 1 < n_prompt ? prompt[i + j + 1] : -1);
        if (i + T == n_prompt) t = tgt->last_tok;   // the argmax, or the sampler's draw
    }
    const double t_start = now_ms();
    if ((int)R.pt.size() > 1 && mtp_flush(R, (int)R.pt.size() - 1, false, nullptr, err, errlen)) return done(-1);
    int produced = 0;
    const bool smp = sampling(tgt);
    while (produced < n_gen) {
        out[produced++] = t;   // t: the token after everything fed so far (xj_spec.c:135-140)
        if (produced == n_gen || is_end(hp, t)) break;   // an end token is returned, never fed
        const int P = tgt->st[0]->s.n_past;
        R.pt.back() = t;
        int kk = k;
        if (kk > n_gen - produced) kk = n_gen - produced;
        for (auto *S : tgt->st) if (kk > S->s.n_ctx - P - 1) kk = S->s.n_ctx - P - 1;
        const int mroom = R.S->s.n_ctx - R.S->s.n_past - (int)R.pt.size() - 1;
        if (kk > mroom) kk = mroom;
        if (smp && kk > tgt->n_rnd - tgt->used - 1) kk = tgt->n_rnd - tgt->used - 1;   // numbers for kk + 1 draws
        if (kk <= 0) {   // no room to speculate: feed t alone (xj_spec.c:145-152)
            int32_t am = -1;
            if (xjh_chain_eval(tgt, &t, 1, 1, 0, nullptr, &am, err, errlen) || push_hidden(R, 1, err, errlen)) return done(-1);
            R.pt.push_back(-1);
            t = tgt->last_tok;
            continue;
        }
        // 1) the MTP stage drafts kk tokens (xj_spec.c:154-171): the pending
        //    positions give draft 1; each further draft comes from the row
        //    [embedding(previous draft) | shared_head_norm(previous MTP output)]
        const double t0 = now_ms();
        int32_t toks[5];
        toks[0] = t;
        const int mtp_pos = R.S->s.n_past + (int)R.pt.size();
        if (mtp_flush(R, (int)R.pt.size(), true, &toks[1], err, errlen)) return done(-1);
        log_draft(toks[1]);
        for (int j = 2; j <= kk; j++) {
            const int32_t id = toks[j - 1];
            const float *prev = R.S->x + (int64_t)R.last_row * E;
            if (mtp_rows(R, &id, nullptr, 1, err, errlen) ||
                (R.chain_post ? norm_rows_launch(2, prev, E, R.S->out_norm, E, 1, hp.eps, R.S->mx + E, 2 * E, R.S->st)
                              : hipMemcpyAsync(R.S->mx + E, prev, 4 * E, hipMemcpyDeviceToDevice, R.S->st) != hipSuccess) ||
                mtp_forward(R, 1, true, &toks[j], err, errlen))
                return done(-1);
            log_draft(toks[j]);
        }
        if (mtp->rollback(mtp, mtp_pos, err, errlen)) return done(-1);
        st.t_draft_ms += now_ms() - t0;
        for (int j = 1; j <= kk && oracle; j++) {   // the driver's test mode (xj_spec.c:173-177)
            const long gi = produced - 1 + j;
            if (gi < n_oracle) toks[j] = oracle[gi];
            if (oracle_miss && (gi * 7 + j) % oracle_miss == 0) toks[j] = (toks[j] + 1) % V;
        }
        // 2) verify [t, d1..dk] in one batch with checkpoints; 3) accept the
        //    agreeing prefix; an accepted end token is returned, and neither it
        //    nor what follows is fed (xj_spec.c:179-201)
        //    (the target's token after each row: its argmax, or the sampler's
        //    draw, row i with number used + i, xj_spec.c:185)
        int32_t am[5];
        if (chain_eval(tgt, toks, kk + 1, kk + 1, 1, nullptr, am, err, errlen) ||
            (smp && chain_draw(tgt, 0, kk + 1, am, err, errlen))) return done(-1);
        int a = 0;
        while (a < kk && am[a] == toks[a + 1]) { st.acc_at[a]++; a++; }
        int fed = a + 1, n_out = a + 1;
        for (int i = 1; i <= a; i++)
            if (is_end(hp, toks[i])) { fed = i; n_out = i + 1; break; }
        if (smp) tgt->used += n_out > fed ? fed : a + 1;   // one number per token produced
        for (int i = 1; i < n_out && produced < n_gen; i++) out[produced++] = toks[i];
        st.n_steps++; st.n_drafted += kk; st.n_accepted += fed - 1 < a ? fed - 1 : a;
        // 4) the fed positions become pending for the MTP stage (xj_spec.c:204-207)
        if (push_hidden(R, fed, err, errlen)) return done(-1);
        for (int i = 1; i < fed; i++) R.pt.push_back(toks[i]);
        R.pt.push_back(-1);
        if (fed < kk + 1 && xjh_chain_rollback(tgt, P + fed, err, errlen)) return done(-1);
        if (n_out > fed) { t = toks[fed]; break; }   // stopped at an accepted end token
        t = am[a];
    }
    tgt->last_tok = t;
    st.t_total_ms = now_ms() - t_start;
    if (stats) *stats = st;
    return done(produced);
}

extern "C" int xjh_chain_time_gemv(xjh_chain *c, int iters, double *ms_per_step, double *bytes_per_step,
                                   int *launches_per_step, char *err, size_t errlen) {
    if (iters < 1) iters = 1;
    Profile pf;
    HStage *head = c->st.back();
    pf.sink = head->logits;   // [max_batch][n_vocab] floats: larger than any GEMV output
    auto enqueue_step = [&](Profile *p) -> int {
        for (auto *S : c->st)
            if (enqueue_layers(S, c->x, 1, 0, false, c->stream, p)) return -1;
        return enqueue_head(head, c->x, 1, head->logits, c->stream, p);
    };
    if (enqueue_step(&pf)) { snprintf(err, errlen, "profile launch failed"); return -1; }   // warm-up, counts bytes
    if (chain_sync(c, err, errlen)) return -1;
    const double bytes = pf.bytes;
    const int launches = pf.launches;
    (void)hipEventRecord(c->ev0, c->stream);
    for (int i = 0; i < iters; i++) {
        Profile q;
        q.sink = pf.sink;
        if (enqueue_step(&q)) { snprintf(err, errlen, "profile launch failed"); return -1; }
    }
    (void)hipEventRecord(c->ev1, c->stream);
    if (chain_sync(c, err, errlen)) return -1;
    float ms = 0;
    (void)hipEventElapsedTime(&ms, c->ev0, c->ev1);
    *ms_per_step = ms / iters;
    *bytes_per_step = bytes;
    *launches_per_step = launches;
    return 0;
}

// ======================================================= per-op entries ==

namespace {
hipStream_t g_stream = nullptr;

hipStream_t ops_stream() {
    if (!g_stream) {
        if (hipStreamCreateWithFlags(&g_stream, hipStreamNonBlocking) != hipSuccess) return nullptr;
        char err[128];
        gemv_init(err, sizeof err);
    }
    return g_stream;
}

int ops_done(char *err, size_t errlen) {
    hipError_t e = hipStreamSynchronize(g_stream);
    if (e == hipSuccess) e = hipGetLastError();
    if (e != hipSuccess) { snprintf(err, errlen, "GPU error: %s", hipGetErrorString(e)); return -1; }
    return 0;
}
}  // namespace

extern "C" void *xjh_malloc(size_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) { snprintf(g_lasterr, sizeof g_lasterr, "hipMalloc(%zu) failed", bytes); return nullptr; }
    return p;
}
extern "C" void xjh_free(void *p) { if (p) (void)hipFree(p); }
extern "C" int xjh_h2d(void *dst, const void *src, size_t n) { return hipMemcpy(dst, src, n, hipMemcpyHostToDevice) == hipSuccess ? 0 : -1; }
extern "C" int xjh_d2h(void *dst, const void *src, size_t n) { return hipMemcpy(dst, src, n, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1; }
extern "C" int xjh_d2d(void *dst, const void *src, size_t n) { return hipMemcpy(dst, src, n, hipMemcpyDeviceToDevice) == hipSuccess ? 0 : -1; }
extern "C" int xjh_sync(void) { return hipDeviceSynchronize() == hipSuccess ? 0 : -1; }
extern "C" const char *xjh_last_error(void) { return g_lasterr; }

extern "C" void *xjh_upload_weight(uint32_t type, const void *host, int64_t n_rows, int64_t k, char *err, size_t errlen) {
    if (!ops_stream()) { snprintf(err, errlen, "no HIP stream"); return nullptr; }
    if (!gemv_type_ok(type)) { snprintf(err, errlen, "type %s has no device layout", xjh_type_name(type)); return nullptr; }
    const uint64_t bytes = xjh_row_bytes(type, k) * (uint64_t)n_rows;
    void *p = nullptr;
    if (hipMalloc(&p, bytes + kWeightPad) != hipSuccess) { snprintf(err, errlen, "hipMalloc failed"); return nullptr; }
    if (upload_repack(type, host, n_rows, k, (uint8_t *)p, g_stream, err, errlen)) { (void)hipFree(p); return nullptr; }
    return p;
}

extern "C" int xjh_dequant(uint32_t type, const void *dw, int64_t n_rows, int64_t k, int64_t r0, int64_t n, float *y,
                           char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if (r0 < 0 || n < 0 || r0 + n > n_rows || k % 32) { snprintf(err, errlen, "bad dequant range"); return -1; }
    DevW w;
    w.p = (const uint8_t *)dw; w.type = type; w.n_rows = n_rows; w.k = k;
    if (dequant_launch(w, r0, n, y, g_stream)) { snprintf(err, errlen, "dequant launch failed"); return -1; }
    return ops_done(err, errlen);
}

// The per-op GEMV on `st`. Its prepared activations (T tokens of
// xq_off(k).stride bytes) go to xq_given when it is not null, otherwise to a
// library buffer grown on demand (the per-op entries are synchronous on one stream).
static int gemv_enqueue(uint32_t type, const void *dw, int64_t n_rows, int64_t k, const float *x, int T, float *y, int add,
                        hipStream_t st, uint8_t *xq_given = nullptr) {
    DevW w;
    w.p = (const uint8_t *)dw; w.type = type; w.n_rows = n_rows; w.k = k;
    static uint8_t *xq_own = nullptr;
    static size_t xq_cap = 0;
    uint8_t *xq = xq_given;
    if (!xq) {
        const size_t need = (size_t)T * xq_off((int)k).stride;
        if (need > xq_cap) {
            if (xq_own) (void)hipFree(xq_own);
            xq_own = nullptr;
            xq_cap = 0;
            if (hipMalloc(&xq_own, need) != hipSuccess) return -1;
            xq_cap = need;
        }
        xq = xq_own;
    }
    Gemv g(xq);
    g.a.x = x; g.a.xs = (int32_t)k; g.a.pro = PRO_NONE;
    // quantized rows, one or two tokens: the GEMV's work-groups build the
    // activations from x (no prep launch); float rows read a prep launch's v,
    // and from three tokens on one prep launch is cheaper than every
    // work-group converting all of them (2560 x 9216 Q6_K, T = 3: 17.6 vs 38 us)
    static const bool inwg = getenv("XJ_GEMV_OP_INWG") == nullptr || atoi(getenv("XJ_GEMV_OP_INWG")) != 0;
    if (inwg && T <= 2 && type != XJ_F32 && type != XJ_F16 && type != XJ_BF16 && !((uintptr_t)x & 15) && k % 4 == 0)
        g.a.pro = PRO_X;
    g.seg(w, y, (int32_t)n_rows, add ? EPI_ADD : EPI_STORE);
    return g.run(T, st);
}

static bool gemv_shape_ok(uint32_t type, int64_t n_rows, int64_t k, int T) {
    return gemv_type_ok(type) && T >= 1 && n_rows >= 1 && k >= 32 && k % 32 == 0 && k <= INT32_MAX / 8 &&
           !((type == XJ_Q4_K || type == XJ_Q6_K || type == XJ_Q5_K) && k % 256);
}

extern "C" int xjh_gemv(uint32_t type, const void *dw, int64_t n_rows, int64_t k, const float *x, int T, float *y, int add,
                        char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if (!gemv_shape_ok(type, n_rows, k, T)) { snprintf(err, errlen, "unsupported GEMV shape/type"); return -1; }
    if (gemv_enqueue(type, dw, n_rows, k, x, T, y, add, g_stream)) { snprintf(err, errlen, "GEMV launch failed"); return -1; }
    return ops_done(err, errlen);
}

// Scratch of xjh_gemv_noalloc: the prepared activations of one call. Each GPU
// holds its own copy of this array from the library's load to the process's
// end; host code reaches it only through the per-device address taken with
// hipGetSymbolAddress (the array's name is not a device address on the host).
constexpr size_t kNoAllocScratchBytes = size_t(1) << 20;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
uint8_t *g_scratch_dev[kMaxDevices];   // device address of `scratch` on each device, set once
std::mutex g_scratch_mu;

// The current device's address of `scratch`, looked up on the first call on that device.
uint8_t *scratch_address(char *err, size_t errlen) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        snprintf(err, errlen, "no usable HIP device (%d)", dev);
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_dev[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            snprintf(err, errlen, "scratch address lookup failed: %s", hipGetErrorString(e));
            return nullptr;
        }
        g_scratch_dev[dev] = (uint8_t *)p;
    }
    return g_scratch_dev[dev];
}
}  // namespace

extern "C" int xjh_gemv_noalloc(uint32_t type, const void *dw, int64_t n_rows, int64_t k, const float *x, int T, float *y,
                                int add, char *err, size_t errlen) {
    if (!gemv_shape_ok(type, n_rows, k, T)) { snprintf(err, errlen, "unsupported GEMV shape/type"); return -1; }
    const size_t need = (size_t)T * (size_t)xq_off((int)k).stride;
    if (need > kNoAllocScratchBytes) {
        snprintf(err, errlen, "xjh_gemv_noalloc: %d tokens of %lld inputs need %zu scratch bytes, above its %zu-byte maximum",
                 T, (long long)k, need, kNoAllocScratchBytes);
        return -1;
    }
    if (!ops_stream()) { snprintf(err, errlen, "no HIP stream"); return -1; }
    uint8_t *xq = scratch_address(err, errlen);
    if (!xq) return -1;
    if (gemv_enqueue(type, dw, n_rows, k, x, T, y, add, g_stream, xq)) { snprintf(err, errlen, "GEMV launch failed"); return -1; }
    return ops_done(err, errlen);
}

// Prepared activations of T tokens (prep launch) and the matrix-core GEMM.
static int gemm_enqueue(uint32_t type, const void *dw, int64_t n_rows, int64_t k, const float *x, int T, float *y, int add,
                        hipStream_t st) {
    static uint8_t *xq = nullptr, *hq = nullptr;   // grown on demand; the per-op entries are synchronous on one stream
    static float *part = nullptr;
    static int32_t *cnt = nullptr;
    static size_t xq_cap = 0, hq_cap = 0, part_cap = 0, cnt_cap = 0;
    const int64_t xs = xq_off((int)k).stride, hs = hq_stride((int)k);
    const size_t need = (size_t)T * xs, hneed = (size_t)T * hs, pneed = (size_t)gemm_part_floats(n_rows, T),
                 cneed = (size_t)gemm_counters(n_rows);
    if (need > xq_cap) {
        if (xq) (void)hipFree(xq);
        xq = nullptr, xq_cap = 0;
        if (hipMalloc(&xq, need) != hipSuccess) return -1;
        xq_cap = need;
    }
    if (hneed > hq_cap) {
        if (hq) (void)hipFree(hq);
        hq = nullptr, hq_cap = 0;
        if (hipMalloc(&hq, hneed) != hipSuccess) return -1;
        hq_cap = hneed;
    }
    if (pneed > part_cap) {
        if (part) (void)hipFree(part);
        part = nullptr, part_cap = 0;
        if (hipMalloc(&part, pneed * 4) != hipSuccess) return -1;
        part_cap = pneed;
    }
    if (cneed > cnt_cap) {   // zero once; the kernel leaves them zero
        if (cnt) (void)hipFree(cnt);
        cnt = nullptr, cnt_cap = 0;
        if (hipMalloc(&cnt, cneed * 4) != hipSuccess || hipMemsetAsync(cnt, 0, cneed * 4, st) != hipSuccess) return -1;
        cnt_cap = cneed;
    }
    GArgs p{};
    p.x = x; p.xs = (int32_t)k; p.pro = PRO_NONE; p.xq = xq; p.K = (int32_t)k; p.T = T; p.hq = hq;
    if (prep_launch(p, st)) return -1;
    GemmArgs g{};
    g.type = type; g.K = (int32_t)k; g.T = T; g.hq = hq; g.hs = hs; g.part = part; g.cnt = cnt;
    g.nseg = 1;
    g.seg[0] = GemmSeg{(const uint8_t *)dw, (int32_t)n_rows, y, (int32_t)n_rows, add};
    return gemm_launch(g, (int64_t)part_cap, (int)cnt_cap, st);
}

extern "C" int xjh_gemm(uint32_t type, const void *dw, int64_t n_rows, int64_t k, const float *x, int T, float *y, int add,
                        char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if ((type != XJ_Q4_K && type != XJ_Q6_K) || T < 1 || T > gemm_max_tokens() || n_rows < 1 || n_rows > INT32_MAX ||
        k < 256 || k % 256) {
        snprintf(err, errlen, "unsupported GEMM shape/type (Q4_K or Q6_K, K %% 256 == 0, 1 <= T <= %d)", gemm_max_tokens());
        return -1;
    }
    if (gemm_enqueue(type, dw, n_rows, k, x, T, y, add, g_stream)) { snprintf(err, errlen, "GEMM launch failed"); return -1; }
    return ops_done(err, errlen);
}

extern "C" double xjh_gemm_time(uint32_t type, void *const *dws, int n_copies, int64_t n_rows, int64_t k, const float *x,
                                int T, float *y, int iters, char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if ((type != XJ_Q4_K && type != XJ_Q6_K) || T < 1 || T > gemm_max_tokens() || k < 256 || k % 256) {
        snprintf(err, errlen, "unsupported GEMM shape/type"); return -1;
    }
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) { snprintf(err, errlen, "event creation failed"); return -1; }
    for (int i = 0; i < n_copies; i++)
        if (gemm_enqueue(type, dws[i], n_rows, k, x, T, y, 0, g_stream)) { snprintf(err, errlen, "GEMM launch failed"); return -1; }
    (void)hipEventRecord(e0, g_stream);
    for (int i = 0; i < iters; i++)
        if (gemm_enqueue(type, dws[i % n_copies], n_rows, k, x, T, y, 0, g_stream)) { snprintf(err, errlen, "GEMM launch failed"); return -1; }
    (void)hipEventRecord(e1, g_stream);
    if (ops_done(err, errlen)) return -1;
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return (double)ms / iters;
}

extern "C" double xjh_gemv_time(uint32_t type, void *const *dws, int n_copies, int64_t n_rows, int64_t k, const float *x,
                                int T, float *y, int iters, char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) { snprintf(err, errlen, "event creation failed"); return -1; }
    for (int i = 0; i < n_copies; i++)   // warm-up pass over every copy
        if (gemv_enqueue(type, dws[i], n_rows, k, x, T, y, 0, g_stream)) { snprintf(err, errlen, "GEMV launch failed"); return -1; }
    (void)hipEventRecord(e0, g_stream);
    for (int i = 0; i < iters; i++)
        if (gemv_enqueue(type, dws[i % n_copies], n_rows, k, x, T, y, 0, g_stream)) { snprintf(err, errlen, "GEMV launch failed"); return -1; }
    (void)hipEventRecord(e1, g_stream);
    if (ops_done(err, errlen)) return -1;
    float ms = 0;
    (void)hipEventElapsedTime(&ms, e0, e1);
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return (double)ms / iters;
}

extern "C" int xjh_norm(int mode, const float *x, const float *w, int n, int rows, float eps, float *out, char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if (norm_launch(mode, x, w, n, rows, eps, out, g_stream)) { snprintf(err, errlen, "norm launch failed"); return -1; }
    return ops_done(err, errlen);
}

extern "C" int xjh_swiglu(float *g, const float *u, int64_t n, char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if (swiglu_launch(g, u, n, g_stream)) { snprintf(err, errlen, "swiglu launch failed (n = %lld)", (long long)n); return -1; }
    return ops_done(err, errlen);
}

extern "C" int xjh_rope(float *x, int T, int n_heads, int64_t tok_stride, int64_t head_stride, int n_rot, int pos0,
                        float base, char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if (T < 0 || n_heads < 0 || n_rot < 2 || n_rot % 2 || pos0 < 0 || head_stride < n_rot) {
        snprintf(err, errlen, "rope: bad shape (T=%d, heads=%d, n_rot=%d, pos0=%d)", T, n_heads, n_rot, pos0);
        return -1;
    }
    if (!T || !n_heads) return 0;
    const int half = n_rot / 2;
    std::vector<float2> cs((size_t)T * half);
    rope_table(pos0, T, n_rot, base, cs.data());
    float2 *d = nullptr;
    if (hipMalloc(&d, cs.size() * sizeof(float2)) != hipSuccess) { snprintf(err, errlen, "hipMalloc failed"); return -1; }
    int rc = 0;
    if (hipMemcpy(d, cs.data(), cs.size() * sizeof(float2), hipMemcpyHostToDevice) != hipSuccess ||
        rope_launch(x, d, T, n_heads, tok_stride, head_stride, n_rot, g_stream)) {
        snprintf(err, errlen, "rope launch failed");
        rc = -1;
    } else {
        rc = ops_done(err, errlen);
    }
    (void)hipFree(d);
    return rc;
}

extern "C" int xjh_conv_silu(float *x, float *state, const float *w, int C, int K, int T, float *ck, int ck_n,
                             char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if (conv_silu_launch(x, state, w, C, K, T, ck, ck_n, g_stream)) {
        snprintf(err, errlen, "conv_silu: bad shape (C=%d, K=%d (2..8), T=%d, ck_n=%d)", C, K, T, ck_n);
        return -1;
    }
    return ops_done(err, errlen);
}

extern "C" int xjh_attn_decode(int T, int H, int Hkv, int D, int n_rot, float rope_base, float eps, int n_past, int n_ctx,
                               const float *qg, const float *k, const float *v, const float *q_norm, const float *k_norm,
                               uint16_t *kc, uint16_t *vc, float *out, char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    const int G = Hkv > 0 ? H / Hkv : 0;
    if (T < 1 || Hkv < 1 || H % Hkv || (G != 1 && G != 2 && G != 4 && G != 8) || (D != 64 && D != 128 && D != 256) ||
        n_rot < 0 || n_rot % 2 || n_rot > D || n_past < 0 || n_past + T > n_ctx || ((uintptr_t)kc | (uintptr_t)vc) & 15) {
        snprintf(err, errlen, "attn_decode: bad shape or unaligned cache (T=%d H=%d Hkv=%d D=%d n_rot=%d n_past=%d n_ctx=%d)",
                 T, H, Hkv, D, n_rot, n_past, n_ctx);
        return -1;
    }
    const int half = n_rot / 2 > 0 ? n_rot / 2 : 1;
    std::vector<float2> cs((size_t)n_ctx * half, float2{1.f, 0.f});
    rope_table(0, n_ctx, n_rot, rope_base, cs.data());
    AttnArgs at{};
    at.n_split = attn_splits(n_ctx);
    // every region 256-byte aligned (the split kernel reads qr with 16-byte loads)
    const size_t b_rope = (cs.size() * sizeof(float2) + 255) & ~(size_t)255, b_qr = ((size_t)T * H * D * 4 + 255) & ~(size_t)255,
                 b_sc = (size_t)T * H * at.n_split * (D + 2) * 4;
    uint8_t *buf = nullptr;
    if (hipMalloc(&buf, 256 + b_rope + b_qr + b_sc) != hipSuccess) { snprintf(err, errlen, "hipMalloc failed"); return -1; }
    int32_t *np = (int32_t *)buf;
    float2 *rope = (float2 *)(buf + 256);
    int rc = 0;
    if (hipMemcpy(np, &n_past, 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(rope, cs.data(), cs.size() * sizeof(float2), hipMemcpyHostToDevice) != hipSuccess) {
        snprintf(err, errlen, "attn_decode: copy failed");
        rc = -1;
    }
    if (!rc) {
        at.qg = qg; at.qg_s = 2 * H * D;
        at.kn = k; at.kn_s = Hkv * D;
        at.vn = v; at.vn_s = Hkv * D;
        at.kc = kc; at.vc = vc; at.qnorm_w = q_norm; at.knorm_w = k_norm; at.rope = rope; at.npast = np;
        at.qr = (float *)(buf + 256 + b_rope);
        at.scores = (float *)(buf + 256 + b_rope + b_qr);
        at.out = out;
        at.T = T; at.H = H; at.Hkv = Hkv; at.D = D; at.n_rot = n_rot; at.n_ctx = n_ctx;
        at.eps = eps; at.scale = 1.0f / sqrtf((float)D);
        at.xq = nullptr;
        if (attn_launch(at, g_stream)) { snprintf(err, errlen, "attn_decode launch failed"); rc = -1; }
        else rc = ops_done(err, errlen);
    }
    (void)hipFree(buf);
    return rc;
}

extern "C" int xjh_delta_step(const float *qkv, int qkv_stride, int k_off, int v_off, const float *beta_raw,
                              const float *alpha_raw, const float *dt, const float *A, int Hk, int Hv, int S, int T,
                              float eps, float qscale, float *state, float *out, float *ck, int ck_n, char *err,
                              size_t errlen) {
    if (!ops_stream()) return -1;
    if ((S != 64 && S != 128) || Hk < 1 || Hv < 1 || T < 1 || ck_n < 0 || ck_n > T || (ck_n && !ck) ||
        ((uintptr_t)state | (uintptr_t)ck) & 15) {
        snprintf(err, errlen, "delta_step: bad shape or unaligned state (S=%d (64|128), Hk=%d, Hv=%d, T=%d, ck_n=%d)", S,
                 Hk, Hv, T, ck_n);
        return -1;
    }
    DeltaArgs d{};
    d.qkv = qkv; d.qkv_s = qkv_stride; d.k_off = k_off; d.v_off = v_off;
    d.beta = beta_raw; d.beta_s = Hv; d.alpha = alpha_raw; d.alpha_s = Hv;
    d.dt = dt; d.A = A; d.state = state; d.ck = ck; d.out = out; d.out_s = Hv * S;
    d.T = T; d.Hk = Hk; d.Hv = Hv; d.S = S; d.keep_n = ck_n; d.eps = eps; d.qscale = qscale;
    // the token loop's default form (32 value rows per work-group); XJ_DELTA_SPLIT=0
    // selects one work-group per value head, read on every call
    const char *e = getenv("XJ_DELTA_SPLIT");
    d.split = e == nullptr || atoi(e) != 0;
    if (delta_launch(d, g_stream)) { snprintf(err, errlen, "delta_step launch failed"); return -1; }
    return ops_done(err, errlen);
}

extern "C" int xjh_sample(const float *logits, int n, int T, float temperature, const uint32_t *rand30, int32_t *out_host,
                          char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if (n < 1 || T < 1) { snprintf(err, errlen, "sample: bad shape (n=%d, T=%d)", n, T); return -1; }
    const bool draw = !(temperature <= 0.f);   // the app's test: temperature <= 0 is greedy, no number drawn
    if (draw && !rand30) { snprintf(err, errlen, "sample: no random numbers"); return -1; }
    for (int t = 0; draw && t < T; t++)
        if (rand30[t] >= (1u << 30)) { snprintf(err, errlen, "sample: random number %u not below 2^30", rand30[t]); return -1; }
    const int prow = sample_part_rows(n), np = (n + prow - 1) / prow;
    uint32_t *d = nullptr;
    if (hipMalloc(&d, 8 * (size_t)T + 8 * (size_t)T * np) != hipSuccess) { snprintf(err, errlen, "hipMalloc failed"); return -1; }
    int32_t *o = (int32_t *)(d + T);
    unsigned long long *part = (unsigned long long *)(d + 2 * T);
    int rc = !draw || hipMemcpy(d, rand30, 4 * (size_t)T, hipMemcpyHostToDevice) == hipSuccess ? 0 : -1;
    SampleArgs sa{};
    sa.lg = logits; sa.V = n; sa.T = T; sa.temp = temperature; sa.rnd = d; sa.out = o;
    sa.part = part; sa.n_part = np; sa.part_rows = prow;
    if (!rc && (sample_part_launch(logits, n, T, part, g_stream) || sample_launch(sa, g_stream))) rc = -1;
    if (!rc) rc = ops_done(err, errlen);
    else snprintf(err, errlen, "sample launch failed");
    if (!rc && hipMemcpy(out_host, o, 4 * (size_t)T, hipMemcpyDeviceToHost) != hipSuccess) rc = -1;
    (void)hipFree(d);
    return rc;
}

extern "C" int xjh_argmax(const float *x, int n, int T, int32_t *out_host, char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    int32_t *d = nullptr;
    if (hipMalloc(&d, 4 * T) != hipSuccess) { snprintf(err, errlen, "hipMalloc failed"); return -1; }
    int rc = argmax_rows_launch(x, n, T, d, g_stream) ? -1 : ops_done(err, errlen);
    if (!rc && hipMemcpy(out_host, d, 4 * T, hipMemcpyDeviceToHost) != hipSuccess) rc = -1;
    (void)hipFree(d);
    return rc;
}

extern "C" int xjh_delta_recurrent(int H, int S, int T, const float *q, const float *k, const float *v, const float *decay,
                                   const float *beta, float qscale, float *state, float *out, char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    if (delta_recurrent_launch(H, S, T, q, k, v, decay, beta, qscale, state, out, g_stream)) {
        snprintf(err, errlen, "delta launch failed (S must be 64 or 128)"); return -1;
    }
    return ops_done(err, errlen);
}

extern "C" int xjh_delta_chunked(int H, int S, int T, int chunk, const float *q, const float *k, const float *v,
                                 const float *decay, const float *beta, float qscale, float *state, float *out,
                                 char *err, size_t errlen) {
    if (!ops_stream()) return -1;
    const size_t wb = delta_chunked_work_bytes(H, S, T, chunk);
    if (!wb) { snprintf(err, errlen, "chunked delta: unsupported shape (S=%d, chunk=%d)", S, chunk); return -1; }
    void *work = nullptr;
    if (hipMalloc(&work, wb) != hipSuccess) { snprintf(err, errlen, "hipMalloc failed"); return -1; }
    int rc = delta_chunked_launch(H, S, T, chunk, q, k, v, decay, beta, qscale, state, out, (float *)work, g_stream);
    if (rc) snprintf(err, errlen, "chunked delta launch failed (q, k, v and state must be 16-byte aligned)");
    else rc = ops_done(err, errlen);
    (void)hipFree(work);
    return rc;
}
