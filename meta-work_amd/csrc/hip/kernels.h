// Host-side launch interface of the gfx950 kernels (internal to the library).
//
// Device weight layouts (produced by upload_repack, read by every kernel):
//   F32   rows of K floats (GGUF layout)
//   Q4_K  GGUF blocks of 144 B (16-byte aligned: 16 B header + 128 B nibbles)
//   Q6_K  four planes over the tensor's blocks g = row*nb + b:
//         ql[g][128] | qh[g][64] | sc[g][16] | d[g] (fp16)
//   Q8_0  two planes: qs[g][32] | d[g] (fp16)
// The repack only moves bytes; every decode reproduces the GGUF block exactly.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "xq.h"

namespace xjk {

constexpr int kMaxSeg = 4;
constexpr int kTileT = 8;        // tokens per GEMV launch (larger T is tiled)
// Bytes allocated after every weight tensor: the GEMV prefetches each lane's
// next units unconditionally, reading up to 3 * 16 + 1 Q4_K blocks past a row.
constexpr size_t kWeightPad = 16384;

// Prologues. RMSNorm(x) * w = sc * (x * w) with sc = 1/sqrt(mean(x^2) + eps):
// the activations are prepared from u = x * w with the per-group sums of x^2,
// and the GEMV scales each row's dot product by sc.
//   PRO_RMSU    the GEMV stages them from a prep launch's xq
//   PRO_RMSU_X  the GEMV's work-groups build them from x in LDS (no prep launch)
//   PRO_X       the GEMV's work-groups build them from the plain input x in
//               LDS (no norm), e.g. the SwiGLU values left by POST_SWIGLU_H
//   PRO_HEADRMS prepared digits of u = o * w * silu(z) whose groups carry the
//               sum of o^2 in ss: every head of `group` elements is scaled by
//               1/sqrt(sum over its groups / group + eps) (a gated RMSNorm per
//               head whose rows were produced by different work-groups)
enum Pro { PRO_NONE = 0, PRO_SWIGLU = 2, PRO_GATED_RMS = 3, PRO_RMSU = 4, PRO_RMSU_X = 5, PRO_X = 6, PRO_HEADRMS = 7 };
enum Epi { EPI_STORE = 0, EPI_ADD = 1, EPI_CONV = 2 };

struct DevW {
    const uint8_t *p = nullptr;
    uint32_t type = 0;
    int64_t n_rows = 0, k = 0;
    size_t bytes = 0;
};

struct GSeg {
    const uint8_t *w;
    uint32_t type;
    int32_t n_rows;
    int32_t wg0, nwg;            // work-group range of this segment
    int64_t nblk;                // blocks in the tensor (plane stride for Q6_K / Q8_0)
    float *y;                    // y[t * ys + row]
    int32_t ys;
    int32_t epi;
    // EPI_CONV: depthwise causal conv + SiLU on this segment's rows
    float *conv_state;           // [rows][conv_k-1]
    const float *conv_w;         // [rows][conv_k]
    float *conv_ck;              // [keep][rows][conv_k-1]
    int32_t conv_k;
    // greedy argmax partials, one key per (token, work-group); may be null
    unsigned long long *amax;
};

// Tails that leave the next GEMV's prepared activations (xq.h) behind, so the
// next GEMV needs no prep launch:
//   POST_SWIGLU  per 32-index group, the last of the work-groups that wrote
//                its gate rows (segment 0) and up rows (segment 1) emits
//                silu(gate) * up
//   POST_SWIGLU_H  single token, per-CU launch: every work-group computes the
//                gate and up rows of the same indices and stores
//                silu(gate) * up as floats into h (the down GEMV reads them
//                with PRO_X); no hand-off between work-groups
enum Post { POST_NONE = 0, POST_SWIGLU = 2, POST_SWIGLU_H = 3 };
struct PostPrep {
    int32_t mode;
    uint8_t *xq;                   // token 0 of this tile
    int32_t *cnt;                  // zero between launches, one per group
    float *h;                      // POST_SWIGLU_H output [n_rows]
};

struct GArgs {
    // prologue inputs (read by the prep kernel, and by the GEMV for PRO_RMSU_X)
    const float *x;  int32_t xs;   // input rows x[t * xs + k]
    const float *x2; int32_t x2s;  // second input (SwiGLU up, gated-RMS z)
    int32_t pro;
    const float *pro_w; float eps; int32_t group;
    uint8_t *xq;                   // prepared activations [T][xq_off(K).stride]
    int32_t K, T;
    int32_t t0;                    // absolute index of token 0 of this tile (checkpoints)
    int32_t keep_n;                // conv checkpoints for absolute tokens t < keep_n
    int32_t *inc_ptr; int32_t inc_by;
    PostPrep post;
    int32_t rpw;                   // rows per work-group (set by the launcher for per-CU launches)
    int32_t nseg;
    GSeg seg[kMaxSeg];
    uint8_t *hq;                   // prep launch, K % 256 == 0: also the GEMM's activations [T][hq_stride(K)]
    int32_t hq_only;               // ... and of xq only the groups' sums of x^2 (PRO_RMSU)
};

// Launch plan of one GEMV over `rows` output rows of inner size K: a team of
// `lanes` lanes per row, `rpt` rows per team, `rows_per_group` rows per
// 256-thread work-group. The plan depends on (K, rows) only, never on T.
struct GemvPlan {
    int lanes, rpt, rows_per_group;
};
GemvPlan gemv_plan(int K, int64_t rows);

// prep kernel: xq for the T tokens of a tile (grid ceil(K/256) x T), and hq
// when a.hq is set
int prep_launch(const GArgs &a, hipStream_t st);
// One GEMV launch (T <= kTileT) over all segments, reading a.xq. Segment i
// covers row groups [wg0, wg0+nwg) with nwg = ceil(n_rows / rows_per_group)
// of gemv_plan(K, total rows of all segments).
int gemv_launch(const GArgs &a, hipStream_t st);
// Whether gemv_launch serves `a` (one token, post.mode = POST_SWIGLU_H,
// gate = segment 0, up = segment 1) with a per-CU launch.
bool gemv_swiglu_h_ok(const GArgs &a);
int gemv_init(char *err, size_t errlen);       // raise the dynamic-LDS limit once
int gemv_max_tile(int K);                       // largest T tile whose activations fit in LDS
size_t gemv_xq_bytes(int K);                    // xq bytes for the largest tile of this K

// Multi-token GEMM on the matrix cores (gemm.hip): for each segment i,
// y_i[t][r] (+)= (W_i[r] . v[t]) (* tsc[t]) for T in 1..gemm_max_tokens()
// tokens of the prep launch's hq records (stride hs per token); every segment of
// one launch has the same type (Q4_K or Q6_K) and inner size K. One
// persistent work-group per CU takes an equal, contiguous share of the
// (row group of 128 rows, 256-element block) units of all segments; a row
// group whose blocks are shared by several work-groups leaves their partial
// sums in `part`, which the last of them to arrive adds in work-group order,
// so results do not depend on timing.
constexpr int kGemmMaxSeg = 4;
struct GemmSeg {
    const uint8_t *w; int32_t N;
    float *y; int32_t ys; int32_t add;   // add: y += instead of y =
};
struct GemmArgs {
    uint32_t type; int32_t K, T;
    const uint8_t *hq; int64_t hs;      // the T tokens' hq records (xq.h), token stride hs
    int32_t nseg;
    GemmSeg seg[kGemmMaxSeg];
    // optional: y[t][r] = (sum) * tsc[t] before the add (an RMSNorm input's
    // per-token scale, applied after the dot product as the GEMV applies it)
    const float *tsc;
    float *part;     // partial sums: gemm_part_floats(rows, T) floats
    int32_t *cnt;    // arrival counters: gemm_counters(rows) ints, zero before the first launch
    int32_t *inc_ptr; int32_t inc_by;   // optional: *inc_ptr += inc_by once
    // n6 > 0: the last n6 segments hold Q6_K rows, the others Q4_K rows (type
    // = XJ_Q4_K); one launch, each type on its own share of the work-groups
    int32_t n6;
    // set by gemm_launch
    int32_t rg0[kGemmMaxSeg + 1];       // first row group of each segment (prefix)
    int32_t nb, G;                      // blocks per row, work-groups
    int64_t P;                          // units
    int32_t G4; int64_t P4;             // the Q4_K work-groups and units of a mixed launch
};
// Capacities for a launch over `rows` rows in all (at most kGemmMaxSeg) segments.
int64_t gemm_part_floats(int64_t rows, int T);
int gemm_counters(int64_t rows);
// Per-token RMSNorm scale of T tokens of PRO_RMSU activations (xq, token
// stride xs): tsc[t] = 1 / sqrt(sum of the groups' ss / K + eps), the
// GEMV's rmsu_scale.
int rms_scale_launch(const uint8_t *xq, int64_t xs, int K, int T, float eps, float *tsc, hipStream_t st);
// hq records (token stride hq_stride(K)) of T tokens of prepared activations
// (xq, token stride xq_off(K).stride) from their v values.
int hq_from_v_launch(const uint8_t *xq, int K, int T, uint8_t *hq, hipStream_t st);
// *p += by on the device, in stream order (one thread).
int inc_launch(int32_t *p, int32_t by, hipStream_t st);
int gemm_max_tokens();
int gemm_launch(const GemmArgs &a, int64_t part_floats, int n_cnt, hipStream_t st);

// Repack a GGUF tensor into the device layout. dst must hold `bytes` =
// n_rows * row_bytes(type, k); src is host memory in GGUF layout.
int upload_repack(uint32_t type, const void *src, int64_t n_rows, int64_t k, uint8_t *dst,
                  hipStream_t st, char *err, size_t errlen);

int dequant_launch(const DevW &w, int64_t r0, int64_t n, float *y, hipStream_t st);

struct AttnArgs {
    const float *qg; int32_t qg_s;      // q|gate interleaved per head, token stride
    const float *kn; int32_t kn_s;      // new keys [T][Hkv*D] (pre-norm)
    const float *vn; int32_t vn_s;
    uint16_t *kc, *vc;                   // fp16 caches [n_ctx][Hkv*D]
    const float *qnorm_w, *knorm_w;
    const float2 *rope;                  // [n_ctx][n_rot/2] (cos, sin) of pos * base^(-2i/n_rot)
    const int32_t *npast;
    float *qr;                           // normalised, rotated queries [T][H][D] (written by kv_store)
    float *scores;                       // split partials [T][H][n_split][D+2]
    float *out;                          // [T][H*D]
    int32_t T, H, Hkv, D, n_rot, n_ctx, n_split;
    float eps, scale;
    uint8_t *xq;                         // optional: prepared activations of out (no prologue)
};
int attn_launch(const AttnArgs &a, hipStream_t st);
int attn_splits(int n_ctx);             // 64-position splits covering n_ctx

struct DeltaArgs {
    const float *qkv; int32_t qkv_s;    // conv+SiLU outputs [T][conv_dim]
    int32_t k_off, v_off;
    const float *beta; int32_t beta_s;  // raw projections [T][Hv]
    const float *alpha; int32_t alpha_s;
    const float *dt, *A;
    float *state;                        // [Hv][S][S] ([value j][key i])
    float *ck;                           // [keep][Hv][S][S]
    float *out; int32_t out_s;           // [T][Hv*S]
    int32_t T, Hk, Hv, S, keep_n;
    float eps, qscale;
    // optional: the prepared activations of norm(out) * norm_w * silu(z)
    // (gated RMSNorm, xj_cpu.c:215-217) into xq (token stride xq_off(Hv*S).stride)
    uint8_t *xq;
    const float *z; int32_t z_s;
    const float *norm_w;
    // split: one work-group per 32 value rows, xq holding the digits of
    // out * norm_w * silu(z) and each group's sum of out^2 (PRO_HEADRMS input)
    int32_t split;
};
int delta_launch(const DeltaArgs &a, hipStream_t st);
// Prefill inputs of the chunked rule from a layer's projections, per token t
// and value head hv (key head hv % Hk): q and k L2-normalised as the
// recurrent kernel normalises them, v gathered, decay = exp(softplus(alpha +
// dt) * A) and sigmoid(beta); q, k, v [T][Hv][S], decay and beta [T][Hv].
struct DeltaPrepArgs {
    const float *qkv; int32_t qkv_s, k_off, v_off;
    const float *beta; int32_t beta_s;
    const float *alpha; int32_t alpha_s;
    const float *dt, *A;
    float *q, *k, *v, *decay, *bt;
    int32_t T, Hk, Hv, S;
    float eps;
};
int delta_prefill_prep_launch(const DeltaPrepArgs &a, hipStream_t st);

// Standalone gated delta rule (decay/beta given), recurrent and chunked.
int delta_recurrent_launch(int H, int S, int T, const float *q, const float *k, const float *v,
                           const float *decay, const float *beta, float qscale, float *state,
                           float *out, hipStream_t st);
int delta_chunked_launch(int H, int S, int T, int chunk, const float *q, const float *k,
                         const float *v, const float *decay, const float *beta, float qscale,
                         float *state, float *out, float *work, hipStream_t st);
size_t delta_chunked_work_bytes(int H, int S, int T, int chunk);

// Several device-to-device copies of float arrays in one launch (the
// recurrent states of every DeltaNet layer of a stage: snapshots, restores,
// rollbacks to a checkpoint). Entries past kCopyMax take further launches.
constexpr int kCopyMax = 48;
struct CopyList {
    const float *src[kCopyMax];
    float *dst[kCopyMax];
    int64_t n[kCopyMax];   // floats
    int32_t cnt;
};
int copy_list_launch(const CopyList &c, hipStream_t st);

// Embedding rows for T tokens: x[t] = dequant(tok_embd row tokens[t]).
struct EmbedArgs {
    const int32_t *tokens;
    DevW w;
    float *x; int32_t T;
};
int embed_launch(const EmbedArgs &a, hipStream_t st);
// out[t] (optional) = greedy argmax over amax[t][0..n_part); tok_out (optional)
// receives the last row's id; hist/step (optional, T == 1 only) append it to a
// device-side history and advance the step counter; embed (optional, T == 1
// only): the id's row of embed->w into embed->x (embed->tokens unused).
int argmax_finalize_launch(const unsigned long long *amax, int n_part, int T, int32_t *out, int32_t *tok_out,
                           int32_t *hist, int32_t *step, hipStream_t st, const EmbedArgs *embed = nullptr);
// Plain argmax of T rows of n floats (first maximum).
int argmax_rows_launch(const float *x, int n, int T, int32_t *out, hipStream_t st);
int norm_launch(int mode, const float *x, const float *w, int n, int rows, float eps, float *out, hipStream_t st);
// The same over rows r < rows of n elements at x + r * xs, into out + r * os.
int norm_rows_launch(int mode, const float *x, int64_t xs, const float *w, int n, int rows, float eps, float *out,
                     int64_t os, hipStream_t st);
// One token per row t of lg [T][V]: the app's top-k 40 / top-p 0.95 draw at
// temperature temp (*temp_dev when given) with rnd[base + t] / 2^30 as the
// uniform number, base = (*rbase if given) + (*step if given); temp <= 0: the
// first maximum (no number read). part [T][n_part]: the largest argmax key of
// each part_rows elements of the row (the LM head's argmax partials, or
// sample_part_launch's). out[t] (optional); tok_out (optional) gets the last
// row's id; hist/step (optional, T == 1) append it to the history and advance
// the step; embed.x (optional, T == 1): the id's embedding row.
struct SampleArgs {
    const float *lg;
    int32_t V, T;
    const unsigned long long *part;
    int32_t n_part, part_rows;
    float temp;
    const float *temp_dev;
    const uint32_t *rnd;
    const int32_t *rbase;
    int32_t *out, *tok_out, *hist, *step;
    EmbedArgs embed;
};
int sample_launch(const SampleArgs &a, hipStream_t st);
// Partials for sample_launch when no LM head made them: sample_part_rows(V)
// elements each, ceil(V / rows) per row, into part [T][n].
int sample_part_rows(int V);
int sample_part_launch(const float *lg, int V, int T, unsigned long long *part, hipStream_t st);
// g = silu(g) * u over n floats.
int swiglu_launch(float *g, const float *u, int64_t n, hipStream_t st);
// NeoX RoPE in place of x[t * tok_stride + h * head_stride + i] for T tokens and
// n_heads heads; cs[t][n_rot/2] holds (cos, sin) of token t's angles.
int rope_launch(float *x, const float2 *cs, int T, int n_heads, int64_t tok_stride, int64_t head_stride, int n_rot,
                hipStream_t st);
// (cos, sin) of theta = pos * base^(-2i/n_rot) for positions pos0 .. pos0+n-1,
// in float as the reference's rope evaluates them: out[p][n_rot/2].
void rope_table(int pos0, int n, int n_rot, float base, float2 *out);
// Depthwise causal conv (kernel K <= 8) + SiLU in place of x [T][C], state
// [C][K-1] carried across calls, ck [ck_n][C][K-1] the state after each of the
// first ck_n tokens (EPI_CONV's code).
int conv_silu_launch(float *x, float *state, const float *w, int C, int K, int T, float *ck, int ck_n, hipStream_t st);

}  // namespace xjk
