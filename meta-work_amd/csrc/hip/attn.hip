// Gated GQA attention over the fp16 KV cache (gfx950).
//
// Computes attn_full of src/xiaoju-pipe/core/xj_cpu.c:83-151 after the q/k/v
// projections, with the cache in fp16 as the Metal backend keeps it
// (xj_kernels.metal:440-452):
//   kv_store_kernel  one work-group per (token, kv head) (several tokens; a single
//                    token leaves this to attn_part_kernel): RMSNorm(k_norm) of the
//                    new key (double sum, x*sc*w), NeoX RoPE of the first n_rot
//                    dims (xj_cpu.c:68-77; cos and sin of theta = pos * base^(-2i/n_rot)
//                    from a table the host fills per position with the
//                    reference's float powf, cosf and sinf), then k and v
//                    rounded to fp16 (RNE) and stored at position
//                    n_past + t; the same for the query heads that read this kv
//                    head (q_norm, RoPE), kept in fp32 for the split kernel.
//   attn_part_kernel one work-group per (kv head, token, 64-position split) for
//                    the G query heads of the kv head: scores q.k_j * scale
//                    (16-lane teams, two positions per team), per head the
//                    split's max, sum of exponentials and unnormalised
//                    sum_j e_j v_j (8 dims x position groups per thread row,
//                    16-byte loads, position groups combined in a fixed order)
//   attn_combine     merges the splits with the usual max rescaling, divides
//                    by the total, applies sigmoid(gate) (xj_cpu.c:128-147:
//                    the same softmax(qK^T/sqrt(D)) V, reassociated by split)
//                    and, when asked, writes the wo GEMV's prepared activations.
// Query rows are [q(D) | gate(D)] per head (xj_cpu.c:118); kv head = h / (H/Hkv).
#include "common.h"
#include "kernels.h"
#include "xq.h"

namespace xjk {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Work-group (t, g): the new key of kv head g and the queries of the
// G = H/Hkv heads that read it, each normalised (RMSNorm * w, double sum) and
// rotated (NeoX RoPE of the first n_rot dims); the sums of all G+1 vectors are
// formed in one block reduction. Thread i < D handles element i of every vector.
constexpr int kMaxGroup = 8;

template <int D>
__global__ __launch_bounds__(256) void kv_store_kernel(const AttnArgs a) {
    const int t = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int G = a.H / a.Hkv, NV = G + 1;       // vector 0 = key, 1..G = queries
    __shared__ float buf[kMaxGroup + 1][D];
    __shared__ float2 cs[D / 2];
    __shared__ double red[4][kMaxGroup + 1];
    const int pos = *a.npast + t, nk = a.Hkv * D, w = tid >> 6;
    const bool in = tid < D;
    float v[kMaxGroup + 1];
#pragma unroll
    for (int i = 0; i <= kMaxGroup; i++) {
        v[i] = 0.f;
        if (in && i < NV)
            v[i] = i == 0 ? a.kn[(int64_t)t * a.kn_s + g * D + tid]
                          : a.qg[(int64_t)t * a.qg_s + (int64_t)(g * G + i - 1) * 2 * D + tid];
    }
    const float vv = in ? a.vn[(int64_t)t * a.vn_s + g * D + tid] : 0.f;
    for (int i = tid; i < a.n_rot / 2; i += 256) cs[i] = a.rope[(int64_t)pos * (a.n_rot / 2) + i];
#pragma unroll
    for (int i = 0; i <= kMaxGroup; i++) {
        const double ss = xjd::wave_sum_d((double)v[i] * v[i]);
        if ((tid & 63) == 0 && i < NV) red[w][i] = ss;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i <= kMaxGroup; i++) {
        if (i >= NV) break;
        const double ss = red[0][i] + red[1][i] + red[2][i] + red[3][i];
        const float sc = 1.0f / sqrtf((float)(ss / D) + a.eps);
        if (in) buf[i][tid] = v[i] * sc * (i == 0 ? a.knorm_w[tid] : a.qnorm_w[tid]);
    }
    __syncthreads();
    const int half = a.n_rot / 2;
    for (int idx = tid; idx < NV * half; idx += 256) {
        const int i = idx / half, j = idx % half;
        const float x0 = buf[i][j], x1 = buf[i][j + half];
        buf[i][j] = x0 * cs[j].x - x1 * cs[j].y;
        buf[i][j + half] = x0 * cs[j].y + x1 * cs[j].x;
    }
    __syncthreads();
    if (in) {
        a.kc[(int64_t)pos * nk + g * D + tid] = xjd::f32_to_f16(buf[0][tid]);
        a.vc[(int64_t)pos * nk + g * D + tid] = xjd::f32_to_f16(vv);
        for (int i = 1; i < NV; i++) a.qr[((int64_t)t * a.H + g * G + i - 1) * D + tid] = buf[i][tid];
    }
}

// Split-K decode attention. Work-group (g, t, s) covers positions
// [s*P, min(s*P+P, pos+1)) for the G query heads of kv head g, token t: it
// writes, per head, the split's maximum score m_s, l_s = sum_j exp(s_j - m_s)
// and the unnormalised o_s = sum_j exp(s_j - m_s) v_j. Splits past pos exit.
// The keys and values of the split are requested at once and read once for
// all G heads. The grid covers n_ctx, so one captured graph serves every
// decode position. P = 64 (4B decode at ~1060 positions: split 6.74 us +
// combine 4.46 us per layer against 6.91 + 4.63 at 32 positions and
// 9.10 + 4.22 at 128; prefill attention 22.4 vs 27.8 us per chunk launch).
constexpr int kSplitP = 64;

// Work-group barrier ordering LDS accesses only (global loads in flight stay
// in flight).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// F (single token): the work-group also does kv_store's work for itself -
// the G queries normalised and rotated into LDS, and in the split holding pos
// the new key (stored to the cache with its value, and used in place of the
// cache bytes read for pos) - with kv_store's arithmetic, so the results are
// those of kv_store + attn_part bit for bit.
template <int D, int G, bool F>
__global__ __launch_bounds__(256) void attn_part_kernel(const AttnArgs a) {
    constexpr int DL = D / 16;           // score dims per lane (16-lane teams, one position each)
    constexpr int NPT = kSplitP / 16;    // positions per team
    constexpr int DG = D / 8;            // PV: 8-dim groups
    constexpr int PG = 256 / DG;         // PV: position groups
    constexpr int NPG = kSplitP / PG;    // PV: positions per group
    constexpr int HC = G < 4 ? G : 4;    // PV: heads per LDS pass
    static_assert(kSplitP % PG == 0 && NPG >= 1, "split size");
    // work-group g takes query heads g G .. g G + G - 1, of kv head gk (the
    // kv head's heads may be split over nsub work-groups)
    const int g = blockIdx.x, t = blockIdx.y, sp = blockIdx.z, tid = threadIdx.x;
    const int nsub = a.H / (a.Hkv * G), gk = g / nsub;
    const int team = tid >> 4, l16 = tid & 15;
    const int nk = a.Hkv * D;
    // the kernel arguments read together (each read would otherwise be
    // waited for in turn)
    asm volatile("" ::"s"(a.npast), "s"(a.kc), "s"(a.vc), "s"(a.qg), "s"(a.kn), "s"(a.vn), "s"(a.qnorm_w),
                 "s"(a.knorm_w), "s"(a.rope), "s"(a.n_rot), "s"(a.qr), "s"(a.scores), "s"(a.n_split));
    // F: the token's raw queries, key, value and norm weights do not depend
    // on the position: they are requested with it and waited for together
    // (lanes past D keep zeros)
    float v[G + 1], vv = 0.f;
    float2 csv = {0.f, 0.f};
    float qnw = 0.f, knw = 0.f;
    const int npast = *a.npast;
    if constexpr (F) {
        const bool in = tid < D;
        const int dc = in ? tid : D - 1;
        const float q_w = a.qnorm_w[dc], k_w = a.knorm_w[dc], kx = a.kn[gk * D + dc], vx = a.vn[gk * D + dc];
        qnw = in ? q_w : 0.f;
        knw = in ? k_w : 0.f;
#pragma unroll
        for (int i = 0; i < G; i++) {
            const float qx = a.qg[(int64_t)(g * G + i) * 2 * D + dc];
            v[i] = in ? qx : 0.f;
            asm volatile("" ::"v"(v[i]));
        }
        v[G] = in ? kx : 0.f;
        vv = in ? vx : 0.f;
        asm volatile("" ::"v"(v[G]), "v"(vv), "v"(qnw), "v"(knw), "v"(npast));
    }
    const int pos = npast + t, j0 = sp * kSplitP;
    if (j0 > pos) return;                       // uniform per work-group
    const int n = (j0 + kSplitP - 1 < pos ? j0 + kSplitP - 1 : pos) - j0 + 1;
    __shared__ float e[G][kSplitP];
    __shared__ float ml[G][2];
    __shared__ float po[PG][HC][D];
    const bool last = F && pos - j0 < kSplitP;   // this split holds pos (uniform)
    if constexpr (F) {   // n_rot <= D <= 256; a clamped read, so the cache reads below need not wait for it
        const int half = a.n_rot / 2, rc = tid < half ? tid : half - 1;
        const float2 cv = a.rope[(int64_t)pos * half + rc];
        csv = tid < half ? cv : float2{0.f, 0.f};
    }
    // every key and value of the split, clamped to valid positions
    u32x4 kw[NPT][(DL + 7) / 8];
    uint2 kw4[NPT];
#pragma unroll
    for (int r = 0; r < NPT; r++) {
        const int jj = team + 16 * r, jc = jj < n ? jj : n - 1;
        const uint16_t *kp = a.kc + (int64_t)(j0 + jc) * nk + gk * D + l16 * DL;
        if constexpr (DL % 8 == 0) {
#pragma unroll
            for (int d = 0; d < DL / 8; d++) kw[r][d] = *(const u32x4 *)(kp + 8 * d);
        } else {
            kw4[r] = *(const uint2 *)kp;   // DL == 4
        }
    }
    const int dg = tid % DG, pg = tid / DG;
    u32x4 vw[NPG];
#pragma unroll
    for (int r = 0; r < NPG; r++) {
        const int jj = pg + PG * r, jc = jj < n ? jj : n - 1;
        vw[r] = *(const u32x4 *)(a.vc + (int64_t)(j0 + jc) * nk + gk * D + 8 * dg);
    }
    float qv[G][DL];
    if constexpr (F) {
        __shared__ float buf[G + 1][D];   // vectors 0..G-1 = queries, G = the new key
        __shared__ float2 cs[D / 2];
        __shared__ double red[4][G + 1];
        __shared__ __align__(16) uint16_t kv16[2][D];   // the new key and value in fp16
        const int NV = last ? G + 1 : G, w = tid >> 6;
        const bool in = tid < D;
        if (tid < a.n_rot / 2) cs[tid] = csv;
#pragma unroll
        for (int i = 0; i <= G; i++) {
            const double ss = xjd::wave_sum_d((double)v[i] * v[i]);
            if ((tid & 63) == 0 && i < NV) red[w][i] = ss;
        }
        lds_barrier();
#pragma unroll
        for (int i = 0; i <= G; i++) {
            if (i >= NV) break;
            const double ss = red[0][i] + red[1][i] + red[2][i] + red[3][i];
            const float sc = 1.0f / sqrtf((float)(ss / D) + a.eps);
            if (in) buf[i][tid] = v[i] * sc * (i == G ? knw : qnw);
        }
        lds_barrier();
        const int half = a.n_rot / 2;
        for (int idx = tid; idx < NV * half; idx += 256) {
            const int i = idx / half, j = idx % half;
            const float x0 = buf[i][j], x1 = buf[i][j + half];
            buf[i][j] = x0 * cs[j].x - x1 * cs[j].y;
            buf[i][j + half] = x0 * cs[j].y + x1 * cs[j].x;
        }
        lds_barrier();
        if (last && in) {
            const uint16_t k16 = xjd::f32_to_f16(buf[G][tid]), v16 = xjd::f32_to_f16(vv);
            if (g % nsub == 0) {   // one of the kv head's work-groups stores the new key and value
                a.kc[(int64_t)pos * nk + gk * D + tid] = k16;
                a.vc[(int64_t)pos * nk + gk * D + tid] = v16;
            }
            kv16[0][tid] = k16;
            kv16[1][tid] = v16;
        }
        lds_barrier();
#pragma unroll
        for (int h = 0; h < G; h++)
#pragma unroll
            for (int d = 0; d < DL; d++) qv[h][d] = buf[h][l16 * DL + d];
        if (last) {   // the cache bytes read for pos (every clamped entry past it too) were stale
#pragma unroll
            for (int r = 0; r < NPT; r++) {
                const int jj = team + 16 * r, jc = jj < n ? jj : n - 1;
                if (j0 + jc != pos) continue;
                const uint16_t *kp = &kv16[0][l16 * DL];
                if constexpr (DL % 8 == 0) {
#pragma unroll
                    for (int d = 0; d < DL / 8; d++) kw[r][d] = *(const u32x4 *)(kp + 8 * d);
                } else {
                    kw4[r] = *(const uint2 *)kp;
                }
            }
#pragma unroll
            for (int r = 0; r < NPG; r++) {
                const int jj = pg + PG * r, jc = jj < n ? jj : n - 1;
                if (j0 + jc == pos) vw[r] = *(const u32x4 *)&kv16[1][8 * dg];
            }
        }
    } else {
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float *qp = a.qr + ((int64_t)t * a.H + g * G + h) * D + l16 * DL;
#pragma unroll
            for (int d = 0; d < DL; d += 4) {
                const float4 q4 = *(const float4 *)(qp + d);
                qv[h][d] = q4.x; qv[h][d + 1] = q4.y; qv[h][d + 2] = q4.z; qv[h][d + 3] = q4.w;
            }
        }
    }
    // scores
#pragma unroll
    for (int r = 0; r < NPT; r++) {
        const int jj = team + 16 * r;
        float kf[DL];
        if constexpr (DL % 8 == 0) {
#pragma unroll
            for (int d = 0; d < DL / 8; d++)
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    kf[8 * d + 2 * c] = xjd::f16_to_f32(kw[r][d][c] & 0xFFFFu);
                    kf[8 * d + 2 * c + 1] = xjd::f16_to_f32(kw[r][d][c] >> 16);
                }
        } else {
            kf[0] = xjd::f16_to_f32(kw4[r].x & 0xFFFFu); kf[1] = xjd::f16_to_f32(kw4[r].x >> 16);
            kf[2] = xjd::f16_to_f32(kw4[r].y & 0xFFFFu); kf[3] = xjd::f16_to_f32(kw4[r].y >> 16);
        }
#pragma unroll
        for (int h = 0; h < G; h++) {
            float s = 0.f;
#pragma unroll
            for (int d = 0; d < DL; d++) s = fmaf(qv[h][d], kf[d], s);
            s = xjd::row16_sum(s) * a.scale;
            if (l16 == 0) e[h][jj] = jj < n ? s : -INFINITY;
        }
    }
    __syncthreads();
    // per head: maximum, exponentials and their sum over the split (32 lanes
    // per head, lane jj holding positions jj, jj + 32, ...)
    if (tid < G * 32) {
        constexpr int PPL = kSplitP / 32;
        const int h = tid >> 5, jj = tid & 31;
        float sv[PPL];
#pragma unroll
        for (int q = 0; q < PPL; q++) sv[q] = e[h][jj + 32 * q];
        float m = sv[0];
#pragma unroll
        for (int q = 1; q < PPL; q++) m = fmaxf(m, sv[q]);
        m = xjd::row16_max(m);
        m = fmaxf(m, __shfl_xor(m, 16, 64));
        float l = 0.f;
#pragma unroll
        for (int q = 0; q < PPL; q++) {
            const float ev = jj + 32 * q < n ? expf(sv[q] - m) : 0.f;
            e[h][jj + 32 * q] = ev;
            l += ev;
        }
        l = xjd::row16_sum(l);
        l += __shfl_xor(l, 16, 64);
        if (jj == 0) { ml[h][0] = m; ml[h][1] = l; }
    }
    __syncthreads();
    // PV: thread (pg, dg) sums positions pg, pg + PG, ... over dims 8dg..8dg+7, HC heads per pass
#pragma unroll
    for (int h0 = 0; h0 < G; h0 += HC) {
        float o[HC][8];
#pragma unroll
        for (int h = 0; h < HC; h++)
#pragma unroll
            for (int c = 0; c < 8; c++) o[h][c] = 0.f;
#pragma unroll
        for (int r = 0; r < NPG; r++) {
            const int jj = pg + PG * r;
            float vf[8];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                vf[2 * c] = xjd::f16_to_f32(vw[r][c] & 0xFFFFu);
                vf[2 * c + 1] = xjd::f16_to_f32(vw[r][c] >> 16);
            }
#pragma unroll
            for (int h = 0; h < HC; h++) {
                const float ej = e[h0 + h][jj];   // 0 past n
#pragma unroll
                for (int c = 0; c < 8; c++) o[h][c] = fmaf(ej, vf[c], o[h][c]);
            }
        }
        if (h0) __syncthreads();   // po of the previous pass consumed
#pragma unroll
        for (int h = 0; h < HC; h++)
#pragma unroll
            for (int c = 0; c < 8; c++) po[pg][h][8 * dg + c] = o[h][c];
        __syncthreads();
        for (int idx = tid; idx < HC * D; idx += 256) {
            const int h = idx / D, d = idx % D;
            float acc = 0.f;
#pragma unroll
            for (int g2 = 0; g2 < PG; g2++) acc += po[g2][h][d];
            float *part = a.scores + (((int64_t)t * a.H + g * G + h0 + h) * a.n_split + sp) * (D + 2);
            part[2 + d] = acc;
            if (d == 0) { part[0] = ml[h0 + h][0]; part[1] = ml[h0 + h][1]; }
        }
    }
}

// out[t][h] = sigmoid(gate) * sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a) {
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    asm volatile("" ::"s"(a.npast), "s"(a.scores), "s"(a.qg), "s"(a.qg_s), "s"(a.out), "s"(a.xq), "s"(a.n_split), "s"(a.H));
    const float *part = a.scores + ((int64_t)t * a.H + h) * a.n_split * (D + 2);
    // the first 64 splits' partials are requested before the position is
    // known (addresses clamped to the buffer; entries past the position are
    // never used, whatever they hold)
    const int d = tid;   // D <= 256
    const bool in = d < D;
    const int dc = in ? d : D - 1;
    const int sl = tid < a.n_split ? tid : a.n_split - 1;
    const float ms_l = part[(int64_t)sl * (D + 2)], ls_l = part[(int64_t)sl * (D + 2) + 1];
    float pv[64];
#pragma unroll
    for (int s = 0; s < 64; s++) pv[s] = part[(int64_t)(s < a.n_split ? s : a.n_split - 1) * (D + 2) + 2 + dc];
    const float gx = a.qg[(int64_t)t * a.qg_s + (int64_t)h * 2 * D + D + dc];   // the output gate
    const int pos = *a.npast + t, ns = pos / kSplitP + 1;
    __shared__ float w[64];
    __shared__ float inv_l;
    if (tid < 64) {
        // split s < 64 on lane s; the weights and the total are formed in a fixed order
        const float ms = tid < ns ? ms_l : -INFINITY;
        const float ls = tid < ns ? ls_l : 0.f;
        float M = ms;
        for (int s = tid + 64; s < ns; s += 64) M = fmaxf(M, part[(int64_t)s * (D + 2)]);
        for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        const float ws = tid < ns ? expf(ms - M) : 0.f;
        w[tid] = ws;
        float L = ws * ls;
        for (int off = 1; off < 64; off <<= 1) L += __shfl_xor(L, off, 64);
        for (int s = 64; s < ns; s++) L = fmaf(expf(part[(int64_t)s * (D + 2)] - M), part[(int64_t)s * (D + 2) + 1], L);
        if (tid == 0) inv_l = 1.0f / L;
    }
    float r = 0.f;
    if (ns <= 64) {
        // every split's value of dim d (requested above), summed in order
        __syncthreads();
        float o = 0.f;
#pragma unroll
        for (int s = 0; s < 64; s++) if (s < ns) o = fmaf(w[s], pv[s], o);
        r = o * inv_l * (in ? xjd::sigm(gx) : 0.f);
    } else {
        __syncthreads();
        if (in) {
            // more splits than cached weights: recompute the maximum
            float o = 0.f, M2 = -INFINITY;
            for (int s = 0; s < ns; s++) M2 = fmaxf(M2, part[(int64_t)s * (D + 2)]);
            for (int s = 0; s < ns; s++) o = fmaf(expf(part[(int64_t)s * (D + 2)] - M2), part[(int64_t)s * (D + 2) + 2 + d], o);
            r = o * inv_l * xjd::sigm(gx);
        }
    }
    if (in) a.out[(int64_t)t * a.H * D + (int64_t)h * D + d] = r;
    // the wo GEMV's prepared activations (no prologue): groups of 32 lie inside the head
    if (a.xq) xjd::emit_xq(r, h * D + d, in, a.xq + (int64_t)t * xq_off(a.H * D).stride, xq_off(a.H * D));
}

template <int D, bool F>
static void launch_part(const AttnArgs &a, hipStream_t st) {
    // a single token: each kv head's query heads over two work-groups (twice
    // the work-groups, the split's keys and values read by both; 4B decode
    // attention 7.36 -> 6.98 us per layer); XJ_ATTN_SUB sets the count
    static const int sub_env = getenv("XJ_ATTN_SUB") ? atoi(getenv("XJ_ATTN_SUB")) : 2;
    const int per = a.H / a.Hkv;
    const int sub = F && sub_env > 1 && per % sub_env == 0 ? sub_env : 1;   // work-groups per kv head
    const dim3 grid(a.Hkv * sub, a.T, a.n_split);
    switch (per / sub) {
    case 1: hipLaunchKernelGGL((attn_part_kernel<D, 1, F>), grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL((attn_part_kernel<D, 2, F>), grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL((attn_part_kernel<D, 4, F>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((attn_part_kernel<D, 8, F>), grid, dim3(256), 0, st, a); break;
    }
}

// A single token: kv_store's work inside the split kernel (XJ_ATTN_FUSE=0
// keeps the separate kv_store launch).
template <int D>
static int launch_d(const AttnArgs &a, hipStream_t st) {
    static const bool fuse = getenv("XJ_ATTN_FUSE") == nullptr || atoi(getenv("XJ_ATTN_FUSE")) != 0;
    if (a.T == 1 && fuse) {
        launch_part<D, true>(a, st);
    } else {
        hipLaunchKernelGGL(kv_store_kernel<D>, dim3(a.T, a.Hkv), dim3(256), 0, st, a);
        launch_part<D, false>(a, st);
    }
    hipLaunchKernelGGL(attn_combine_kernel<D>, dim3(a.H, a.T), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// NeoX RoPE in place (xj_cpu.c:68-77) of T tokens x n_heads heads, one
// thread per pair (i, i + n_rot/2), with cos and sin of position pos0 + t from
// the same kind of table kv_store reads (cs[t][n_rot/2]).
__global__ __launch_bounds__(256) void rope_kernel(float *x, const float2 *cs, int T, int nh, int64_t tok_s, int64_t head_s,
                                                   int n_rot) {
    const int half = n_rot / 2;
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= (int64_t)T * nh * half) return;
    const int i = (int)(gid % half), h = (int)((gid / half) % nh), t = (int)(gid / ((int64_t)half * nh));
    const float2 c = cs[(int64_t)t * half + i];
    float *p = x + t * tok_s + h * head_s;
    const float x0 = p[i], x1 = p[i + half];
    p[i] = x0 * c.x - x1 * c.y;
    p[i + half] = x0 * c.y + x1 * c.x;
}

void rope_table(int pos0, int n, int n_rot, float base, float2 *out) {
    const int half = n_rot / 2;
    for (int p = 0; p < n; p++)
        for (int i = 0; i < half; i++) {
            const float theta = (pos0 + p) * powf(base, -2.0f * i / n_rot);
            out[(size_t)p * half + i] = float2{cosf(theta), sinf(theta)};
        }
}

int rope_launch(float *x, const float2 *cs, int T, int n_heads, int64_t tok_stride, int64_t head_stride, int n_rot,
                hipStream_t st) {
    if (T < 0 || n_heads < 0 || n_rot < 2 || n_rot % 2) return -1;
    const int64_t n = (int64_t)T * n_heads * (n_rot / 2);
    if (n == 0) return 0;
    hipLaunchKernelGGL(rope_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, cs, T, n_heads, tok_stride,
                       head_stride, n_rot);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int attn_splits(int n_ctx) { return (n_ctx + kSplitP - 1) / kSplitP; }

int attn_launch(const AttnArgs &a, hipStream_t st) {
    const int G = a.Hkv > 0 ? a.H / a.Hkv : 0;
    if (a.Hkv < 1 || a.H % a.Hkv || (G != 1 && G != 2 && G != 4 && G != 8) || a.n_rot > a.D || a.n_rot % 2 ||
        a.n_split != attn_splits(a.n_ctx) ||
        !a.qr)
        return -1;
    switch (a.D) {
    case 64: return launch_d<64>(a, st);
    case 128: return launch_d<128>(a, st);
    case 256: return launch_d<256>(a, st);
    default: return -1;
    }
}

}  // namespace xjk
