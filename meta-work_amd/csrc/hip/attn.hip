// Gated GQA attention over the fp16 KV cache (gfx950).
//
// Computes attn_full of src/xiaoju-pipe/core/xj_cpu.c:83-151 after the q/k/v
// projections, with the cache in fp16 as the Metal backend keeps it
// (xj_kernels.metal:440-452):
//   kv_store_kernel  one work-group per (token, kv head): RMSNorm(k_norm) of the
//                    new key (double sum, x*sc*w), NeoX RoPE of the first n_rot
//                    dims (xj_cpu.c:68-77; theta = pos * inv_freq[i] with
//                    inv_freq = base^(-2i/n_rot) computed on the host exactly as
//                    the reference's powf, cos/sin of theta evaluated in double),
//                    then k and v rounded to fp16 (RNE) and stored at position
//                    n_past + t; the same for the query heads that read this kv
//                    head (q_norm, RoPE), kept in fp32 for the split kernel.
//   attn_part_kernel one work-group per (query head, token, 64-position split):
//                    scores q.k_j * scale (16-lane teams, one position per team),
//                    the split's max, sum of exponentials and unnormalised
//                    sum_j e_j v_j (8 dims x 8 position groups per thread row,
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
    for (int i = tid; i < a.n_rot / 2; i += 256) {
        const float theta = (float)pos * a.inv_freq[i];
        cs[i] = float2{(float)cos((double)theta), (float)sin((double)theta)};
    }
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

// Split-K decode attention. Work-group (h, t, s) covers positions
// [s*P, min(s*P+P, pos+1)) of query head h, token t: it writes the split's
// maximum score m_s, l_s = sum_j exp(s_j - m_s) and the unnormalised
// o_s = sum_j exp(s_j - m_s) v_j. Splits past pos exit.
// The grid covers n_ctx, so one captured graph serves every decode position.
constexpr int kSplitP = 64;

template <int D>
__global__ __launch_bounds__(256) void attn_part_kernel(const AttnArgs a) {
    constexpr int DL = D / 16;           // score dims per lane
    constexpr int DG = D / 8;            // PV: 8-dim groups
    constexpr int PG = 256 / DG;         // PV: position groups
    const int h = blockIdx.x, t = blockIdx.y, sp = blockIdx.z, tid = threadIdx.x;
    const int team = tid >> 4, l16 = tid & 15;
    const int kvh = h / (a.H / a.Hkv), nk = a.Hkv * D;
    const int pos = *a.npast + t, j0 = sp * kSplitP;
    if (j0 > pos) return;                       // uniform per work-group
    const int n = (j0 + kSplitP - 1 < pos ? j0 + kSplitP - 1 : pos) - j0 + 1;
    __shared__ float q[D];
    __shared__ float e[kSplitP];
    __shared__ float redf[4];
    __shared__ float po[PG][D];
    for (int i = tid; i < D; i += 256) q[i] = a.qr[((int64_t)t * a.H + h) * D + i];
    __syncthreads();
    float qv[DL];
#pragma unroll
    for (int d = 0; d < DL; d++) qv[d] = q[l16 * DL + d];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < kSplitP / 16; r++) {
        const int jj = team + 16 * r;
        if (jj < n) {
            const uint16_t *kp = a.kc + (int64_t)(j0 + jj) * nk + kvh * D + l16 * DL;
            float s = 0.f;
            if constexpr (DL % 8 == 0) {
#pragma unroll
                for (int d = 0; d < DL; d += 8) {
                    const u32x4 kw = *(const u32x4 *)(kp + d);
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const uint32_t w2 = kw[c];
                        s = fmaf(qv[d + 2 * c], xjd::f16_to_f32(w2 & 0xFFFFu), s);
                        s = fmaf(qv[d + 2 * c + 1], xjd::f16_to_f32(w2 >> 16), s);
                    }
                }
            } else {
#pragma unroll
                for (int d = 0; d < DL; d++) s = fmaf(qv[d], xjd::f16_to_f32(kp[d]), s);
            }
            s = xjd::row16_sum(s) * a.scale;
            if (l16 == 0) e[jj] = s;
            mx = fmaxf(mx, s);
        }
    }
    mx = xjd::block_max(mx, redf);
    __syncthreads();
    float lsum = 0.f;
    if (tid < 64) {
        const float ev = tid < n ? expf(e[tid] - mx) : 0.f;
        if (tid < n) e[tid] = ev;
        lsum = ev;
        for (int off = 32; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off, 64);
    }
    __syncthreads();
    // PV: thread (pg, dg) sums positions pg, pg + PG, ... over dims 8dg..8dg+7
    {
        const int dg = tid % DG, pg = tid / DG;
        float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        const uint16_t *vp = a.vc + (int64_t)j0 * nk + kvh * D + 8 * dg;
#pragma unroll
        for (int r = 0; r < kSplitP / PG; r++) {
            const int jj = pg + PG * r;
            if (jj < n) {
                const u32x4 vw = *(const u32x4 *)(vp + (int64_t)jj * nk);
                const float ej = e[jj];
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    o[2 * c] = fmaf(ej, xjd::f16_to_f32(vw[c] & 0xFFFFu), o[2 * c]);
                    o[2 * c + 1] = fmaf(ej, xjd::f16_to_f32(vw[c] >> 16), o[2 * c + 1]);
                }
            }
        }
#pragma unroll
        for (int c = 0; c < 8; c++) po[pg][8 * dg + c] = o[c];
    }
    __syncthreads();
    float *part = a.scores + (((int64_t)t * a.H + h) * a.n_split + sp) * (D + 2);
    for (int d = tid; d < D; d += 256) {
        float o = 0.f;
#pragma unroll
        for (int g2 = 0; g2 < PG; g2++) o += po[g2][d];
        part[2 + d] = o;
    }
    if (tid == 0) { part[0] = mx; part[1] = lsum; }
}

// out[t][h] = sigmoid(gate) * sum_s e^(m_s - M) o_s / sum_s e^(m_s - M) l_s
template <int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(const AttnArgs a) {
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x;
    const int pos = *a.npast + t, ns = pos / kSplitP + 1;
    const float *part = a.scores + ((int64_t)t * a.H + h) * a.n_split * (D + 2);
    __shared__ float w[64];
    __shared__ float inv_l;
    if (tid < 64) {
        // split s < 64 on lane s; the weights and the total are formed in a fixed order
        const float ms = tid < ns ? part[(int64_t)tid * (D + 2)] : -INFINITY;
        const float ls = tid < ns ? part[(int64_t)tid * (D + 2) + 1] : 0.f;
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
    __syncthreads();
    const float *qr = a.qg + (int64_t)t * a.qg_s + (int64_t)h * 2 * D;
    const int d = tid;   // D <= 256
    const bool in = d < D;
    float r = 0.f;
    if (in) {
        float o = 0.f, M2 = -INFINITY;
        if (ns > 64)   // more splits than cached weights: recompute the maximum
            for (int s = 0; s < ns; s++) M2 = fmaxf(M2, part[(int64_t)s * (D + 2)]);
        if (ns <= 64) {
            for (int s0 = 0; s0 < ns; s0 += 8) {   // eight loads in flight, summed in order
                float pv[8];
#pragma unroll
                for (int j = 0; j < 8; j++) pv[j] = s0 + j < ns ? part[(int64_t)(s0 + j) * (D + 2) + 2 + d] : 0.f;
#pragma unroll
                for (int j = 0; j < 8; j++) if (s0 + j < ns) o = fmaf(w[s0 + j], pv[j], o);
            }
        } else {
            for (int s = 0; s < ns; s++) o = fmaf(expf(part[(int64_t)s * (D + 2)] - M2), part[(int64_t)s * (D + 2) + 2 + d], o);
        }
        r = o * inv_l * xjd::sigm(qr[D + d]);
        a.out[(int64_t)t * a.H * D + (int64_t)h * D + d] = r;
    }
    // the wo GEMV's prepared activations (no prologue): groups of 32 lie inside the head
    if (a.xq) xjd::emit_xq(r, h * D + d, in, a.xq + (int64_t)t * xq_off(a.H * D).stride, xq_off(a.H * D));
}

template <int D>
static int launch_d(const AttnArgs &a, hipStream_t st) {
    hipLaunchKernelGGL(kv_store_kernel<D>, dim3(a.T, a.Hkv), dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_part_kernel<D>, dim3(a.H, a.T, a.n_split), dim3(256), 0, st, a);
    hipLaunchKernelGGL(attn_combine_kernel<D>, dim3(a.H, a.T), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int attn_splits(int n_ctx) { return (n_ctx + kSplitP - 1) / kSplitP; }

int attn_launch(const AttnArgs &a, hipStream_t st) {
    if (a.H % a.Hkv || a.H / a.Hkv > kMaxGroup || a.n_rot > a.D || a.n_rot % 2 || a.n_split != attn_splits(a.n_ctx) ||
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
