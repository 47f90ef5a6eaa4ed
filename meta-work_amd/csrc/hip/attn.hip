// Gated GQA attention over the fp16 KV cache (gfx950).
//
// Computes attn_full of src/xiaoju-pipe/core/xj_cpu.c:83-151 after the q/k/v
// projections, with the cache in fp16 as the Metal backend keeps it
// (xj_kernels.metal:440-452):
//   kv_store_kernel  one work-group per (token, kv head): RMSNorm(k_norm) of the
//                    new key (double sum, x*sc*w), NeoX RoPE of the first n_rot
//                    dims (xj_cpu.c:68-77; theta = pos * inv_freq[i] with
//                    inv_freq = base^(-2i/n_rot) computed on the host exactly as
//                    the reference's powf), then k and v rounded to fp16 (RNE)
//                    and stored at position n_past + t.
//   attn_part_kernel one work-group per (query head, token, 64-position split):
//                    q_norm + RoPE, scores q.k_j * scale (16-lane teams, one
//                    position per team), the split's max, sum of exponentials
//                    and unnormalised sum_j e_j v_j (positions in order)
//   attn_combine     merges the splits with the usual max rescaling, divides
//                    by the total, applies sigmoid(gate) (xj_cpu.c:128-147:
//                    the same softmax(qK^T/sqrt(D)) V, reassociated by split)
//                    and, when asked, writes the wo GEMV's prepared activations.
// Query rows are [q(D) | gate(D)] per head (xj_cpu.c:118); kv head = h / (H/Hkv).
#include "common.h"
#include "kernels.h"
#include "xq.h"

namespace xjk {

template <int D>
__global__ __launch_bounds__(256) void kv_store_kernel(const AttnArgs a) {
    const int t = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    __shared__ float kk[D];
    __shared__ double red[4];
    const int pos = *a.npast + t, nk = a.Hkv * D;
    const float *kr = a.kn + (int64_t)t * a.kn_s + g * D, *vr = a.vn + (int64_t)t * a.vn_s + g * D;
    double ss = 0;
    for (int i = tid; i < D; i += 256) ss += (double)kr[i] * kr[i];
    ss = xjd::block_sum_d(ss, red);
    const float sc = 1.0f / sqrtf((float)(ss / D) + a.eps);
    for (int i = tid; i < D; i += 256) kk[i] = kr[i] * sc * a.knorm_w[i];
    __syncthreads();
    const int half = a.n_rot / 2;
    for (int i = tid; i < half; i += 256) {
        const float theta = (float)pos * a.inv_freq[i];
        const float c = (float)cos((double)theta), s = (float)sin((double)theta);
        const float x0 = kk[i], x1 = kk[i + half];
        kk[i] = x0 * c - x1 * s;
        kk[i + half] = x0 * s + x1 * c;
    }
    __syncthreads();
    uint16_t *kd = a.kc + (int64_t)pos * nk + g * D, *vd = a.vc + (int64_t)pos * nk + g * D;
    for (int i = tid; i < D; i += 256) {
        kd[i] = xjd::f32_to_f16(kk[i]);
        vd[i] = xjd::f32_to_f16(vr[i]);
    }
}

// Split-K decode attention. Work-group (h, t, s) covers positions
// [s*P, min(s*P+P, pos+1)) of query head h, token t: it writes the split's
// maximum score m_s, l_s = sum_j exp(s_j - m_s) and the unnormalised
// o_s = sum_j exp(s_j - m_s) v_j (positions in order). Splits past pos exit.
// The grid covers n_ctx, so one captured graph serves every decode position.
constexpr int kSplitP = 64;

template <int D>
__global__ __launch_bounds__(256) void attn_part_kernel(const AttnArgs a) {
    constexpr int DL = D / 16;
    const int h = blockIdx.x, t = blockIdx.y, sp = blockIdx.z, tid = threadIdx.x;
    const int team = tid >> 4, l16 = tid & 15;
    const int kvh = h / (a.H / a.Hkv), nk = a.Hkv * D;
    const int pos = *a.npast + t, j0 = sp * kSplitP;
    if (j0 > pos) return;                       // uniform per work-group
    const int j1 = j0 + kSplitP - 1 < pos ? j0 + kSplitP - 1 : pos;
    __shared__ float q[D];
    __shared__ float e[kSplitP];
    __shared__ double red[4];
    __shared__ float redf[4];
    const float *qr = a.qg + (int64_t)t * a.qg_s + (int64_t)h * 2 * D;
    double ss = 0;
    for (int i = tid; i < D; i += 256) ss += (double)qr[i] * qr[i];
    ss = xjd::block_sum_d(ss, red);
    const float sc = 1.0f / sqrtf((float)(ss / D) + a.eps);
    for (int i = tid; i < D; i += 256) q[i] = qr[i] * sc * a.qnorm_w[i];
    __syncthreads();
    const int half = a.n_rot / 2;
    for (int i = tid; i < half; i += 256) {
        const float theta = (float)pos * a.inv_freq[i];
        const float c = (float)cos((double)theta), s = (float)sin((double)theta);
        const float x0 = q[i], x1 = q[i + half];
        q[i] = x0 * c - x1 * s;
        q[i + half] = x0 * s + x1 * c;
    }
    __syncthreads();
    float qv[DL];
#pragma unroll
    for (int d = 0; d < DL; d++) qv[d] = q[l16 * DL + d];
    float mx = -INFINITY;
    for (int j = j0 + team; j <= j1; j += 16) {
        const uint16_t *kp = a.kc + (int64_t)j * nk + kvh * D + l16 * DL;
        float s = 0.f;
#pragma unroll
        for (int d = 0; d < DL; d++) s = fmaf(qv[d], xjd::f16_to_f32(kp[d]), s);
        s = xjd::row16_sum(s) * a.scale;
        if (l16 == 0) e[j - j0] = s;
        mx = fmaxf(mx, s);
    }
    mx = xjd::block_max(mx, redf);
    __syncthreads();
    const int n = j1 - j0 + 1;
    float lsum = 0.f;
    if (tid < 64) {
        const float ev = tid < n ? expf(e[tid] - mx) : 0.f;
        if (tid < n) e[tid] = ev;
        lsum = ev;
        for (int off = 32; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off, 64);
    }
    __syncthreads();
    float *part = a.scores + (((int64_t)t * a.H + h) * a.n_split + sp) * (D + 2);
    for (int d = tid; d < D; d += 256) {
        const uint16_t *vp = a.vc + (int64_t)j0 * nk + kvh * D + d;
        float o = 0.f;
        for (int j = 0; j < n; j++) o = fmaf(e[j], xjd::f16_to_f32(vp[(int64_t)j * nk]), o);
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
        float M = -INFINITY;
        for (int s = tid; s < ns; s += 64) M = fmaxf(M, part[(int64_t)s * (D + 2)]);
        for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        float L = 0.f;
        for (int s = 0; s < ns; s++) {   // fixed order: every thread forms the same sum
            const float ws = expf(part[(int64_t)s * (D + 2)] - M);
            if (tid == 0 && s < 64) w[s] = ws;
            L = fmaf(ws, part[(int64_t)s * (D + 2) + 1], L);
        }
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
        for (int s = 0; s < ns; s++) {
            const float ws = ns > 64 ? expf(part[(int64_t)s * (D + 2)] - M2) : w[s];
            o = fmaf(ws, part[(int64_t)s * (D + 2) + 2 + d], o);
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
    if (a.H % a.Hkv || a.n_rot > a.D || a.n_rot % 2 || a.n_split != attn_splits(a.n_ctx)) return -1;
    switch (a.D) {
    case 64: return launch_d<64>(a, st);
    case 128: return launch_d<128>(a, st);
    case 256: return launch_d<256>(a, st);
    default: return -1;
    }
}

}  // namespace xjk
