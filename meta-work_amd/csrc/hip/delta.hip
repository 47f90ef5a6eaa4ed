// Gated DeltaNet recurrent update (gfx950).
//
// delta_head_kernel: the per-token body of attn_linear (src/xiaoju-pipe/core/xj_cpu.c:183-219)
// after the conv (which the qkv GEMV epilogue already applied): L2-normalise
// q and k of key head hk = hv % Hk (double sum, x / sqrt(sum + eps)), then for
// every value row j of head hv
//     S_j <- exp(softplus(alpha + dt) * A) * S_j
//     delta_j = (v_j - S_j . k) * sigmoid(beta)
//     S_j <- S_j + k * delta_j,   o_j = (S_j . q) / sqrt(S)
// With a.xq set, the kernel also applies the gated RMSNorm of o
// (xj_cpu.c:215-217) and writes the ssm_out GEMV's prepared activations, so
// that GEMV needs no prep launch.
//
// Mapping: one work-group per value head; a 16-lane team owns S/64 rows, and
// each lane keeps S/16 consecutive entries of each in registers across all T
// tokens, so the 64 KB (S=128) head state is read and written once per call.
// Per element the updates are the reference's own: m*eg, fma(m, k, sk),
// fma(k, delta, m), fma(m, q, acc); only the 16 lane partial sums are combined
// in a fixed butterfly instead of one running sum. With keep, the state after
// each token t < keep_n is written to checkpoint t (xj_cpu.c:218).
//
// delta_part_kernel: the same per row, split over 32-row work-groups (below).
//
// delta_rec_kernel: the same rule with decay and beta given per token and head
// (the standalone layer test), q and k used as given.
#include "common.h"
#include "kernels.h"
#include "xq.h"

namespace xjk {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int S>
__device__ __forceinline__ void load_row(const float *p, float (&m)[S / 16]) {
#pragma unroll
    for (int i = 0; i < S / 16; i += 4) {
        const f32x4 v = *(const f32x4 *)(p + i);
        m[i] = v.x; m[i + 1] = v.y; m[i + 2] = v.z; m[i + 3] = v.w;
    }
}
template <int S>
__device__ __forceinline__ void store_row(float *p, const float (&m)[S / 16]) {
#pragma unroll
    for (int i = 0; i < S / 16; i += 4) {
        f32x4 v = {m[i], m[i + 1], m[i + 2], m[i + 3]};
        *(f32x4 *)(p + i) = v;
    }
}

// one token of the rule for the row held in m; returns o_j (unscaled) in every lane
template <int S>
__device__ __forceinline__ float rule_step(float (&m)[S / 16], const float *ks, const float *qs, int i0,
                                           float eg, float b, float vj) {
    constexpr int IPL = S / 16;
    float sk = 0.f;
#pragma unroll
    for (int i = 0; i < IPL; i++) {
        m[i] = m[i] * eg;
        sk = fmaf(m[i], ks[i0 + i], sk);
    }
    sk = xjd::row16_sum(sk);
    const float delta = (vj - sk) * b;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < IPL; i++) {
        m[i] = fmaf(ks[i0 + i], delta, m[i]);
        acc = fmaf(m[i], qs[i0 + i], acc);
    }
    return xjd::row16_sum(acc);
}

// 1024 threads: team r16 = tid / 16 (of 64) owns rows j = r16 + 64 * r,
// r < S / 64, so 16 wavefronts share the head's latency; every operand of a
// token is loaded at once. The work-group holds all of the head's outputs, so
// the gated RMSNorm needs no hand-off between work-groups.
template <int S>
__global__ __launch_bounds__(1024) void delta_head_kernel(const DeltaArgs a) {
    constexpr int IPL = S / 16, NR = S / 64, NW = 1024 / 64;
    const int hv = blockIdx.x, tid = threadIdx.x, r16 = tid >> 4, l16 = tid & 15, i0 = l16 * IPL;
    const int hk = hv % a.Hk;
    __shared__ float qs[S], ks[S], os[S];
    __shared__ double red[2 * NW];
    float m[NR][IPL];
#pragma unroll
    for (int r = 0; r < NR; r++) load_row<S>(a.state + ((int64_t)hv * S + r16 + 64 * r) * S + i0, m[r]);
    const float dt = a.dt[hv], A = a.A[hv];
    const bool in = tid < S;
    const float nw = a.norm_w && in ? a.norm_w[tid] : 0.f;
    for (int t = 0; t < a.T; t++) {
        const float *row = a.qkv + (int64_t)t * a.qkv_s;
        const float qv = in ? row[hk * S + tid] : 0.f, kv = in ? row[a.k_off + hk * S + tid] : 0.f;
        const float bt = a.beta[(int64_t)t * a.beta_s + hv], al = a.alpha[(int64_t)t * a.alpha_s + hv];
        float vj[NR];
#pragma unroll
        for (int r = 0; r < NR; r++) vj[r] = row[a.v_off + hv * S + r16 + 64 * r];
        const float zv = a.xq && in ? a.z[(int64_t)t * a.z_s + hv * S + tid] : 0.f;
        // the q and k sums over the S threads that hold them (S / 64 wavefronts)
        __syncthreads();   // red and qs / ks of the previous token consumed
        const double sq = xjd::head_sum_d<(S + 63) / 64>((double)qv * qv, red);
        const double sk2 = xjd::head_sum_d<(S + 63) / 64>((double)kv * kv, red + 4);
        if (in) {
            qs[tid] = qv * (1.0f / sqrtf((float)sq + a.eps));
            ks[tid] = kv * (1.0f / sqrtf((float)sk2 + a.eps));
        }
        const float b = xjd::sigm(bt);
        const float eg = expf(xjd::softplus(al + dt) * A);
        __syncthreads();
#pragma unroll
        for (int r = 0; r < NR; r++) {
            const float o = rule_step<S>(m[r], ks, qs, i0, eg, b, vj[r]) * a.qscale;
            const int j = r16 + 64 * r;
            if (l16 == 0) {
                os[j] = o;
                a.out[(int64_t)t * a.out_s + hv * S + j] = o;
            }
            if (t < a.keep_n) store_row<S>(a.ck + (((int64_t)t * a.Hv + hv) * S + j) * S + i0, m[r]);
        }
        __syncthreads();
        if (a.xq) {
            // gated RMSNorm (xj_cpu.c:215-217) of the head's outputs into the
            // ssm_out GEMV's prepared activations
            const float ov = in ? os[tid] : 0.f;
            const double ss = xjd::head_sum_d<(S + 63) / 64>((double)ov * ov, red + 8);
            const float gsc = 1.0f / sqrtf((float)(ss / S) + a.eps);
            if (tid < (S + 63) / 64 * 64) {   // wavefronts holding outputs
                const XqOff o = xq_off(a.Hv * S);
                const float v = in ? ov * gsc * nw * xjd::silu(zv) : 0.f;
                xjd::emit_xq(v, hv * S + tid, in, a.xq + (int64_t)t * o.stride, o);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < NR; r++) store_row<S>(a.state + ((int64_t)hv * S + r16 + 64 * r) * S + i0, m[r]);
}

// The same update split over value rows: work-group (hv, p) owns the 32 rows
// p*32 .. p*32+31 of head hv (one activation group), 16 lanes per row; q and
// k are normalised by every work-group of the head. The gated RMSNorm couples
// the head's rows, so with a.xq set each work-group writes the digits of
// u_j = o_j * norm_w_j * silu(z_j) for its group and the group's sum of o_j^2
// (double, fixed order) into the group's ss field; the ssm_out GEMV
// (PRO_HEADRMS) folds 1/sqrt(sum over the head's groups / S + eps) into the
// head's group scales - the same product in another order.
template <int S>
__global__ __launch_bounds__(512) void delta_part_kernel(const DeltaArgs a) {
    constexpr int IPL = S / 16, RW = 32;
    const int hv = blockIdx.x, p = blockIdx.y, tid = threadIdx.x, team = tid >> 4, l16 = tid & 15, i0 = l16 * IPL;
    const int hk = hv % a.Hk, j = p * RW + team;
    // the kernel arguments of the token loop read together, with the state
    // (each read would otherwise be waited for in turn before the inputs are
    // requested)
    asm volatile("" ::"s"(a.qkv), "s"(a.qkv_s), "s"(a.k_off), "s"(a.v_off), "s"(a.beta), "s"(a.beta_s), "s"(a.alpha),
                 "s"(a.alpha_s), "s"(a.out), "s"(a.out_s), "s"(a.T), "s"(a.xq), "s"(a.z), "s"(a.z_s), "s"(a.norm_w),
                 "s"(a.keep_n), "s"(a.dt), "s"(a.A));
    __shared__ float qs[S], ks[S], os[RW];
    __shared__ double red[16];
    float m[IPL];
    load_row<S>(a.state + ((int64_t)hv * S + j) * S + i0, m);
    const float dt = a.dt[hv], A = a.A[hv];
    const bool in = tid < S;
    const bool emit = a.xq && tid < RW;   // lanes of wavefront 0 that emit the group
    const float nw = emit ? a.norm_w[p * RW + tid] : 0.f;
    for (int t = 0; t < a.T; t++) {
        const float *row = a.qkv + (int64_t)t * a.qkv_s;
        const float qv = in ? row[hk * S + tid] : 0.f, kv = in ? row[a.k_off + hk * S + tid] : 0.f;
        const float bt = a.beta[(int64_t)t * a.beta_s + hv], al = a.alpha[(int64_t)t * a.alpha_s + hv];
        const float vj = row[a.v_off + hv * S + j];
        const float zv = emit ? a.z[(int64_t)t * a.z_s + hv * S + p * RW + tid] : 0.f;
        __syncthreads();   // red and qs / ks / os of the previous token consumed
        const double sq = xjd::head_sum_d<(S + 63) / 64>((double)qv * qv, red);
        const double sk2 = xjd::head_sum_d<(S + 63) / 64>((double)kv * kv, red + 4);
        if (in) {
            qs[tid] = qv * (1.0f / sqrtf((float)sq + a.eps));
            ks[tid] = kv * (1.0f / sqrtf((float)sk2 + a.eps));
        }
        const float b = xjd::sigm(bt);
        const float eg = expf(xjd::softplus(al + dt) * A);
        __syncthreads();
        const float o = rule_step<S>(m, ks, qs, i0, eg, b, vj) * a.qscale;
        if (l16 == 0) {
            os[team] = o;
            a.out[(int64_t)t * a.out_s + hv * S + j] = o;
        }
        if (t < a.keep_n) store_row<S>(a.ck + (((int64_t)t * a.Hv + hv) * S + j) * S + i0, m);
        if (a.xq) {
            __syncthreads();
            if (tid < 64) {   // wavefront 0: lanes 0..31 hold the group
                const XqOff o = xq_off(a.Hv * S);
                const float ov = emit ? os[tid] : 0.f;
                const double ss = xjd::group_ss(ov);
                const int k = hv * S + p * RW + tid;
                uint8_t *dst = a.xq + (int64_t)t * o.stride;
                xjd::emit_xq(emit ? ov * nw * xjd::silu(zv) : 0.f, k, emit, dst, o);
                if (tid == 0) ((double *)(dst + o.ss_off))[k >> 5] = ss;
            }
        }
    }
    store_row<S>(a.state + ((int64_t)hv * S + j) * S + i0, m);
}

// Work-group (t, hv), S threads (element i): the inputs of the chunked rule
// with the recurrent kernels' expressions (head_sum_d over the same S
// threads, x * (1 / sqrt(sum + eps)), expf(softplus(alpha + dt) * A), sigm).
template <int S>
__global__ __launch_bounds__(S) void delta_prefill_prep_kernel(const DeltaPrepArgs a) {
    const int t = blockIdx.x, hv = blockIdx.y, i = threadIdx.x, hk = hv % a.Hk;
    __shared__ double red[8];
    const float *row = a.qkv + (int64_t)t * a.qkv_s;
    const float qv = row[hk * S + i], kv = row[a.k_off + hk * S + i];
    const double sq = xjd::head_sum_d<S / 64>((double)qv * qv, red);
    const double sk2 = xjd::head_sum_d<S / 64>((double)kv * kv, red + 4);
    const int64_t o = ((int64_t)t * a.Hv + hv) * S + i;
    a.q[o] = qv * (1.0f / sqrtf((float)sq + a.eps));
    a.k[o] = kv * (1.0f / sqrtf((float)sk2 + a.eps));
    a.v[o] = row[a.v_off + hv * S + i];
    if (i == 0) {
        a.decay[(int64_t)t * a.Hv + hv] = expf(xjd::softplus(a.alpha[(int64_t)t * a.alpha_s + hv] + a.dt[hv]) * a.A[hv]);
        a.bt[(int64_t)t * a.Hv + hv] = xjd::sigm(a.beta[(int64_t)t * a.beta_s + hv]);
    }
}

int delta_prefill_prep_launch(const DeltaPrepArgs &a, hipStream_t st) {
    if (a.T < 1 || a.Hk < 1 || a.Hv < 1) return -1;
    if (a.S == 128) hipLaunchKernelGGL(delta_prefill_prep_kernel<128>, dim3(a.T, a.Hv), dim3(128), 0, st, a);
    else if (a.S == 64) hipLaunchKernelGGL(delta_prefill_prep_kernel<64>, dim3(a.T, a.Hv), dim3(64), 0, st, a);
    else return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int S>
__global__ __launch_bounds__(256) void delta_rec_kernel(int H, int T, const float *q, const float *k, const float *v,
                                                        const float *decay, const float *beta, float qscale,
                                                        float *state, float *out) {
    constexpr int IPL = S / 16;
    const int hh = blockIdx.x, tid = threadIdx.x;
    const int j = blockIdx.y * 16 + (tid >> 4), l16 = tid & 15, i0 = l16 * IPL;
    __shared__ float qs[S], ks[S];
    float m[IPL];
    float *Mp = state + ((int64_t)hh * S + j) * S + i0;
    load_row<S>(Mp, m);
    for (int t = 0; t < T; t++) {
        const int64_t base = ((int64_t)t * H + hh) * S;
        if (tid < S) { qs[tid] = q[base + tid]; ks[tid] = k[base + tid]; }
        __syncthreads();
        const float o = rule_step<S>(m, ks, qs, i0, decay[(int64_t)t * H + hh], beta[(int64_t)t * H + hh], v[base + j]);
        if (l16 == 0) out[base + j] = o * qscale;
        __syncthreads();
    }
    store_row<S>(Mp, m);
}

int delta_launch(const DeltaArgs &a, hipStream_t st) {
    if (a.xq && (!a.z || !a.norm_w)) return -1;
    if (a.split) {   // one work-group per 32 value rows; the norm's scale is left to the consumer
        if (a.S == 128) hipLaunchKernelGGL(delta_part_kernel<128>, dim3(a.Hv, 4), dim3(512), 0, st, a);
        else if (a.S == 64) hipLaunchKernelGGL(delta_part_kernel<64>, dim3(a.Hv, 2), dim3(512), 0, st, a);
        else return -1;
    } else if (a.S == 128) {
        hipLaunchKernelGGL(delta_head_kernel<128>, dim3(a.Hv), dim3(1024), 0, st, a);
    } else if (a.S == 64) {
        hipLaunchKernelGGL(delta_head_kernel<64>, dim3(a.Hv), dim3(1024), 0, st, a);
    } else {
        return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int delta_recurrent_launch(int H, int S, int T, const float *q, const float *k, const float *v, const float *decay,
                           const float *beta, float qscale, float *state, float *out, hipStream_t st) {
    if (S == 128)
        hipLaunchKernelGGL(delta_rec_kernel<128>, dim3(H, 128 / 16), dim3(256), 0, st, H, T, q, k, v, decay, beta, qscale, state, out);
    else if (S == 64)
        hipLaunchKernelGGL(delta_rec_kernel<64>, dim3(H, 64 / 16), dim3(256), 0, st, H, T, q, k, v, decay, beta, qscale, state, out);
    else
        return -1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace xjk
