// Fused dequant-GEMV for gfx950 (Q4_K / Q6_K / Q8_0 / F32), 1..8 activation rows.
//
// Computes the reference's matmul (src/xiaoju-pipe/core/xj_cpu.c:36-54,
// y[t][r] = dot(dequant(W[r]), x[t])) with the neighbouring element-wise work
// folded in:
//   prologue (activations into LDS): RMSNorm (xj_cpu.c:56-61, double sum),
//     SwiGLU silu(g)*u (xj_cpu.c:273), per-head gated RMSNorm
//     norm(o)*w*silu(z) (xj_cpu.c:215-217)
//   epilogue: store, residual add (xj_cpu.c:268,275), depthwise causal conv +
//     SiLU with state carry and checkpoints (xj_cpu.c:172-182,220), and greedy
//     argmax partials for the LM head (xj_spec.c:12-16 tie rule).
// One launch serves up to four weight segments that share K (e.g. qkv, gate,
// beta and alpha of a DeltaNet layer) so a layer needs few launches.
//
// Work mapping. A team of TS lanes (16, 32 or 64, chosen from K so that each
// lane owns about four 32-element chunks) owns one row; a 256-thread
// work-group holds 256/TS teams. One chunk is 16 B of Q4_K nibbles (+ the
// block header), 3 x 8 B of Q6_K planes, 32 B of Q8_0 quants or 128 B of F32.
// A lane loads all of its chunks (up to NPF) before using any, and the first
// round is issued before the activations are staged in LDS, so the weight
// latency overlaps the prologue. Quantized products are factored per
// sub-block, sum_l (d*sc*q_l - dmin*m) x_l = d*sc*sum q_l x_l - dmin*m*sum x_l,
// with the sums of x precomputed per 8 elements in the prologue. Lane partials
// are combined in a fixed butterfly (DPP within 16 lanes, then cross-row
// shuffles), so a row's result does not depend on T, on the grid, or on which
// work-group computed it. Work-groups loop over row groups when there are
// more than eight per CU, so the LDS fill is amortised on the LM head.
#include "common.h"
#include "dequant.h"
#include "kernels.h"
#include "xj_hip.h"

#include <cstring>
#include <vector>

namespace xjk {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

static int g_lds_max = 64 * 1024;
static int g_grid_cap = 256 * 8;

// x is stored in LDS with 4 floats of padding per 64 so that the chunk
// pattern of a team spreads over the banks.
__device__ __forceinline__ int xpad(int e) { return e + 4 * (e >> 6); }
__host__ __device__ inline int kpad(int K) { return K + 4 * ((K + 63) / 64); }

// byte i of w as float (selected into one v_cvt_f32_ubyte{0..3})
__device__ __forceinline__ float ub(uint32_t w, int i) { return (float)((w >> (8 * i)) & 0xFFu); }

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

// s = sum_i bytes(w)[i] * x[i] over 4 elements, in order
__device__ __forceinline__ float dot4(uint32_t w, f32x4 x, float s) {
    s = fmaf(ub(w, 0), x.x, s);
    s = fmaf(ub(w, 1), x.y, s);
    s = fmaf(ub(w, 2), x.z, s);
    s = fmaf(ub(w, 3), x.w, s);
    return s;
}

// Raw bytes of one 32-element chunk, fetched ahead of use (9 dwords):
//   Q4_K  r0..3 block header (d|dmin, 12 scale bytes), r4..7 the chunk's 16 nibble bytes
//   Q6_K  r0..1 ql (low-half group), r2..3 ql (+32), r4..5 qh, r6..7 the half's 8 scales, r8 d
//   Q8_0  r0..7 the 32 quants, r8 d
struct Raw {
    uint32_t r[9];
};

__device__ __forceinline__ void put4(uint32_t *d, u32x4 v) { d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w; }
__device__ __forceinline__ void put2(uint32_t *d, u32x2 v) { d[0] = v.x; d[1] = v.y; }

// chunk c of a row whose first block index is rowblk (row * blocks_per_row)
__device__ __forceinline__ void load_chunk(uint32_t type, const uint8_t *__restrict__ W, int64_t nblk, int64_t rowblk,
                                           int c, Raw &raw) {
    if (type == XJ_Q4_K) {
        const uint8_t *blk = W + (rowblk + (c >> 3)) * 144;
        put4(raw.r, __builtin_nontemporal_load((const u32x4 *)blk));
        put4(raw.r + 4, __builtin_nontemporal_load((const u32x4 *)(blk + 16 + 16 * (c & 7))));
    } else if (type == XJ_Q6_K) {
        const int q = c & 7, h = q >> 2, l0 = (q & 3) * 8;
        const int64_t g = rowblk + (c >> 3);
        const uint8_t *ql = W + g * 128 + 64 * h + l0;
        put2(raw.r, __builtin_nontemporal_load((const u32x2 *)ql));
        put2(raw.r + 2, __builtin_nontemporal_load((const u32x2 *)(ql + 32)));
        put2(raw.r + 4, __builtin_nontemporal_load((const u32x2 *)(W + nblk * 128 + g * 64 + 32 * h + l0)));
        put2(raw.r + 6, __builtin_nontemporal_load((const u32x2 *)(W + nblk * 192 + g * 16 + 8 * h)));
        raw.r[8] = *(const uint16_t *)(W + nblk * 208 + g * 2);
    } else {  // Q8_0
        const int64_t g = rowblk + c;
        put4(raw.r, __builtin_nontemporal_load((const u32x4 *)(W + g * 32)));
        put4(raw.r + 4, __builtin_nontemporal_load((const u32x4 *)(W + g * 32 + 16)));
        raw.r[8] = *(const uint16_t *)(W + nblk * 32 + g * 2);
    }
}

// acc[t] += sum over the chunk's 32 elements of dequant(w) * x[t]
template <int T>
__device__ __forceinline__ void dot_q4k(const Raw &raw, int c, const float *xl, const float *xs8, int KP, int K8, float (&acc)[T]) {
    const int q = c & 7, p = q >> 1, jm = (2 * p) & 3;
    const bool hi4 = p >= 2;
    const int e0 = (c >> 3) * 256 + 64 * p + (q & 1) * 16;
    const float d = xjd::f16_to_f32(raw.r[0] & 0xFFFFu), dmin = xjd::f16_to_f32(raw.r[0] >> 16);
    float ds[2], dm[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint32_t A = byte_of(raw.r[1], jm + s), B = byte_of(raw.r[2], jm + s), C = byte_of(raw.r[3], jm + s);
        const uint32_t sc = hi4 ? ((C & 0xF) | ((A >> 6) << 4)) : (A & 63);
        const uint32_t mn = hi4 ? ((C >> 4) | ((B >> 6) << 4)) : (B & 63);
        ds[s] = d * (float)sc;
        dm[s] = dmin * (float)mn;
    }
    float s0[T], s1[T];
#pragma unroll
    for (int t = 0; t < T; t++) { s0[t] = 0.f; s1[t] = 0.f; }
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const uint32_t w = raw.r[4 + u];
        const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int t = 0; t < T; t++) {
            const f32x4 xa = *(const f32x4 *)(xl + t * KP + xpad(e0 + 4 * u));
            const f32x4 xb = *(const f32x4 *)(xl + t * KP + xpad(e0 + 32 + 4 * u));
            s0[t] = dot4(lo, xa, s0[t]);
            s1[t] = dot4(hi, xb, s1[t]);
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++) {
        const float xsa = xs8[t * K8 + (e0 >> 3)] + xs8[t * K8 + (e0 >> 3) + 1];
        const float xsb = xs8[t * K8 + ((e0 + 32) >> 3)] + xs8[t * K8 + ((e0 + 32) >> 3) + 1];
        acc[t] += ds[0] * s0[t] - dm[0] * xsa + (ds[1] * s1[t] - dm[1] * xsb);
    }
}

template <int T>
__device__ __forceinline__ void dot_q6k(const Raw &raw, int c, const float *xl, const float *xs8, int KP, int K8, float (&acc)[T]) {
    const int q = c & 7, h = q >> 2, l0 = (q & 3) * 8, is = l0 >> 4;
    const int e0 = (c >> 3) * 256 + 128 * h + l0;
    const float d = xjd::f16_to_f32(raw.r[8]);
    float dsc[4];
#pragma unroll
    for (int G = 0; G < 4; G++) {
        const int bi = is + 2 * G;
        dsc[G] = d * (float)(int8_t)byte_of(bi < 4 ? raw.r[6] : raw.r[7], bi & 3);
    }
    float sq[T][4];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int G = 0; G < 4; G++) sq[t][G] = 0.f;
#pragma unroll
    for (int v = 0; v < 2; v++) {
        const uint32_t la = raw.r[v], lb = raw.r[2 + v], hb = raw.r[4 + v];
#pragma unroll
        for (int G = 0; G < 4; G++) {
            const uint32_t nib = (G == 0) ? (la & 0x0F0F0F0Fu) : (G == 1) ? (lb & 0x0F0F0F0Fu)
                               : (G == 2) ? ((la >> 4) & 0x0F0F0F0Fu) : ((lb >> 4) & 0x0F0F0F0Fu);
            const uint32_t q6 = nib | (((hb >> (2 * G)) & 0x03030303u) << 4);
#pragma unroll
            for (int t = 0; t < T; t++)
                sq[t][G] = dot4(q6, *(const f32x4 *)(xl + t * KP + xpad(e0 + 32 * G + 4 * v)), sq[t][G]);
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int G = 0; G < 4; G++) acc[t] += dsc[G] * (sq[t][G] - 32.0f * xs8[t * K8 + ((e0 + 32 * G) >> 3)]);
}

template <int T>
__device__ __forceinline__ void dot_q80(const Raw &raw, int c, const float *xl, int KP, float (&acc)[T]) {
    const int e0 = c * 32;
    const float d = xjd::f16_to_f32(raw.r[8]);
    float s[T];
#pragma unroll
    for (int t = 0; t < T; t++) s[t] = 0.f;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const uint32_t w = raw.r[u];
#pragma unroll
        for (int t = 0; t < T; t++) {
            const f32x4 xv = *(const f32x4 *)(xl + t * KP + xpad(e0 + 4 * u));
            float a = s[t];
            a = fmaf((float)(int8_t)(w & 0xFF), xv.x, a);
            a = fmaf((float)(int8_t)((w >> 8) & 0xFF), xv.y, a);
            a = fmaf((float)(int8_t)((w >> 16) & 0xFF), xv.z, a);
            a = fmaf((float)(int8_t)(w >> 24), xv.w, a);
            s[t] = a;
        }
    }
#pragma unroll
    for (int t = 0; t < T; t++) acc[t] += d * s[t];
}

template <int T>
__device__ __forceinline__ void dot_f32(const uint8_t *__restrict__ W, int K, int64_t row, int c, const float *xl, int KP,
                                        float (&acc)[T]) {
    const int e0 = c * 32;
#pragma unroll
    for (int u = 0; u < 8; u++) {
        const f32x4 w = __builtin_nontemporal_load((const f32x4 *)(W + (row * K + e0 + 4 * u) * 4));
#pragma unroll
        for (int t = 0; t < T; t++) {
            const f32x4 xv = *(const f32x4 *)(xl + t * KP + xpad(e0 + 4 * u));
            float a = acc[t];
            a = fmaf(w.x, xv.x, a);
            a = fmaf(w.y, xv.y, a);
            a = fmaf(w.z, xv.z, a);
            a = fmaf(w.w, xv.w, a);
            acc[t] = a;
        }
    }
}

// ------------------------------------------------------------ prologue --
template <int T>
__device__ void prologue(const GArgs &a, float *xl, float *xs8, float *gsc, int KP, int K8) {
    const int K = a.K, tid = threadIdx.x;
    __shared__ double red[4];
    if (a.pro == PRO_RMS) {
        for (int t = 0; t < T; t++) {
            const float *x = a.x + (int64_t)t * a.xs;
            double ss = 0;
            for (int k = tid; k < K; k += 256) ss += (double)x[k] * x[k];
            ss = xjd::block_sum_d(ss, red);
            const float sc = 1.0f / sqrtf((float)(ss / K) + a.eps);
            for (int k = tid; k < K; k += 256) xl[t * KP + xpad(k)] = x[k] * sc * a.pro_w[k];
        }
    } else if (a.pro == PRO_SWIGLU) {
        for (int t = 0; t < T; t++) {
            const float *g = a.x + (int64_t)t * a.xs, *u = a.x2 + (int64_t)t * a.x2s;
            for (int k = tid; k < K; k += 256) xl[t * KP + xpad(k)] = xjd::silu(g[k]) * u[k];
        }
    } else if (a.pro == PRO_GATED_RMS) {
        // one wavefront per (token, group); group = head size S
        const int G = a.group, ng = K / G, w = tid >> 6, ln = tid & 63;
        for (int tg = w; tg < T * ng; tg += 4) {
            const int t = tg / ng, g = tg % ng;
            const float *o = a.x + (int64_t)t * a.xs + g * G;
            double ss = 0;
            for (int k = ln; k < G; k += 64) ss += (double)o[k] * o[k];
            ss = xjd::wave_sum_d(ss);
            if (ln == 0) gsc[tg] = 1.0f / sqrtf((float)(ss / G) + a.eps);
        }
        __syncthreads();
        for (int t = 0; t < T; t++) {
            const float *o = a.x + (int64_t)t * a.xs, *z = a.x2 + (int64_t)t * a.x2s;
            for (int k = tid; k < K; k += 256)
                xl[t * KP + xpad(k)] = o[k] * gsc[t * ng + k / G] * a.pro_w[k % G] * xjd::silu(z[k]);
        }
    } else {
        for (int t = 0; t < T; t++) {
            const float *x = a.x + (int64_t)t * a.xs;
            for (int k = tid; k < K; k += 256) xl[t * KP + xpad(k)] = x[k];
        }
    }
    __syncthreads();
    for (int i = tid; i < T * K8; i += 256) {
        const int t = i / K8, g = i % K8;
        const float *p = xl + t * KP + xpad(8 * g);   // 8 consecutive elements never straddle a pad
        xs8[i] = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    }
    __syncthreads();
}

// Team reduction over TS lanes (16, 32 or 64) in a fixed order.
template <int TS>
__device__ __forceinline__ float team_sum(float v) {
    v = xjd::row16_sum(v);
    if (TS >= 32) v += __shfl_xor(v, 16, 64);
    if (TS >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// -------------------------------------------------------------- kernel --
// A row group is 256/TS rows, one per TS-lane team. Lanes take chunks
// c = lane, lane+TS, ...; NPF of them are loaded before any is used, and the
// first round of the first row group is issued before the LDS prologue so
// both latencies overlap.
constexpr int NPF = 5;

template <int T, int TS>
__global__ __launch_bounds__(256) void gemv_kernel(const GArgs a) {
    extern __shared__ float lds[];
    constexpr int NT = 256 / TS;
    __shared__ unsigned long long amax_sh[NT][T];
    const int K = a.K, KP = kpad(K), K8 = K / 8, nch = K / 32;
    const int tid = threadIdx.x, team = tid / TS, lane = tid % TS;
    float *xl = lds, *xs8 = lds + T * KP, *gsc = xs8 + T * K8;
    const int n_rg = a.seg[a.nseg - 1].wg0 + a.seg[a.nseg - 1].nwg;

    auto seg_of = [&](int rg) {
        int si = 0;
        while (si + 1 < a.nseg && rg >= a.seg[si + 1].wg0) si++;
        return si;
    };
    auto row_of = [&](const GSeg &sg, int rg) {
        const int64_t r = (int64_t)(rg - sg.wg0) * NT + team;
        return r < sg.n_rows ? r : (int64_t)sg.n_rows - 1;
    };

    Raw raw[NPF];
    int rg = blockIdx.x;
    if (rg < n_rg) {   // first round of the first row group, before the prologue
        const GSeg &sg = a.seg[seg_of(rg)];
        if (sg.type != XJ_F32) {
            const int64_t rowblk = row_of(sg, rg) * (sg.type == XJ_Q8_0 ? K / 32 : K / 256);
#pragma unroll
            for (int i = 0; i < NPF; i++) {
                const int c = lane + i * TS;
                if (c < nch) load_chunk(sg.type, sg.w, sg.nblk, rowblk, c, raw[i]);
            }
        }
    }
    prologue<T>(a, xl, xs8, gsc, KP, K8);

    bool first = true;
    for (; rg < n_rg; rg += gridDim.x) {
        const GSeg &sg = a.seg[seg_of(rg)];
        const int64_t row = row_of(sg, rg);
        const int64_t rowblk = row * (sg.type == XJ_Q8_0 ? K / 32 : K / 256);
        float acc[T];
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] = 0.f;
        if (sg.type == XJ_F32) {
            for (int c = lane; c < nch; c += TS) dot_f32<T>(sg.w, K, row, c, xl, KP, acc);
        } else {
            for (int base = 0; base < nch; base += NPF * TS) {
                if (!first) {
#pragma unroll
                    for (int i = 0; i < NPF; i++) {
                        const int c = base + lane + i * TS;
                        if (c < nch) load_chunk(sg.type, sg.w, sg.nblk, rowblk, c, raw[i]);
                    }
                }
                first = false;
#pragma unroll
                for (int i = 0; i < NPF; i++) {
                    const int c = base + lane + i * TS;
                    if (c >= nch) break;
                    if (sg.type == XJ_Q4_K) dot_q4k<T>(raw[i], c, xl, xs8, KP, K8, acc);
                    else if (sg.type == XJ_Q6_K) dot_q6k<T>(raw[i], c, xl, xs8, KP, K8, acc);
                    else dot_q80<T>(raw[i], c, xl, KP, acc);
                }
            }
        }
        first = false;
#pragma unroll
        for (int t = 0; t < T; t++) acc[t] = team_sum<TS>(acc[t]);

        // epilogue: lane 0 of the team owns the row
        const int64_t r = (int64_t)(rg - sg.wg0) * NT + team;
        unsigned long long best[T];
#pragma unroll
        for (int t = 0; t < T; t++) best[t] = 0ull;
        if (lane == 0 && r < sg.n_rows) {
            if (sg.epi == EPI_CONV) {
                const int KC = sg.conv_k;
                float st[8], wc[8];
                for (int k = 0; k + 1 < KC; k++) st[k] = sg.conv_state[r * (KC - 1) + k];
                for (int k = 0; k < KC; k++) wc[k] = sg.conv_w[r * KC + k];
#pragma unroll
                for (int t = 0; t < T; t++) {
                    const float xv = acc[t];
                    float s = 0.f;
                    for (int k = 0; k + 1 < KC; k++) s = fmaf(st[k], wc[k], s);
                    s = fmaf(xv, wc[KC - 1], s);
                    for (int k = 0; k + 2 < KC; k++) st[k] = st[k + 1];
                    st[KC - 2] = xv;
                    sg.y[(int64_t)t * sg.ys + r] = xjd::silu(s);
                    const int ta = a.t0 + t;
                    if (ta < a.keep_n)
                        for (int k = 0; k + 1 < KC; k++) sg.conv_ck[((int64_t)ta * sg.n_rows + r) * (KC - 1) + k] = st[k];
                }
                for (int k = 0; k + 1 < KC; k++) sg.conv_state[r * (KC - 1) + k] = st[k];
            } else {
#pragma unroll
                for (int t = 0; t < T; t++) {
                    float *yp = sg.y + (int64_t)t * sg.ys + r;
                    *yp = sg.epi == EPI_ADD ? *yp + acc[t] : acc[t];
                    if (sg.amax) best[t] = xjd::argmax_key(acc[t], (uint32_t)r);
                }
            }
        }
        if (sg.amax) {  // uniform per work-group
            if (lane == 0)
#pragma unroll
                for (int t = 0; t < T; t++) amax_sh[team][t] = best[t];
            __syncthreads();
            if (tid < T) {
                unsigned long long m = 0ull;
                for (int j = 0; j < NT; j++) m = amax_sh[j][tid] > m ? amax_sh[j][tid] : m;
                sg.amax[(int64_t)tid * sg.nwg + (rg - sg.wg0)] = m;
            }
            __syncthreads();
        }
    }
    if (a.inc_ptr && blockIdx.x == 0 && tid == 0) *a.inc_ptr += a.inc_by;
}

// -------------------------------------------------------------- host side --
int gemv_team_lanes(int K) {
    const int nch = K / 32;
    return nch <= 16 * NPF ? 16 : nch <= 32 * NPF ? 32 : 64;
}

int gemv_rows_per_group(int K) { return 256 / gemv_team_lanes(K); }

static size_t lds_bytes(const GArgs &a, int T) {
    size_t n = (size_t)T * kpad(a.K) + (size_t)T * (a.K / 8);
    if (a.pro == PRO_GATED_RMS) n += (size_t)T * (a.K / a.group);
    return n * 4;
}

int gemv_max_tile(int K) {
    const size_t per_t = (size_t)(kpad(K) + K / 8 + K / 64) * 4;
    int t = (int)(g_lds_max / per_t);
    return t < 1 ? 0 : t > kTileT ? kTileT : t;
}

template <int T, int TS>
static hipError_t launch_t(const GArgs &a, hipStream_t st) {
    const int n_rg = a.seg[a.nseg - 1].wg0 + a.seg[a.nseg - 1].nwg;
    const int grid = n_rg < g_grid_cap ? n_rg : g_grid_cap;
    hipLaunchKernelGGL((gemv_kernel<T, TS>), dim3(grid), dim3(256), lds_bytes(a, T), st, a);
    return hipGetLastError();
}

template <int TS>
static hipError_t launch_ts(const GArgs &a, hipStream_t st) {
    switch (a.T) {
    case 1: return launch_t<1, TS>(a, st);
    case 2: return launch_t<2, TS>(a, st);
    case 3: return launch_t<3, TS>(a, st);
    case 4: return launch_t<4, TS>(a, st);
    case 5: return launch_t<5, TS>(a, st);
    case 6: return launch_t<6, TS>(a, st);
    case 7: return launch_t<7, TS>(a, st);
    case 8: return launch_t<8, TS>(a, st);
    default: return hipErrorInvalidValue;
    }
}

int gemv_launch(const GArgs &a, hipStream_t st) {
    if (a.T < 1 || a.T > kTileT || a.nseg < 1 || a.nseg > kMaxSeg || a.K % 32) return -1;
    if (lds_bytes(a, a.T) > (size_t)g_lds_max) return -1;
    const int rows = gemv_rows_per_group(a.K);
    for (int i = 0; i < a.nseg; i++) {
        const GSeg &s = a.seg[i];
        if ((s.type == XJ_Q4_K || s.type == XJ_Q6_K) && a.K % 256) return -1;
        if (s.type != XJ_Q4_K && s.type != XJ_Q6_K && s.type != XJ_Q8_0 && s.type != XJ_F32) return -1;
        if (s.n_rows < 1 || s.nwg != (s.n_rows + rows - 1) / rows) return -1;
        if (i > 0 && s.wg0 != a.seg[i - 1].wg0 + a.seg[i - 1].nwg) return -1;
    }
    if (a.seg[0].wg0 != 0) return -1;
    const int ts = gemv_team_lanes(a.K);
    hipError_t e = ts == 16 ? launch_ts<16>(a, st) : ts == 32 ? launch_ts<32>(a, st) : launch_ts<64>(a, st);
    return e == hipSuccess ? 0 : -1;
}

template <int T, int TS>
static void raise_lds(int bytes) {
    (void)hipFuncSetAttribute((const void *)gemv_kernel<T, TS>, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <int TS>
static void raise_all(int bytes) {
    raise_lds<1, TS>(bytes); raise_lds<2, TS>(bytes); raise_lds<3, TS>(bytes); raise_lds<4, TS>(bytes);
    raise_lds<5, TS>(bytes); raise_lds<6, TS>(bytes); raise_lds<7, TS>(bytes); raise_lds<8, TS>(bytes);
}

int gemv_init(char *err, size_t errlen) {
    static bool done = false;
    if (done) return 0;
    int dev = 0, cus = 0, lds = 0;
    XJ_CHECK(hipGetDevice(&dev), err, errlen, -1);
    XJ_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), err, errlen, -1);
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) lds = 65536;
    if (cus > 0) g_grid_cap = cus * 8;
    // keep 4 KB for the static reduction buffers
    int want = lds > 65536 ? lds - 4096 : 65536 - 4096;
    raise_all<16>(want); raise_all<32>(want); raise_all<64>(want);
    (void)hipGetLastError();
    g_lds_max = want;
    done = true;
    return 0;
}

// ------------------------------------------------------------- upload --
int upload_repack(uint32_t type, const void *src, int64_t n_rows, int64_t k, uint8_t *dst, hipStream_t st,
                  char *err, size_t errlen) {
    const uint8_t *s = (const uint8_t *)src;
    const uint64_t bytes = xj_row_bytes(type, k) * (uint64_t)n_rows;
    if (type == XJ_F32 || type == XJ_Q4_K) {
        XJ_CHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st), err, errlen, -1);
        XJ_CHECK(hipStreamSynchronize(st), err, errlen, -1);
        return 0;
    }
    std::vector<uint8_t> tmp(bytes);
    if (type == XJ_Q6_K) {
        const int64_t nblk = n_rows * (k / 256);
        uint8_t *ql = tmp.data(), *qh = ql + nblk * 128, *sc = ql + nblk * 192, *dd = ql + nblk * 208;
        for (int64_t g = 0; g < nblk; g++) {
            const uint8_t *b = s + g * 210;
            memcpy(ql + g * 128, b, 128);
            memcpy(qh + g * 64, b + 128, 64);
            memcpy(sc + g * 16, b + 192, 16);
            memcpy(dd + g * 2, b + 208, 2);
        }
    } else if (type == XJ_Q8_0) {
        const int64_t nblk = n_rows * (k / 32);
        uint8_t *qs = tmp.data(), *dd = qs + nblk * 32;
        for (int64_t g = 0; g < nblk; g++) {
            memcpy(dd + g * 2, s + g * 34, 2);
            memcpy(qs + g * 32, s + g * 34 + 2, 32);
        }
    } else {
        snprintf(err, errlen, "no device layout for %s tensors", xj_type_name(type));
        return -1;
    }
    XJ_CHECK(hipMemcpyAsync(dst, tmp.data(), bytes, hipMemcpyHostToDevice, st), err, errlen, -1);
    XJ_CHECK(hipStreamSynchronize(st), err, errlen, -1);
    return 0;
}

// ------------------------------------------------------------ dequant --
// One thread per 32-element chunk, bit-identical to xj_dequant_row.
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ W, uint32_t type, int64_t K,
                                                      int64_t nblk, int64_t r0, int64_t n, float *__restrict__ y) {
    const int64_t nch = K / 32;
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= n * nch) return;
    const int64_t rr = idx / nch, c = idx % nch;
    xjd::dequant_chunk(W, type, K, nblk, r0 + rr, c, y + rr * K + c * 32);
}

int dequant_launch(const DevW &w, int64_t r0, int64_t n, float *y, hipStream_t st) {
    const int64_t nch = w.k / 32, total = n * nch;
    const int64_t nblk = xjd::dev_nblk(w.type, w.n_rows, w.k);
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, w.p, w.type, w.k,
                       nblk, r0, n, y);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace xjk
