// Multi-token dequant-GEMM on the matrix cores (gfx950), for prefill chunks of
// 16..64 tokens (the reference's matmul, src/xiaoju-pipe/core/xj_cpu.c:36-54,
// y[t][r] = sum_k deq(W_r)[k] x[t][k], over a whole chunk of tokens).
//
// The arithmetic is the GEMV's: activations in the prepared form (xq.h: three
// int8 digit planes of X = rint(v 2^(20-E)) per 32-element group), and for
// every quantization sub-block the exact integer sum of q * X, now formed by
// v_mfma_i32_16x16x32_i8 (A = 16 weight rows x 32 elements, B = 32 elements x
// 16 tokens, one digit plane per instruction), then scaled once in fp32 with
// the same expressions as the GEMV's q4k_unit / q6k_unit:
//   Q4_K  (S ds - SX dm) f        Q6_K  (S - 32 SX_half) dsc f
// Only the order in which the fp32 sub-block terms are added differs from the
// GEMV (sequential over each K split here, lane-strided plus a butterfly
// there), so the two agree to fp32 rounding.
//
// Q6_K sub-blocks are 16 elements, so each 32-element group takes two
// instructions per plane with the other half of A zeroed.
//
// Work split: one wavefront = 16 rows x up to 64 tokens (four 16-token
// column groups) over a range of whole 256-element blocks; four wavefronts
// per work-group, which stage each block's activations of all tokens in LDS
// with one round of copies (864 bytes per token) while the weights arrive. Short weights (few row groups) split K over blockIdx.y and
// write partial sums that gemm_reduce adds in split order, so results do not
// depend on timing.
#include "common.h"
#include "kernels.h"
#include "xj_hip.h"
#include "xq.h"

#include <cstdint>

namespace xjk {
namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(long a, long b) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, v4i{0, 0, 0, 0}, 0, 0, 0);
}

__device__ __forceinline__ uint32_t byte_at(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }
__device__ __forceinline__ uint32_t byte16(const uint4 &v, int i) {
    const uint32_t w = i < 4 ? v.x : i < 8 ? v.y : i < 12 ? v.z : v.w;
    return byte_at(w, i & 3);
}

constexpr int kGemmMaxT = 64;
// One token's activations for one 256-element block, as staged in LDS:
// digits of the block's 8 groups (8 x 96 bytes), their f (8 x 4) and the
// half-group sums of X (16 x 4): 54 chunks of 16 bytes.
constexpr int kBlkTok = 864, kBlkChunks = kBlkTok / 16;

template <bool Q6, int NTG>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(const GemmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int rb = (blockIdx.x * 4 + wv) * 16;
    const bool active = rb < a.N;   // idle wavefronts still stage and meet the barriers
    const int li = lane & 15, kq = lane >> 4;
    const int nb = a.K / 256;
    const int sp = blockIdx.y;
    const int b0 = (int)((int64_t)sp * nb / a.nsplit), b1 = (int)((int64_t)(sp + 1) * nb / a.nsplit);
    const XqOff o = xq_off(a.K);
    // operand rows and tokens, clamped so every load stays inside the buffers
    // (lanes past N or T compute values that are never stored)
    const int rowA = min(rb + li, a.N - 1);
    int rowC[4];
#pragma unroll
    for (int i = 0; i < 4; i++) rowC[i] = min(rb + 4 * kq + i, a.N - 1);
    int tok[NTG];
#pragma unroll
    for (int tg = 0; tg < NTG; tg++) tok[tg] = min(16 * tg + li, a.T - 1);

    float acc[NTG][4];
#pragma unroll
    for (int tg = 0; tg < NTG; tg++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[tg][i] = 0.f;

    const int64_t NB = (int64_t)a.N * nb;
    const uint8_t *ql = a.w, *qh = a.w + NB * 128, *scp = a.w + NB * 192, *dp = a.w + NB * 208;   // Q6_K planes
    const int nchunks = a.T * kBlkChunks;
    for (int blk = b0; blk < b1; blk++) {
        // this wavefront's weights for the block, requested before the staging copies
        uint64_t qa[4];
        uint4 hc[4];
        float dC[4];
        if constexpr (!Q6) {
            const uint8_t *wa = a.w + ((int64_t)rowA * nb + blk) * 144;
#pragma unroll
            for (int p = 0; p < 4; p++) qa[p] = *(const uint64_t *)(wa + 16 + 32 * p + 8 * kq);
#pragma unroll
            for (int i = 0; i < 4; i++) hc[i] = *(const uint4 *)(a.w + ((int64_t)rowC[i] * nb + blk) * 144);
        } else {
            const int64_t bA = (int64_t)rowA * nb + blk;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                qa[2 * h] = *(const uint64_t *)(ql + bA * 128 + h * 64 + 8 * kq);
                qa[2 * h + 1] = *(const uint64_t *)(ql + bA * 128 + h * 64 + 32 + 8 * kq);
            }
            uint64_t hb0 = *(const uint64_t *)(qh + bA * 64 + 8 * kq), hb1 = *(const uint64_t *)(qh + bA * 64 + 32 + 8 * kq);
            hc[0].x = (uint32_t)hb0; hc[0].y = (uint32_t)(hb0 >> 32); hc[0].z = (uint32_t)hb1; hc[0].w = (uint32_t)(hb1 >> 32);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int64_t bC = (int64_t)rowC[i] * nb + blk;
                dC[i] = xjd::f16_to_f32(*(const uint16_t *)(dp + bC * 2));
                if (i) hc[i] = *(const uint4 *)(scp + bC * 16);
            }
        }
        uint4 scC0 = {0, 0, 0, 0};
        if constexpr (Q6) scC0 = *(const uint4 *)(scp + ((int64_t)rowC[0] * nb + blk) * 16);
        // stage the block's activations of all T tokens, straight into LDS
        // (global_load_lds: lane l of a wavefront writes base + 16 l, so chunk c
        // lands at 16 c); every copy is in flight at once, behind the weights
        __syncthreads();   // the previous block's reads of LDS are done
        for (int j0 = 0; j0 < nchunks; j0 += 256) {
            const int c = j0 + (int)threadIdx.x;
            if (c < nchunks) {
                const int t = c / kBlkChunks, q = c - t * kBlkChunks;
                const uint8_t *xt = a.xq + (int64_t)t * a.xs;
                const uint8_t *src = q < 48 ? xt + blk * 768 + 16 * q
                                   : q < 50 ? xt + o.f_off + blk * 32 + 16 * (q - 48)
                                            : xt + o.sx_off + blk * 64 + 16 * (q - 50);
                __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1))) *)src,
                                                 (void __attribute__((address_space(3))) *)(lds + 16 * (j0 + 64 * wv)), 16, 0, 0);
            }
        }
        __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));   // vmcnt(0): copies (and weights) landed
        __syncthreads();
        if (!active) continue;
        if constexpr (!Q6) {
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const long A[2] = {(long)(qa[p] & 0x0F0F0F0F0F0F0F0Full), (long)((qa[p] >> 4) & 0x0F0F0F0F0F0F0F0Full)};
                // scale / min of sub-blocks 2p, 2p+1 for the four output rows
                // (get_scale_min_k4, xj_quant.h:49-52)
                float ds[4][2], dm[4][2];
                const int jm = (2 * p) & 3;
                const bool hi4 = p >= 2;
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float d = xjd::f16_to_f32(hc[i].x & 0xFFFFu), dmin = xjd::f16_to_f32(hc[i].x >> 16);
#pragma unroll
                    for (int s = 0; s < 2; s++) {
                        const uint32_t Ab = byte_at(hc[i].y, jm + s), Bb = byte_at(hc[i].z, jm + s), Cb = byte_at(hc[i].w, jm + s);
                        const uint32_t sc = hi4 ? ((Cb & 0xF) | ((Ab >> 6) << 4)) : (Ab & 63);
                        const uint32_t mn = hi4 ? ((Cb >> 4) | ((Bb >> 6) << 4)) : (Bb & 63);
                        ds[i][s] = d * (float)sc;
                        dm[i][s] = dmin * (float)mn;
                    }
                }
#pragma unroll
                for (int s = 0; s < 2; s++) {
                    const int gl = 2 * p + s;
#pragma unroll
                    for (int tg = 0; tg < NTG; tg++) {
                        const uint8_t *xt = lds + tok[tg] * kBlkTok;
                        const uint8_t *xb = xt + gl * kDigStride + 8 * kq;
                        const v4i Sa = mfma_i8(A[s], *(const long *)xb);
                        const v4i Sb = mfma_i8(A[s], *(const long *)(xb + 32));
                        const v4i Sc = mfma_i8(A[s], *(const long *)(xb + 64));
                        const float f = ((const float *)(xt + 768))[gl];
                        const int2 sxp = ((const int2 *)(xt + 800))[gl];
                        const float SX = (float)(sxp.x + sxp.y);
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int S = (Sa[i] * 128 + Sb[i]) * 128 + Sc[i];
                            const float part = (float)S * ds[i][s] - SX * dm[i][s];
                            acc[tg][i] = fmaf(part, f, acc[tg][i]);
                        }
                    }
                }
            }
        } else {
            const uint64_t hbs[2] = {(uint64_t)hc[0].x | ((uint64_t)hc[0].y << 32), (uint64_t)hc[0].z | ((uint64_t)hc[0].w << 32)};
            const uint4 scC[4] = {scC0, hc[1], hc[2], hc[3]};
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint64_t l0 = qa[2 * h], l1 = qa[2 * h + 1], hb = hbs[h];
#pragma unroll
                for (int G = 0; G < 4; G++) {
                    // dequantize_row_q6_K bit layout: q = low nibble | 2 high bits << 4
                    const uint64_t M4 = 0x0F0F0F0F0F0F0F0Full, M2 = 0x3030303030303030ull;
                    const uint64_t q6 = G == 0 ? (l0 & M4) | ((hb << 4) & M2)
                                      : G == 1 ? (l1 & M4) | ((hb << 2) & M2)
                                      : G == 2 ? ((l0 >> 4) & M4) | (hb & M2)
                                               : ((l1 >> 4) & M4) | ((hb >> 2) & M2);
                    // elements 0..15 of the group (lanes kq < 2) and 16..31 are two sub-blocks
                    const long Alo = kq < 2 ? (long)q6 : 0, Ahi = kq < 2 ? 0 : (long)q6;
                    const int gl = 4 * h + G;
#pragma unroll
                    for (int tg = 0; tg < NTG; tg++) {
                        const uint8_t *xt = lds + tok[tg] * kBlkTok;
                        const uint8_t *xb = xt + gl * kDigStride + 8 * kq;
                        const long Ba = *(const long *)xb, Bb = *(const long *)(xb + 32), Bc = *(const long *)(xb + 64);
                        const v4i La = mfma_i8(Alo, Ba), Lb = mfma_i8(Alo, Bb), Lc = mfma_i8(Alo, Bc);
                        const v4i Ha = mfma_i8(Ahi, Ba), Hb = mfma_i8(Ahi, Bb), Hc = mfma_i8(Ahi, Bc);
                        const float f = ((const float *)(xt + 768))[gl];
                        const int2 sxp = ((const int2 *)(xt + 800))[gl];
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int SL = (La[i] * 128 + Lb[i]) * 128 + Lc[i] - 32 * sxp.x;
                            const int SH = (Ha[i] * 128 + Hb[i]) * 128 + Hc[i] - 32 * sxp.y;
                            const float dl = dC[i] * (float)(int8_t)byte16(scC[i], 8 * h + 2 * G);
                            const float dh = dC[i] * (float)(int8_t)byte16(scC[i], 8 * h + 2 * G + 1);
                            acc[tg][i] = fmaf((float)SL * dl, f, acc[tg][i]);
                            acc[tg][i] = fmaf((float)SH * dh, f, acc[tg][i]);
                        }
                    }
                }
            }
        }
    }
    if (!active) return;
    // lane holds rows rb + 4 kq + i of token 16 tg + li
#pragma unroll
    for (int tg = 0; tg < NTG; tg++) {
        const int t = 16 * tg + li;
        if (t >= a.T) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = rb + 4 * kq + i;
            if (r >= a.N) continue;
            if (a.nsplit > 1) {
                a.part[((int64_t)sp * a.T + t) * a.N + r] = acc[tg][i];
            } else {
                float *yp = a.y + (int64_t)t * a.ys + r;
                const float v = a.tsc ? acc[tg][i] * a.tsc[t] : acc[tg][i];
                *yp = a.add ? *yp + v : v;
            }
        }
    }
}

// y[t][r] (+)= sum over splits 0..nsplit-1 of part[s][t][r], in that order.
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const GemmArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)a.T * a.N) return;
    const int t = (int)(idx / a.N), r = (int)(idx % a.N);
    float s = 0.f;
    for (int k = 0; k < a.nsplit; k++) s += a.part[((int64_t)k * a.T + t) * a.N + r];
    if (a.tsc) s *= a.tsc[t];
    float *yp = a.y + (int64_t)t * a.ys + r;
    *yp = a.add ? *yp + s : s;
}

// PRO_RMSU scale per token (one wavefront per token): the groups' sums of
// x^2 in double, lane-strided then the wavefront sum, as rmsu_scale.
__global__ __launch_bounds__(64) void rms_scale_kernel(const uint8_t *xq, int64_t xs, int K, float eps, float *tsc) {
    const int t = blockIdx.x, lane = threadIdx.x;
    const XqOff o = xq_off(K);
    const double *ss = (const double *)(xq + (int64_t)t * xs + o.ss_off);
    double s = 0;
    for (int g = lane; g < o.G; g += 64) s += ss[g];
    s = xjd::wave_sum_d(s);
    if (lane == 0) tsc[t] = 1.0f / sqrtf((float)(s / K) + eps);
}

__global__ void inc_kernel(int32_t *p, int32_t by) { *p += by; }

template <bool Q6, int NTG>
void launch_g(const GemmArgs &a, dim3 grid, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL((gemm_mfma_kernel<Q6, NTG>), grid, dim3(256), lds, st, a);
}

int cu_count() {
    static int n = 0;
    if (!n) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n < 1)
            n = 256;
    }
    return n;
}

}  // namespace

int gemm_max_tokens() { return kGemmMaxT; }

int gemm_splits(int N, int K, int T, int64_t part_floats) {
    const int nb = K / 256, wgs = (N + 63) / 64;
    int ns = (2 * cu_count() + wgs - 1) / wgs;
    if (ns > nb) ns = nb;
    if (ns < 1) ns = 1;
    while (ns > 1 && (int64_t)ns * T * N > part_floats) ns--;
    return ns;
}

int gemm_launch(const GemmArgs &in, int64_t part_floats, hipStream_t st) {
    GemmArgs a = in;
    if ((a.type != XJ_Q4_K && a.type != XJ_Q6_K) || a.K < 256 || a.K % 256 || a.N < 1 || a.T < 1 || a.T > kGemmMaxT)
        return -1;
    if (!a.w || !a.xq || !a.y || (a.xs & 255) || ((uintptr_t)a.w & 15) || ((uintptr_t)a.xq & 255)) return -1;
    if (a.xs < xq_off(a.K).stride) return -1;
    a.nsplit = a.part ? gemm_splits(a.N, a.K, a.T, part_floats) : 1;
    const dim3 grid((a.N + 63) / 64, a.nsplit);
    const size_t lds = (size_t)a.T * kBlkTok;
    const bool q6 = a.type == XJ_Q6_K;
    switch ((a.T + 15) / 16) {
    case 1: q6 ? launch_g<true, 1>(a, grid, lds, st) : launch_g<false, 1>(a, grid, lds, st); break;
    case 2: q6 ? launch_g<true, 2>(a, grid, lds, st) : launch_g<false, 2>(a, grid, lds, st); break;
    case 3: q6 ? launch_g<true, 3>(a, grid, lds, st) : launch_g<false, 3>(a, grid, lds, st); break;
    default: q6 ? launch_g<true, 4>(a, grid, lds, st) : launch_g<false, 4>(a, grid, lds, st); break;
    }
    if (hipGetLastError() != hipSuccess) return -1;
    if (a.nsplit > 1) {
        const int64_t n = (int64_t)a.T * a.N;
        hipLaunchKernelGGL(gemm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a);
        if (hipGetLastError() != hipSuccess) return -1;
    }
    if (a.inc_ptr) {
        hipLaunchKernelGGL(inc_kernel, dim3(1), dim3(1), 0, st, a.inc_ptr, a.inc_by);
        if (hipGetLastError() != hipSuccess) return -1;
    }
    return 0;
}

int inc_launch(int32_t *p, int32_t by, hipStream_t st) {
    hipLaunchKernelGGL(inc_kernel, dim3(1), dim3(1), 0, st, p, by);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int rms_scale_launch(const uint8_t *xq, int64_t xs, int K, int T, float eps, float *tsc, hipStream_t st) {
    if (T < 1 || K < 32 || K % 32 || !xq || !tsc) return -1;
    hipLaunchKernelGGL(rms_scale_kernel, dim3(T), dim3(64), 0, st, xq, xs, K, eps, tsc);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace xjk
