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
// column groups), eight wavefronts = a row group of 128 rows. The units, a
// (row group, 256-element block) pair each over every segment of the launch,
// are dealt out in equal contiguous ranges to one persistent work-group per
// CU. A work-group requests a unit's weights and stages its activations of
// all tokens in LDS (864 bytes per token), half of the copies before and half
// in the middle of computing the previous unit from the other LDS buffer.
// A row group covered by one work-group is stored directly; one shared by
// several leaves a partial sum per work-group, and the last to arrive adds
// them in work-group order (the hand-off of the GEMV's SwiGLU tail:
// system-scope stores and loads, a device-scope arrival counter).
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


constexpr int kGemmMaxT = 64;
// One token's activations for one 256-element block, as staged in LDS:
// digits of the block's 8 groups (8 x 96 bytes), their f (8 x 4) and the
// half-group sums of X (16 x 4): 54 chunks of 16 bytes, at a stride of 55
// chunks per token (880 bytes = 220 banks mod 32 = 28: the 8-byte digit
// reads of 16 tokens x 2 column quarters in a half-wavefront fall on 16
// distinct bank pairs; at 864 bytes they fell on 8).
constexpr int kBlkChunks = 54, kTokChunks = 55, kTokStride = 16 * kTokChunks;
constexpr int kRG = 128, kWaves = kRG / 16, kThreads = 64 * kWaves;   // rows and wavefronts per row group
constexpr int kScaleBytes = kWaves * 64 * 16;                          // scale tables, one per wavefront

// 16 bytes from global g to LDS at the wavefront-uniform lds_off + 16 * lane,
// issued as assembly: a copy the compiler cannot see is never waited for
// before unrelated LDS reads (it would wait for every outstanding vector
// request at each). Every wait for these copies is explicit (vmcnt drains in
// issue order; the compiler's own waits only ever count fewer requests, so
// they stay sufficient); the memory clobber keeps LDS accesses from moving
// across it. M0 is restored once the copy is issued.
__device__ __forceinline__ void dma16(const uint8_t *g, uint32_t lds_off) {
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %2, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "s"(lds_off), "v"(g)
                 : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const uint8_t *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

// The T tokens' activations of block blk into buf: slot c = 55 t + q (chunk
// q < 54 of token t; q = 54 is padding) at buf + 16 c, slot c by thread c
// mod blockDim; `part` 0 / 1 issues the first / second half of the rounds.
__device__ __forceinline__ void stage_blk(const GemmArgs &a, const XqOff &o, int blk, uint8_t *buf, int part) {
    const int nslots = a.T * kTokChunks, wv = threadIdx.x >> 6;
    const int rounds = (nslots + kThreads - 1) / kThreads, r0 = part ? rounds / 2 : 0, r1 = part ? rounds : rounds / 2;
    for (int j0 = r0 * kThreads; j0 < r1 * kThreads; j0 += kThreads) {
        const int c = j0 + (int)threadIdx.x;
        const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(buf + 16 * (j0 + 64 * wv)));
        const int t = c / kTokChunks, q = c - t * kTokChunks;
        if (c < nslots && q < kBlkChunks) {
            const uint8_t *xt = a.xq + (int64_t)t * a.xs;
            const uint8_t *src = q < 48 ? xt + blk * 768 + 16 * q
                               : q < 50 ? xt + o.f_off + blk * 32 + 16 * (q - 48)
                                        : xt + o.sx_off + blk * 64 + 16 * (q - 50);
            dma16(src, base);
        }
    }
}

// A wavefront's weights of one block: lane (li, kq) supplies A for row rowA
// (bytes 8 kq.. of each 32-element group) and the scales of rows rowC[i] =
// rb + 4 kq + i, whose outputs it holds.
struct WReg {
    uint64_t qa[4];
    uint4 hc[4];
    float dC[4];
    uint4 sc0;
};

template <bool Q6>
__device__ __forceinline__ void load_w(const uint8_t *w, int64_t NB, int nb, int rowA, const int (&rowC)[4], int blk,
                                       int kq, WReg &r) {
    if constexpr (!Q6) {
        const uint8_t *wa = w + ((int64_t)rowA * nb + blk) * 144;
#pragma unroll
        for (int p = 0; p < 4; p++) r.qa[p] = *(const uint64_t *)(wa + 16 + 32 * p + 8 * kq);
#pragma unroll
        for (int i = 0; i < 4; i++) r.hc[i] = *(const uint4 *)(w + ((int64_t)rowC[i] * nb + blk) * 144);
    } else {
        const uint8_t *ql = w, *qh = w + NB * 128, *scp = w + NB * 192, *dp = w + NB * 208;   // Q6_K planes
        const int64_t bA = (int64_t)rowA * nb + blk;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            r.qa[2 * h] = *(const uint64_t *)(ql + bA * 128 + h * 64 + 8 * kq);
            r.qa[2 * h + 1] = *(const uint64_t *)(ql + bA * 128 + h * 64 + 32 + 8 * kq);
        }
        const uint64_t hb0 = *(const uint64_t *)(qh + bA * 64 + 8 * kq), hb1 = *(const uint64_t *)(qh + bA * 64 + 32 + 8 * kq);
        r.hc[0].x = (uint32_t)hb0; r.hc[0].y = (uint32_t)(hb0 >> 32); r.hc[0].z = (uint32_t)hb1; r.hc[0].w = (uint32_t)(hb1 >> 32);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int64_t bC = (int64_t)rowC[i] * nb + blk;
            r.dC[i] = xjd::f16_to_f32(*(const uint16_t *)(dp + bC * 2));
            if (i) r.hc[i] = *(const uint4 *)(scp + bC * 16);
        }
        r.sc0 = *(const uint4 *)(scp + ((int64_t)rowC[0] * nb + blk) * 16);
    }
}

// Q4_K: the wavefront's table of (ds, dm) = (d sc, dmin m) for sub-blocks
// 2p, 2p+1 of its 16 rows (get_scale_min_k4, xj_quant.h:49-52), float4
// [row][p] = (ds_2p, ds_2p+1, dm_2p, dm_2p+1): lane (li, kq) decodes row
// 4 kq + li / 4, p = li % 4 from the header it holds for its output rows
// (rowC[li / 4]), and the 16 lanes that hold a row's outputs read its entry.
__device__ __forceinline__ void q4k_scales(const WReg &r, int li, int kq, float4 *scl) {
    const int i = li >> 2, p = li & 3;
    // the header of rowC[i], chosen word by word (a lane-dependent index into
    // the registers would put them in scratch memory)
    auto pick = [&](uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
        const uint32_t lo = (i & 1) ? w1 : w0, hi = (i & 1) ? w3 : w2;
        return (i & 2) ? hi : lo;
    };
    const uint4 h = {pick(r.hc[0].x, r.hc[1].x, r.hc[2].x, r.hc[3].x), pick(r.hc[0].y, r.hc[1].y, r.hc[2].y, r.hc[3].y),
                     pick(r.hc[0].z, r.hc[1].z, r.hc[2].z, r.hc[3].z), pick(r.hc[0].w, r.hc[1].w, r.hc[2].w, r.hc[3].w)};
    const float d = xjd::f16_to_f32(h.x & 0xFFFFu), dmin = xjd::f16_to_f32(h.x >> 16);
    const int jm = (2 * p) & 3;
    float ds[2], dm[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint32_t Ab = (h.y >> (8 * (jm + s))) & 0xFFu, Bb = (h.z >> (8 * (jm + s))) & 0xFFu,
                       Cb = (h.w >> (8 * (jm + s))) & 0xFFu;
        const uint32_t sc = p >= 2 ? ((Cb & 0xF) | ((Ab >> 6) << 4)) : (Ab & 63);
        const uint32_t mn = p >= 2 ? ((Cb >> 4) | ((Bb >> 6) << 4)) : (Bb & 63);
        ds[s] = d * (float)sc;
        dm[s] = dmin * (float)mn;
    }
    scl[(4 * kq + i) * 4 + p] = float4{ds[0], ds[1], dm[0], dm[1]};
}

// Q6_K: the wavefront's table of d * sc for the 16 sub-blocks of its 16 rows,
// float4 [row][quad] = sub-blocks 4 quad .. 4 quad + 3: lane (li, kq) decodes
// row 4 kq + li / 4, quad li % 4.
__device__ __forceinline__ void q6k_scales(const WReg &r, int li, int kq, float4 *scl) {
    const int i = li >> 2, qd = li & 3;
    // word qd of row i's scales, by conditional moves over compile-time
    // indices (a lane-dependent index into the registers would put them in
    // scratch memory)
    uint32_t w = 0;
    float d = 0.f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint4 v = c == 0 ? r.sc0 : r.hc[c];
        const uint32_t x[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; q++) w = c == i && q == qd ? x[q] : w;
        d = c == i ? r.dC[c] : d;
    }
    scl[(4 * kq + i) * 4 + qd] = float4{d * (float)(int8_t)(w & 0xFFu), d * (float)(int8_t)((w >> 8) & 0xFFu),
                                        d * (float)(int8_t)((w >> 16) & 0xFFu), d * (float)(int8_t)(w >> 24)};
}

// Half HALF (32-element groups 4 HALF .. 4 HALF + 3) of one block of one
// wavefront: acc[tg][i] += the terms of row rb + 4 kq + i and token tok[tg]
// (= 16 tg + li).
template <bool Q6, int NTG, int HALF>
__device__ __forceinline__ void compute_blk(const WReg &r, const uint8_t *buf, const float4 *scl, const int (&tok)[NTG],
                                            int kq, float (&acc)[NTG][4]) {
    if constexpr (!Q6) {
#pragma unroll
        for (int p = 2 * HALF; p < 2 * HALF + 2; p++) {
            const long A[2] = {(long)(r.qa[p] & 0x0F0F0F0F0F0F0F0Full), (long)((r.qa[p] >> 4) & 0x0F0F0F0F0F0F0F0Full)};
            // ds, dm of sub-blocks 2p, 2p+1 for the four output rows (q4k_scales)
            float4 sd[4];
#pragma unroll
            for (int i = 0; i < 4; i++) sd[i] = scl[(4 * kq + i) * 4 + p];
#pragma unroll
            for (int s = 0; s < 2; s++) {
                const int gl = 2 * p + s;
#pragma unroll
                for (int tg = 0; tg < NTG; tg++) {
                    const uint8_t *xt = buf + tok[tg] * kTokStride;
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
                        const float ds = s ? sd[i].y : sd[i].x, dm = s ? sd[i].w : sd[i].z;
                        const float part = (float)S * ds - SX * dm;
                        acc[tg][i] = fmaf(part, f, acc[tg][i]);
                    }
                }
            }
        }
    } else {
        const uint64_t hbs[2] = {(uint64_t)r.hc[0].x | ((uint64_t)r.hc[0].y << 32), (uint64_t)r.hc[0].z | ((uint64_t)r.hc[0].w << 32)};
        {
            constexpr int h = HALF;
            const uint64_t l0 = r.qa[2 * h], l1 = r.qa[2 * h + 1], hb = hbs[h];
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
                // d * sc of sub-blocks 2 gl, 2 gl + 1 for the four output rows
                float dl[4], dh[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float4 q = scl[(4 * kq + i) * 4 + (gl >> 1)];
                    dl[i] = (gl & 1) ? q.z : q.x;
                    dh[i] = (gl & 1) ? q.w : q.y;
                }
#pragma unroll
                for (int tg = 0; tg < NTG; tg++) {
                    const uint8_t *xt = buf + tok[tg] * kTokStride;
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
                        acc[tg][i] = fmaf((float)SL * dl[i], f, acc[tg][i]);
                        acc[tg][i] = fmaf((float)SH * dh[i], f, acc[tg][i]);
                    }
                }
            }
        }
    }
}

// Work-group holding unit u: the w whose range [w P / G, (w + 1) P / G) holds u.
__device__ __forceinline__ int wg_of(int u, int P, int G) { return ((u + 1) * G - 1) / P; }

template <bool Q6, int NTG>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(const GemmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int last_sh;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 15, kq = lane >> 4;
    const int nb = a.nb, G = a.G, w = blockIdx.x, P = (int)a.P;
    const int u0 = w * P / G, u1 = (w + 1) * P / G;
    const XqOff o = xq_off(a.K);
    uint8_t *const buf0 = lds, *const buf1 = lds + a.T * kTokStride;
    float4 *const scl = (float4 *)(lds + 2 * a.T * kTokStride) + wv * 64;   // this wavefront's scale table
    int tok[NTG];
#pragma unroll
    for (int tg = 0; tg < NTG; tg++) tok[tg] = min(16 * tg + li, a.T - 1);
    // row group g (global) -> segment s; this wavefront's rows (clamped so that
    // every load stays inside the weights; rows past N compute values that
    // are never stored)
    auto rows_of = [&](int g, int &s, int &rb, int &rowA, int (&rowC)[4]) {
        s = 0;
#pragma unroll
        for (int i = 1; i < kGemmMaxSeg; i++) s += i < a.nseg && g >= a.rg0[i];
        const int N = a.seg[s].N;
        rb = (g - a.rg0[s]) * kRG + wv * 16;
        rowA = min(rb + li, N - 1);
#pragma unroll
        for (int i = 0; i < 4; i++) rowC[i] = min(rb + 4 * kq + i, N - 1);
    };
    int g = u0 / nb, blk = u0 - g * nb, s, rb, rowA, rowC[4];
    rows_of(g, s, rb, rowA, rowC);
    WReg cur, nxt;
    load_w<Q6>(a.seg[s].w, (int64_t)a.seg[s].N * nb, nb, rowA, rowC, blk, kq, cur);
    stage_blk(a, o, blk, buf0, 0);
    stage_blk(a, o, blk, buf0, 1);
    float acc[NTG][4];
#pragma unroll
    for (int tg = 0; tg < NTG; tg++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[tg][i] = 0.f;
    for (int u = u0; u < u1; u++) {
        uint8_t *const bc = ((u - u0) & 1) ? buf1 : buf0, *const bn = ((u - u0) & 1) ? buf0 : buf1;
        __builtin_amdgcn_s_waitcnt(0);   // unit u's weights and staged activations have landed
        __syncthreads();                 // ... for every wavefront; unit u - 1's reads of bn are done
        // unit u + 1's requests are in flight while unit u computes: its
        // weights, then half of its activation copies before each half of
        // the computation
        const bool more = u + 1 < u1;
        int g2 = blk + 1 == nb ? g + 1 : g, blk2 = blk + 1 == nb ? 0 : blk + 1, s2 = s, rb2 = rb, rowA2 = rowA;
        int rowC2[4] = {rowC[0], rowC[1], rowC[2], rowC[3]};
        if (more) {
            if (g2 != g) rows_of(g2, s2, rb2, rowA2, rowC2);
            load_w<Q6>(a.seg[s2].w, (int64_t)a.seg[s2].N * nb, nb, rowA2, rowC2, blk2, kq, nxt);
            stage_blk(a, o, blk2, bn, 0);
        }
        const GemmSeg &sg = a.seg[s];
        const bool act = rb < sg.N;
        if (act) {
            if constexpr (Q6) q6k_scales(cur, li, kq, scl);
            else q4k_scales(cur, li, kq, scl);
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // the table, written by other lanes of the wavefront
            compute_blk<Q6, NTG, 0>(cur, bc, scl, tok, kq, acc);
        }
        if (more) stage_blk(a, o, blk2, bn, 1);
        if (act) compute_blk<Q6, NTG, 1>(cur, bc, scl, tok, kq, acc);
        if (u + 1 == u1 || blk == nb - 1) {   // the last of this row group's blocks here (uniform)
            const int first = g * nb;
            const int wf = wg_of(first, P, G), wl = wg_of(first + nb - 1, P, G);
            const int r0 = (g - a.rg0[s]) * kRG;
            if (wf == wl) {
                // lane holds rows rb + 4 kq + i of token 16 tg + li
#pragma unroll
                for (int tg = 0; tg < NTG; tg++) {
                    const int t = 16 * tg + li;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int r = rb + 4 * kq + i;
                        if (t >= a.T || r >= sg.N) continue;
                        float *yp = sg.y + (int64_t)t * sg.ys + r;
                        const float v = a.tsc ? acc[tg][i] * a.tsc[t] : acc[tg][i];
                        *yp = sg.add ? *yp + v : v;
                    }
                }
            } else {
                // this work-group's partial sum of the row group, [t][row - r0]
                float *slot = a.part + (int64_t)(w + g) * a.T * kRG;
#pragma unroll
                for (int tg = 0; tg < NTG; tg++) {
                    const int t = 16 * tg + li;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int r = rb + 4 * kq + i;
                        if (t < a.T && r < sg.N) xjd::store_sys(slot + (int64_t)t * kRG + (r - r0), acc[tg][i]);
                    }
                }
                if (xjd::arrive_last(a.cnt + g, wl - wf + 1, &last_sh)) {
                    // the last to arrive adds the partial sums in work-group order: thread
                    // tid owns elements tid + j kThreads of [t][row], eight at a time, and
                    // the loads of four work-groups' partial sums are in flight at once
                    constexpr int kPer = 8;
                    const int nrow = min(kRG, sg.N - r0), ne = a.T * kRG;
                    for (int e0 = 0; e0 < ne; e0 += kPer * kThreads) {
                        float v[kPer];
#pragma unroll
                        for (int j = 0; j < kPer; j++) v[j] = 0.f;
                        for (int w0 = wf; w0 <= wl; w0 += 4) {
                            float pv[4][kPer];
#pragma unroll
                            for (int q = 0; q < 4; q++)
#pragma unroll
                                for (int j = 0; j < kPer; j++) {
                                    const int idx = e0 + tid + j * kThreads, rr = idx % kRG;
                                    const bool in = w0 + q <= wl && idx < ne && rr < nrow;
                                    pv[q][j] = in ? xjd::load_sys(a.part + (int64_t)(w0 + q + g) * a.T * kRG + idx) : 0.f;
                                }
#pragma unroll
                            for (int q = 0; q < 4; q++)
#pragma unroll
                                for (int j = 0; j < kPer; j++)
                                    if (w0 + q <= wl) v[j] += pv[q][j];
                        }
#pragma unroll
                        for (int j = 0; j < kPer; j++) {
                            const int idx = e0 + tid + j * kThreads, t = idx / kRG, rr = idx - t * kRG;
                            if (idx >= ne || rr >= nrow) continue;
                            const float x = a.tsc ? v[j] * a.tsc[t] : v[j];
                            float *yp = sg.y + (int64_t)t * sg.ys + r0 + rr;
                            *yp = sg.add ? *yp + x : x;
                        }
                    }
                }
            }
#pragma unroll
            for (int tg = 0; tg < NTG; tg++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[tg][i] = 0.f;
        }
        cur = nxt;
        s = s2; g = g2; blk = blk2; rb = rb2; rowA = rowA2;
#pragma unroll
        for (int i = 0; i < 4; i++) rowC[i] = rowC2[i];
    }
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
void launch_g(const GemmArgs &a, size_t lds, hipStream_t st) {
    static const bool raised =
        hipFuncSetAttribute((const void *)gemm_mfma_kernel<Q6, NTG>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            2 * kGemmMaxT * kTokStride + kScaleBytes) == hipSuccess;
    (void)raised;
    hipLaunchKernelGGL((gemm_mfma_kernel<Q6, NTG>), dim3(a.G), dim3(kThreads), lds, st, a);
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

// Partial-sum slots are indexed w + g (work-group, row group): for one row
// group the work-groups are consecutive, and a work-group's row groups too,
// so the index is unique and below G + row groups.
int64_t gemm_part_floats(int64_t rows, int T) {
    return (int64_t)(cu_count() + gemm_counters(rows)) * T * kRG;
}
int gemm_counters(int64_t rows) { return (int)(rows / kRG) + kGemmMaxSeg; }

int gemm_launch(const GemmArgs &in, int64_t part_floats, int n_cnt, hipStream_t st) {
    GemmArgs a = in;
    if ((a.type != XJ_Q4_K && a.type != XJ_Q6_K) || a.K < 256 || a.K % 256 || a.T < 1 || a.T > kGemmMaxT ||
        a.nseg < 1 || a.nseg > kGemmMaxSeg)
        return -1;
    if (!a.xq || !a.part || !a.cnt || (a.xs & 255) || ((uintptr_t)a.xq & 255) || a.xs < xq_off(a.K).stride) return -1;
    a.rg0[0] = 0;
    for (int i = 0; i < a.nseg; i++) {
        const GemmSeg &sg = a.seg[i];
        if (!sg.w || !sg.y || sg.N < 1 || ((uintptr_t)sg.w & 15)) return -1;
        a.rg0[i + 1] = a.rg0[i] + (sg.N + kRG - 1) / kRG;
    }
    for (int i = a.nseg + 1; i <= kGemmMaxSeg; i++) a.rg0[i] = a.rg0[a.nseg];
    a.nb = a.K / 256;
    a.P = (int64_t)a.rg0[a.nseg] * a.nb;
    a.G = (int)(a.P < cu_count() ? a.P : cu_count());
    if (a.P >= (1 << 23)) return -1;   // unit indices times G stay in 32 bits
    if (a.rg0[a.nseg] > n_cnt || (int64_t)(a.G + a.rg0[a.nseg]) * a.T * kRG > part_floats) return -1;
    const size_t lds = 2 * (size_t)a.T * kTokStride + kScaleBytes;
    const bool q6 = a.type == XJ_Q6_K;
    switch ((a.T + 15) / 16) {
    case 1: q6 ? launch_g<true, 1>(a, lds, st) : launch_g<false, 1>(a, lds, st); break;
    case 2: q6 ? launch_g<true, 2>(a, lds, st) : launch_g<false, 2>(a, lds, st); break;
    case 3: q6 ? launch_g<true, 3>(a, lds, st) : launch_g<false, 3>(a, lds, st); break;
    default: q6 ? launch_g<true, 4>(a, lds, st) : launch_g<false, 4>(a, lds, st); break;
    }
    if (hipGetLastError() != hipSuccess) return -1;
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
