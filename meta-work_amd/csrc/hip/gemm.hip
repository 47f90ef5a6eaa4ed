// Multi-token dequant-GEMM on the matrix cores (gfx950), for prefill chunks of
// 16..64 tokens (the reference's matmul, src/xiaoju-pipe/core/xj_cpu.c:36-54,
// y[t][r] = sum_k deq(W_r)[k] x[t][k], over a whole chunk of tokens).
//
// Activations: the prep launch's hq records (xq.h): per token and 256-element
// block, v * 2^-e = hi + lo in two f16 planes (e the block's exponent) and
// the groups' sums of v. The weights enter v_mfma_f32_16x16x32_f16 as small
// integers, exact in f16, so every product is exact and the matrix cores
// accumulate a whole block in fp32 without per-group scaling:
//   Q4_K (xj_quant.h:49-52 and the Q4_K dequantization, w = d sc_j q -
//        dmin m_j): A = sc_j q (at most 945), one MFMA per plane, S = sum of
//        sc_j q (hi + lo) over the block, added as d 2^e S; the minimum term
//        sum_j dmin m_j sx_j of every block accumulates on
//        v_mfma_f32_16x16x4_f32 (A = dmin m_j, B = the group sums).
//   Q6_K (w = d sc_s (q - 32), int8 sc_s per 16 elements): sc (q - 32) needs
//        13 bits, so with sc = 16 sc_hi + sc_lo the operands A_hi = sc_hi (q -
//        32) and A_lo = sc_lo (q - 32) are exact and S = 16 (A_hi . hi) +
//        A_lo . hi + (16 A_hi + A_lo) . lo, the last operand rounded to f16 (it
//        multiplies the low plane only, so its rounding is 2^-23 of a product).
// Only fp32 accumulation rounds: results agree with the fp64 product of the
// dequantized weights to ~1e-7 relative; the dot-product GEMV, whose
// activations are 21-bit integers per 32-element group, agrees to ~1e-6.
//
// Work split: a row group of 128 rows per work-group of eight wavefronts.
// Above 32 tokens a wavefront takes 32 rows (two 16-row tiles) x 32 tokens
// (two 16-token tiles), the eight being four row pairs x two token halves;
// otherwise 16 rows x every token. The units, a (row group, 256-element
// block) pair each over every segment of the launch, are dealt out in equal
// contiguous ranges to one persistent work-group per CU. A work-group
// requests a unit's weights and stages its activations of all tokens in LDS
// (one kHqBlk record per token), half of the copies before and half in the
// middle of computing the previous unit from the other LDS buffer. A row
// group covered by one work-group is stored directly; one shared by several
// leaves a partial sum per work-group, and the last to arrive adds them in
// work-group order (system-scope stores and loads, a device-scope arrival
// counter).
#include "common.h"
#include "kernels.h"
#include "xj_hip.h"
#include "xq.h"

#include <algorithm>
#include <cstdint>

namespace xjk {
namespace {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned int u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma_h(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ f4 mfma_s(float a, float b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }

__device__ __forceinline__ h2 as_h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
__device__ __forceinline__ h8 cat8(h2 a, h2 b, h2 c, h2 d) {
    return __builtin_shufflevector(__builtin_shufflevector(a, b, 0, 1, 2, 3), __builtin_shufflevector(c, d, 0, 1, 2, 3), 0,
                                   1, 2, 3, 4, 5, 6, 7);
}
// f16 pairs (1024 + byte 0, 1024 + byte 1) and (1024 + byte 2, 1024 + byte 3)
// of w: an f16 whose high byte is 0x64 has the value 1024 + its low byte.
__device__ __forceinline__ h2 biased01(uint32_t w) { return as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04010400u)); }
__device__ __forceinline__ h2 biased23(uint32_t w) { return as_h2(__builtin_amdgcn_perm(0x64646464u, w, 0x04030402u)); }

constexpr int kGemmMaxT = 64;
constexpr int kTokChunks = kHqBlk / 16;   // 16-byte chunks per token record
constexpr int kRG = 128, kWaves = 8, kThreads = 64 * kWaves;   // rows and wavefronts per row group

// A block's activations of all T tokens pass through registers: thread tid
// loads chunks c = tid + kThreads j (16 bytes each; token c / 67, chunk c % 67
// of its record) two units ahead, and writes them to the LDS buffer of the
// next unit at the top of each unit, where chunk c lands at 16 c.
template <int NTG>
struct ActRegs {
    static constexpr int R = (kTokChunks * 16 * NTG + kThreads - 1) / kThreads;   // rounds for 16 NTG tokens
    u4 v[R];
    int32_t off[R];   // t * hs + 16 q of chunk c (chunk 0 past the T tokens, loaded but not stored)
    bool in[R];
};
template <int NTG>
__device__ __forceinline__ void act_offsets(const GemmArgs &a, ActRegs<NTG> &r) {
#pragma unroll
    for (int j = 0; j < ActRegs<NTG>::R; j++) {
        const int c = (int)threadIdx.x + kThreads * j, t = c / kTokChunks, q = c - t * kTokChunks;
        r.in[j] = c < a.T * kTokChunks;
        r.off[j] = r.in[j] ? (int32_t)(t * a.hs + 16 * q) : 0;
    }
}
template <int NTG>
__device__ __forceinline__ void act_load(const GemmArgs &a, int blk, ActRegs<NTG> &r) {
    const uint8_t *base = a.hq + (int64_t)blk * kHqBlk;
#pragma unroll
    for (int j = 0; j < ActRegs<NTG>::R; j++) r.v[j] = *(const u4 *)(base + r.off[j]);
}
template <int NTG>
__device__ __forceinline__ void act_store(const ActRegs<NTG> &r, uint8_t *buf) {
#pragma unroll
    for (int j = 0; j < ActRegs<NTG>::R; j++)
        if (r.in[j]) *(u4 *)(buf + 16 * ((int)threadIdx.x + kThreads * j)) = r.v[j];
}

// Partial sums cross work-groups on other XCDs: 8-byte system-scope stores
// (written through every cache level) and loads (which bypass the caches).
__device__ __forceinline__ void store_sys2(float *p, float x, float y) {
    const unsigned long long v = (unsigned long long)__float_as_uint(x) | ((unsigned long long)__float_as_uint(y) << 32);
    __hip_atomic_store((unsigned long long *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ unsigned long long load_sys2(const float *p) {
    return __hip_atomic_load((unsigned long long *)const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// A wavefront's weights of one block for its RT row tiles: lane (li, kq)
// supplies A for row rowA[rt] (elements 8 kq .. 8 kq + 7 of each 32-element
// group).
template <bool Q6, int RT>
struct WReg {
    // Q4_K: q[rt][2p + i] = nibble bytes 8 kq + 4 i .. of the block's 32-byte chunk p
    // Q6_K: q[rt][4h + 2c + i] = ql bytes 64 h + 32 c + 8 kq + 4 i ..,
    //       qh[rt][2h + i] = qh bytes 32 h + 8 kq + 4 i ..
    uint32_t q[RT][8];
    uint32_t qh[RT][Q6 ? 4 : 1];
    uint4 hd[RT];       // Q4_K: the 16-byte header (d, dmin, scales); Q6_K: the 16 scales
    uint32_t d6[RT];    // Q6_K: d (fp16 bits)
};

template <bool Q6, int RT>
__device__ __forceinline__ void load_w(const uint8_t *w, int64_t NB, int nb, const int (&rowA)[RT], int blk, int kq,
                                       WReg<Q6, RT> &r) {
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        if constexpr (!Q6) {
            const uint8_t *wa = w + ((int64_t)rowA[rt] * nb + blk) * 144;
#pragma unroll
            for (int p = 0; p < 4; p++) {
                const uint2 v = *(const uint2 *)(wa + 16 + 32 * p + 8 * kq);
                r.q[rt][2 * p] = v.x;
                r.q[rt][2 * p + 1] = v.y;
            }
            r.hd[rt] = *(const uint4 *)wa;
        } else {
            const uint8_t *ql = w, *qh = w + NB * 128, *scp = w + NB * 192, *dp = w + NB * 208;   // Q6_K planes
            const int64_t b = (int64_t)rowA[rt] * nb + blk;
#pragma unroll
            for (int h = 0; h < 2; h++) {
#pragma unroll
                for (int c = 0; c < 2; c++) {
                    const uint2 v = *(const uint2 *)(ql + b * 128 + 64 * h + 32 * c + 8 * kq);
                    r.q[rt][4 * h + 2 * c] = v.x;
                    r.q[rt][4 * h + 2 * c + 1] = v.y;
                }
                const uint2 u = *(const uint2 *)(qh + b * 64 + 32 * h + 8 * kq);
                r.qh[rt][2 * h] = u.x;
                r.qh[rt][2 * h + 1] = u.y;
            }
            r.hd[rt] = *(const uint4 *)(scp + b * 16);
            r.d6[rt] = *(const uint16_t *)(dp + b * 2);
        }
    }
}

// Q4_K: the 6-bit scales and minimums of a header, four per word
// (get_scale_min_k4, xj_quant.h:49-52): sc[0] = sub-blocks 0..3, sc[1] = 4..7.
struct Q4Scales {
    uint32_t sc[2], m[2];
};
__device__ __forceinline__ Q4Scales q4k_scmin(const uint4 h) {
    Q4Scales s;
    s.sc[0] = h.y & 0x3F3F3F3Fu;
    s.m[0] = h.z & 0x3F3F3F3Fu;
    s.sc[1] = (h.w & 0x0F0F0F0Fu) | ((h.y >> 2) & 0x30303030u);
    s.m[1] = ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u);
    return s;
}

// Groups 4 HALF .. 4 HALF + 3 of one block: s1[rt][tt] (and s16, Q6_K) +=
// the tile's products for rows rowA[rt] and tokens tok[tt].
template <bool Q6, int RT, int TT, int HALF>
__device__ __forceinline__ void compute_half(const WReg<Q6, RT> &r, const Q4Scales (&qs)[RT], const uint8_t *buf,
                                             const int (&tok)[TT], int kq, f4 (&s1)[RT][TT], f4 (&s16)[RT][TT]) {
#pragma unroll
    for (int G = 0; G < 4; G++) {
        const int j = 4 * HALF + G;
        h8 bh[TT], bl[TT];
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            const uint8_t *xb = buf + tok[tt] * kHqBlk + 64 * j + 16 * kq;
            bh[tt] = *(const h8 *)xb;
            bl[tt] = *(const h8 *)(xb + 512);
        }
#pragma unroll
        for (int rt = 0; rt < RT; rt++) {
            if constexpr (!Q6) {
                // sub-block j: (sc, sc) from the byte next to 0x64, minus 1024
                const uint32_t sel = 0x04000400u | ((uint32_t)(j & 3) << 16) | (uint32_t)(j & 3);
                const h2 s2 = as_h2(__builtin_amdgcn_perm(0x64646464u, qs[rt].sc[j >> 2], sel)) - h2{1024, 1024};
                const h2 n2 = s2 * h2{-1024, -1024};
                const int p = j >> 1;
                const uint32_t w0 = (j & 1) ? r.q[rt][2 * p] >> 4 : r.q[rt][2 * p];
                const uint32_t w1 = (j & 1) ? r.q[rt][2 * p + 1] >> 4 : r.q[rt][2 * p + 1];
                const uint32_t n0 = w0 & 0x0F0F0F0Fu, n1 = w1 & 0x0F0F0F0Fu;
                // (1024 + q) sc - 1024 sc = q sc, exact
                const h8 A = cat8(__builtin_elementwise_fma(biased01(n0), s2, n2), __builtin_elementwise_fma(biased23(n0), s2, n2),
                                  __builtin_elementwise_fma(biased01(n1), s2, n2), __builtin_elementwise_fma(biased23(n1), s2, n2));
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    s1[rt][tt] = mfma_h(A, bh[tt], s1[rt][tt]);
                    s1[rt][tt] = mfma_h(A, bl[tt], s1[rt][tt]);
                }
            } else {
                // q6 bytes of the lane's 8 elements (the Q6_K bit layout: low
                // nibble from ql, two high bits from qh)
                const uint64_t l0 = (uint64_t)r.q[rt][4 * HALF] | ((uint64_t)r.q[rt][4 * HALF + 1] << 32);
                const uint64_t l1 = (uint64_t)r.q[rt][4 * HALF + 2] | ((uint64_t)r.q[rt][4 * HALF + 3] << 32);
                const uint64_t hb = (uint64_t)r.qh[rt][2 * HALF] | ((uint64_t)r.qh[rt][2 * HALF + 1] << 32);
                const uint64_t M4 = 0x0F0F0F0F0F0F0F0Full, M2 = 0x3030303030303030ull;
                const uint64_t q6 = G == 0 ? (l0 & M4) | ((hb << 4) & M2)
                                  : G == 1 ? (l1 & M4) | ((hb << 2) & M2)
                                  : G == 2 ? ((l0 >> 4) & M4) | (hb & M2)
                                           : ((l1 >> 4) & M4) | ((hb >> 2) & M2);
                const uint32_t u0 = (uint32_t)q6, u1 = (uint32_t)(q6 >> 32);
                // scale of sub-block 2 j + kq / 2: byte 2 (j & 1) + kq / 2 of word j / 2
                const uint32_t sw = (j >> 1) == 0 ? r.hd[rt].x : (j >> 1) == 1 ? r.hd[rt].y : (j >> 1) == 2 ? r.hd[rt].z : r.hd[rt].w;
                const int sc = __builtin_amdgcn_sbfe((int)sw, 16 * (j & 1) + 8 * (kq >> 1), 8);
                const _Float16 fhi = (_Float16)(sc >> 4), flo = (_Float16)(sc & 15);
                const h2 shi = {fhi, fhi}, slo = {flo, flo};
                const h2 nhi = shi * h2{-1056, -1056}, nlo = slo * h2{-1056, -1056};   // exact
                const h2 b0 = biased01(u0), b1 = biased23(u0), b2 = biased01(u1), b3 = biased23(u1);
                // (1024 + q) s - 1056 s = (q - 32) s, exact
                const h2 h0 = __builtin_elementwise_fma(b0, shi, nhi), h1 = __builtin_elementwise_fma(b1, shi, nhi),
                         h2_ = __builtin_elementwise_fma(b2, shi, nhi), h3 = __builtin_elementwise_fma(b3, shi, nhi);
                const h2 o0 = __builtin_elementwise_fma(b0, slo, nlo), o1 = __builtin_elementwise_fma(b1, slo, nlo),
                         o2 = __builtin_elementwise_fma(b2, slo, nlo), o3 = __builtin_elementwise_fma(b3, slo, nlo);
                const h2 sixteen = {16, 16};
                const h8 Ahi = cat8(h0, h1, h2_, h3), Alo = cat8(o0, o1, o2, o3);
                const h8 Afl = cat8(__builtin_elementwise_fma(h0, sixteen, o0), __builtin_elementwise_fma(h1, sixteen, o1),
                                    __builtin_elementwise_fma(h2_, sixteen, o2), __builtin_elementwise_fma(h3, sixteen, o3));
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    s16[rt][tt] = mfma_h(Ahi, bh[tt], s16[rt][tt]);
                    s1[rt][tt] = mfma_h(Alo, bh[tt], s1[rt][tt]);
                    s1[rt][tt] = mfma_h(Afl, bl[tt], s1[rt][tt]);
                }
            }
        }
    }
}

// The end of a block: acc[rt][tt] += d 2^e S for the lane's output rows
// (rb + 16 rt + 4 kq + i, whose d the lanes li = 4 kq + i hold) and, Q4_K,
// accm[rt][tt] += the block's minimum terms; s1 and s16 are cleared.
template <bool Q6, int RT, int TT>
__device__ __forceinline__ void end_blk(const WReg<Q6, RT> &r, const Q4Scales (&qs)[RT], const uint8_t *buf,
                                        const int (&tok)[TT], int kq, f4 (&s1)[RT][TT], f4 (&s16)[RT][TT],
                                        f4 (&acc)[RT][TT], f4 (&accm)[RT][TT]) {
    int e[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) e[tt] = *(const int *)(buf + tok[tt] * kHqBlk + 1056);
#pragma unroll
    for (int rt = 0; rt < RT; rt++) {
        const float dA = xjd::f16_to_f32(Q6 ? r.d6[rt] : r.hd[rt].x & 0xFFFFu);
        float dC[4];
#pragma unroll
        for (int i = 0; i < 4; i++) dC[i] = __shfl(dA, 4 * kq + i, 64);
#pragma unroll
        for (int tt = 0; tt < TT; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float S = Q6 ? fmaf(16.f, s16[rt][tt][i], s1[rt][tt][i]) : s1[rt][tt][i];
                acc[rt][tt][i] = fmaf(dC[i], ldexpf(S, e[tt]), acc[rt][tt][i]);
            }
        if constexpr (!Q6) {
            // sum over the block's groups g = 4 h + kq of dmin m_g sx_g (A: row li, k = kq; B: k = kq, token li)
            const float dminA = xjd::f16_to_f32(r.hd[rt].x >> 16);
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const float am = dminA * (float)((qs[rt].m[h] >> (8 * kq)) & 0xFFu);
#pragma unroll
                for (int tt = 0; tt < TT; tt++) {
                    const float bm = ((const float *)(buf + tok[tt] * kHqBlk + 1024))[4 * h + kq];
                    accm[rt][tt] = mfma_s(am, bm, accm[rt][tt]);
                }
            }
        }
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            s1[rt][tt] = f4{0.f, 0.f, 0.f, 0.f};
            s16[rt][tt] = f4{0.f, 0.f, 0.f, 0.f};
        }
    }
}

// Work-group holding unit u: the w whose range [w P / G, (w + 1) P / G) holds u.
__device__ __forceinline__ int wg_of(int u, int P, int G) { return ((u + 1) * G - 1) / P; }

// The units of one weight type: work-group wb + w of this type's G takes its
// equal contiguous share of the type's P units, which start at unit ub (and
// at row group ub / nb) of the launch.
template <bool Q6, int NTG>
__device__ __forceinline__ void gemm_units(const GemmArgs &a, uint8_t *lds, int *last_sh_p, int wb, int w, int G,
                                           int P, int ub) {
    // NTG 16-token column groups: above two, a wavefront takes two row tiles x
    // two token tiles (four row pairs x two token halves), else one row tile x
    // all of them
    constexpr int RT = NTG > 2 ? 2 : 1, TT = NTG > 2 ? 2 : NTG;
    int &last_sh = *last_sh_p;
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 15, kq = lane >> 4;
    const int nb = a.nb;
    const int u0 = ub + w * P / G, u1 = ub + (w + 1) * P / G;
    uint8_t *const buf0 = lds, *const buf1 = lds + a.T * kHqBlk;
    const int wrow = RT == 2 ? 32 * (wv >> 1) : 16 * wv;   // this wavefront's first row in the row group
    const int tile0 = RT == 2 ? TT * (wv & 1) : 0;          // ... and first token tile
    int tok[TT];
#pragma unroll
    for (int tt = 0; tt < TT; tt++) tok[tt] = min(16 * (tile0 + tt) + li, a.T - 1);
    // row group g (global) -> segment s; this wavefront's rows (clamped so that
    // every load stays inside the weights; rows past N compute values that
    // are never stored)
    auto rows_of = [&](int g, int &s, int &rb, int (&rowA)[RT]) {
        s = 0;
#pragma unroll
        for (int i = 1; i < kGemmMaxSeg; i++) s += i < a.nseg && g >= a.rg0[i];
        const int N = a.seg[s].N;
        rb = (g - a.rg0[s]) * kRG + wrow;
#pragma unroll
        for (int rt = 0; rt < RT; rt++) rowA[rt] = min(rb + 16 * rt + li, N - 1);
    };
    int g = u0 / nb, blk = u0 - g * nb, s, rb, rowA[RT];
    rows_of(g, s, rb, rowA);
    WReg<Q6, RT> cur, nxt;
    load_w<Q6, RT>(a.seg[s].w, (int64_t)a.seg[s].N * nb, nb, rowA, blk, kq, cur);
    // unit u0's activations into buf0; unit u0 + 1's in registers
    ActRegs<NTG> ar;
    act_offsets(a, ar);
    act_load(a, blk, ar);
    __builtin_amdgcn_s_waitcnt(0);
    act_store(ar, buf0);
    if (u0 + 1 < u1) act_load(a, (u0 + 1) % nb, ar);
    f4 acc[RT][TT], accm[RT][TT], s1[RT][TT], s16[RT][TT];
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
        for (int tt = 0; tt < TT; tt++) {
            acc[rt][tt] = accm[rt][tt] = s1[rt][tt] = s16[rt][tt] = f4{0.f, 0.f, 0.f, 0.f};
        }
    for (int u = u0; u < u1; u++) {
        uint8_t *const bc = ((u - u0) & 1) ? buf1 : buf0, *const bn = ((u - u0) & 1) ? buf0 : buf1;
        __builtin_amdgcn_s_waitcnt(0);   // unit u's weights and unit u + 1's activations have landed
        __syncthreads();                 // unit u's LDS buffer is written; unit u - 1's reads of bn are done
        // unit u + 1's activations into bn, then the requests for unit u + 1's
        // weights and unit u + 2's activations, in flight while unit u computes
        const bool more = u + 1 < u1;
        int g2 = blk + 1 == nb ? g + 1 : g, blk2 = blk + 1 == nb ? 0 : blk + 1, s2 = s, rb2 = rb, rowA2[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) rowA2[rt] = rowA[rt];
        if (more) {
            act_store(ar, bn);
            if (g2 != g) rows_of(g2, s2, rb2, rowA2);
            load_w<Q6, RT>(a.seg[s2].w, (int64_t)a.seg[s2].N * nb, nb, rowA2, blk2, kq, nxt);
            if (u + 2 < u1) act_load(a, blk2 + 1 == nb ? 0 : blk2 + 1, ar);
        }
        const GemmSeg &sg = a.seg[s];
        const bool act = rb < sg.N;   // uniform over the wavefront
        Q4Scales qs[RT];
#pragma unroll
        for (int rt = 0; rt < RT; rt++) qs[rt] = q4k_scmin(cur.hd[rt]);
        if (act) compute_half<Q6, RT, TT, 0>(cur, qs, bc, tok, kq, s1, s16);
        if (act) {
            compute_half<Q6, RT, TT, 1>(cur, qs, bc, tok, kq, s1, s16);
            end_blk<Q6, RT, TT>(cur, qs, bc, tok, kq, s1, s16, acc, accm);
        }
        if (u + 1 == u1 || blk == nb - 1) {   // the last of this row group's blocks here (uniform)
            const int first = g * nb;
            const int wf = wb + wg_of(first - ub, P, G), wl = wb + wg_of(first + nb - 1 - ub, P, G);
            const int r0 = (g - a.rg0[s]) * kRG;
            if (wf == wl) {
                // lane holds rows rb + 16 rt + 4 kq + i of token 16 (tile0 + tt) + li
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
#pragma unroll
                    for (int tt = 0; tt < TT; tt++) {
                        const int t = 16 * (tile0 + tt) + li;
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int r = rb + 16 * rt + 4 * kq + i;
                            if (t >= a.T || r >= sg.N) continue;
                            float *yp = sg.y + (int64_t)t * sg.ys + r;
                            const float y = acc[rt][tt][i] - accm[rt][tt][i];
                            const float v = a.tsc ? y * a.tsc[t] : y;
                            *yp = sg.add ? *yp + v : v;
                        }
                    }
            } else {
                // this work-group's partial sum of the row group, [t][row - r0]
                // (rows past N too: in bounds of the slot, never read)
                float *slot = a.part + (int64_t)(wb + w + g) * a.T * kRG;
#pragma unroll
                for (int rt = 0; rt < RT; rt++)
#pragma unroll
                    for (int tt = 0; tt < TT; tt++) {
                        const int t = 16 * (tile0 + tt) + li;
                        if (t >= a.T) continue;
                        float *sp = slot + (int64_t)t * kRG + (rb - r0 + 16 * rt + 4 * kq);
                        const f4 y = acc[rt][tt] - accm[rt][tt];
                        store_sys2(sp, y[0], y[1]);
                        store_sys2(sp + 2, y[2], y[3]);
                    }
                if (xjd::arrive_last(a.cnt + g, wl - wf + 1, &last_sh)) {
                    // the last to arrive adds the partial sums in work-group order:
                    // thread tid owns element pairs tid + j kThreads of [t][row], and
                    // the loads of four work-groups' partial sums are in flight at once
                    constexpr int kPer = 8;
                    const int nrow = min(kRG, sg.N - r0), np = a.T * kRG / 2;
                    for (int e0 = 0; e0 < np; e0 += kPer * kThreads) {
                        float v[kPer][2];
#pragma unroll
                        for (int j = 0; j < kPer; j++) v[j][0] = v[j][1] = 0.f;
                        for (int w0 = wf; w0 <= wl; w0 += 4) {
                            unsigned long long pv[4][kPer];
#pragma unroll
                            for (int q = 0; q < 4; q++)
#pragma unroll
                                for (int j = 0; j < kPer; j++) {
                                    const int idx = e0 + tid + j * kThreads;
                                    const bool in = w0 + q <= wl && idx < np;
                                    pv[q][j] = in ? load_sys2(a.part + (int64_t)(w0 + q + g) * a.T * kRG + 2 * idx) : 0ull;
                                }
#pragma unroll
                            for (int q = 0; q < 4; q++)
#pragma unroll
                                for (int j = 0; j < kPer; j++)
                                    if (w0 + q <= wl) {
                                        v[j][0] += __uint_as_float((uint32_t)pv[q][j]);
                                        v[j][1] += __uint_as_float((uint32_t)(pv[q][j] >> 32));
                                    }
                        }
#pragma unroll
                        for (int j = 0; j < kPer; j++) {
                            const int idx = e0 + tid + j * kThreads, t = 2 * idx / kRG, rr = 2 * idx - t * kRG;
                            if (idx >= np) continue;
#pragma unroll
                            for (int h = 0; h < 2; h++) {
                                if (rr + h >= nrow) continue;
                                const float x = a.tsc ? v[j][h] * a.tsc[t] : v[j][h];
                                float *yp = sg.y + (int64_t)t * sg.ys + r0 + rr + h;
                                *yp = sg.add ? *yp + x : x;
                            }
                        }
                    }
                }
            }
#pragma unroll
            for (int rt = 0; rt < RT; rt++)
#pragma unroll
                for (int tt = 0; tt < TT; tt++) acc[rt][tt] = accm[rt][tt] = f4{0.f, 0.f, 0.f, 0.f};
        }
        cur = nxt;
        s = s2; g = g2; blk = blk2; rb = rb2;
#pragma unroll
        for (int rt = 0; rt < RT; rt++) rowA[rt] = rowA2[rt];
    }
}

template <bool Q6, int NTG>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(const GemmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int last_sh;
    gemm_units<Q6, NTG>(a, lds, &last_sh, 0, blockIdx.x, a.G, (int)a.P, 0);
}

// Q4_K segments then Q6_K segments sharing the activations in one launch:
// work-groups [0, G4) take the Q4_K units [0, P4), the others the Q6_K units
// (each type's work-groups its own instruction sequence, so a row's sums are
// formed as in a single-type launch over the same work-group shares).
template <int NTG>
__global__ __launch_bounds__(kThreads) void gemm_mfma_mixed_kernel(const GemmArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int last_sh;
    const int w = blockIdx.x;
    if (w < a.G4) gemm_units<false, NTG>(a, lds, &last_sh, 0, w, a.G4, (int)a.P4, 0);
    else gemm_units<true, NTG>(a, lds, &last_sh, a.G4, w - a.G4, a.G - a.G4, (int)(a.P - a.P4), (int)a.P4);
}

// The hq records of T tokens from the v values of prepared activations (xq,
// token stride xs): for inputs whose producer wrote only xq.
__global__ __launch_bounds__(256) void hq_from_v_kernel(const uint8_t *xq, int64_t xs, int K, uint8_t *hq) {
    __shared__ float red[4];
    const int t = blockIdx.y, tid = threadIdx.x;
    const float v = ((const float *)(xq + (int64_t)t * xs + xq_off(K).v_off))[blockIdx.x * 256 + tid];
    xjd::emit_hq(v, tid, hq + (int64_t)t * hq_stride(K) + (int64_t)blockIdx.x * kHqBlk, red);
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
                            2 * kGemmMaxT * kHqBlk) == hipSuccess;
    (void)raised;
    hipLaunchKernelGGL((gemm_mfma_kernel<Q6, NTG>), dim3(a.G), dim3(kThreads), lds, st, a);
}
template <int NTG>
void launch_m(const GemmArgs &a, size_t lds, hipStream_t st) {
    static const bool raised =
        hipFuncSetAttribute((const void *)gemm_mfma_mixed_kernel<NTG>, hipFuncAttributeMaxDynamicSharedMemorySize,
                            2 * kGemmMaxT * kHqBlk) == hipSuccess;
    (void)raised;
    hipLaunchKernelGGL((gemm_mfma_mixed_kernel<NTG>), dim3(a.G), dim3(kThreads), lds, st, a);
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
        a.nseg < 1 || a.nseg > kGemmMaxSeg || a.n6 < 0 || a.n6 >= a.nseg || (a.n6 && a.type != XJ_Q4_K))
        return -1;
    if (!a.hq || !a.part || !a.cnt || (a.hs & 255) || ((uintptr_t)a.hq & 255) || a.hs < hq_stride(a.K)) return -1;
    a.rg0[0] = 0;
    for (int i = 0; i < a.nseg; i++) {
        const GemmSeg &sg = a.seg[i];
        if (!sg.w || !sg.y || sg.N < 1 || ((uintptr_t)sg.w & 15)) return -1;
        a.rg0[i + 1] = a.rg0[i] + (sg.N + kRG - 1) / kRG;
    }
    for (int i = a.nseg + 1; i <= kGemmMaxSeg; i++) a.rg0[i] = a.rg0[a.nseg];
    a.nb = a.K / 256;
    a.P = (int64_t)a.rg0[a.nseg] * a.nb;
    // the fewest work-groups (at most one per CU) that give none more units
    // than a work-group per CU would: every share then has the same length,
    // and a row group's blocks are split over fewer partial sums (Q4_K
    // 2560 x 4096 at T = 64, 320 units: 160 work-groups 26.8 us, 256 31.6 us)
    {
        const int64_t g = a.P < cu_count() ? a.P : cu_count(), per = (a.P + g - 1) / g;
        a.G = (int)((a.P + per - 1) / per);
    }
    if (a.P >= (1 << 23)) return -1;   // unit indices times G stay in 32 bits
    // mixed: the CUs shared out so that the longer of the two types' shares
    // is shortest, a Q6_K unit counted as 3/2 of a Q4_K unit (its three
    // products per group against two), then each type on the fewest
    // work-groups that keep its share
    a.P4 = (int64_t)a.rg0[a.nseg - a.n6] * a.nb;
    a.G4 = a.G;
    if (a.n6) {
        const int64_t P6 = a.P - a.P4, ncu = cu_count();
        int64_t best = -1, b4 = 1, b6 = 1;
        for (int64_t g6 = 1; g6 < ncu && g6 <= P6; g6++) {
            const int64_t g4 = ncu - g6 < a.P4 ? ncu - g6 : a.P4;
            if (g4 < 1) break;
            const int64_t c = std::max(2 * ((a.P4 + g4 - 1) / g4), 3 * ((P6 + g6 - 1) / g6));
            if (best < 0 || c < best) best = c, b4 = g4, b6 = g6;
        }
        const int64_t s4 = (a.P4 + b4 - 1) / b4, s6 = (P6 + b6 - 1) / b6;
        a.G4 = (int)((a.P4 + s4 - 1) / s4);
        a.G = a.G4 + (int)((P6 + s6 - 1) / s6);
    }
    if (a.rg0[a.nseg] > n_cnt || (int64_t)(a.G + a.rg0[a.nseg]) * a.T * kRG > part_floats) return -1;
    const size_t lds = 2 * (size_t)a.T * kHqBlk;
    const bool q6 = a.type == XJ_Q6_K;
    const int ntg = (a.T + 15) / 16;
    if (a.n6) {
        switch (ntg) {
        case 1: launch_m<1>(a, lds, st); break;
        case 2: launch_m<2>(a, lds, st); break;
        case 3: launch_m<3>(a, lds, st); break;
        default: launch_m<4>(a, lds, st); break;
        }
    } else {
        switch (ntg) {
        case 1: q6 ? launch_g<true, 1>(a, lds, st) : launch_g<false, 1>(a, lds, st); break;
        case 2: q6 ? launch_g<true, 2>(a, lds, st) : launch_g<false, 2>(a, lds, st); break;
        case 3: q6 ? launch_g<true, 3>(a, lds, st) : launch_g<false, 3>(a, lds, st); break;
        default: q6 ? launch_g<true, 4>(a, lds, st) : launch_g<false, 4>(a, lds, st); break;
        }
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

int hq_from_v_launch(const uint8_t *xq, int K, int T, uint8_t *hq, hipStream_t st) {
    if (T < 1 || K < 256 || K % 256 || !xq || !hq) return -1;
    hipLaunchKernelGGL(hq_from_v_kernel, dim3(K / 256, T), dim3(256), 0, st, xq, (int64_t)xq_off(K).stride, K, hq);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int rms_scale_launch(const uint8_t *xq, int64_t xs, int K, int T, float eps, float *tsc, hipStream_t st) {
    if (T < 1 || K < 32 || K % 32 || !xq || !tsc) return -1;
    hipLaunchKernelGGL(rms_scale_kernel, dim3(T), dim3(64), 0, st, xq, xs, K, eps, tsc);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace xjk
