// Fused dequant-GEMV for gfx950 (Q4_K / Q6_K / Q8_0 / F32), 1..8 activation rows.
//
// Computes the reference's matmul (src/xiaoju-pipe/core/xj_cpu.c:36-54,
// y[t][r] = dot(dequant(W[r]), x[t])) with the neighbouring element-wise work
// folded in, in two launches:
//   prep  the prologue, once per launch: RMSNorm (xj_cpu.c:56-61, double
//         sum), SwiGLU silu(g)*u (xj_cpu.c:273) or per-head gated RMSNorm
//         norm(o)*w*silu(z) (xj_cpu.c:215-217); the result v is written as
//         21-bit integers X = rint(v * 2^(20-E)) per 32-element group (E the
//         group's binary exponent), split into three int8 digit planes.
//   gemv  weights x activations with v_dot4_i32_i8: for every quantization
//         sub-block, sum_l q_l X_l is formed exactly in 32-bit integers, then
//         scaled once in fp32 (d*sc, the group's 2^(E-20)) and the block
//         minimum term dmin*m*sum(X) subtracted. Epilogues: store, residual
//         add (xj_cpu.c:268,275), depthwise causal conv + SiLU with state
//         carry and checkpoints (xj_cpu.c:172-182,220), greedy argmax
//         partials for the LM head (xj_spec.c:12-16 tie rule).
// The activation digits add at most 2^-21 of the group maximum per element,
// about 2e-6 relative on a dot product, below the 1e-3 parity bar by three
// orders of magnitude (fp32 accumulation itself is ~1e-6).
//
// Work mapping. A team of `lanes` lanes owns `rpt` rows; a 256-thread
// work-group holds 256/lanes teams. A lane takes 64-element units (one Q4_K
// scale pair, one Q6_K half-block column of 16, two Q8_0 blocks) of its rows
// with stride `lanes`, so consecutive lanes read consecutive weight bytes.
// Each unit's activation digits are read from LDS once per token and used for
// all of the team's rows. Lane partials are combined in a fixed butterfly
// (DPP within 16 lanes, then cross-row shuffles), so a row's result does not
// depend on T, on the grid, or on which work-group computed it. One launch
// serves up to four weight segments that share K (e.g. qkv, gate, beta and
// alpha of a DeltaNet layer).
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
constexpr int kCuMaxT = 5;   // tokens of a per-CU launch (speculative verify widths)
static int g_cus = 256;
static int g_grid_cap = 256 * 8;     // work-groups of a looping multi-token launch
static int g_grid_cap1 = 256 * 3;    // ... of a looping single-token launch
static bool g_grid_forced = false;   // XJ_GEMV_WG_PER_CU given: one cap for every launch

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ u32x4 ld16(const uint8_t *p) { return *(const u32x4 *)p; }
__device__ __forceinline__ u32x4 lds16(const uint8_t *p) { return *(const u32x4 *)p; }

// ---------------------------------------------------------------- prep --
// One thread per input element k of token blockIdx.y; 32 consecutive lanes
// form one digit group.
__global__ __launch_bounds__(256) void prep_kernel(const GArgs a) {
    const int K = a.K, t = blockIdx.y, tid = threadIdx.x, k = blockIdx.x * 256 + tid;
    const XqOff o = xq_off(K);
    const bool in = k < K;
    __shared__ double red[4];
    const float *x = a.x + (int64_t)t * a.xs;
    float v = 0.f;
    float xr = 0.f;   // PRO_RMSU: the raw input, for the group's sum of squares
    if (a.pro == PRO_RMSU) {
        if (in) {
            xr = x[k];
            v = xr * a.pro_w[k];
        }
    } else if (a.pro == PRO_SWIGLU) {
        if (in) v = xjd::silu(x[k]) * a.x2[(int64_t)t * a.x2s + k];
    } else if (a.pro == PRO_GATED_RMS) {
        const int G = a.group;
        float gsc;
        if (G % 64 == 0 && 256 % G == 0) {
            // each wavefront lies inside one head: combine the wavefront sums of the head
            const float o1 = in ? x[k] : 0.f;
            const double ws = xjd::wave_sum_d((double)o1 * o1);
            if ((tid & 63) == 0) red[tid >> 6] = ws;
            __syncthreads();
            const int w0 = (tid / G) * (G / 64);
            double ss = 0;
            for (int w = w0; w < w0 + G / 64; w++) ss += red[w];
            gsc = 1.0f / sqrtf((float)(ss / G) + a.eps);
        } else {
            const int h0 = in ? (k / G) * G : 0;
            double ss = 0;
            for (int i = h0; in && i < h0 + G; i++) ss += (double)x[i] * x[i];
            gsc = 1.0f / sqrtf((float)(ss / G) + a.eps);
        }
        if (in) v = x[k] * gsc * a.pro_w[k % G] * xjd::silu(a.x2[(int64_t)t * a.x2s + k]);
    } else {
        if (in) v = x[k];
    }
    uint8_t *dst = a.xq + (int64_t)t * o.stride;
    if (!a.hq_only) xjd::emit_xq(v, k, in, dst, o);
    if (a.pro == PRO_RMSU) {
        const double ss = xjd::group_ss(xr);
        if (in && (k & 31) == 0) ((double *)(dst + o.ss_off))[k >> 5] = ss;
    }
    if (a.hq) {   // K % 256 == 0: every thread holds an element
        __shared__ float hred[4];
        xjd::emit_hq(v, tid, a.hq + (int64_t)t * hq_stride(K) + (int64_t)blockIdx.x * kHqBlk, hred);
    }
}

// -------------------------------------------------------- unit kernels --
// Exact integer sum over 4N elements of q (packed signed bytes) times X,
// whose digit planes start at p, p + 32 and p + 64:
//   ((sum q*a) * 128 + sum q*b) * 128 + sum q*c.
// Q4_K (q <= 15, 32 elements) and Q6_K (q <= 63, 16 elements) stay below
// 2^31 at every step.
template <int N>
__device__ __forceinline__ int qdot(const uint32_t (&q)[N], const u32x4 (&pa)[N / 4], const u32x4 (&pb)[N / 4],
                                    const u32x4 (&pc)[N / 4]) {
    int s = 0;
#pragma unroll
    for (int j = 0; j < N; j++) s = sdot4(q[j], pa[j >> 2][j & 3], s);
    s *= 128;
#pragma unroll
    for (int j = 0; j < N; j++) s = sdot4(q[j], pb[j >> 2][j & 3], s);
    s *= 128;
#pragma unroll
    for (int j = 0; j < N; j++) s = sdot4(q[j], pc[j >> 2][j & 3], s);
    return s;
}

template <int N>
__device__ __forceinline__ void planes(const uint8_t *p, u32x4 (&pa)[N / 4], u32x4 (&pb)[N / 4], u32x4 (&pc)[N / 4]) {
#pragma unroll
    for (int j = 0; j < N / 4; j++) {
        pa[j] = lds16(p + 16 * j);
        pb[j] = lds16(p + 32 + 16 * j);
        pc[j] = lds16(p + 64 + 16 * j);
    }
}

// Raw bytes of one 64-element unit of a Q4_K or Q6_K row:
//   Q4_K  a = block header (d|dmin, 12 scale bytes), b, c = the pair's 32 nibble bytes
//   Q6_K  a, b = ql columns (+0, +32), c = qh column, e = the half's 8 scales, f = d
struct RawU {
    u32x4 a, b, c;
    u32x2 e;
    uint32_t f;
};

// One Q4_K sub-block term S ds - SX dm: SX dm rounded, then one fused
// multiply-add (the rounding the compiler gives the plain expression), written
// out so that every kernel forming it rounds alike.
__device__ __forceinline__ float q4k_part(int S, float ds, float SX, float dm) {
    return __builtin_fmaf((float)S, ds, -(SX * dm));
}

// Q4_K unit = scale pair p of a block: elements 64p..64p+63, i.e. sub-blocks
// 2p (low nibbles of qs[32p..32p+31]) and 2p+1 (high nibbles), whose
// activations are x-groups g0 and g0+1. Scale/min decoding as
// get_scale_min_k4 (xj_quant.h:49-52).
template <int T>
__device__ __forceinline__ void q4k_unit(const RawU &w, int p, int g0, const uint8_t *xl, int ldsT, const XqOff &o,
                                         float (&acc)[T]) {
    const int jm = (2 * p) & 3;
    const bool hi4 = p >= 2;
    const float d = xjd::f16_to_f32(w.a.x & 0xFFFFu), dmin = xjd::f16_to_f32(w.a.x >> 16);
    float ds[2], dm[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
        const uint32_t A = byte_of(w.a.y, jm + s), B = byte_of(w.a.z, jm + s), C = byte_of(w.a.w, jm + s);
        const uint32_t sc = hi4 ? ((C & 0xF) | ((A >> 6) << 4)) : (A & 63);
        const uint32_t mn = hi4 ? ((C >> 4) | ((B >> 6) << 4)) : (B & 63);
        ds[s] = d * (float)sc;
        dm[s] = dmin * (float)mn;
    }
    const uint32_t q[8] = {w.b.x, w.b.y, w.b.z, w.b.w, w.c.x, w.c.y, w.c.z, w.c.w};
#pragma unroll
    for (int s = 0; s < 2; s++) {
        uint32_t nib[8];
#pragma unroll
        for (int j = 0; j < 8; j++) nib[j] = s ? (q[j] >> 4) & 0x0F0F0F0Fu : q[j] & 0x0F0F0F0Fu;
        const int g = g0 + s;
#pragma unroll
        for (int t = 0; t < T; t++) {
            const uint8_t *xt = xl + t * ldsT;
            u32x4 pa[2], pb[2], pc[2];
            planes<8>(xt + g * kDigStride, pa, pb, pc);
            const float f = ((const float *)(xt + o.f_off))[g];
            const int2 sxp = ((const int2 *)(xt + o.sx_off))[g];
            const float SX = (float)(sxp.x + sxp.y);
            const int S = qdot<8>(nib, pa, pb, pc);
            const float part = q4k_part(S, ds[s], SX, dm[s]);
            acc[t] = fmaf(part, f, acc[t]);
        }
    }
}

// Q6_K unit = column half hl of half h of a block: for each 32-element group
// G of the half, the 16 elements 128h + 32G + 16hl .. +15 (one scale
// sub-block each), activations in x-group gb + G. Bit layout as
// dequantize_row_q6_K: q = (ql & 15 | ql >> 4) | qh bit pair << 4, value q - 32.
template <int T>
__device__ __forceinline__ void q6k_unit(const RawU &w, int hl, int gb, const uint8_t *xl, int ldsT, const XqOff &o,
                                         float (&acc)[T]) {
    const float d = xjd::f16_to_f32(w.f);
#pragma unroll
    for (int G = 0; G < 4; G++) {
        uint32_t q6[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t a0 = w.a[j], a1 = w.b[j], hb = w.c[j];
            q6[j] = G == 0 ? (a0 & 0x0F0F0F0Fu) | ((hb << 4) & 0x30303030u)
                  : G == 1 ? (a1 & 0x0F0F0F0Fu) | ((hb << 2) & 0x30303030u)
                  : G == 2 ? ((a0 >> 4) & 0x0F0F0F0Fu) | (hb & 0x30303030u)
                           : ((a1 >> 4) & 0x0F0F0F0Fu) | ((hb >> 2) & 0x30303030u);
        }
        const uint32_t sw = G < 2 ? w.e.x : w.e.y;
        const float dsc = d * (float)(int8_t)byte_of(sw, 2 * (G & 1) + hl);
        const int g = gb + G;
#pragma unroll
        for (int t = 0; t < T; t++) {
            const uint8_t *xt = xl + t * ldsT;
            u32x4 pa[1], pb[1], pc[1];
            planes<4>(xt + g * kDigStride + 16 * hl, pa, pb, pc);
            const float f = ((const float *)(xt + o.f_off))[g];
            const int sxh = ((const int *)(xt + o.sx_off))[2 * g + hl];
            const int S = qdot<4>(q6, pa, pb, pc) - 32 * sxh;
            acc[t] = fmaf((float)S * dsc, f, acc[t]);
        }
    }
}

// The same units of two rows (same lane position, so the same x-groups):
// each activation read from LDS serves both rows. Every row's arithmetic is
// q4k_unit's / q6k_unit's, statement for statement, so a row's result does
// not depend on whether it was computed alone or in a pair.
template <int T>
__device__ __forceinline__ void q4k_unit2(const RawU &w0, const RawU &w1, int p, int g0, const uint8_t *xl, int ldsT,
                                          const XqOff &o, float (&acc0)[T], float (&acc1)[T]) {
    const int jm = (2 * p) & 3;
    const bool hi4 = p >= 2;
    float ds[2][2], dm[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const RawU &w = i ? w1 : w0;
        const float d = xjd::f16_to_f32(w.a.x & 0xFFFFu), dmin = xjd::f16_to_f32(w.a.x >> 16);
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const uint32_t A = byte_of(w.a.y, jm + s), B = byte_of(w.a.z, jm + s), C = byte_of(w.a.w, jm + s);
            const uint32_t sc = hi4 ? ((C & 0xF) | ((A >> 6) << 4)) : (A & 63);
            const uint32_t mn = hi4 ? ((C >> 4) | ((B >> 6) << 4)) : (B & 63);
            ds[i][s] = d * (float)sc;
            dm[i][s] = dmin * (float)mn;
        }
    }
    const uint32_t q0[8] = {w0.b.x, w0.b.y, w0.b.z, w0.b.w, w0.c.x, w0.c.y, w0.c.z, w0.c.w};
    const uint32_t q1[8] = {w1.b.x, w1.b.y, w1.b.z, w1.b.w, w1.c.x, w1.c.y, w1.c.z, w1.c.w};
#pragma unroll
    for (int s = 0; s < 2; s++) {
        uint32_t n0[8], n1[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            n0[j] = s ? (q0[j] >> 4) & 0x0F0F0F0Fu : q0[j] & 0x0F0F0F0Fu;
            n1[j] = s ? (q1[j] >> 4) & 0x0F0F0F0Fu : q1[j] & 0x0F0F0F0Fu;
        }
        const int g = g0 + s;
#pragma unroll
        for (int t = 0; t < T; t++) {
            const uint8_t *xt = xl + t * ldsT;
            u32x4 pa[2], pb[2], pc[2];
            planes<8>(xt + g * kDigStride, pa, pb, pc);
            const float f = ((const float *)(xt + o.f_off))[g];
            const int2 sxp = ((const int2 *)(xt + o.sx_off))[g];
            const float SX = (float)(sxp.x + sxp.y);
            const int S0 = qdot<8>(n0, pa, pb, pc), S1 = qdot<8>(n1, pa, pb, pc);
            const float part0 = q4k_part(S0, ds[0][s], SX, dm[0][s]);
            const float part1 = q4k_part(S1, ds[1][s], SX, dm[1][s]);
            acc0[t] = fmaf(part0, f, acc0[t]);
            acc1[t] = fmaf(part1, f, acc1[t]);
        }
    }
}

template <int T>
__device__ __forceinline__ void q6k_unit2(const RawU &w0, const RawU &w1, int hl, int gb, const uint8_t *xl, int ldsT,
                                          const XqOff &o, float (&acc0)[T], float (&acc1)[T]) {
    const float d0 = xjd::f16_to_f32(w0.f), d1 = xjd::f16_to_f32(w1.f);
#pragma unroll
    for (int G = 0; G < 4; G++) {
        uint32_t q6[2][4];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const RawU &w = i ? w1 : w0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t a0 = w.a[j], a1 = w.b[j], hb = w.c[j];
                q6[i][j] = G == 0 ? (a0 & 0x0F0F0F0Fu) | ((hb << 4) & 0x30303030u)
                         : G == 1 ? (a1 & 0x0F0F0F0Fu) | ((hb << 2) & 0x30303030u)
                         : G == 2 ? ((a0 >> 4) & 0x0F0F0F0Fu) | (hb & 0x30303030u)
                                  : ((a1 >> 4) & 0x0F0F0F0Fu) | ((hb >> 2) & 0x30303030u);
            }
        }
        const uint32_t sw0 = G < 2 ? w0.e.x : w0.e.y, sw1 = G < 2 ? w1.e.x : w1.e.y;
        const float dsc0 = d0 * (float)(int8_t)byte_of(sw0, 2 * (G & 1) + hl);
        const float dsc1 = d1 * (float)(int8_t)byte_of(sw1, 2 * (G & 1) + hl);
        const int g = gb + G;
#pragma unroll
        for (int t = 0; t < T; t++) {
            const uint8_t *xt = xl + t * ldsT;
            u32x4 pa[1], pb[1], pc[1];
            planes<4>(xt + g * kDigStride + 16 * hl, pa, pb, pc);
            const float f = ((const float *)(xt + o.f_off))[g];
            const int sxh = ((const int *)(xt + o.sx_off))[2 * g + hl];
            const int S0 = qdot<4>(q6[0], pa, pb, pc) - 32 * sxh;
            const int S1 = qdot<4>(q6[1], pa, pb, pc) - 32 * sxh;
            acc0[t] = fmaf((float)S0 * dsc0, f, acc0[t]);
            acc1[t] = fmaf((float)S1 * dsc1, f, acc1[t]);
        }
    }
}

// Q8_0 unit u = block u (32 elements). |q| <= 128 can reach 2^32 over 32
// elements, so the c plane is added in fp32: ((sum q*a) * 128 + sum q*b) * 128 + sum q*c.
template <int T, int RPT>
__device__ __forceinline__ void unit_q80(const u32x4 (&qa)[RPT], const u32x4 (&qb)[RPT], const uint32_t (&dd)[RPT], int u,
                                         const uint8_t *xl, int ldsT, const XqOff &o, float (&acc)[RPT][T]) {
#pragma unroll
    for (int t = 0; t < T; t++) {
        const uint8_t *xt = xl + t * ldsT;
        u32x4 pa[2], pb[2], pc[2];
        planes<8>(xt + u * kDigStride, pa, pb, pc);
        const float f = ((const float *)(xt + o.f_off))[u];
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const uint32_t q[8] = {qa[i].x, qa[i].y, qa[i].z, qa[i].w, qb[i].x, qb[i].y, qb[i].z, qb[i].w};
            int sa = 0, sb = 0, sc = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                sa = sdot4(q[j], pa[j >> 2][j & 3], sa);
                sb = sdot4(q[j], pb[j >> 2][j & 3], sb);
                sc = sdot4(q[j], pc[j >> 2][j & 3], sc);
            }
            const float S = (float)(sa * 128 + sb) * 128.0f + (float)sc;
            acc[i][t] = fmaf(S * xjd::f16_to_f32(dd[i]), f, acc[i][t]);
        }
    }
}

// ---------------------------------------------------------- row loops --
// Unit u of a row, for either K-quant type, with the same five loads and
// addresses chosen without branches (a load whose result reaches a register
// through a control-flow merge must complete before the merge); used for the
// window issued before a work-group's LDS setup. Q4_K re-reads header bytes
// for e and f, other types read the row's first bytes; the extra values are
// ignored. Q4 (a launch whose rows are all Q4_K): the three Q4_K loads only.
template <bool Q4>
__device__ __forceinline__ RawU load_unit(uint32_t type, const uint8_t *__restrict__ W, int64_t nblk, int64_t rb, int u) {
    if constexpr (Q4) {
        const uint8_t *blk = W + (rb + (u >> 2)) * 144;
        RawU r;
        r.a = ld16(blk);
        r.b = ld16(blk + 16 + 32 * (u & 3));
        r.c = ld16(blk + 32 + 32 * (u & 3));
        r.e = u32x2{0u, 0u};
        r.f = 0u;
        return r;
    }
    const bool q4 = type == XJ_Q4_K, q6 = type == XJ_Q6_K;
    const int h = (u >> 1) & 1, hl = u & 1;
    const int64_t b = rb + (u >> 2);
    const uint8_t *blk = W + b * 144, *ql = W + b * 128 + 64 * h + 16 * hl, *w0 = W + rb * 32;
    const uint8_t *pa = q4 ? blk : q6 ? ql : w0;
    const uint8_t *pb = q4 ? blk + 16 + 32 * (u & 3) : q6 ? ql + 32 : w0;
    const uint8_t *pc = q4 ? blk + 32 + 32 * (u & 3) : q6 ? W + nblk * 128 + b * 64 + 32 * h + 16 * hl : w0;
    const uint8_t *pe = q6 ? W + nblk * 192 + b * 16 + 8 * h : pa;
    const uint8_t *pf = q6 ? W + nblk * 208 + b * 2 : pa;
    RawU r;
    r.a = ld16(pa);
    r.b = ld16(pb);
    r.c = ld16(pc);
    r.e = *(const u32x2 *)pe;
    r.f = *(const uint16_t *)pf;
    return r;
}

// Q4_K / Q6_K rows: lane `lane` takes units u = lane, lane + TS, ... Since
// TS is a multiple of 4, the lane's position inside a block (Q4_K scale pair,
// Q6_K half and column half) is the same for all its units, so every pointer
// advances by a constant stride. `cur` holds unit `lane` on entry.
//
// MU > 0 (single-token launches, at most MU <= 4 units per lane): the loop over
// the lane's units is unrolled, so every unit has its own registers and PD
// units ahead of the one being computed are in flight; the loads are
// unconditional (units past the row read the padding after the tensor,
// kWeightPad) and only the arithmetic is predicated. A rolled loop that
// rotated a register ring would have to wait for each load at the rotation.
// MU == 0: rolled loop with the next unit in flight.
__device__ __forceinline__ RawU ld_q4k(const uint8_t *blk, int p) {
    RawU r;
    r.a = ld16(blk);
    r.b = ld16(blk + 16 + 32 * p);
    r.c = ld16(blk + 32 + 32 * p);
    return r;
}

struct Q6Ptr {
    const uint8_t *ql, *qh, *sc, *dd;
};

// unit k steps (of TS/4 blocks) after the one q points at
__device__ __forceinline__ RawU ld_q6k(const Q6Ptr &q, int64_t k) {
    RawU r;
    r.a = ld16(q.ql + k * 128);
    r.b = ld16(q.ql + k * 128 + 32);
    r.c = ld16(q.qh + k * 64);
    r.e = *(const u32x2 *)(q.sc + k * 16);
    r.f = *(const uint16_t *)(q.dd + k * 2);
    return r;
}

// Units a lane has in flight ahead of the one it computes (MU > 0), and the
// window of units loaded before the work-group's LDS setup. Two units: deeper
// windows (up to all MU units up front) measured slower on decode-sized
// launches, whose activation copies then queue behind more weight requests.
// Q4 (Q4_K-only launches): three loads per unit instead of five.
template <int MU, bool Q4>
struct Win {
    static constexpr int PD = MU <= 1 ? 0 : 1;
    static constexpr int N = PD + 1;
    static constexpr int LOADS = (Q4 ? 3 : 5) * N;   // vector-memory instructions of the window
};

template <int T, int TS, int MU, int PD>
__device__ __forceinline__ void rows_q4k(const uint8_t *__restrict__ W, int64_t rb, int nu, int lane,
                                         const RawU (&win)[PD + 1], const uint8_t *xl, int ldsT, const XqOff &o,
                                         float (&acc)[T]) {
    constexpr int DB = TS / 4;
    const int p = lane & 3;
    const int g0 = 8 * (lane >> 2) + 2 * p;
    const uint8_t *blk = W + (rb + (lane >> 2)) * 144;
    RawU cur = win[0];
    if constexpr (MU > 0) {
        RawU r[MU];
#pragma unroll
        for (int m = 0; m <= PD; m++) r[m] = win[m];
#pragma unroll
        for (int m = 0; m < MU; m++) {
            __builtin_amdgcn_sched_barrier(0);   // keep each prefetch in its step (register budget)
            if (m + PD + 1 < MU) r[m + PD + 1] = ld_q4k(blk + (m + PD + 1) * DB * 144, p);
            if (lane + m * TS < nu) q4k_unit<T>(r[m], p, g0 + 8 * DB * m, xl, ldsT, o, acc);
        }
    } else {
        // the next unit of the row is requested during this one; after the
        // row's last unit that is the same unit again (a cache hit, where the
        // next row's bytes would come back from HBM long after that row's own
        // reads)
        int g = g0;
        for (int u = lane; u < nu; u += TS) {
            blk += u + TS < nu ? DB * 144 : 0;
            const RawU nxt = ld_q4k(blk, p);
            q4k_unit<T>(cur, p, g, xl, ldsT, o, acc);
            g += 8 * DB;
            cur = nxt;
        }
    }
}

template <int T, int TS, int MU, int PD>
__device__ __forceinline__ void rows_q6k(const uint8_t *__restrict__ W, int64_t nblk, int64_t rb, int nu, int lane,
                                         const RawU (&win)[PD + 1], const uint8_t *xl, int ldsT, const XqOff &o,
                                         float (&acc)[T]) {
    constexpr int DB = TS / 4;
    const int h = (lane >> 1) & 1, hl = lane & 1;
    const int64_t b = rb + (lane >> 2);
    Q6Ptr q{W + b * 128 + 64 * h + 16 * hl, W + nblk * 128 + b * 64 + 32 * h + 16 * hl,
            W + nblk * 192 + b * 16 + 8 * h, W + nblk * 208 + b * 2};
    const int gb0 = 8 * (lane >> 2) + 4 * h;
    RawU cur = win[0];
    if constexpr (MU > 0) {
        RawU r[MU];
#pragma unroll
        for (int m = 0; m <= PD; m++) r[m] = win[m];
#pragma unroll
        for (int m = 0; m < MU; m++) {
            __builtin_amdgcn_sched_barrier(0);   // keep each prefetch in its step (register budget)
            if (m + PD + 1 < MU) r[m + PD + 1] = ld_q6k(q, (m + PD + 1) * DB);
            if (lane + m * TS < nu) q6k_unit<T>(r[m], hl, gb0 + 8 * DB * m, xl, ldsT, o, acc);
        }
    } else {
        int gb = gb0;
        for (int u = lane; u < nu; u += TS) {
            const int st = u + TS < nu ? DB : 0;   // after the row's last unit: the same unit again
            q.ql += st * 128; q.qh += st * 64; q.sc += st * 16; q.dd += st * 2;
            const RawU nxt = ld_q6k(q, 0);
            q6k_unit<T>(cur, hl, gb, xl, ldsT, o, acc);
            gb += 8 * DB;
            cur = nxt;
        }
    }
}

// Two rows of a team in the rolled loop (several tokens): rows rb0 and rb1 at
// the same lane positions, the next unit of both in flight; `w0`, `w1` hold
// unit `lane` of each on entry.
template <int T, int TS>
__device__ __forceinline__ void rows2_q4k(const uint8_t *__restrict__ W, int64_t rb0, int64_t rb1, int nu, int lane,
                                          const RawU &w0, const RawU &w1, const uint8_t *xl, int ldsT, const XqOff &o,
                                          float (&acc0)[T], float (&acc1)[T]) {
    constexpr int DB = TS / 4;
    const int p = lane & 3;
    const uint8_t *b0 = W + (rb0 + (lane >> 2)) * 144, *b1 = W + (rb1 + (lane >> 2)) * 144;
    RawU c0 = w0, c1 = w1;
    int g = 8 * (lane >> 2) + 2 * p;
    for (int u = lane; u < nu; u += TS) {
        const int st = u + TS < nu ? DB * 144 : 0;   // after the rows' last unit: the same unit again
        b0 += st;
        b1 += st;
        const RawU n0 = ld_q4k(b0, p), n1 = ld_q4k(b1, p);
        q4k_unit2<T>(c0, c1, p, g, xl, ldsT, o, acc0, acc1);
        g += 8 * DB;
        c0 = n0;
        c1 = n1;
    }
}

template <int T, int TS>
__device__ __forceinline__ void rows2_q6k(const uint8_t *__restrict__ W, int64_t nblk, int64_t rb0, int64_t rb1, int nu,
                                          int lane, const RawU &w0, const RawU &w1, const uint8_t *xl, int ldsT,
                                          const XqOff &o, float (&acc0)[T], float (&acc1)[T]) {
    constexpr int DB = TS / 4;
    const int h = (lane >> 1) & 1, hl = lane & 1;
    const int64_t b0 = rb0 + (lane >> 2), b1 = rb1 + (lane >> 2);
    Q6Ptr q0{W + b0 * 128 + 64 * h + 16 * hl, W + nblk * 128 + b0 * 64 + 32 * h + 16 * hl,
             W + nblk * 192 + b0 * 16 + 8 * h, W + nblk * 208 + b0 * 2};
    Q6Ptr q1{W + b1 * 128 + 64 * h + 16 * hl, W + nblk * 128 + b1 * 64 + 32 * h + 16 * hl,
             W + nblk * 192 + b1 * 16 + 8 * h, W + nblk * 208 + b1 * 2};
    int gb = 8 * (lane >> 2) + 4 * h;
    RawU c0 = w0, c1 = w1;
    for (int u = lane; u < nu; u += TS) {
        const int st = u + TS < nu ? DB : 0;   // after the rows' last unit: the same unit again
        q0.ql += st * 128; q0.qh += st * 64; q0.sc += st * 16; q0.dd += st * 2;
        q1.ql += st * 128; q1.qh += st * 64; q1.sc += st * 16; q1.dd += st * 2;
        const RawU n0 = ld_q6k(q0, 0), n1 = ld_q6k(q1, 0);
        q6k_unit2<T>(c0, c1, hl, gb, xl, ldsT, o, acc0, acc1);
        gb += 8 * DB;
        c0 = n0;
        c1 = n1;
    }
}

template <int T, int TS, int RPT>
__device__ __forceinline__ void rows_q80(const uint8_t *__restrict__ W, int64_t nblk, const int64_t (&rb)[RPT], int nu,
                                         int lane, const uint8_t *xl, int ldsT, const XqOff &o, float (&acc)[RPT][T]) {
    for (int u = lane; u < nu; u += TS) {
        u32x4 qa[RPT], qb[RPT];
        uint32_t dd[RPT];
#pragma unroll
        for (int i = 0; i < RPT; i++) {
            const int64_t g = rb[i] + u;
            qa[i] = ld16(W + g * 32);
            qb[i] = ld16(W + g * 32 + 16);
            dd[i] = *(const uint16_t *)(W + nblk * 32 + g * 2);
        }
        unit_q80<T, RPT>(qa, qb, dd, u, xl, ldsT, o, acc);
    }
}

// F32 rows (small tensors and tests): fp32 products with the prepared v, read from global memory.
template <int T, int TS, int RPT>
__device__ __forceinline__ void rows_f32(const uint8_t *__restrict__ W, const int64_t (&row)[RPT], int K, int lane,
                                         const uint8_t *xq, const XqOff &o, float (&acc)[RPT][T]) {
    for (int c = lane; c < K / 32; c += TS) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            const float *v = (const float *)(xq + (int64_t)t * o.stride + o.v_off) + c * 32;
#pragma unroll
            for (int i = 0; i < RPT; i++) {
                const float *w = (const float *)W + row[i] * K + c * 32;
                float s = acc[i][t];
#pragma unroll
                for (int e = 0; e < 32; e += 4) {
                    const f32x4 wv = *(const f32x4 *)(w + e), xv = *(const f32x4 *)(v + e);
                    s = fmaf(wv.x, xv.x, s);
                    s = fmaf(wv.y, xv.y, s);
                    s = fmaf(wv.z, xv.z, s);
                    s = fmaf(wv.w, xv.w, s);
                }
                acc[i][t] = s;
            }
        }
    }
}

// F16 / BF16 rows (no configuration uses them): widened exactly, fp32
// products with the prepared v, read from global memory.
template <int T, int TS, int RPT>
__device__ __forceinline__ void rows_h16(const uint8_t *__restrict__ W, const int64_t (&row)[RPT], int K, int lane,
                                         bool bf, const uint8_t *xq, const XqOff &o, float (&acc)[RPT][T]) {
    for (int c = lane; c < K / 32; c += TS) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            const float *v = (const float *)(xq + (int64_t)t * o.stride + o.v_off) + c * 32;
#pragma unroll
            for (int i = 0; i < RPT; i++) {
                const uint8_t *w = W + (row[i] * K + c * 32) * 2;
                float s = acc[i][t];
#pragma unroll
                for (int e = 0; e < 32; e += 8) {
                    const u32x4 wv = ld16(w + 2 * e);
                    const f32x4 x0 = *(const f32x4 *)(v + e), x1 = *(const f32x4 *)(v + e + 4);
                    const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int h = 0; h < 8; h++) {
                        const uint32_t b = (wv[h >> 1] >> (16 * (h & 1))) & 0xFFFFu;
                        s = fmaf(bf ? __uint_as_float(b << 16) : xjd::f16_to_f32(b), xs[h], s);
                    }
                }
                acc[i][t] = s;
            }
        }
    }
}

// Q5_K rows (no configuration uses them): a unit is scale pair p of a block,
// as for Q4_K, with bit j of qh[l] as the fifth bit of element l of sub-block
// j (xj_quant.h:83-98). |q| <= 31 keeps the digit-plane sums within 32 bits.
// Blocks stay in the GGUF layout (176 bytes: d, dmin, scales[12], qh[32], qs[128]).
template <int T, int TS>
__device__ __forceinline__ void rows_q5k(const uint8_t *__restrict__ W, int64_t rb, int nu, int lane,
                                         const uint8_t *xl, int ldsT, const XqOff &o, float (&acc)[T]) {
    for (int u = lane; u < nu; u += TS) {
        const int p = u & 3, jm = (2 * p) & 3;
        const bool hi4 = p >= 2;
        const uint8_t *blk = W + (rb + (u >> 2)) * 176;
        const u32x4 hdr = ld16(blk), h0 = ld16(blk + 16), h1 = ld16(blk + 32);
        const u32x4 qa = ld16(blk + 48 + 32 * p), qb = ld16(blk + 64 + 32 * p);
        const float d = xjd::f16_to_f32(hdr.x & 0xFFFFu), dmin = xjd::f16_to_f32(hdr.x >> 16);
        const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
        const uint32_t hb[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        const int g0 = 8 * (u >> 2) + 2 * p;
#pragma unroll
        for (int sb = 0; sb < 2; sb++) {
            const uint32_t A = byte_of(hdr.y, jm + sb), B = byte_of(hdr.z, jm + sb), C = byte_of(hdr.w, jm + sb);
            const uint32_t sc = hi4 ? ((C & 0xF) | ((A >> 6) << 4)) : (A & 63);
            const uint32_t mn = hi4 ? ((C >> 4) | ((B >> 6) << 4)) : (B & 63);
            const float ds = d * (float)sc, dm = dmin * (float)mn;
            const int j = 2 * p + sb;
            uint32_t q5[8];
#pragma unroll
            for (int k = 0; k < 8; k++)
                q5[k] = (sb ? (q[k] >> 4) & 0x0F0F0F0Fu : q[k] & 0x0F0F0F0Fu) | (((hb[k] >> j) & 0x01010101u) << 4);
            const int g = g0 + sb;
#pragma unroll
            for (int t = 0; t < T; t++) {
                const uint8_t *xt = xl + t * ldsT;
                u32x4 pa[2], pb[2], pc[2];
                planes<8>(xt + g * kDigStride, pa, pb, pc);
                const float f = ((const float *)(xt + o.f_off))[g];
                const int2 sxp = ((const int2 *)(xt + o.sx_off))[g];
                const int S = qdot<8>(q5, pa, pb, pc);
                acc[t] = fmaf((float)S * ds - (float)(sxp.x + sxp.y) * dm, f, acc[t]);
            }
        }
    }
}

// Team reduction over TS lanes (8, 16, 32 or 64) in a fixed order.
template <int TS>
__device__ __forceinline__ float team_sum(float v) {
    v += xjd::dpp<0xB1>(v);
    v += xjd::dpp<0x4E>(v);
    v += xjd::dpp<0x141>(v);
    if (TS >= 16) v += xjd::dpp<0x140>(v);
    if (TS >= 32) v += __shfl_xor(v, 16, 64);
    if (TS >= 64) v += __shfl_xor(v, 32, 64);
    return v;
}

// Segment of row group rg (the looping kernels: one segment costs one read).
__device__ __forceinline__ int seg_of(const GArgs &a, int rg) {
    int si = 0;
    while (si + 1 < a.nseg && rg >= a.seg[si + 1].wg0) si++;
    return si;
}
// The same with every segment's first work-group read at once (a loop over
// the segments waits for each read in turn); the ranges ascend, so the count
// of later segments starting at or before rg is its index.
__device__ __forceinline__ int seg_of_flat(const GArgs &a, int rg) {
    int si = 0;
#pragma unroll
    for (int i = 1; i < kMaxSeg; i++) si += i < a.nseg && rg >= a.seg[i].wg0 ? 1 : 0;
    return si;
}

// Team-reduced results acc[i][t] of rows (rg - wg0) * ROWS + team * RPT + i:
// lane i of the team stores row i (plain, residual add or conv + SiLU), and
// the work-group's greedy argmax partial is written when the segment has one.
// Operands of the epilogue of one row, loaded before the row's dot products
// so their latency overlaps the weight stream: the residual (EPI_ADD) or,
// for kernel sizes up to 4, the conv state and weights (EPI_CONV; larger
// kernels load them in the epilogue).
constexpr int kConvPre = 4;
template <int T>
struct EpiIn {
    float y[T];
    float st[kConvPre - 1], wc[kConvPre];
};

template <int T>
__device__ __forceinline__ void epi_load(const GSeg &sg, int64_t r, EpiIn<T> &e) {
    // Unconditional loads at clamped in-row addresses (a loaded value that
    // reaches its register through a branch would make the first use of the
    // weight window wait for every outstanding load); values an epilogue does
    // not use are ignored. y is valid memory for every epilogue.
    const bool conv = sg.epi == EPI_CONV && sg.conv_k <= kConvPre;
    const int KC = conv ? sg.conv_k : 2;
    const float *ps = conv ? sg.conv_state + r * (KC - 1) : sg.y + r;
    const float *pw = conv ? sg.conv_w + r * KC : sg.y + r;
#pragma unroll
    for (int t = 0; t < T; t++) e.y[t] = sg.y[(int64_t)t * sg.ys + r];
#pragma unroll
    for (int k = 0; k < kConvPre; k++) {
        if (k < kConvPre - 1) e.st[k < kConvPre - 1 ? k : 0] = ps[k < KC - 2 ? k : KC - 2];
        e.wc[k] = pw[k < KC - 1 ? k : KC - 1];
    }
}

// Epilogue of row r (one lane): conv + SiLU, residual add or plain store.
template <int T>
__device__ __forceinline__ void epi_row(const GArgs &a, const GSeg &sg, int64_t r, const float (&acc)[T],
                                        const EpiIn<T> &e) {
    if (sg.epi == EPI_CONV) {
        // register arrays with compile-time indices only (KC is a runtime value <= 8)
        const int KC = sg.conv_k;
        float st[8], wc[8];
#pragma unroll
        for (int k = 0; k < 8; k++) {
            if (KC <= kConvPre) {
                st[k] = k < kConvPre - 1 ? e.st[k < kConvPre - 1 ? k : 0] : 0.f;
                wc[k] = k < kConvPre ? e.wc[k < kConvPre ? k : 0] : 0.f;
            } else {
                st[k] = k + 1 < KC ? sg.conv_state[r * (KC - 1) + k] : 0.f;
                wc[k] = k < KC ? sg.conv_w[r * KC + k] : 0.f;
            }
        }
        float wl = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) if (k == KC - 1) wl = wc[k];
#pragma unroll
        for (int t = 0; t < T; t++) {
            const float xv = acc[t];
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < 7; k++) if (k + 1 < KC) s = fmaf(st[k], wc[k], s);
            s = fmaf(xv, wl, s);
#pragma unroll
            for (int k = 0; k < 6; k++) if (k + 2 < KC) st[k] = st[k + 1];
#pragma unroll
            for (int k = 0; k < 7; k++) if (k == KC - 2) st[k] = xv;
            sg.y[(int64_t)t * sg.ys + r] = xjd::silu(s);
            const int ta = a.t0 + t;
            if (ta < a.keep_n)
#pragma unroll
                for (int k = 0; k < 7; k++)
                    if (k + 1 < KC) sg.conv_ck[((int64_t)ta * sg.n_rows + r) * (KC - 1) + k] = st[k];
        }
#pragma unroll
        for (int k = 0; k < 7; k++) if (k + 1 < KC) sg.conv_state[r * (KC - 1) + k] = st[k];
    } else {
#pragma unroll
        for (int t = 0; t < T; t++) {
            float *yp = sg.y + (int64_t)t * sg.ys + r;
            const float yv = sg.epi == EPI_ADD ? e.y[t] + acc[t] : acc[t];
            if (a.post.mode != POST_NONE) xjd::store_sys(yp, yv);   // read by this launch's tail
            else *yp = yv;
        }
    }
}

template <int T, int TS, int RPT>
__device__ __forceinline__ void epilogue(const GArgs &a, const GSeg &sg, int rg, int team, int lane, int tid,
                                         const float (&acc)[RPT][T], unsigned long long (*amax_sh)[T],
                                         const EpiIn<T> &e) {
    constexpr int NT = 256 / TS, ROWS = NT * RPT;
    unsigned long long best[T];
#pragma unroll
    for (int t = 0; t < T; t++) best[t] = 0ull;
#pragma unroll
    for (int i = 0; i < RPT; i++) {
        const int64_t r = (int64_t)(rg - sg.wg0) * ROWS + team * RPT + i;
        if (lane != i || r >= sg.n_rows) continue;
        epi_row<T>(a, sg, r, acc[i], e);
        if (sg.amax)
#pragma unroll
            for (int t = 0; t < T; t++) best[t] = xjd::argmax_key(acc[i][t], (uint32_t)r);
    }
    if (sg.amax) {  // uniform per work-group
        // lanes 0..RPT-1 of each team hold one row's key each: reduce them
        // first, then the teams of each wavefront (lane 0 of each team meets
        // the same lane of the others), then the four wavefronts' maxima
#pragma unroll
        for (int t = 0; t < T; t++) {
#pragma unroll
            for (int off = 1; off < RPT; off <<= 1) {
                const unsigned long long q = __shfl_xor(best[t], off, 64);
                best[t] = q > best[t] ? q : best[t];
            }
#pragma unroll
            for (int off = TS; off < 64; off <<= 1) {
                const unsigned long long q = __shfl_xor(best[t], off, 64);
                best[t] = q > best[t] ? q : best[t];
            }
        }
        if ((tid & 63) == 0)
#pragma unroll
            for (int t = 0; t < T; t++) amax_sh[tid >> 6][t] = best[t];
        __syncthreads();
        if (tid < T) {
            unsigned long long m = 0ull;
#pragma unroll
            for (int j = 0; j < 4; j++) m = amax_sh[j][tid] > m ? amax_sh[j][tid] : m;
            sg.amax[(int64_t)tid * sg.nwg + (rg - sg.wg0)] = m;
        }
        __syncthreads();
    }
}

// POST_SWIGLU tail of row group rg: the last of the 2 * 32/ROWS work-groups
// that wrote gate (segment 0) and up (segment 1) rows of its 32-index group
// emits silu(gate) * up for the group's T tokens (xj_cpu.c:273).
template <int T, int ROWS>
__device__ __forceinline__ void tail_swiglu(const GArgs &a, int rg, int *flag_sh) {
    const GSeg &g = a.seg[0], &u = a.seg[1];
    const int j = rg < u.wg0 ? rg - g.wg0 : rg - u.wg0;
    const int grp = j * ROWS / 32;
    if (!xjd::arrive_last(a.post.cnt + grp, 2 * (32 / ROWS), flag_sh)) return;
    const int tid = threadIdx.x, t = tid >> 5, k = grp * 32 + (tid & 31);
    const bool in = t < T;
    float v = 0.f;
    if (in) v = xjd::silu(xjd::load_sys(g.y + (int64_t)t * g.ys + k)) * xjd::load_sys(u.y + (int64_t)t * u.ys + k);
    const XqOff o = xq_off(g.n_rows);
    xjd::emit_xq(v, k, in, a.post.xq + (int64_t)(in ? t : 0) * o.stride, o);
}

// Asynchronous global -> LDS copy of n16 16-byte chunks by the work-group
// (global_load_lds_dwordx4: lane l of a wavefront writes LDS base + 16 * l).
// Issued before the weight window, the copies hold no registers, and waiting
// for them (vmcnt drains in issue order) does not wait for the weights.
// Completion: the caller's wait for vmcnt and barrier. nthr = the
// work-group's threads, read once by the kernel (each read of blockDim.x is
// a scalar load that would wait before every copy loop).
__device__ __forceinline__ void dma_lds(const uint8_t *src, uint8_t *lds, int n16, int nthr) {
    const int w = threadIdx.x >> 6;
    for (int j0 = 0; j0 < n16; j0 += nthr) {
        const int i = j0 + threadIdx.x;
        if (i < n16)
            __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1))) *)(src + 16 * (int64_t)i),
                                             (void __attribute__((address_space(3))) *)(lds + 16 * (j0 + 64 * w)),
                                             16, 0, 0);
    }
}

// Waits until at most N vector-memory operations of the wavefront are
// outstanding (gfx9 s_waitcnt encoding; expcnt and lgkmcnt not waited for).
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
// Work-group barrier without a memory fence (which would wait for every
// outstanding load, the weight window included); the LDS-DMA data it
// publishes is complete once each wavefront's vmcnt covers it.
__device__ __forceinline__ void barrier_raw() { asm volatile("s_barrier" ::: "memory"); }
// Work-group barrier ordering LDS accesses only.
__device__ __forceinline__ void barrier_lds() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The T tokens' prepared activations, [0, v_off) of each, into LDS.
template <int T>
__device__ __forceinline__ void dma_xq(const GArgs &a, const XqOff &o, uint8_t *lds, int nthr) {
#pragma unroll
    for (int t = 0; t < T; t++) dma_lds(a.xq + (int64_t)t * o.stride, lds + t * o.v_off, o.v_off >> 4, nthr);
}

// PRO_RMSU_X / PRO_X: eight consecutive inputs k..k+7 of one token (u = x * w,
// or u = x for PRO_X) into its LDS copy at dst: the digits, scale and
// half-group sums that emit_xq gives for u, and (RMS) the group's sum of x^2.
// Called by all 64 lanes of a wavefront with k = k0 + 8 * lane (4 lanes per
// 32-element group, 2 per half); lanes with in == false (whole groups, since
// K % 32 == 0) store nothing.
template <bool RMS>
__device__ __forceinline__ void emit8(const f32x4 (&x)[2], const f32x4 (&w)[2], int k, bool in, uint8_t *dst,
                                      const XqOff &o) {
    const float xv[8] = {x[0].x, x[0].y, x[0].z, x[0].w, x[1].x, x[1].y, x[1].z, x[1].w};
    float u[8];
    if (RMS) {
        const float wv[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
        for (int c = 0; c < 8; c++) u[c] = xv[c] * wv[c];
    } else {
#pragma unroll
        for (int c = 0; c < 8; c++) u[c] = xv[c];
    }
    float m = 0.f;
#pragma unroll
    for (int c = 0; c < 8; c++) m = fmaxf(m, fabsf(u[c]));
    m = fmaxf(m, xjd::dpp<0xB1>(m));   // the group's 4 lanes (one quad)
    m = fmaxf(m, xjd::dpp<0x4E>(m));
    int E = 0;
    (void)frexpf(m, &E);
    if (E < -100) E = -100;
    const float sc = ldexpf(1.0f, 20 - E);
    // X = rint(u * sc), |X| <= 2^20: u * sc + 1.5 * 2^23 rounds once (to
    // nearest even) to an integer whose float bits are 0x4B400000 + X. The
    // base-128 digits of Xb = X + 64 * (2^14 + 2^7 + 1) >= 0 are the balanced
    // digits + 64.
    constexpr uint32_t kBias = 0x102040u;
    uint32_t xb[8], sum = 0;
#pragma unroll
    for (int c = 0; c < 8; c++) {
        xb[c] = __float_as_uint(__builtin_fmaf(u[c], sc, 12582912.0f)) - (0x4B400000u - kBias);
        sum += xb[c];
    }
    int sx = (int)sum - 8 * (int)kBias;
    sx += xjd::dpp_i<0xB1>(sx);   // the 16-element half (2 lanes)
    // digit bytes of four inputs: t = the low 16 bits of two Xb side by side,
    // s = bits 8..23; c = bits 0..6, b = bits 7..13, a = bits 14..21 of Xb
    uint32_t pa[2], pb[2], pc[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t *q = xb + 4 * h;
        const uint32_t t01 = __builtin_amdgcn_perm(q[1], q[0], 0x05040100u);
        const uint32_t t23 = __builtin_amdgcn_perm(q[3], q[2], 0x05040100u);
        const uint32_t s01 = __builtin_amdgcn_perm(q[1], q[0], 0x06050201u);
        const uint32_t s23 = __builtin_amdgcn_perm(q[3], q[2], 0x06050201u);
        pc[h] = xjd::unbias_bytes(__builtin_amdgcn_perm(t23, t01, 0x06040200u) & 0x7F7F7F7Fu);
        pb[h] = xjd::unbias_bytes(__builtin_amdgcn_perm(t23 >> 7, t01 >> 7, 0x06040200u) & 0x7F7F7F7Fu);
        pa[h] = xjd::unbias_bytes(__builtin_amdgcn_perm(s23 >> 6, s01 >> 6, 0x06040200u));
    }
    double ss = 0;
    if (RMS) {
        double q[4];
#pragma unroll
        for (int c = 0; c < 4; c++) q[c] = (double)xv[2 * c] * xv[2 * c] + (double)xv[2 * c + 1] * xv[2 * c + 1];
        ss = (q[0] + q[1]) + (q[2] + q[3]);
        ss += xjd::dpp_d<0xB1>(ss);
        ss += xjd::dpp_d<0x4E>(ss);
    }
    if (!in) return;
    const int g = k >> 5, l = k & 31;
    uint8_t *d = dst + g * kDigStride + l;
    *(uint2 *)d = make_uint2(pa[0], pa[1]);
    *(uint2 *)(d + 32) = make_uint2(pb[0], pb[1]);
    *(uint2 *)(d + 64) = make_uint2(pc[0], pc[1]);
    if (l == 0) {
        ((float *)(dst + o.f_off))[g] = ldexpf(1.0f, E - 20);
        if (RMS) ((double *)(dst + o.ss_off))[g] = ss;
    }
    if ((k & 15) == 0) ((int *)(dst + o.sx_off))[k >> 4] = sx;
}

__device__ __forceinline__ f32x4 ld4f(const float *p) { return *(const f32x4 *)p; }

// Prologues whose activations the GEMV's work-groups build from x in LDS.
__device__ __forceinline__ bool pro_inwg(int pro) { return pro == PRO_RMSU_X || pro == PRO_X; }

// PRO_RMSU_X / PRO_X for T tokens of a per-CU launch (or one token of the
// 256-thread form): x of token t is copied into LDS after the T tokens'
// activations (at xl + T * v_off + t * 4K bytes), w after those copies (at
// xl + T * v_off + T * 4K), then converted into token t's activations
// (PRO_X: u = x * 1, exact).
template <int T>
__device__ __forceinline__ void rmsx1_issue(const GArgs &a, const XqOff &o, uint8_t *xl, int nthr) {
    uint8_t *base = xl + T * o.v_off;
#pragma unroll
    for (int t = 0; t < T; t++) dma_lds((const uint8_t *)(a.x + (int64_t)t * a.xs), base + t * 4 * a.K, a.K >> 2, nthr);
    if (a.pro == PRO_RMSU_X) dma_lds((const uint8_t *)a.pro_w, base + T * 4 * a.K, a.K >> 2, nthr);
}

template <int T>
__device__ __forceinline__ void rmsx1_finish(const GArgs &a, const XqOff &o, uint8_t *xl, int nthr) {
    const uint8_t *base = xl + T * o.v_off;
    const f32x4 *ws = (const f32x4 *)(base + T * 4 * a.K);
    const int n8 = a.K >> 3;
#pragma unroll
    for (int t = 0; t < T; t++) {
        const f32x4 *xs = (const f32x4 *)(base + t * 4 * a.K);
        for (int i0 = 0; i0 < n8; i0 += nthr) {
            const int i = i0 + threadIdx.x, ic = i < n8 ? i : n8 - 1;
            const f32x4 x[2] = {xs[2 * ic], xs[2 * ic + 1]};
            if (a.pro == PRO_X) {
                emit8<false>(x, x, 8 * i, i < n8, xl + t * o.v_off, o);
            } else {
                const f32x4 w[2] = {ws[2 * ic], ws[2 * ic + 1]};
                emit8<true>(x, w, 8 * i, i < n8, xl + t * o.v_off, o);
            }
        }
    }
}

// PRO_RMSU_X / PRO_X setup for T tokens and any K, loads after the weight window.
template <int T>
__device__ __forceinline__ void rmsx_stage(const GArgs &a, const XqOff &o, uint8_t *xl) {
    const int n8 = a.K >> 3;
    const bool rms = a.pro == PRO_RMSU_X;
    for (int t = 0; t < T; t++) {
        const float *x = a.x + (int64_t)t * a.xs;
        for (int i0 = 0; i0 < n8; i0 += 512) {
            f32x4 xv[2][2], wv[2][2];
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int i = i0 + threadIdx.x + 256 * j, ic = i < n8 ? i : n8 - 1;
                xv[j][0] = ld4f(x + 8 * ic);
                xv[j][1] = ld4f(x + 8 * ic + 4);
                if (rms) {
                    wv[j][0] = ld4f(a.pro_w + 8 * ic);
                    wv[j][1] = ld4f(a.pro_w + 8 * ic + 4);
                }
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const int i = i0 + threadIdx.x + 256 * j;
                if (rms) emit8<true>(xv[j], wv[j], 8 * i, i < n8, xl + t * o.v_off, o);
                else emit8<false>(xv[j], xv[j], 8 * i, i < n8, xl + t * o.v_off, o);
            }
        }
    }
}

// PRO_HEADRMS: every head of a.group elements of staged token t gets the
// scale 1/sqrt(sum of its groups' ss / group + eps), folded into the f of
// each of its groups (each thread sums the head's doubles in the same order).
// Completion: the caller's barrier.
__device__ __forceinline__ void head_scale(const GArgs &a, const XqOff &o, uint8_t *xl, int t, int nthr) {
    uint8_t *x = xl + t * o.v_off;
    const int gph = a.group >> 5;
    for (int g = threadIdx.x; g < o.G; g += nthr) {
        const double *ss = (const double *)(x + o.ss_off) + g / gph * gph;
        double s = 0;
        for (int i = 0; i < gph; i++) s += ss[i];
        ((float *)(x + o.f_off))[g] *= 1.0f / sqrtf((float)(s / a.group) + a.eps);
    }
}

// PRO_RMSU / PRO_RMSU_X: the norm scale of staged token t from its group sums of x^2
// (double, fixed order). Called by every lane of a wavefront; each wavefront
// computes it for itself and keeps it in a scalar register.
__device__ __forceinline__ float rmsu_scale(const GArgs &a, const XqOff &o, const uint8_t *xl, int t) {
    const double *ss = (const double *)(xl + t * o.v_off + o.ss_off);
    const int lane = threadIdx.x & 63;
    double s = 0;
    for (int g = lane; g < o.G; g += 64) s += ss[g];
    s = xjd::wave_sum_d(s);   // uniform: the wavefront's scale lives in scalar registers
    return 1.0f / sqrtf((float)(s / a.K) + a.eps);
}

// -------------------------------------------------------------- kernels --
// A row group is 256/TS rows, one per team of TS lanes. MU > 0 (single-token
// launches with one work-group per row group, kept to three work-groups per
// CU so that up to 3 x CUs of them run in one wave): every lane owns at most
// MU units of its row, and the work-group issues the weight window of its row
// group while the T tokens' activations are copied into LDS (single-token
// rows of at most two units per lane also loop, below). MU == 0: the same
// for the first unit, then a loop over row groups with stride gridDim.x
// that requests each next group's first unit before the current group's
// epilogue. Q4: Q4_K rows only; K6: Q4_K and Q6_K rows only (fewer
// registers than the kernel for every type).
template <int T, int TS, int MU, bool Q4, bool K6 = false>
__global__ __launch_bounds__(256, T == 1 ? 3 : 1) void gemv_kernel(const GArgs a) {
    extern __shared__ u32x4 lds_v[];
    constexpr int NT = 256 / TS;
    __shared__ unsigned long long amax_sh[NT][T];
    __shared__ int flag_sh;
    const int K = a.K, nu = K / 64;
    const XqOff o = xq_off(K);
    const int tid = threadIdx.x, team = tid / TS, lane = tid % TS;
    const int n_rg = a.seg[a.nseg - 1].wg0 + a.seg[a.nseg - 1].nwg;   // gridDim.x <= n_rg
    auto row_of = [&](const GSeg &sg, int rg) {
        const int64_t r = (int64_t)(rg - sg.wg0) * NT + team;
        return r < sg.n_rows ? r : (int64_t)sg.n_rows - 1;
    };
    auto blocks_per_row = [&](uint32_t type) {
        return (type == XJ_Q4_K || type == XJ_Q6_K || type == XJ_Q5_K) ? K / 256 : K / 32;
    };
    // the lane's first units of row group rg, loaded before the work that
    // precedes their use (units past the row read the tensor's padding)
    constexpr int NW = Win<MU, Q4>::N;
    // LW: single-token Q4_K / Q6_K rows of at most two units per lane in a
    // looping launch: the next row group's whole window is requested before
    // this group's dot products, so the work-group's stream never waits on
    // its own epilogue
    constexpr bool LW = T == 1 && MU > 0 && MU <= 2 && (Q4 || K6);
    RawU win[NW], wnx[NW];
    auto units_into = [&](int rg, RawU (&dst)[NW]) {
        const GSeg &sg = a.seg[seg_of(a, rg)];
        const int64_t rb = row_of(sg, rg) * blocks_per_row(sg.type);
        const int u0 = lane < nu ? lane : nu - 1;
#pragma unroll
        for (int m = 0; m < NW; m++) dst[m] = load_unit<Q4>(sg.type, sg.w, sg.nblk, rb, u0 + m * TS);
    };
    auto first_units = [&](int rg) { units_into(rg, win); };
    int rg = blockIdx.x;
    uint8_t *lds = (uint8_t *)lds_v;
    if (pro_inwg(a.pro) && T > 1) {
        first_units(rg);
        rmsx_stage<T>(a, o, lds);
        __syncthreads();
    } else {
        // LDS copies first, then the window's loads: waiting for vmcnt <=
        // their number completes the copies only
        if (pro_inwg(a.pro)) rmsx1_issue<1>(a, o, lds, 256);
        else dma_xq<T>(a, o, lds, 256);
        barrier_raw();   // the group's copies are queued ahead of its weight requests
        first_units(rg);
        __builtin_amdgcn_sched_barrier(0);
        wait_vm<Win<MU, Q4>::LOADS>();
        barrier_raw();
        if (pro_inwg(a.pro)) {
            rmsx1_finish<1>(a, o, lds, 256);
            barrier_lds();
        }
        if (a.pro == PRO_HEADRMS) {
#pragma unroll
            for (int t = 0; t < T; t++) head_scale(a, o, lds, t, 256);
            barrier_lds();
        }
    }
    const uint8_t *xl = (const uint8_t *)lds_v;
    float sc[T];
#pragma unroll
    for (int t = 0; t < T; t++) sc[t] = a.pro == PRO_RMSU || a.pro == PRO_RMSU_X ? rmsu_scale(a, o, xl, t) : 1.f;

    for (;;) {
        const GSeg &sg = a.seg[seg_of(a, rg)];
        const int64_t row = row_of(sg, rg), rb = row * blocks_per_row(sg.type);
        EpiIn<T> ein;
        epi_load<T>(sg, row, ein);
        float acc[1][T];
#pragma unroll
        for (int t = 0; t < T; t++) acc[0][t] = 0.f;
        const int rn = rg + gridDim.x;
        if constexpr (LW) {
            if (rn < n_rg) units_into(rn, wnx);
        }
        if (Q4 || sg.type == XJ_Q4_K) {
            rows_q4k<T, TS, MU, Win<MU, Q4>::PD>(sg.w, rb, nu, lane, win, xl, o.v_off, o, acc[0]);
        } else if constexpr (Q4) {
        } else if (K6 || sg.type == XJ_Q6_K) {
            rows_q6k<T, TS, MU, Win<MU, false>::PD>(sg.w, sg.nblk, rb, nu, lane, win, xl, o.v_off, o, acc[0]);
        } else if constexpr (!K6) {
            const int64_t rr[1] = {row}, rbb[1] = {rb};
            if (sg.type == XJ_Q8_0) rows_q80<T, TS, 1>(sg.w, sg.nblk, rbb, K / 32, lane, xl, o.v_off, o, acc);
            // the types no configuration uses come one token per launch (their
            // loops would raise the register count of every multi-token kernel)
            else if (sg.type == XJ_Q5_K) { if constexpr (T == 1) rows_q5k<T, TS>(sg.w, rb, nu, lane, xl, o.v_off, o, acc[0]); }
            else if (sg.type == XJ_F16 || sg.type == XJ_BF16) {
                if constexpr (T == 1) rows_h16<T, TS, 1>(sg.w, rr, K, lane, sg.type == XJ_BF16, a.xq, o, acc);
            } else rows_f32<T, TS, 1>(sg.w, rr, K, lane, a.xq, o, acc);
        }
        // MU == 0: the next row group's first units are requested before this
        // group's epilogue (its barriers), not after it
        if constexpr (MU == 0) {
            if (rn < n_rg) first_units(rn);
        }
#pragma unroll
        for (int t = 0; t < T; t++) {
            acc[0][t] = team_sum<TS>(acc[0][t]);
            acc[0][t] *= sc[t];
        }
        epilogue<T, TS, 1>(a, sg, rg, team, lane, tid, acc, amax_sh, ein);
        if (a.post.mode == POST_SWIGLU) tail_swiglu<T, NT>(a, rg, &flag_sh);
        rg = rn;
        // MU > 0 (but LW): one row group per work-group (the launch covers
        // them all), so no window is carried around a loop edge
        if ((MU > 0 && !LW) || rg >= n_rg) break;
        if constexpr (LW) {
            for (int m = 0; m < NW; m++) win[m] = wnx[m];
        }
    }
    if (a.inc_ptr && blockIdx.x == 0 && tid == 0) *a.inc_ptr += a.inc_by;
}

// POST_SWIGLU tail of a per-CU launch over T tokens (rpw rows per work-group,
// gate = segment 0, up = segment 1): the work-group arrives once on every
// 32-index group its rows touch; the last of the group's work-groups (those
// of both segments covering its 32 rows) emits silu(gate) * up
// (xj_cpu.c:273). At most 8 groups per work-group (rpw <= 226).
template <int T>
__device__ __forceinline__ void tail_swiglu_cu(const GArgs &a, int rg, const GSeg &sg) {
    __shared__ int last_sh[8];
    const int tid = threadIdx.x, j = rg - sg.wg0;
    const int r_lo = j * a.rpw, r_hi = (r_lo + a.rpw < sg.n_rows ? r_lo + a.rpw : sg.n_rows) - 1;
    const int ga = r_lo / 32, ng = r_hi / 32 - ga + 1;
    __builtin_amdgcn_s_waitcnt(0);   // this group's system-scope stores of y are complete
    __syncthreads();
    if (tid < ng) {
        const int grp = ga + tid;
        const int target = 2 * ((32 * grp + 31) / a.rpw - (32 * grp) / a.rpw + 1);
        const int n = __hip_atomic_fetch_add(a.post.cnt + grp, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = n == target - 1;
        if (last) __hip_atomic_store(a.post.cnt + grp, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last_sh[tid] = last;
    }
    __syncthreads();
    const GSeg &g = a.seg[0], &u = a.seg[1];
    const XqOff o = xq_off(g.n_rows);
    for (int i = 0; i < ng; i++) {
        if (!last_sh[i]) continue;   // uniform
        // half-wavefront t emits token t: the T tokens' loads are in flight together
        if (tid < (T * 32 + 63) / 64 * 64) {
            const int t = tid >> 5, k = 32 * (ga + i) + (tid & 31);
            const bool in = t < T;
            const float v = in ? xjd::silu(xjd::load_sys(g.y + (int64_t)t * g.ys + k)) *
                                     xjd::load_sys(u.y + (int64_t)t * u.ys + k)
                               : 0.f;
            xjd::emit_xq(v, k, in, a.post.xq + (int64_t)(in ? t : 0) * o.stride, o);
        }
    }
}

// POST_SWIGLU_H: the gate results of the work-group's rows (teams [0, rpw))
// and the up results of the same rows (teams [ho, ho + rpw)) meet in LDS, and
// silu(gate) * up (xj_cpu.c:273) is stored for each row.
__device__ __forceinline__ void swiglu_h_cu(const GArgs &a, int rg, int ho, int team, int lane, float y) {
    __shared__ float ys[128];   // one per team (TS >= 8)
    if (lane == 0) ys[team] = y;
    barrier_lds();
    const int i = threadIdx.x;
    const int64_t r = (int64_t)rg * a.rpw + i;
    if (i < a.rpw && r < a.seg[0].n_rows) a.post.h[r] = xjd::silu(ys[i]) * ys[ho + i];
}

// Single-token launch with one work-group per CU (per-segment ranges of
// work-groups): work-group g of segment i (g in [wg0, wg0 + nwg)) takes rows
// (g - wg0) * rpw + team, one per team of TS lanes (blockDim.x / TS >= rpw
// teams; the others repeat a valid row and store nothing); with T >= 4
// tokens and TS >= 16, rows (g - wg0) * rpw + 2 team + i, i = 0, 1 (rpw / 2
// teams, rounded up), each row's lanes and arithmetic as for one token.
// POST_SWIGLU_H:
// work-group g takes rows g * rpw + team of the gate (segment 0) in teams
// [0, rpw) and the same rows of the up (segment 1) in teams [ho, ho + rpw),
// ho = rpw rounded up to whole wavefronts. The activations (prepared, or
// the x (and w) of an input built in the work-group: PRO_RMSU_X, PRO_X) are
// copied into LDS once per CU; WF (inputs built in the work-group, and
// prepared inputs without a tail) requests one unit of every lane right
// behind the copies and converts x while it arrives; otherwise (a prepared
// input with the cross-work-group tail) the copies complete first and every
// lane then requests all its MU units. The gate|up launch ends with the
// SwiGLU tail (or its work-group-local form, POST_SWIGLU_H); no argmax
// partials.
template <int T, int TS, int MU, bool Q4, bool WF>
__global__ __launch_bounds__(T >= 4 && TS >= 16 ? 512 : 1024, 1) void gemv_cu_kernel(const GArgs a) {
    extern __shared__ u32x4 lds_v[];
    // rows per team: with four or five tokens and teams of 16+ lanes (few
    // rows per work-group), each activation digit read from LDS serves two
    // rows (Q6_K 2560 x 9216, T = 4: 22.8 -> 20.7 us; T = 2, 3 lose with half
    // the wavefronts: 14.0 -> 15.6, 17.7 -> 18.0 us). 8-lane teams (many rows)
    // keep one row each: pairing their rows halves their wavefronts (18432 x
    // 2560 Q4_K, T = 5: 23.7 -> 24.6 us), and pairing them in two groups of
    // teams that split the tokens keeps the wavefronts but loads every weight
    // twice (24.8 us)
    constexpr int R = T >= 4 && TS >= 16 ? 2 : 1;
    // WF: one unit requested right behind the activation copies, the rest
    // from the unit loop one ahead (more in flight before the conversion
    // delays it, more ahead in the loop congests: both measured slower);
    // otherwise the copies complete first, then all units. MU == 0 (several
    // tokens): a rolled unit loop with the next unit in flight.
    constexpr int NW = WF || MU == 0 ? 1 : MU, PD = NW - 1;
    const int K = a.K, nu = K / 64;
    // prepared inputs need no group sums of x^2 in LDS: each token is staged
    // without them (v_off here is the LDS bytes per token), so that five
    // tokens of K = 9216 fit
    XqOff o = xq_off(K);
    if (a.pro == PRO_NONE) o.v_off = o.ss_off;
    const int tid = threadIdx.x, team = tid / TS, lane = tid % TS;
    const int nthr = blockDim.x;   // read once (a scalar load)
    // the activation copies go first (they need no segment field), with the
    // kernel arguments they read loaded together rather than each waited for
    // in turn
    asm volatile("" ::"s"(a.x), "s"(a.pro_w), "s"(a.xq), "s"(a.xs), "s"(nthr), "s"(a.post.mode), "s"(a.rpw), "s"(a.nseg),
                 "s"(a.seg[1].wg0), "s"(a.seg[2].wg0), "s"(a.seg[3].wg0));
    uint8_t *lds = (uint8_t *)lds_v;
    const bool inwg = pro_inwg(a.pro);
    if (inwg) rmsx1_issue<T>(a, o, lds, nthr);
    else dma_xq<T>(a, o, lds, nthr);
    const int rg = blockIdx.x;
    const bool H = a.post.mode == POST_SWIGLU_H;
    constexpr int TPW = 64 / TS;   // teams per wavefront
    const int ho = (a.rpw + TPW - 1) / TPW * TPW;
    // uniform over the wavefront (ho is a multiple of TPW)
    const int si = H ? __builtin_amdgcn_readfirstlane((int)(team >= ho)) : seg_of_flat(a, rg);
    // one token: the segment copied by value (its fields read together, never
    // reloaded; several tokens keep the reference, which spills less)
    const GSeg sg_v = a.seg[si];
    const GSeg &sg = T == 1 ? sg_v : a.seg[si];
    const int tr = H && si ? team - ho : team;
    bool mine[R];
    int64_t row[R], rb[R];
#pragma unroll
    for (int i = 0; i < R; i++) {
        const int64_t r0 = (int64_t)(rg - sg.wg0) * a.rpw + tr * R + i;
        mine[i] = tr * R + i < a.rpw && r0 < sg.n_rows;
        row[i] = mine[i] ? r0 : (int64_t)sg.n_rows - 1;
        rb[i] = row[i] * (K / 256);
    }
    if (!WF) wait_vm<0>();   // the activations complete before any weight request
    barrier_raw();
    RawU win[R][NW];
    const int u0 = lane < nu ? lane : nu - 1;
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int m = 0; m < NW; m++) win[i][m] = load_unit<Q4>(sg.type, sg.w, sg.nblk, rb[i], u0 + m * TS);
    if (WF) {   // the copies complete, the window's loads stay in flight
        __builtin_amdgcn_sched_barrier(0);
        wait_vm<(Q4 ? 3 : 5) * NW * R>();
        barrier_raw();
    }
    if (inwg) {
        rmsx1_finish<T>(a, o, lds, nthr);
        barrier_lds();
    }
    if (a.pro == PRO_HEADRMS) {   // prepared: the copies completed before the weight requests
#pragma unroll
        for (int t = 0; t < T; t++) head_scale(a, o, lds, t, nthr);
        barrier_lds();
    }
    float sc[T];
#pragma unroll
    for (int t = 0; t < T; t++) sc[t] = a.pro == PRO_RMSU || a.pro == PRO_RMSU_X ? rmsu_scale(a, o, lds, t) : 1.f;
    EpiIn<T> ein[R];
#pragma unroll
    for (int i = 0; i < R; i++) epi_load<T>(sg, row[i], ein[i]);
    float acc[R][T];
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int t = 0; t < T; t++) acc[i][t] = 0.f;
    if (Q4 || sg.type == XJ_Q4_K) {
        if constexpr (R == 2) rows2_q4k<T, TS>(sg.w, rb[0], rb[1], nu, lane, win[0][0], win[1][0], lds, o.v_off, o, acc[0], acc[1]);
        else rows_q4k<T, TS, MU, PD>(sg.w, rb[0], nu, lane, win[0], lds, o.v_off, o, acc[0]);
    } else if constexpr (!Q4) {
        if constexpr (R == 2)
            rows2_q6k<T, TS>(sg.w, sg.nblk, rb[0], rb[1], nu, lane, win[0][0], win[1][0], lds, o.v_off, o, acc[0], acc[1]);
        else rows_q6k<T, TS, MU, PD>(sg.w, sg.nblk, rb[0], nu, lane, win[0], lds, o.v_off, o, acc[0]);
    }
#pragma unroll
    for (int i = 0; i < R; i++)
#pragma unroll
        for (int t = 0; t < T; t++) acc[i][t] = team_sum<TS>(acc[i][t]) * sc[t];
    if (T == 1 && H) {
        swiglu_h_cu(a, rg, ho, team, lane, acc[0][0]);
    } else {
        // lane i of the team stores row i
#pragma unroll
        for (int i = 0; i < R; i++)
            if (mine[i] && lane == i) epi_row<T>(a, sg, row[i], acc[i], ein[i]);
        if (a.post.mode == POST_SWIGLU) tail_swiglu_cu<T>(a, rg, sg);
    }
    if (a.inc_ptr && blockIdx.x == 0 && tid == 0) *a.inc_ptr += a.inc_by;
}

// -------------------------------------------------------------- host side --
static int env_or(const char *k, int d) {
    const char *v = getenv(k);
    return v ? atoi(v) : d;
}

// Lanes per row: among 8..64, the team that wastes the fewest lane slots with
// at most five 64-element units per lane (ties: the smaller team), widened
// while the grid is short of two work-groups per CU. One row per team.
GemvPlan gemv_plan(int K, int64_t rows) {
    const int nu = K / 64 > 0 ? K / 64 : 1;
    int ts = 64;
    double best = -1;
    for (int c = 8; c <= 64; c *= 2) {
        const int upl = (nu + c - 1) / c;
        if (upl > 5 && c < 64) continue;
        const double eff = (double)nu / ((double)c * upl);
        if (eff > best + 1e-9) { best = eff; ts = c; }
    }
    const int64_t want = 2LL * g_cus;
    while (ts < 64 && (rows + (256 / ts) - 1) / (256 / ts) < want) ts *= 2;
    const int fts = env_or("XJ_GEMV_TS", 0);
    if (fts == 8 || fts == 16 || fts == 32 || fts == 64) ts = fts;
    return GemvPlan{ts, 1, 256 / ts};
}

int gemv_max_tile(int K) {
    static const int cap = env_or("XJ_GEMV_TILE", kCuMaxT);
    // the per-CU launches of prepared inputs stage ss_off bytes per token
    const int per_t = xq_off(K).ss_off;
    int t = (int)(g_lds_max / per_t);
    const int c = cap < 1 ? 1 : cap > kTileT ? kTileT : cap;
    return t < 1 ? 0 : t > c ? c : t;
}

size_t gemv_xq_bytes(int K) { return (size_t)(gemv_max_tile(K) > 0 ? gemv_max_tile(K) : 1) * xq_off(K).stride; }

int prep_launch(const GArgs &a, hipStream_t st) {
    if (a.T < 1 || a.K < 32 || a.K % 32 || !a.xq) return -1;
    if (a.pro == PRO_GATED_RMS && (a.group < 1 || a.K % a.group)) return -1;
    if ((a.pro == PRO_RMSU || a.pro == PRO_GATED_RMS) && !a.pro_w) return -1;
    if (a.hq && a.K % 256) return -1;
    if (a.hq_only && !a.hq) return -1;
    hipLaunchKernelGGL(prep_kernel, dim3((a.K + 255) / 256, a.T), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Dynamic LDS of a launch: the T tokens' activations, and for a single-token
// PRO_RMSU_X (PRO_X) launch the copies of x and w (x) after them.
static size_t gemv_lds_bytes(const GArgs &a) {
    const size_t b = (size_t)a.T * xq_off(a.K).v_off;
    if (a.T > 1) return b;
    return a.pro == PRO_RMSU_X ? b + 8 * (size_t)a.K : a.pro == PRO_X ? b + 4 * (size_t)a.K : b;
}

template <int T, int TS, int MU = 0, bool Q4 = false, bool K6 = false>
static hipError_t launch_v(const GArgs &a, int grid, hipStream_t st) {
    hipLaunchKernelGGL((gemv_kernel<T, TS, MU, Q4, K6>), dim3(grid), dim3(256), gemv_lds_bytes(a), st, a);
    return hipGetLastError();
}

// Single-token Q4_K / Q6_K rows of at most two units per lane loop over row
// groups with the next group's window in flight (XJ_GEMV_LW=0: one row group
// per work-group, as many work-groups as row groups)
static bool loop_window() {
    static const bool on = env_or("XJ_GEMV_LW", 1) != 0;
    return on;
}

static bool all_q4k(const GArgs &a) {
    for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].type != XJ_Q4_K) return false;
    return true;
}

static bool all_k(const GArgs &a) {   // Q4_K and Q6_K rows only
    for (int i = 0; i < a.nseg; i++)
        if (a.seg[i].type != XJ_Q4_K && a.seg[i].type != XJ_Q6_K) return false;
    return true;
}

template <int TS>
static hipError_t launch_ts(const GArgs &a, int grid, hipStream_t st) {
    const int upl = (a.K / 64 + TS - 1) / TS;   // 64-element units per lane
    const int n_rg = a.seg[a.nseg - 1].wg0 + a.seg[a.nseg - 1].nwg;
    switch (a.T) {
    case 1:
        if (grid < n_rg) {   // work-groups loop over row groups
            if (upl <= 2 && loop_window() && all_k(a)) {
                if (all_q4k(a)) return upl == 1 ? launch_v<1, TS, 1, true>(a, grid, st) : launch_v<1, TS, 2, true>(a, grid, st);
                return upl == 1 ? launch_v<1, TS, 1, false, true>(a, grid, st) : launch_v<1, TS, 2, false, true>(a, grid, st);
            }
            return launch_v<1, TS, 0>(a, grid, st);
        }
        if (all_q4k(a) && upl <= 5) switch (upl) {
            case 1: return launch_v<1, TS, 1, true>(a, grid, st);
            case 2: return launch_v<1, TS, 2, true>(a, grid, st);
            case 3: return launch_v<1, TS, 3, true>(a, grid, st);
            case 4: return launch_v<1, TS, 4, true>(a, grid, st);
            default: return launch_v<1, TS, 5, true>(a, grid, st);
        }
        switch (upl) {
        case 1: return launch_v<1, TS, 1>(a, grid, st);
        case 2: return launch_v<1, TS, 2>(a, grid, st);
        case 3: return launch_v<1, TS, 3>(a, grid, st);
        case 4: return launch_v<1, TS, 4>(a, grid, st);
        default: return launch_v<1, TS, 0>(a, grid, st);
        }
    case 2: return launch_v<2, TS>(a, grid, st);
    case 3: return launch_v<3, TS>(a, grid, st);
    case 4: return launch_v<4, TS>(a, grid, st);
    case 5: return launch_v<5, TS>(a, grid, st);
    case 6: return launch_v<6, TS>(a, grid, st);
    case 7: return launch_v<7, TS>(a, grid, st);
    case 8: return launch_v<8, TS>(a, grid, st);
    default: return hipErrorInvalidValue;
    }
}

// Threads of a per-CU work-group whose teams need `need`: an input built in
// the work-group is converted eight elements per thread, in one round where a
// work-group of K / 8 threads is allowed.
static int cu_threads(const GArgs &a, int need) {
    int t = (need + 63) / 64 * 64;
    if (a.pro == PRO_RMSU_X || a.pro == PRO_X) {
        const int one = (a.K / 8 + 63) / 64 * 64;
        if (t < one && one <= 1024) t = one;
    }
    return t;
}

// Dynamic LDS of a per-CU launch: the T tokens' activations, and for an
// input built in the work-group the copies of x (one per token) and of w.
static size_t cu_lds_bytes(const GArgs &a) {
    const XqOff o = xq_off(a.K);
    const size_t b = (size_t)a.T * (a.pro == PRO_NONE ? o.ss_off : o.v_off);   // prepared: staged without ss
    return a.pro == PRO_RMSU_X ? b + (size_t)(a.T + 1) * 4 * a.K : a.pro == PRO_X ? b + (size_t)a.T * 4 * a.K : b;
}

// Teams of a per-CU work-group with rpw rows (POST_SWIGLU_H: rpw gate rows
// from team 0 and rpw up rows from the first whole wavefront after them).
static int cu_teams(int rpw, int ts, bool h) {
    const int tpw = 64 / ts;
    return h ? (rpw + tpw - 1) / tpw * tpw + rpw : rpw;
}

// Two rows per team (four or five tokens, teams of 16+ lanes); that kernel is
// compiled for at most 512 threads per work-group.
static bool cu_row_pairs(int T, int ts) { return T >= 4 && ts >= 16; }

// Threads of a per-CU work-group of rpw rows at ts lanes per row: its teams,
// raised for an input converted in the work-group and for the SwiGLU tail,
// which emits token t from half-wavefront t.
static int cu_block_threads(const GArgs &a, int rpw, int ts) {
    const bool h = a.post.mode == POST_SWIGLU_H;
    const int teams = h ? cu_teams(rpw, ts, true) : cu_row_pairs(a.T, ts) ? (rpw + 1) / 2 : rpw;
    int threads = cu_threads(a, teams * ts);
    if (a.post.mode == POST_SWIGLU && threads < (a.T * 32 + 63) / 64 * 64) threads = (a.T * 32 + 63) / 64 * 64;
    return threads;
}

// Per-CU launch (gemv_cu_kernel) of a single-token GEMV under its plan
// (cu_plan): lanes per row TS with at most 5 units per lane, rows per
// work-group rpw with teams * TS <= 1024, every segment's work-groups counted
// (POST_SWIGLU_H: shared by both segments), at most one per CU in total.
template <int TS>
static int launch_cu_ts(GArgs b, int rpw, int upl, bool q4, bool wf, hipStream_t st) {
    int wg = 0;
    if (b.post.mode == POST_SWIGLU_H) {   // gate and up rows of the same indices in each work-group
        wg = (b.seg[0].n_rows + rpw - 1) / rpw;
        for (int i = 0; i < 2; i++) b.seg[i].wg0 = 0, b.seg[i].nwg = wg;
    } else {
        for (int i = 0; i < b.nseg; i++) {
            b.seg[i].wg0 = wg;
            b.seg[i].nwg = (b.seg[i].n_rows + rpw - 1) / rpw;
            wg += b.seg[i].nwg;
        }
    }
    b.rpw = rpw;
    const int threads = cu_block_threads(b, rpw, TS);
    if (threads > (cu_row_pairs(b.T, TS) ? 512 : 1024)) return -1;
    size_t lds = cu_lds_bytes(b);
    // more than half of a CU's LDS keeps each work-group on a CU of its own
    if (b.pro != PRO_RMSU_X && g_lds_max > 80 * 1024 && lds < 80 * 1024 + 256) lds = 80 * 1024 + 256;
    void (*k)(GArgs) = nullptr;
#define XJ_CU_K(Q, W)                                                   \
    switch (b.T) {                                                       \
    case 1:                                                              \
        switch (upl) {                                                   \
        case 1: k = gemv_cu_kernel<1, TS, 1, Q, W>; break;               \
        case 2: k = gemv_cu_kernel<1, TS, 2, Q, W>; break;               \
        case 3: k = gemv_cu_kernel<1, TS, 3, Q, W>; break;               \
        case 4: k = gemv_cu_kernel<1, TS, 4, Q, W>; break;               \
        default: k = gemv_cu_kernel<1, TS, 5, Q, W>; break;              \
        }                                                                \
        break;                                                           \
    case 2: k = gemv_cu_kernel<2, TS, 0, Q, W>; break;                   \
    case 3: k = gemv_cu_kernel<3, TS, 0, Q, W>; break;                   \
    case 4: k = gemv_cu_kernel<4, TS, 0, Q, W>; break;                   \
    default: k = gemv_cu_kernel<5, TS, 0, Q, W>; break;                  \
    }
    if (q4 && wf) { XJ_CU_K(true, true) }
    else if (q4) { XJ_CU_K(true, false) }
    else if (wf) { XJ_CU_K(false, true) }
    else { XJ_CU_K(false, false) }
#undef XJ_CU_K
    hipLaunchKernelGGL(k, dim3(wg), dim3(threads), lds, st, b);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// Per-CU plan of a single-token launch: rows per work-group (per segment
// for POST_SWIGLU_H), lanes per row, units per lane, all-Q4_K, and whether
// the weight window is requested behind the activation copies.
struct CuPlan {
    int rpw, ts, upl;
    bool q4, wf;
};

static bool cu_plan(const GArgs &a, CuPlan &p) {
    static const bool on = env_or("XJ_GEMV_CU", 1) != 0;
    static const int rms_k = env_or("XJ_GEMV_RMS_WG_PER_CU", 1);
    if (!on || a.T < 1 || a.T > kCuMaxT) return false;
    const bool H = a.post.mode == POST_SWIGLU_H;
    if (H && a.T != 1) return false;
    if (a.post.mode == POST_SWIGLU) {
        if (!a.post.xq || !a.post.cnt || a.nseg != 2 || a.seg[0].n_rows != a.seg[1].n_rows || a.seg[0].n_rows % 32)
            return false;
    } else if (H) {
        if (!a.post.h || a.nseg != 2 || a.seg[0].n_rows != a.seg[1].n_rows || a.seg[0].type != a.seg[1].type ||
            a.seg[0].epi != EPI_STORE || a.seg[1].epi != EPI_STORE)
            return false;
    } else if (a.post.mode != POST_NONE) {
        return false;
    }
    if (a.pro != PRO_NONE && a.pro != PRO_RMSU && a.pro != PRO_RMSU_X && a.pro != PRO_X && a.pro != PRO_HEADRMS)
        return false;
    if ((a.pro == PRO_RMSU_X || a.pro == PRO_X) && (!a.x || ((uintptr_t)a.x & 15))) return false;
    // the weight window requested right behind the activation copies for
    // inputs built in the work-group and for prepared inputs without a tail
    // (before: the copies completed first; 702 vs 707 tok/s); RMSNorm inputs:
    // rms_k balanced work-groups per CU
    const bool wf = a.pro == PRO_RMSU_X || a.pro == PRO_X || a.post.mode == POST_NONE;
    if (a.pro == PRO_RMSU_X && (rms_k < 1 || !a.pro_w || ((uintptr_t)a.pro_w & 15))) return false;
    const int nwg_max = a.pro == PRO_RMSU_X ? rms_k * g_cus : g_cus;
    int64_t total = 0;
    bool q4 = true;
    for (int i = 0; i < a.nseg; i++) {
        const GSeg &s = a.seg[i];
        if ((s.type != XJ_Q4_K && s.type != XJ_Q6_K) || s.amax || s.n_rows < 1) return false;
        if (s.epi == EPI_CONV && (s.conv_k < 2 || s.conv_k > 8)) return false;
        q4 = q4 && s.type == XJ_Q4_K;
        total += s.n_rows;
    }
    if (a.K % 256 || a.K > 16384 || cu_lds_bytes(a) > (size_t)g_lds_max) return false;
    // the fewest rows per work-group whose work-groups fit nwg_max
    int rpw;
    if (H) {
        rpw = (a.seg[0].n_rows + nwg_max - 1) / nwg_max;
    } else {
        rpw = (int)((total + nwg_max - 1) / nwg_max);
        for (;; rpw++) {
            int64_t wg = 0;
            for (int i = 0; i < a.nseg; i++) wg += (a.seg[i].n_rows + rpw - 1) / rpw;
            if (wg <= nwg_max) break;
        }
    }
    // the most lanes per row (more wavefronts) with at most 5 units per lane
    const int nu = a.K / 64;
    for (int ts = 64; ts >= 8; ts /= 2) {
        const int upl = (nu + ts - 1) / ts;
        if (upl > 5 || cu_teams(rpw, ts, H) * ts > 1024 || (a.post.mode == POST_SWIGLU && rpw > 226)) continue;
        // the row-pair kernel's bound (an input built in the work-group can
        // ask for K / 8 threads)
        if (cu_block_threads(a, rpw, ts) > (cu_row_pairs(a.T, ts) ? 512 : 1024)) continue;
        p = CuPlan{rpw, ts, upl, q4, wf};
        return true;
    }
    return false;
}

// Returns 1 when no per-CU plan applies.
static int gemv_launch_cu(const GArgs &a, hipStream_t st) {
    CuPlan p;
    if (!cu_plan(a, p)) return 1;
    switch (p.ts) {
    case 8: return launch_cu_ts<8>(a, p.rpw, p.upl, p.q4, p.wf, st);
    case 16: return launch_cu_ts<16>(a, p.rpw, p.upl, p.q4, p.wf, st);
    case 32: return launch_cu_ts<32>(a, p.rpw, p.upl, p.q4, p.wf, st);
    default: return launch_cu_ts<64>(a, p.rpw, p.upl, p.q4, p.wf, st);
    }
}

bool gemv_swiglu_h_ok(const GArgs &a) {
    static const bool on = env_or("XJ_GEMV_SWIGLU_H", 1) != 0;
    CuPlan p;
    return on && a.post.mode == POST_SWIGLU_H && cu_plan(a, p);
}

// Tokens [t0, t0 + n) of a launch: their activations, inputs, outputs and
// argmax partials; the position increment stays with the last tokens.
static GArgs token_range(const GArgs &a, int t0, int n) {
    GArgs b = a;
    b.T = n;
    b.t0 = a.t0 + t0;
    b.xq = a.xq + t0 * xq_off(a.K).stride;
    if (a.x) b.x = a.x + (int64_t)t0 * a.xs;
    if (a.x2) b.x2 = a.x2 + (int64_t)t0 * a.x2s;
    if (a.post.mode != POST_NONE && a.post.xq) b.post.xq = a.post.xq + t0 * xq_off(a.seg[0].n_rows).stride;
    for (int i = 0; i < a.nseg; i++) {
        b.seg[i].y = a.seg[i].y + (int64_t)t0 * a.seg[i].ys;
        if (a.seg[i].amax) b.seg[i].amax = a.seg[i].amax + (int64_t)t0 * a.seg[i].nwg;
    }
    if (t0 + n < a.T) b.inc_ptr = nullptr;
    return b;
}

int gemv_launch(const GArgs &a, hipStream_t st) {
    if (a.T < 1 || a.T > kTileT || a.nseg < 1 || a.nseg > kMaxSeg || a.K < 32 || a.K % 32 || !a.xq) return -1;
    // (the per-CU launch stages prepared tokens in fewer bytes; several
    // tokens are split below when only that launch would fit them)
    if (a.T == 1 && gemv_lds_bytes(a) > (size_t)g_lds_max && cu_lds_bytes(a) > (size_t)g_lds_max) return -1;
    int64_t total = 0;
    for (int i = 0; i < a.nseg; i++) total += a.seg[i].n_rows;
    const GemvPlan p = gemv_plan(a.K, total);
    for (int i = 0; i < a.nseg; i++) {
        const GSeg &s = a.seg[i];
        if ((s.type == XJ_Q4_K || s.type == XJ_Q6_K || s.type == XJ_Q5_K) && a.K % 256) return -1;
        if (s.type != XJ_Q4_K && s.type != XJ_Q6_K && s.type != XJ_Q8_0 && s.type != XJ_F32 && s.type != XJ_Q5_K &&
            s.type != XJ_F16 && s.type != XJ_BF16)
            return -1;
        if (s.n_rows < 1 || s.nwg != (s.n_rows + p.rows_per_group - 1) / p.rows_per_group) return -1;
        if (s.wg0 != (i ? a.seg[i - 1].wg0 + a.seg[i - 1].nwg : 0)) return -1;
        if (s.epi == EPI_CONV && (s.conv_k < 2 || s.conv_k > 8)) return -1;
        // float rows read v from a prep launch's xq
        if ((s.type == XJ_F32 || s.type == XJ_F16 || s.type == XJ_BF16) && (a.pro == PRO_RMSU_X || a.pro == PRO_X))
            return -1;
    }
    if (a.post.mode != POST_NONE && a.post.mode != POST_SWIGLU && a.post.mode != POST_SWIGLU_H) return -1;
    // other prologues come prepared
    if (a.pro != PRO_NONE && a.pro != PRO_RMSU && a.pro != PRO_RMSU_X && a.pro != PRO_X && a.pro != PRO_HEADRMS)
        return -1;
    if (a.pro == PRO_HEADRMS && (a.group < 32 || a.group % 32 || a.K % a.group)) return -1;
    if ((a.pro == PRO_RMSU_X || a.pro == PRO_X) && (!a.x || ((uintptr_t)a.x & 15) || (a.xs & 3))) return -1;
    if (a.pro == PRO_RMSU_X && (!a.pro_w || ((uintptr_t)a.pro_w & 15))) return -1;
    // POST_SWIGLU_H exists in the per-CU launch only
    if (a.post.mode == POST_SWIGLU_H) return gemv_launch_cu(a, st) == 0 ? 0 : -1;
    if (a.post.mode == POST_SWIGLU &&
        (!a.post.xq || !a.post.cnt || a.nseg != 2 || a.seg[0].n_rows != a.seg[1].n_rows || a.seg[0].n_rows % 32 ||
         32 % p.rows_per_group)) return -1;
    if (a.T > 1) {
        bool secondary = false;
        for (int i = 0; i < a.nseg; i++)
            secondary = secondary || a.seg[i].type == XJ_Q5_K || a.seg[i].type == XJ_F16 || a.seg[i].type == XJ_BF16;
        if (secondary) {   // one launch per token (multi-token kernels carry no Q5_K / F16 / BF16 rows)
            for (int t = 0; t < a.T; t++)
                if (gemv_launch(token_range(a, t, 1), st)) return -1;
            return 0;
        }
    }
    if (a.T <= kCuMaxT) {
        const int rc = gemv_launch_cu(a, st);
        if (rc <= 0) return rc;
    }
    if (gemv_lds_bytes(a) > (size_t)g_lds_max) {
        // the looping kernel stages v_off bytes per token: as many tokens per
        // launch as fit (a row's result does not depend on the split)
        const int fit = a.T > 1 ? (int)((size_t)g_lds_max / xq_off(a.K).v_off) : 0;
        if (fit < 1) return -1;
        for (int t0 = 0; t0 < a.T; t0 += fit)
            if (gemv_launch(token_range(a, t0, a.T - t0 < fit ? a.T - t0 : fit), st)) return -1;
        return 0;
    }
    const int n_rg = a.seg[a.nseg - 1].wg0 + a.seg[a.nseg - 1].nwg;
    int grid = a.T == 1 ? (n_rg < g_grid_cap1 ? n_rg : g_grid_cap1) : (n_rg < g_grid_cap ? n_rg : g_grid_cap);
    // a single token with at most two units per lane: Q4_K / Q6_K rows loop
    // with the next row group's whole window in flight (151936 x 1024 Q4_K
    // 23.6 -> 21.4 us, Q6_K 67.8 -> 55.2 us against one row group per
    // work-group); other rows take one row group per work-group, whose whole
    // window is requested at once, which streams faster than work-groups that
    // loop with one unit in flight (Q4_K: 30.4 -> 22.1 us)
    if (a.T == 1 && !g_grid_forced && (a.K / 64 + p.lanes - 1) / p.lanes <= 2 && n_rg <= 64 * g_cus &&
        !(all_k(a) && loop_window()))
        grid = n_rg;
    // Q4_K-only rows looping with their window in flight: four work-groups
    // per CU (151936 x 1024: 21.1 / 19.7 / 22.0 us at 3 / 4 / 5 per CU; the
    // Q6_K rows of that shape 30.4 / 33.9 us at 3 / 4)
    if (a.T == 1 && !g_grid_forced && (a.K / 64 + p.lanes - 1) / p.lanes <= 2 && all_q4k(a) && loop_window())
        grid = n_rg < 4 * g_cus ? n_rg : 4 * g_cus;
    hipError_t e;
    switch (p.lanes) {
    case 8: e = launch_ts<8>(a, grid, st); break;
    case 16: e = launch_ts<16>(a, grid, st); break;
    case 32: e = launch_ts<32>(a, grid, st); break;
    default: e = launch_ts<64>(a, grid, st); break;
    }
    return e == hipSuccess ? 0 : -1;
}

template <int TS>
static void raise_ts(int bytes) {
    const void *f[] = {(const void *)gemv_kernel<1, TS, 0, false>, (const void *)gemv_kernel<1, TS, 1, false>,
                       (const void *)gemv_kernel<1, TS, 2, false>, (const void *)gemv_kernel<1, TS, 3, false>,
                       (const void *)gemv_kernel<1, TS, 4, false>,
                       (const void *)gemv_kernel<1, TS, 1, true>, (const void *)gemv_kernel<1, TS, 2, true>,
                       (const void *)gemv_kernel<1, TS, 3, true>, (const void *)gemv_kernel<1, TS, 4, true>,
                       (const void *)gemv_kernel<1, TS, 5, true>, (const void *)gemv_kernel<1, TS, 1, false, true>,
                       (const void *)gemv_kernel<1, TS, 2, false, true>, (const void *)gemv_kernel<2, TS, 0, false>, (const void *)gemv_kernel<3, TS, 0, false>,
                       (const void *)gemv_kernel<4, TS, 0, false>, (const void *)gemv_kernel<5, TS, 0, false>,
                       (const void *)gemv_kernel<6, TS, 0, false>, (const void *)gemv_kernel<7, TS, 0, false>,
                       (const void *)gemv_kernel<8, TS, 0, false>};
    for (const void *k : f) (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}

template <int TS, bool WF>
static void raise_cu_wf(int bytes) {
    const void *f[] = {(const void *)gemv_cu_kernel<1, TS, 1, true, WF>, (const void *)gemv_cu_kernel<1, TS, 2, true, WF>,
                       (const void *)gemv_cu_kernel<1, TS, 3, true, WF>, (const void *)gemv_cu_kernel<1, TS, 4, true, WF>,
                       (const void *)gemv_cu_kernel<1, TS, 5, true, WF>, (const void *)gemv_cu_kernel<1, TS, 1, false, WF>,
                       (const void *)gemv_cu_kernel<1, TS, 2, false, WF>, (const void *)gemv_cu_kernel<1, TS, 3, false, WF>,
                       (const void *)gemv_cu_kernel<1, TS, 4, false, WF>, (const void *)gemv_cu_kernel<1, TS, 5, false, WF>,
                       (const void *)gemv_cu_kernel<2, TS, 0, true, WF>, (const void *)gemv_cu_kernel<3, TS, 0, true, WF>,
                       (const void *)gemv_cu_kernel<4, TS, 0, true, WF>, (const void *)gemv_cu_kernel<5, TS, 0, true, WF>,
                       (const void *)gemv_cu_kernel<2, TS, 0, false, WF>, (const void *)gemv_cu_kernel<3, TS, 0, false, WF>,
                       (const void *)gemv_cu_kernel<4, TS, 0, false, WF>, (const void *)gemv_cu_kernel<5, TS, 0, false, WF>};
    for (const void *k : f) (void)hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
}
template <int TS>
static void raise_cu(int bytes) {
    raise_cu_wf<TS, false>(bytes);
    raise_cu_wf<TS, true>(bytes);
}

int gemv_init(char *err, size_t errlen) {
    static bool done = false;
    if (done) return 0;
    int dev = 0, cus = 0, lds = 0;
    XJ_CHECK(hipGetDevice(&dev), err, errlen, -1);
    XJ_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), err, errlen, -1);
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess) lds = 65536;
    if (cus > 0) {
        g_cus = cus;
        const int forced = env_or("XJ_GEMV_WG_PER_CU", 0);
        g_grid_forced = forced > 0;
        // a looping single-token launch (the LM head): three work-groups per
        // CU, one resident round that pays the activation prologue once per
        // work-group (151936 x 2560 Q6_K: 65.2 / 60.4 / 74.4 / 62.9 us at
        // 8 / 3 / 4 / 6 per CU)
        g_grid_cap1 = cus * (forced > 0 ? forced : env_or("XJ_GEMV_WG_PER_CU_1", 3));
        // several tokens stage T x 3 digit bytes per weight element from LDS:
        // fewer work-groups per CU contend less (151936 x 1024 Q4_K, T = 2:
        // 39.2 / 42.2 / 48.7 us at 2 / 4 / 8 per CU)
        g_grid_cap = cus * (forced > 0 ? forced : env_or("XJ_GEMV_WG_PER_CU_T", 2));
    }
    // keep 4 KB for the static reduction buffers
    int want = lds > 65536 ? lds - 4096 : 65536 - 4096;
    raise_ts<8>(want); raise_ts<16>(want); raise_ts<32>(want); raise_ts<64>(want);
    raise_cu<8>(want); raise_cu<16>(want); raise_cu<32>(want); raise_cu<64>(want);
    (void)hipGetLastError();
    g_lds_max = want;
    done = true;
    return 0;
}

// ------------------------------------------------------------- upload --
int upload_repack(uint32_t type, const void *src, int64_t n_rows, int64_t k, uint8_t *dst, hipStream_t st,
                  char *err, size_t errlen) {
    const uint8_t *s = (const uint8_t *)src;
    const uint64_t bytes = xjh_row_bytes(type, k) * (uint64_t)n_rows;
    if (type == XJ_F32 || type == XJ_F16 || type == XJ_BF16 || type == XJ_Q4_K || type == XJ_Q5_K) {
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
        snprintf(err, errlen, "no device layout for %s tensors", xjh_type_name(type));
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

// Depthwise causal conv + SiLU of T tokens in place (xj_cpu.c:164-181), one
// thread per channel walking the tokens with the window in registers: the
// EPI_CONV epilogue's expressions (s = sum over k of st[k] * wc[k] in k
// order, then fma(x, wc[KC-1], s); the window shifted, the input appended),
// so results equal the epilogue's bit for bit. The inputs of 16 tokens are
// requested at once (the stores of earlier tokens go to other addresses).
// Checkpoint t (t < ck_n) holds the state after token t.
template <int KC>
__global__ __launch_bounds__(64) void conv_silu_kernel(float *x, float *state, const float *w, int C, int T, float *ck,
                                                       int ck_n) {
    const int64_t r = (int64_t)blockIdx.x * 64 + threadIdx.x;
    if (r >= C) return;
    float st[KC - 1], wc[KC];
#pragma unroll
    for (int k = 0; k < KC - 1; k++) st[k] = state[r * (KC - 1) + k];
#pragma unroll
    for (int k = 0; k < KC; k++) wc[k] = w[r * KC + k];
    for (int t0 = 0; t0 < T; t0 += 16) {
        float xv[16];
#pragma unroll
        for (int i = 0; i < 16; i++) xv[i] = x[(int64_t)(t0 + i < T ? t0 + i : T - 1) * C + r];
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int t = t0 + i;
            if (t >= T) break;
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < KC - 1; k++) s = fmaf(st[k], wc[k], s);
            s = fmaf(xv[i], wc[KC - 1], s);
#pragma unroll
            for (int k = 0; k + 1 < KC - 1; k++) st[k] = st[k + 1];
            st[KC - 2] = xv[i];
            x[(int64_t)t * C + r] = xjd::silu(s);
            if (t < ck_n)
#pragma unroll
                for (int k = 0; k < KC - 1; k++) ck[((int64_t)t * C + r) * (KC - 1) + k] = st[k];
        }
    }
#pragma unroll
    for (int k = 0; k < KC - 1; k++) state[r * (KC - 1) + k] = st[k];
}

int conv_silu_launch(float *x, float *state, const float *w, int C, int K, int T, float *ck, int ck_n, hipStream_t st) {
    if (C < 1 || T < 1 || K < 2 || K > 8 || ck_n < 0 || ck_n > T || (ck_n && !ck)) return -1;
    const dim3 g((C + 63) / 64), b(64);
    switch (K) {
    case 2: hipLaunchKernelGGL(conv_silu_kernel<2>, g, b, 0, st, x, state, w, C, T, ck, ck_n); break;
    case 3: hipLaunchKernelGGL(conv_silu_kernel<3>, g, b, 0, st, x, state, w, C, T, ck, ck_n); break;
    case 4: hipLaunchKernelGGL(conv_silu_kernel<4>, g, b, 0, st, x, state, w, C, T, ck, ck_n); break;
    case 5: hipLaunchKernelGGL(conv_silu_kernel<5>, g, b, 0, st, x, state, w, C, T, ck, ck_n); break;
    case 6: hipLaunchKernelGGL(conv_silu_kernel<6>, g, b, 0, st, x, state, w, C, T, ck, ck_n); break;
    case 7: hipLaunchKernelGGL(conv_silu_kernel<7>, g, b, 0, st, x, state, w, C, T, ck, ck_n); break;
    default: hipLaunchKernelGGL(conv_silu_kernel<8>, g, b, 0, st, x, state, w, C, T, ck, ck_n); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

int dequant_launch(const DevW &w, int64_t r0, int64_t n, float *y, hipStream_t st) {
    const int64_t nch = w.k / 32, total = n * nch;
    const int64_t nblk = xjd::dev_nblk(w.type, w.n_rows, w.k);
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, w.p, w.type, w.k,
                       nblk, r0, n, y);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace xjk
