/*
 * Oracle (test infrastructure only): block decoding, restated from
 * src/xiaoju-pipe/core/xj_quant.h.
 *
 *   xjo_f16          <- xj_quant.h:9-23   exact fp16 -> fp32, subnormals normalised
 *   xjo_to_f16       <- xj_quant.h:25-43  fp32 -> fp16, round to nearest even, overflow -> inf
 *   scale_min_k4     <- xj_quant.h:49-52  6-bit (scale, min) j of a K-quant block
 *   xjo_dequant_row  <- xj_quant.h:55-118 F32 / F16 / BF16 / Q8_0 / Q4_K / Q5_K / Q6_K
 *   xjo_row_bytes    <- src/xiaoju-pipe/core/gguf.c:12-50
 *
 * The evaluation order of every product is the reference's: Q4_K/Q5_K use
 * (d*sc)*q - dmin*m, Q6_K uses (d*sc)*q (the second product can round, so
 * the order matters), Q8_0 uses d*q.
 *
 * Pinned by: the reference's own known-answer tests (unit.c:17-51, restated in
 * tests/test_oracle.py), golden vectors written by the reference compiled from
 * source (tests/golden/dequant_golden.bin), and live bit-for-bit comparison
 * with oracle/_ref when that library is built.
 */
#include "xjo.h"

#include <string.h>

float xjo_f16(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (e == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else if (e != 0) {
        bits = sign | ((e + 112u) << 23) | (man << 13);
    } else if (man == 0) {
        bits = sign;
    } else {
        /* subnormal: shift the mantissa up until the implicit bit appears */
        int shift = 0;
        while (!(man & 0x400u)) { man <<= 1; shift++; }
        bits = sign | ((uint32_t)(113 - shift) << 23) | ((man & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t xjo_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, fexp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (fexp == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    const int e = (int)fexp - 112;             /* rebias 127 -> 15 */
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;      /* below half the smallest subnormal */
        man |= 0x800000u;
        const uint32_t sh = (uint32_t)(14 - e);
        uint32_t h = man >> sh;
        const uint32_t rem = man & ((1u << sh) - 1u), half = 1u << (sh - 1);
        h += (rem > half || (rem == half && (h & 1u)));
        return (uint16_t)(sign | h);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    h += (rem > 0x1000u || (rem == 0x1000u && (h & 1u)));  /* carry may roll into inf */
    return (uint16_t)h;
}

static float bf16(uint16_t h) {
    uint32_t b = (uint32_t)h << 16;
    float f;
    memcpy(&f, &b, 4);
    return f;
}

static uint16_t ld16(const uint8_t *p) {
    uint16_t v;
    memcpy(&v, p, 2);
    return v;
}

static void scale_min_k4(int j, const uint8_t *s, uint8_t *sc, uint8_t *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4));
        *mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

uint64_t xjo_row_bytes(uint32_t type, int64_t n) {
    switch (type) {
    case XJ_F32: return (uint64_t)n * 4;
    case XJ_F16: case XJ_BF16: return (uint64_t)n * 2;
    case XJ_Q8_0: return (uint64_t)(n / 32) * 34;
    case XJ_Q4_K: return (uint64_t)(n / 256) * 144;
    case XJ_Q5_K: return (uint64_t)(n / 256) * 176;
    case XJ_Q6_K: return (uint64_t)(n / 256) * 210;
    default: return 0;
    }
}

void xjo_dequant_row(uint32_t type, const void *src, float *y, int64_t n) {
    const uint8_t *b = (const uint8_t *)src;
    if (type == XJ_F32) {
        memcpy(y, src, (size_t)n * 4);
    } else if (type == XJ_F16) {
        for (int64_t i = 0; i < n; i++) y[i] = xjo_f16(ld16(b + 2 * i));
    } else if (type == XJ_BF16) {
        for (int64_t i = 0; i < n; i++) y[i] = bf16(ld16(b + 2 * i));
    } else if (type == XJ_Q8_0) {
        for (int64_t blk = 0; blk < n / 32; blk++) {
            const uint8_t *p = b + 34 * blk;
            const float d = xjo_f16(ld16(p));
            for (int l = 0; l < 32; l++) y[32 * blk + l] = d * (float)(int8_t)p[2 + l];
        }
    } else if (type == XJ_Q4_K || type == XJ_Q5_K) {
        const int q5 = type == XJ_Q5_K, bb = q5 ? 176 : 144;
        for (int64_t blk = 0; blk < n / 256; blk++) {
            const uint8_t *p = b + (int64_t)bb * blk;
            const float d = xjo_f16(ld16(p)), dmin = xjo_f16(ld16(p + 2));
            const uint8_t *sc = p + 4, *qh = p + 16, *ql = p + (q5 ? 48 : 16);
            float *o = y + 256 * blk;
            for (int pair = 0; pair < 4; pair++) {
                for (int half = 0; half < 2; half++) {
                    const int j = 2 * pair + half;
                    uint8_t s, m;
                    scale_min_k4(j, sc, &s, &m);
                    const float dj = d * s, mj = dmin * m;
                    for (int l = 0; l < 32; l++) {
                        const uint8_t byte = ql[32 * pair + l];
                        int q = half ? byte >> 4 : byte & 0x0f;
                        if (q5 && (qh[l] & (1u << j))) q += 16;
                        o[64 * pair + 32 * half + l] = dj * q - mj;
                    }
                }
            }
        }
    } else if (type == XJ_Q6_K) {
        for (int64_t blk = 0; blk < n / 256; blk++) {
            const uint8_t *p = b + 210 * blk;
            const uint8_t *ql = p, *qh = p + 128;
            const int8_t *sc = (const int8_t *)(p + 192);
            const float d = xjo_f16(ld16(p + 208));
            float *o = y + 256 * blk;
            for (int e = 0; e < 256; e++) {
                /* element e = 128 h + 32 g + l : nibble (g&1 ? ql[64h+32+l] : ql[64h+l]),
                 * low half for g < 2, high half for g >= 2; 2 high bits at qh[32h+l] >> 2g */
                const int h = e >> 7, g = (e >> 5) & 3, l = e & 31;
                const uint8_t lo = ql[64 * h + 32 * (g & 1) + l];
                const int nib = g < 2 ? (lo & 0x0f) : (lo >> 4);
                const int q = (nib | (((qh[32 * h + l] >> (2 * g)) & 3) << 4)) - 32;
                o[e] = d * sc[e >> 4] * q;
            }
        }
    } else {
        memset(y, 0, (size_t)n * 4);
    }
}
