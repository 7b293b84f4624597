// TEST INFRASTRUCTURE ONLY: part of the CPU oracle (see ts5_oracle.h).
//
// Block formats and fp16 conversion, restated from engine/src/quants.cpp
// (fp16_to_fp32 :10-32, fp32_to_fp16 :34-56, scale_min_k4 :64-72,
// dequantize_row :74-205) and engine/src/gguf.cpp:25-48 (block sizes).
#include <cstring>

#include "ts5_oracle.h"

namespace {

// An f16's exact fp32 value: normal, subnormal (renormalised), zero, inf, NaN.
float half_value(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 31u, f = h & 0x3ffu, bits;
    if (e == 31) {
        bits = s | 0x7f800000u | (f << 13);
    } else if (e != 0) {
        bits = s | ((e + 112u) << 23) | (f << 13);
    } else if (f == 0) {
        bits = s;
    } else {
        // Shift the leading one up to bit 10; each shift halves the exponent.
        int shift = 0;
        while ((f & 0x400u) == 0) { f <<= 1; shift++; }
        bits = s | ((uint32_t)(113 - shift) << 23) | ((f & 0x3ffu) << 13);
    }
    float out;
    std::memcpy(&out, &bits, 4);
    return out;
}

// fp32 to f16, round to nearest even, with f16 subnormals, overflow to inf
// and NaN kept quiet.
uint16_t half_bits(float v) {
    uint32_t x;
    std::memcpy(&x, &v, 4);
    const uint32_t s = (x >> 16) & 0x8000u, raw_e = (x >> 23) & 0xffu, f = x & 0x7fffffu;
    if (raw_e == 0xff) return (uint16_t)(s | 0x7c00u | (f != 0 ? 0x200u : 0u));
    const int e = (int)raw_e - 112;  // rebased to f16's bias
    if (e >= 31) return (uint16_t)(s | 0x7c00u);
    if (e > 0) {
        uint32_t h = s | ((uint32_t)e << 10) | (f >> 13);
        const uint32_t rest = f & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;  // a carry may reach inf: correct
        return (uint16_t)h;
    }
    if (e < -10) return (uint16_t)s;  // below half the smallest subnormal
    const uint32_t m = f | 0x800000u, sh = (uint32_t)(14 - e);
    uint32_t h = m >> sh;
    const uint32_t rest = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rest > half || (rest == half && (h & 1u))) h++;
    return (uint16_t)(s | h);
}

inline float f16_at(const uint8_t *p) {
    uint16_t h;
    std::memcpy(&h, p, 2);
    return half_value(h);
}

// The 6-bit scale and min of sub-block j from a K-quant's 12 packed bytes:
// sub-blocks 0-3 keep theirs in the low 6 bits of bytes j and j+4; 4-7 take
// their low 4 bits from byte j+4 (low/high nibble) and their top 2 bits from
// the top bits of bytes j-4 and j.
inline void kq_scale_min(const uint8_t *sc, int j, int &scale, int &min) {
    if (j < 4) {
        scale = sc[j] & 63;
        min = sc[j + 4] & 63;
    } else {
        scale = (sc[j + 4] & 15) | ((sc[j - 4] >> 6) << 4);
        min = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

}  // namespace

extern "C" {

float ts5o_fp16_to_fp32(uint16_t h) { return half_value(h); }
uint16_t ts5o_fp32_to_fp16(float f) { return half_bits(f); }

int ts5o_block_values(uint32_t t) {
    switch (t) {
        case TS5O_F32: case TS5O_F16: case TS5O_BF16: return 1;
        case TS5O_Q4_0: case TS5O_Q4_1: case TS5O_Q5_0: case TS5O_Q5_1: case TS5O_Q8_0: return 32;
        case TS5O_Q4_K: case TS5O_Q5_K: case TS5O_Q6_K: return 256;
        default: return 0;
    }
}

int ts5o_block_bytes(uint32_t t) {
    switch (t) {
        case TS5O_F32: return 4;
        case TS5O_F16: case TS5O_BF16: return 2;
        case TS5O_Q4_0: return 18;
        case TS5O_Q4_1: return 20;
        case TS5O_Q5_0: return 22;
        case TS5O_Q5_1: return 24;
        case TS5O_Q8_0: return 34;
        case TS5O_Q4_K: return 144;
        case TS5O_Q5_K: return 176;
        case TS5O_Q6_K: return 210;
        default: return 0;
    }
}

int ts5o_dequantize_row(uint32_t type, const void *src, float *y, int64_t n) {
    const uint8_t *b = (const uint8_t *)src;
    switch (type) {
    case TS5O_F32:
        std::memcpy(y, b, (size_t)n * 4);
        return 0;
    case TS5O_F16:
        for (int64_t i = 0; i < n; i++) y[i] = f16_at(b + 2 * i);
        return 0;
    case TS5O_BF16:
        for (int64_t i = 0; i < n; i++) {
            const uint32_t bits = ((uint32_t)b[2 * i] | ((uint32_t)b[2 * i + 1] << 8)) << 16;
            std::memcpy(&y[i], &bits, 4);
        }
        return 0;
    case TS5O_Q4_0:  // d, 16 bytes: value (nibble - 8) * d; low nibbles first
        for (int64_t blk = 0; blk < n / 32; blk++, b += 18, y += 32) {
            const float d = f16_at(b);
            for (int i = 0; i < 16; i++) {
                y[i] = ((b[2 + i] & 15) - 8) * d;
                y[i + 16] = ((b[2 + i] >> 4) - 8) * d;
            }
        }
        return 0;
    case TS5O_Q4_1:  // d, m, 16 bytes: value nibble * d + m
        for (int64_t blk = 0; blk < n / 32; blk++, b += 20, y += 32) {
            const float d = f16_at(b), m = f16_at(b + 2);
            for (int i = 0; i < 16; i++) {
                y[i] = (b[4 + i] & 15) * d + m;
                y[i + 16] = (b[4 + i] >> 4) * d + m;
            }
        }
        return 0;
    case TS5O_Q5_0:
    case TS5O_Q5_1: {  // [d(, m)], 32 fifth bits, 16 bytes of nibbles
        const bool with_min = type == TS5O_Q5_1;
        const int bb = with_min ? 24 : 22, hoff = with_min ? 4 : 2;
        for (int64_t blk = 0; blk < n / 32; blk++, b += bb, y += 32) {
            const float d = f16_at(b), m = with_min ? f16_at(b + 2) : 0.0f;
            const uint32_t hb = (uint32_t)b[hoff] | ((uint32_t)b[hoff + 1] << 8) | ((uint32_t)b[hoff + 2] << 16) |
                                ((uint32_t)b[hoff + 3] << 24);
            const uint8_t *qs = b + hoff + 4;
            for (int i = 0; i < 16; i++) {
                const int lo = (qs[i] & 15) | (int)(((hb >> i) & 1u) << 4);
                const int hi = (qs[i] >> 4) | (int)(((hb >> (i + 16)) & 1u) << 4);
                if (with_min) {
                    y[i] = lo * d + m;
                    y[i + 16] = hi * d + m;
                } else {
                    y[i] = (lo - 16) * d;
                    y[i + 16] = (hi - 16) * d;
                }
            }
        }
        return 0;
    }
    case TS5O_Q8_0:  // d, 32 int8: value q * d
        for (int64_t blk = 0; blk < n / 32; blk++, b += 34, y += 32) {
            const float d = f16_at(b);
            for (int i = 0; i < 32; i++) y[i] = (int8_t)b[2 + i] * d;
        }
        return 0;
    case TS5O_Q4_K:
        // d, dmin, 12 bytes of scales/mins, 128 bytes of nibbles. Each 32-byte
        // group g holds sub-block 2g in its low nibbles and 2g+1 in its high.
        for (int64_t blk = 0; blk < n / 256; blk++, b += 144) {
            const float d = f16_at(b), dmin = f16_at(b + 2);
            const uint8_t *sc = b + 4;
            for (int g = 0; g < 4; g++) {
                const uint8_t *q = b + 16 + 32 * g;
                int s, m;
                kq_scale_min(sc, 2 * g, s, m);
                const float dl = d * s, ml = dmin * m;
                kq_scale_min(sc, 2 * g + 1, s, m);
                const float dh = d * s, mh = dmin * m;
                for (int i = 0; i < 32; i++) y[i] = dl * (q[i] & 15) - ml;
                for (int i = 0; i < 32; i++) y[32 + i] = dh * (q[i] >> 4) - mh;
                y += 64;
            }
        }
        return 0;
    case TS5O_Q5_K:
        // d, dmin, 12 bytes of scales/mins, 32 bytes of fifth bits (bit 2g
        // of byte i for group g's low value, 2g+1 for its high), 128 of nibbles.
        for (int64_t blk = 0; blk < n / 256; blk++, b += 176) {
            const float d = f16_at(b), dmin = f16_at(b + 2);
            const uint8_t *sc = b + 4, *hb = b + 16;
            for (int g = 0; g < 4; g++) {
                const uint8_t *q = b + 48 + 32 * g;
                int s, m;
                kq_scale_min(sc, 2 * g, s, m);
                const float dl = d * s, ml = dmin * m;
                kq_scale_min(sc, 2 * g + 1, s, m);
                const float dh = d * s, mh = dmin * m;
                for (int i = 0; i < 32; i++) y[i] = dl * ((q[i] & 15) + ((hb[i] >> (2 * g)) & 1 ? 16 : 0)) - ml;
                for (int i = 0; i < 32; i++) y[32 + i] = dh * ((q[i] >> 4) + ((hb[i] >> (2 * g + 1)) & 1 ? 16 : 0)) - mh;
                y += 64;
            }
        }
        return 0;
    case TS5O_Q6_K:
        // ql[128], qh[64], int8 scales[16], d. Two halves of 128 values; in a
        // half, value 32*c + i (c = 0..3) takes 4 bits from ql (byte i or
        // 32+i, low or high nibble) and 2 bits from qh[i] bits 2c..2c+1.
        for (int64_t blk = 0; blk < n / 256; blk++, b += 210) {
            const float d = f16_at(b + 208);
            for (int half = 0; half < 2; half++) {
                const uint8_t *ql = b + 64 * half, *qh = b + 128 + 32 * half;
                const int8_t *sc = (const int8_t *)(b + 192 + 8 * half);
                for (int i = 0; i < 32; i++) {
                    const int sub = i / 16;
                    const int v0 = (int)((ql[i] & 15) | (((qh[i] >> 0) & 3) << 4)) - 32;
                    const int v1 = (int)((ql[i + 32] & 15) | (((qh[i] >> 2) & 3) << 4)) - 32;
                    const int v2 = (int)((ql[i] >> 4) | (((qh[i] >> 4) & 3) << 4)) - 32;
                    const int v3 = (int)((ql[i + 32] >> 4) | (((qh[i] >> 6) & 3) << 4)) - 32;
                    y[i] = d * sc[sub] * v0;
                    y[i + 32] = d * sc[sub + 2] * v1;
                    y[i + 64] = d * sc[sub + 4] * v2;
                    y[i + 96] = d * sc[sub + 6] * v3;
                }
                y += 128;
            }
        }
        return 0;
    default:
        return -1;
    }
}

}  // extern "C"
