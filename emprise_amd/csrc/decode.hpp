// Element decoders for the device weight layouts (see layout.hpp).
#pragma once
#include "common.hpp"
#include "layout.hpp"

namespace emprise {

// Q4_K 6-bit scale and min of sub-block j from the 12 packed bytes (quant.cpp:48-52).
__device__ __forceinline__ void q4_scale_min(const uint8_t* s, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// The element formulas of dequantize() (quant.cpp:25-61), shared by every decoder so
// each forms the value with the same operations in the same order: Q6_K (d*sc)*(q-32),
// Q4_K (d*sc)*q - dmin*m.
__device__ __forceinline__ float q6k_weight(float d, int8_t sc, int code) { return d * (float)sc * (float)(code - 32); }
__device__ __forceinline__ float q4k_weight(float dd, float dm, int sc, int mn, int code) {
    return (dd * (float)sc) * (float)code - dm * (float)mn;
}

// Weight (row r, column k) of a matrix with `cols` inputs, exactly as the CPU
// dequantize() produces it (quant.cpp:25-78): the Q6_K product (d*sc)*q and the Q4_K
// (d*sc)*q - dmin*m are formed in the same order.
__device__ __forceinline__ float decode_element(const uint8_t* w, uint32_t type, int cols, uint64_t r, int k) {
    const int nb = cols / 256;
    if (type == kQ6K && cols % kChunkCols == 0) {
        const uint8_t* ch = w + r * (uint64_t)nb * 210 + (size_t)(k / kChunkCols) * 3360;
        const int kk = k % kChunkCols, u = kk >> 4, t = kk & 15;
        int code;
        if (t < 12) {
            code = ch[(t >> 2) * 1024 + 4 * u + (t & 3)] & 63;
        } else {
            const int b = t - 12;
            code = (ch[4 * u + b] >> 6) | ((ch[1024 + 4 * u + b] >> 6) << 2) | ((ch[2048 + 4 * u + b] >> 6) << 4);
        }
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(ch + 3328 + 2 * (u >> 4)));
        return q6k_weight(d, (int8_t)ch[3072 + u], code);
    }
    if (type == kQ4K && cols % kChunkCols == 0) {
        const uint8_t* ch = w + r * (uint64_t)nb * 144 + (size_t)(k / kChunkCols) * 2304;
        const int kk = k % kChunkCols, u = kk >> 5, t = kk & 31;
        const uint8_t byte = ch[(u & 1) * 1024 + 16 * (u >> 1) + 4 * ((t & 15) >> 2) + (t & 3)];
        const int code = t < 16 ? (byte & 15) : (byte >> 4);
        const uint8_t* s = ch + 2048 + 12 * (u >> 3);
        const int j = u & 7;
        const int sc = s[j] & 63, mn = ((s[j] >> 6) << 4) | ((s[8 + (j >> 1)] >> (4 * (j & 1))) & 15);
        const uint8_t* dp = ch + 2240 + 4 * (u >> 3);
        const float dd = half_bits_to_float(*reinterpret_cast<const uint16_t*>(dp));
        const float dm = half_bits_to_float(*reinterpret_cast<const uint16_t*>(dp + 2));
        return q4k_weight(dd, dm, sc, mn, code);
    }
    if (type == kQ6K) {
        const uint8_t* row = w + r * (uint64_t)nb * 210;
        const int u = k >> 4, t = k & 15;
        const uint8_t* q = row + (size_t)u * 12;
        int code;
        if (t < 12) code = q[t] & 63;
        else code = (q[t - 12] >> 6) | ((q[t - 8] >> 6) << 2) | ((q[t - 4] >> 6) << 4);
        const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(row + (size_t)nb * 208 + 2 * (u >> 4)));
        return q6k_weight(d, (int8_t)row[(size_t)nb * 192 + u], code);
    }
    if (type == kQ4K) {
        const uint8_t* row = w + r * (uint64_t)nb * 144;
        const int u = k >> 5, t = k & 31;
        const uint8_t byte = row[(size_t)u * 16 + 4 * ((t & 15) >> 2) + (t & 3)];
        const int code = t < 16 ? (byte & 15) : (byte >> 4);
        int sc, mn;
        q4_scale_min(row + (size_t)nb * 128 + (size_t)(u >> 3) * 12, u & 7, sc, mn);
        const uint8_t* dp = row + (size_t)nb * 140 + (size_t)(u >> 3) * 4;
        const float dd = half_bits_to_float(*reinterpret_cast<const uint16_t*>(dp));
        const float dm = half_bits_to_float(*reinterpret_cast<const uint16_t*>(dp + 2));
        return q4k_weight(dd, dm, sc, mn, code);
    }
    const uint64_t i = r * (uint64_t)cols + (uint64_t)k;
    if (type == kF32) return reinterpret_cast<const float*>(w)[i];
    if (type == kF16) return half_bits_to_float(reinterpret_cast<const uint16_t*>(w)[i]);
    return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(w)[i] << 16);
}

}  // namespace emprise
