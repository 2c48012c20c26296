// Device weight layouts. Both quantised layouts keep exactly the GGUF byte count
// (210 B per 256 Q6_K weights, 144 B per 256 Q4_K weights): blocks are rearranged per
// row into planes, never padded (the reference pads Q6_K to 216 B and Q4_K to 160 B,
// cuda.cpp:640-690).
//
// A matrix of `rows` x `cols` (nb = cols/256 super-blocks per row) is row-major; row r
// starts at r * nb * block_bytes, and inside a row:
//
// Q6_K (block_bytes 210), 16-weight "units" u = 0 .. 16*nb-1 (unit u = sub-block u%16 of
// block u/16, the granularity of one int8 scale):
//   [0, 192*nb)      quants: unit u at 12*u, three dwords D0 D1 D2. With q[i] the 6-bit
//                    code (0..63) of weight 16u+i:  byte 4j+k of the unit (j<3, k<4) =
//                    q[4j+k] | ((q[12+k] >> 2j) & 3) << 6.  So Dj & 0x3F3F3F3F gives
//                    weights 4j..4j+3 as bytes, and weights 12..15 are gathered from the
//                    top two bits of D0, D1, D2.
//   [192*nb, 208*nb) int8 scales, one per unit (the GGUF scale bytes, in order)
//   [208*nb, 210*nb) fp16 d, one per block
//
// Q4_K (block_bytes 144), 32-weight units u = 0 .. 8*nb-1 (unit u = sub-block u%8 of block
// u/8, the granularity of one 6-bit scale/min pair):
//   [0, 128*nb)      nibbles: unit u at 16*u, four dwords; byte k of dword j holds weight
//                    4j+k in its low nibble and weight 16+4j+k in its high nibble
//   [128*nb, 140*nb) the GGUF 12-byte packed scales/mins of each block, unchanged
//   [140*nb, 144*nb) fp16 d, fp16 dmin of each block
//
// F32 / F16 / BF16 weights keep the GGUF row-major bytes.
//
// Rows of a multiple of 4096 inputs use a chunked layout instead: the row is a sequence
// of 4096-column chunks (16 super-blocks), each laid out for one wave of 64 lanes
// (lane l handles 64 consecutive weights of every chunk):
//
// Q6_K chunk (3360 B): three planes of 256 dwords, plane p holding dword Dp of unit u
//   (u = 0..255, the unit encoding above) at p*1024 + 4u, so lane l reads its four units
//   with one 16-byte load per plane; then the 256 int8 scales in unit order (3072), then
//   the 16 fp16 d (3328).
// Q4_K chunk (2304 B): two planes of 64 x 16 B, unit u at (u%2)*1024 + 16*(u/2) (lane l
//   reads units 2l and 2l+1); then 16 x 12 B of scales/mins re-packed per block as bytes
//   0-7: sc_j | (m_j >> 4) << 6 and bytes 8-11: (m_2t & 15) | (m_2t+1 & 15) << 4 (2048);
//   then 16 x (fp16 d, fp16 dmin) (2240).
#pragma once
#include <stdint.h>
#include <string.h>

namespace emprise {

constexpr int kChunkCols = 4096;
inline bool chunked_cols(uint64_t cols) { return cols % kChunkCols == 0; }

enum WeightType : uint32_t { kF32 = 0, kF16 = 1, kQ4K = 12, kQ6K = 14, kBF16 = 30 };

inline uint64_t type_block_bytes(uint32_t t) { return t == kQ6K ? 210 : t == kQ4K ? 144 : 0; }

// GGUF encoded size (gguf.cpp:72-85); 0 = not representable.
inline uint64_t encoded_bytes(uint32_t type, uint64_t n) {
    switch (type) {
    case kF32: return n > UINT64_MAX / 4 ? 0 : n * 4;
    case kF16:
    case kBF16: return n > UINT64_MAX / 2 ? 0 : n * 2;
    case kQ6K: return n % 256 ? 0 : n / 256 * 210;
    case kQ4K: return n % 256 ? 0 : n / 256 * 144;
    default: return 0;
    }
}

// 6-bit code of element i of a GGUF Q6_K block (quant.cpp:32-35, before the -32).
inline int q6_code(const uint8_t* blk, int i) {
    const int half = i / 128, g = (i % 128) / 32, l = i % 32;
    const int low = (blk[half * 64 + (g & 1) * 32 + l] >> (g >= 2 ? 4 : 0)) & 15;
    const int high = (blk[128 + half * 32 + l] >> (g * 2)) & 3;
    return low | (high << 4);
}

// GGUF row (nb blocks) -> device row.
inline void q6_row_to_device(const uint8_t* src, uint8_t* dst, uint64_t nb) {
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t* blk = src + b * 210;
        for (int su = 0; su < 16; ++su) {
            int q[16];
            for (int i = 0; i < 16; ++i) q[i] = q6_code(blk, su * 16 + i);
            uint8_t* unit = dst + (b * 16 + su) * 12;
            for (int j = 0; j < 3; ++j)
                for (int k = 0; k < 4; ++k)
                    unit[4 * j + k] = (uint8_t)(q[4 * j + k] | (((q[12 + k] >> (2 * j)) & 3) << 6));
        }
        memcpy(dst + nb * 192 + b * 16, blk + 192, 16);
        memcpy(dst + nb * 208 + b * 2, blk + 208, 2);
    }
}

// Device row -> GGUF row (inverse of the above).
inline void q6_row_from_device(const uint8_t* src, uint8_t* dst, uint64_t nb) {
    for (uint64_t b = 0; b < nb; ++b) {
        uint8_t* blk = dst + b * 210;
        memset(blk, 0, 192);
        for (int su = 0; su < 16; ++su) {
            const uint8_t* unit = src + (b * 16 + su) * 12;
            int q[16];
            for (int j = 0; j < 3; ++j)
                for (int k = 0; k < 4; ++k) q[4 * j + k] = unit[4 * j + k] & 63;
            for (int k = 0; k < 4; ++k)
                q[12 + k] = (unit[k] >> 6) | ((unit[4 + k] >> 6) << 2) | ((unit[8 + k] >> 6) << 4);
            for (int t = 0; t < 16; ++t) {
                const int i = su * 16 + t;
                const int half = i / 128, g = (i % 128) / 32, l = i % 32;
                blk[half * 64 + (g & 1) * 32 + l] |= (uint8_t)((q[t] & 15) << (g >= 2 ? 4 : 0));
                blk[128 + half * 32 + l] |= (uint8_t)(((q[t] >> 4) & 3) << (2 * g));
            }
        }
        memcpy(blk + 192, src + nb * 192 + b * 16, 16);
        memcpy(blk + 208, src + nb * 208 + b * 2, 2);
    }
}

// 4-bit code of element i of a GGUF Q4_K block (quant.cpp:53-60).
inline int q4_code(const uint8_t* blk, int i) {
    const int chunk = i / 64, within = i % 64;
    const uint8_t byte = blk[16 + chunk * 32 + (within % 32)];
    return within < 32 ? (byte & 15) : (byte >> 4);
}

inline void q4_row_to_device(const uint8_t* src, uint8_t* dst, uint64_t nb) {
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t* blk = src + b * 144;
        for (int su = 0; su < 8; ++su) {
            uint8_t* unit = dst + (b * 8 + su) * 16;
            for (int j = 0; j < 4; ++j)
                for (int k = 0; k < 4; ++k)
                    unit[4 * j + k] = (uint8_t)(q4_code(blk, su * 32 + 4 * j + k) |
                                                (q4_code(blk, su * 32 + 16 + 4 * j + k) << 4));
        }
        memcpy(dst + nb * 128 + b * 12, blk + 4, 12);
        memcpy(dst + nb * 140 + b * 4, blk, 4);
    }
}

inline void q4_row_from_device(const uint8_t* src, uint8_t* dst, uint64_t nb) {
    for (uint64_t b = 0; b < nb; ++b) {
        uint8_t* blk = dst + b * 144;
        memset(blk + 16, 0, 128);
        for (int su = 0; su < 8; ++su) {
            const uint8_t* unit = src + (b * 8 + su) * 16;
            for (int t = 0; t < 32; ++t) {
                const int j = (t % 16) / 4, k = t % 4;
                const int q = t < 16 ? (unit[4 * j + k] & 15) : (unit[4 * j + k] >> 4);
                const int i = su * 32 + t, chunk = i / 64, within = i % 64;
                blk[16 + chunk * 32 + within % 32] |= (uint8_t)(within < 32 ? q : q << 4);
            }
        }
        memcpy(blk + 4, src + nb * 128 + b * 12, 12);
        memcpy(blk, src + nb * 140 + b * 4, 4);
    }
}

// ---- chunked rows (cols % 4096 == 0) ----

// Q6_K: unit-major row (the layout above, nb = 16 per chunk) -> chunked row.
inline void q6_unitrow_to_chunked(const uint8_t* src, uint8_t* dst, uint64_t nb) {
    const uint64_t chunks = nb / 16;
    for (uint64_t c = 0; c < chunks; ++c) {
        uint8_t* out = dst + c * 3360;
        for (int u = 0; u < 256; ++u) {
            const uint8_t* unit = src + (c * 256 + u) * 12;
            for (int p = 0; p < 3; ++p) memcpy(out + p * 1024 + 4 * u, unit + 4 * p, 4);
        }
        memcpy(out + 3072, src + nb * 192 + c * 256, 256);
        memcpy(out + 3328, src + nb * 208 + c * 32, 32);
    }
}

inline void q6_chunked_to_unitrow(const uint8_t* src, uint8_t* dst, uint64_t nb) {
    const uint64_t chunks = nb / 16;
    for (uint64_t c = 0; c < chunks; ++c) {
        const uint8_t* in = src + c * 3360;
        for (int u = 0; u < 256; ++u) {
            uint8_t* unit = dst + (c * 256 + u) * 12;
            for (int p = 0; p < 3; ++p) memcpy(unit + 4 * p, in + p * 1024 + 4 * u, 4);
        }
        memcpy(dst + nb * 192 + c * 256, in + 3072, 256);
        memcpy(dst + nb * 208 + c * 32, in + 3328, 32);
    }
}

// Q4_K scale/min pairs of a GGUF block (quant.cpp:48-52).
inline void q4_scales_mins(const uint8_t* s, int sc[8], int mn[8]) {
    for (int j = 0; j < 8; ++j) {
        if (j < 4) {
            sc[j] = s[j] & 63;
            mn[j] = s[j + 4] & 63;
        } else {
            sc[j] = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
            mn[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
        }
    }
}

// Inverse of q4_scales_mins: the GGUF 12-byte packing.
inline void q4_pack_scales(const int sc[8], const int mn[8], uint8_t* s) {
    for (int j = 0; j < 4; ++j) {
        s[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
        s[j + 4] = (uint8_t)((mn[j] & 63) | ((mn[j + 4] >> 4) << 6));
        s[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
}

inline void q4_unitrow_to_chunked(const uint8_t* src, uint8_t* dst, uint64_t nb) {
    const uint64_t chunks = nb / 16;
    for (uint64_t c = 0; c < chunks; ++c) {
        uint8_t* out = dst + c * 2304;
        for (int u = 0; u < 128; ++u) memcpy(out + (u % 2) * 1024 + 16 * (u / 2), src + (c * 128 + u) * 16, 16);
        for (int b = 0; b < 16; ++b) {
            int sc[8], mn[8];
            q4_scales_mins(src + nb * 128 + (c * 16 + b) * 12, sc, mn);
            uint8_t* s = out + 2048 + 12 * b;
            for (int j = 0; j < 8; ++j) s[j] = (uint8_t)(sc[j] | ((mn[j] >> 4) << 6));
            for (int t = 0; t < 4; ++t) s[8 + t] = (uint8_t)((mn[2 * t] & 15) | ((mn[2 * t + 1] & 15) << 4));
            memcpy(out + 2240 + 4 * b, src + nb * 140 + (c * 16 + b) * 4, 4);
        }
    }
}

inline void q4_chunked_to_unitrow(const uint8_t* src, uint8_t* dst, uint64_t nb) {
    const uint64_t chunks = nb / 16;
    for (uint64_t c = 0; c < chunks; ++c) {
        const uint8_t* in = src + c * 2304;
        for (int u = 0; u < 128; ++u) memcpy(dst + (c * 128 + u) * 16, in + (u % 2) * 1024 + 16 * (u / 2), 16);
        for (int b = 0; b < 16; ++b) {
            const uint8_t* s = in + 2048 + 12 * b;
            int sc[8], mn[8];
            for (int j = 0; j < 8; ++j) {
                sc[j] = s[j] & 63;
                mn[j] = ((s[j] >> 6) << 4) | ((s[8 + j / 2] >> (4 * (j % 2))) & 15);
            }
            q4_pack_scales(sc, mn, dst + nb * 128 + (c * 16 + b) * 12);
            memcpy(dst + nb * 140 + (c * 16 + b) * 4, in + 2240 + 4 * b, 4);
        }
    }
}

// Whole row GGUF <-> device, choosing the layout by width.
inline void row_to_device(uint32_t type, const uint8_t* src, uint8_t* dst, uint64_t cols, uint8_t* tmp) {
    const uint64_t nb = cols / 256;
    if (type == kQ6K) {
        if (chunked_cols(cols)) {
            q6_row_to_device(src, tmp, nb);
            q6_unitrow_to_chunked(tmp, dst, nb);
        } else {
            q6_row_to_device(src, dst, nb);
        }
    } else {
        if (chunked_cols(cols)) {
            q4_row_to_device(src, tmp, nb);
            q4_unitrow_to_chunked(tmp, dst, nb);
        } else {
            q4_row_to_device(src, dst, nb);
        }
    }
}

inline void row_from_device(uint32_t type, const uint8_t* src, uint8_t* dst, uint64_t cols, uint8_t* tmp) {
    const uint64_t nb = cols / 256;
    if (type == kQ6K) {
        if (chunked_cols(cols)) {
            q6_chunked_to_unitrow(src, tmp, nb);
            q6_row_from_device(tmp, dst, nb);
        } else {
            q6_row_from_device(src, dst, nb);
        }
    } else {
        if (chunked_cols(cols)) {
            q4_chunked_to_unitrow(src, tmp, nb);
            q4_row_from_device(tmp, dst, nb);
        } else {
            q4_row_from_device(src, dst, nb);
        }
    }
}

}  // namespace emprise
