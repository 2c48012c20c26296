// Streaming dequant-matvec building blocks of the per-projection kernels (matvec.hip):
// the chunked weight layout's per-wave loads and per-unit FP32 arithmetic.
//
// Arithmetic (FP32 path): weight = (d*sc)*(q-32) for Q6_K (quant.cpp:25-40) and
// (d*sc)*q - dmin*m for Q4_K (quant.cpp:41-61). A unit's contribution is computed as
// (d*sc) * (sum q*x - 32*sum x) and (d*sc)*(sum q*x) - (dmin*m)*(sum x): the same
// products as the CPU path, grouped per unit.
#pragma once
#include "common.hpp"
#include "kernels.hpp"
#include "layout.hpp"

namespace emprise {
namespace {

template <int T> struct Fmt;
template <> struct Fmt<kQ6K> { static constexpr int unit = 16, block = 210; };
template <> struct Fmt<kQ4K> { static constexpr int unit = 32, block = 144; };

__device__ __forceinline__ float dot4(uint32_t q, const float4& x, float acc) {
    acc = fmaf(ubyte_f(q, 0), x.x, acc);
    acc = fmaf(ubyte_f(q, 1), x.y, acc);
    acc = fmaf(ubyte_f(q, 2), x.z, acc);
    acc = fmaf(ubyte_f(q, 3), x.w, acc);
    return acc;
}

// Hides a value's known-zero bits from the optimiser, so byte-to-float conversions of
// masked codes select v_cvt_f32_ubyte{0..3} (one instruction per weight) instead of a
// bit-field extract plus a conversion.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

// seed + sum over the 16 codes of a Q6_K unit times x (codes 0..63, no zero point)
__device__ __forceinline__ float q6_unit(uint32_t d0, uint32_t d1, uint32_t d2, const float4* x, float seed = 0.f) {
    const uint32_t a = opaque(d0 & 0x3F3F3F3Fu), b = opaque(d1 & 0x3F3F3F3Fu), c = opaque(d2 & 0x3F3F3F3Fu);
    const uint32_t e = opaque(((d0 >> 6) & 0x03030303u) | ((d1 >> 4) & 0x0C0C0C0Cu) | ((d2 >> 2) & 0x30303030u));
    float s0 = dot4(a, x[0], seed);
    float s1 = dot4(b, x[1], 0.f);
    s0 = dot4(c, x[2], s0);
    s1 = dot4(e, x[3], s1);
    return s0 + s1;
}

// sum over the 32 codes of a Q4_K unit times x
__device__ __forceinline__ float q4_unit(const uint4& d, const float4* x) {
    float s0 = dot4(opaque(d.x & 0x0F0F0F0Fu), x[0], 0.f);
    float s1 = dot4(opaque(d.y & 0x0F0F0F0Fu), x[1], 0.f);
    s0 = dot4(opaque(d.z & 0x0F0F0F0Fu), x[2], s0);
    s1 = dot4(opaque(d.w & 0x0F0F0F0Fu), x[3], s1);
    s0 = dot4(opaque((d.x >> 4) & 0x0F0F0F0Fu), x[4], s0);
    s1 = dot4(opaque((d.y >> 4) & 0x0F0F0F0Fu), x[5], s1);
    s0 = dot4(opaque((d.z >> 4) & 0x0F0F0F0Fu), x[6], s0);
    s1 = dot4(opaque((d.w >> 4) & 0x0F0F0F0Fu), x[7], s1);
    return s0 + s1;
}

// Orders floats as unsigned ints so that a larger key means a larger float; the low
// word holds ~index so that equal values prefer the smaller index (std::max_element).
__device__ __forceinline__ unsigned long long argmax_key(float v, int index) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)(~(uint32_t)index);
}

// LDS slot of input float4 e in the streaming kernels: lane l's 16 float4 of chunk c
// sit at (c*16 + i)*64 + l, so a wave reading float4 i of its lanes touches 1 KiB of
// consecutive bytes (no bank conflicts).
__device__ __forceinline__ int chunk_slot(int e) { return (((e >> 10) << 4) + (e & 15)) * 64 + ((e & 1023) >> 4); }

template <int T, int NA> struct SChunk;
template <int NA> struct SChunk<kQ6K, NA> {
    uint4 q[NA][3];    // plane p: D_p of the lane's units 4l..4l+3
    uint32_t sc[NA];   // the four int8 scales
    uint32_t d[NA];    // fp16 d of the block
};
template <int NA> struct SChunk<kQ4K, NA> {
    uint4 q[NA][2];    // units 2l and 2l+1
    uint32_t s2[NA];   // bytes j0, j0+1 of the re-packed scales (sc | m_hi << 6)
    uint32_t m4[NA];   // m low nibbles of sub-blocks j0 (low) and j0+1 (high)
    uint32_t dd[NA];   // fp16 d | fp16 dmin << 16
};

// Weight bytes are read once per token: non-temporal loads stream them past the caches.
// The pointers are cast to the global address space so the loads are global_load_*:
// through a generic pointer they become flat_load_*, which also count against lgkmcnt,
// so every wait for an LDS read would drain the next item's weight loads as well.
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
#define EMPRISE_GLOBAL __attribute__((address_space(1)))
__device__ __forceinline__ uint4 nt_u4(const uint8_t* p) {
    const u32x4_t v = __builtin_nontemporal_load((const EMPRISE_GLOBAL u32x4_t*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t nt_u32(const uint8_t* p) {
    return __builtin_nontemporal_load((const EMPRISE_GLOBAL uint32_t*)p);
}
__device__ __forceinline__ uint32_t nt_u16(const uint8_t* p) {
    return __builtin_nontemporal_load((const EMPRISE_GLOBAL uint16_t*)p);
}
__device__ __forceinline__ uint32_t nt_u8(const uint8_t* p) { return __builtin_nontemporal_load((const EMPRISE_GLOBAL uint8_t*)p); }

template <int T, int NA>
__device__ __forceinline__ void sload(SChunk<T, NA>& ch, const uint8_t* const* rp, int c, int lane) {
    if constexpr (T == kQ6K) {
#pragma unroll
        for (int r = 0; r < NA; ++r) {
            const uint8_t* base = rp[r] + (size_t)c * 3360;
#pragma unroll
            for (int p = 0; p < 3; ++p) ch.q[r][p] = nt_u4(base + p * 1024 + 16 * lane);
            ch.sc[r] = nt_u32(base + 3072 + 4 * lane);
            ch.d[r] = nt_u16(base + 3328 + 2 * (lane >> 2));
        }
    } else {
#pragma unroll
        for (int r = 0; r < NA; ++r) {
            const uint8_t* base = rp[r] + (size_t)c * 2304;
            ch.q[r][0] = nt_u4(base + 16 * lane);
            ch.q[r][1] = nt_u4(base + 1024 + 16 * lane);
            const uint8_t* s = base + 2048 + 12 * (lane >> 2);
            ch.s2[r] = nt_u16(s + 2 * (lane & 3));
            ch.m4[r] = nt_u8(s + 8 + (lane & 3));
            ch.dd[r] = nt_u32(base + 2240 + 4 * (lane >> 2));
        }
    }
}

// The per-unit input sum as the streaming kernels keep it in LDS: for Q6_K units (16
// values) the zero-point term -32 * sum x itself (exact: a power-of-two scaling), which
// seeds each unit's dot product; for Q4_K units (32 values) the plain sum, which the
// dmin * m term multiplies.
template <int UNIT> __device__ __forceinline__ float stored_unit_sum(float t) { return UNIT == 16 ? -32.f * t : t; }

__device__ __forceinline__ uint32_t lane_word(const uint4& v, int j) {
    return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

template <int T, int NA>
__device__ __forceinline__ void scompute(const SChunk<T, NA>& ch, float* acc, const float* xs, const float* usum, int c,
                                         int lane) {
    const float4* x4 = reinterpret_cast<const float4*>(xs) + (size_t)c * 1024 + lane;
    if constexpr (T == kQ6K) {
        // (d*sc_u) * (sum q x - 32 sum x) per unit u: the first of the unit's two product
        // chains starts from the stored -32 * sum x
        const float4 off4 = reinterpret_cast<const float4*>(usum)[c * 64 + lane];
        const float off[4] = {off4.x, off4.y, off4.z, off4.w};
        float dv[NA];
#pragma unroll
        for (int r = 0; r < NA; ++r) dv[r] = half_bits_to_float((uint16_t)ch.d[r]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float4 xv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) xv[i] = x4[(j * 4 + i) * 64];
#pragma unroll
            for (int r = 0; r < NA; ++r) {
                const float s = q6_unit(lane_word(ch.q[r][0], j), lane_word(ch.q[r][1], j), lane_word(ch.q[r][2], j), xv,
                                        off[j]);
                const float sc = (float)(int)(int8_t)(ch.sc[r] >> (8 * j));
                acc[r] = fmaf(dv[r] * sc, s, acc[r]);
            }
        }
    } else {
        const float2 xsum = reinterpret_cast<const float2*>(usum)[c * 64 + lane];
        const float xsv[2] = {xsum.x, xsum.y};
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            float4 xv[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = x4[(p * 8 + i) * 64];
#pragma unroll
            for (int r = 0; r < NA; ++r) {
                const uint32_t b = (ch.s2[r] >> (8 * p)) & 0xff;
                const int sc = b & 63;
                const int mn = ((b >> 6) << 4) | ((ch.m4[r] >> (4 * p)) & 15);
                const float dd = half_bits_to_float((uint16_t)(ch.dd[r] & 0xffff));
                const float dm = half_bits_to_float((uint16_t)(ch.dd[r] >> 16));
                const float s = q4_unit(ch.q[r][p], xv);
                acc[r] += (dd * (float)sc) * s - (dm * (float)mn) * xsv[p];
            }
        }
    }
}

// Work item of the streaming kernel: row group g (R rows, or R gate/up row pairs) x
// 4096-column chunk c, with the row pointers of the group and, for the conv epilogue,
// lane r*conv_width + j's history slot j and tap j of row row0 + r.
template <int NA> struct SItem {
    int g, c, seg, row0;
    const uint8_t* rp[NA];
    float conv_h, conv_k;
};

}  // namespace
}  // namespace emprise
