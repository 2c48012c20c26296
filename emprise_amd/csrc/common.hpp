// Shared device helpers for the gfx950 decode kernels (wave64, CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace emprise {

constexpr int kWave = 64;

// Exact IEEE fp16 -> fp32 (subnormals kept). The hardware conversion v_cvt_f32_f16 is
// exact for every fp16 input, including subnormals, inf and NaN (quant.cpp:8-17).
__device__ __forceinline__ float half_bits_to_float(uint16_t bits) {
    _Float16 h;
    __builtin_memcpy(&h, &bits, 2);
    return (float)h;
}

// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32 with the default mode).
__device__ __forceinline__ uint16_t float_to_half_bits(float f) {
    _Float16 h = (_Float16)f;
    uint16_t bits;
    __builtin_memcpy(&bits, &h, 2);
    return bits;
}

// Wave64 reductions on DPP lane shifts (ALU only, no LDS round trips): inclusive
// prefix within each row of 16 lanes (row_shr 1, 2, 4, 8), then row_bcast:15 and
// row_bcast:31 carry the row totals up to lane 63, which is broadcast to the wave.
// Lanes whose DPP source is out of range keep `old` (0 for sums, the value for max).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float old, float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v), CTRL, ROW_MASK, 0xf, false));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_f<0x111, 0xf>(0.f, v);  // row_shr:1
    v += dpp_f<0x112, 0xf>(0.f, v);  // row_shr:2
    v += dpp_f<0x114, 0xf>(0.f, v);  // row_shr:4
    v += dpp_f<0x118, 0xf>(0.f, v);  // row_shr:8
    v += dpp_f<0x142, 0xa>(0.f, v);  // row_bcast:15 into rows 1, 3
    v += dpp_f<0x143, 0xc>(0.f, v);  // row_bcast:31 into rows 2, 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, dpp_f<0x111, 0xf>(v, v));
    v = fmaxf(v, dpp_f<0x112, 0xf>(v, v));
    v = fmaxf(v, dpp_f<0x114, 0xf>(v, v));
    v = fmaxf(v, dpp_f<0x118, 0xf>(v, v));
    v = fmaxf(v, dpp_f<0x142, 0xa>(v, v));
    v = fmaxf(v, dpp_f<0x143, 0xc>(v, v));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `red` holds >= 16 floats.
// Workgroup barrier that orders LDS accesses only. __syncthreads() also carries a
// global-memory release, which waits for every outstanding vector memory operation of
// the wave, loads included: a kernel that has weight loads in flight would drain them
// at the barrier.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum over the workgroup (red: one float per wave) with LDS-only barriers.
__device__ __forceinline__ float block_sum_lds(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    v = wave_sum(v);
    lds_barrier();
    if (lane == 0) red[wave] = v;
    lds_barrier();
    float t = 0.f;
    for (int i = 0; i < waves; ++i) t += red[i];
    return t;
}

__device__ __forceinline__ float block_sum(float v, float* red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < waves; ++i) t += red[i];
    return t;
}

// The Q8 codes of a block's values v for its scale s (quantize_x, cuda.cpp:547-559):
// round(v / s), ties away from zero, with v / s the correctly rounded IEEE quotient. With y = 1 / s
// (itself correctly rounded, once per block) the quotient comes from Markstein's
// correction instead of a division per value: q = v*y, r = v - q*s (exact, one fused
// multiply-add), v/s = q + r*y rounded once -- the correctly rounded quotient whenever s
// and 1/s are normal (P. Markstein, "Computation of elementary functions on the IBM RISC
// System/6000 processor", IBM J. Res. Dev. 34(1), 1990; J.-M. Muller et al., Handbook of
// Floating-Point Arithmetic, the theorem on the correction step of division). Scales
// below 2^-125 take the division itself.
template <int N>
__device__ __forceinline__ void q8_codes(const float (&v)[N], float s, int (&q)[N]) {
    float t[N];
    if (s >= 0x1p-125f) {  // one branch per block: every value takes the same path
        const float y = 1.f / s;
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const float c = v[i] * y;
            t[i] = fmaf(fmaf(-c, s, v[i]), y, c);
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) t[i] = s != 0.f ? v[i] / s : 0.f;
    }
#pragma unroll
    for (int i = 0; i < N; ++i) q[i] = (int)roundf(t[i]);
}

// Numerically stable forms used by the reference (backend.cpp:10-12, cuda.cpp:414-416).
__device__ __forceinline__ float sigmoidf_(float x) {
    return x >= 0.f ? 1.f / (1.f + expf(-x)) : expf(x) / (1.f + expf(x));
}
__device__ __forceinline__ float siluf_(float x) { return x * sigmoidf_(x); }
__device__ __forceinline__ float softplusf_(float x) { return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x))); }

// Byte j of a dword as float (v_cvt_f32_ubyte{j}).
__device__ __forceinline__ float ubyte_f(uint32_t v, int j) { return (float)((v >> (8 * j)) & 0xffu); }

// ---- Gated DeltaNet on 16-lane rows --------------------------------------------------
//
// Every GDN kernel (the decode kernels and the prefill scan) keeps
// a vector of SD = 16*NE columns -- a state row, q, k -- on the 16 lanes of a DPP row,
// lane j holding columns NE*j .. NE*j + NE-1, so a wave carries four rows side by side.
// A row sum is NE sequential FMAs per lane, then row16_sum; all the kernels use these
// helpers, so they give the same bits.

// Sum over the 16 lanes of each DPP row, left in all 16: swaps within quads, then the
// half-row and row mirrors. Each step adds two equal partial sums (in either order, so
// every lane gets the same bits).
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f<0xb1, 0xf>(0.f, v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4e, 0xf>(0.f, v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x141, 0xf>(0.f, v);  // row_half_mirror
    v += dpp_f<0x140, 0xf>(0.f, v);  // row_mirror
    return v;
}
// lane U of each DPP row, in every lane of that row (row_newbcast)
template <int U> __device__ __forceinline__ float row16_bcast(float v) { return dpp_f<0x150 + U, 0xf>(0.f, v); }

// q/k L2 normalisation (backend.cpp:30-35): q / sqrt(sum q^2 + eps) / sqrt(SD) and
// k / sqrt(sum k^2 + eps).
template <int NE> __device__ __forceinline__ void gdn16_qk_norm(float (&q)[NE], float (&k)[NE], float eps) {
    float qs = 0.f, ks = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        qs = fmaf(q[i], q[i], qs);
        ks = fmaf(k[i], k[i], ks);
    }
    qs = row16_sum(qs);
    ks = row16_sum(ks);
    const float qscale = 1.f / sqrtf(qs + eps) / sqrtf((float)(16 * NE)), kscale = 1.f / sqrtf(ks + eps);
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        q[i] *= qscale;
        k[i] *= kscale;
    }
}

// The delta rule on one state row (backend.cpp:36-56) with normalised q/k, the head's
// decay and beta gate b and the row's v: S *= decay; mem = S.k; S += k * (v - mem) * b;
// returns S.q (in all 16 lanes of the row).
template <int NE>
__device__ __forceinline__ float gdn16_row(float (&s)[NE], const float (&q)[NE], const float (&k)[NE], float decay,
                                           float b, float v) {
    float mem = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        s[i] *= decay;
        mem = fmaf(s[i], k[i], mem);
    }
    mem = row16_sum(mem);
    const float delta = (v - mem) * b;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NE; ++i) {
        s[i] = fmaf(k[i], delta, s[i]);
        sum = fmaf(s[i], q[i], sum);
    }
    return row16_sum(sum);
}

// NE consecutive floats (NE a multiple of 4) as 16-byte accesses.
template <int NE> __device__ __forceinline__ void ld16v(float (&d)[NE], const float* p) {
#pragma unroll
    for (int i = 0; i < NE; i += 4) {
        const float4 v = *reinterpret_cast<const float4*>(p + i);
        d[i] = v.x, d[i + 1] = v.y, d[i + 2] = v.z, d[i + 3] = v.w;
    }
}
template <int NE> __device__ __forceinline__ void st16v(float* p, const float (&d)[NE]) {
#pragma unroll
    for (int i = 0; i < NE; i += 4) *reinterpret_cast<float4*>(p + i) = make_float4(d[i], d[i + 1], d[i + 2], d[i + 3]);
}

}  // namespace emprise
