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

// Numerically stable forms used by the reference (backend.cpp:10-12, cuda.cpp:414-416).
__device__ __forceinline__ float sigmoidf_(float x) {
    return x >= 0.f ? 1.f / (1.f + expf(-x)) : expf(x) / (1.f + expf(x));
}
__device__ __forceinline__ float siluf_(float x) { return x * sigmoidf_(x); }
__device__ __forceinline__ float softplusf_(float x) { return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x))); }

// Byte j of a dword as float (v_cvt_f32_ubyte{j}).
__device__ __forceinline__ float ubyte_f(uint32_t v, int j) { return (float)((v >> (8 * j)) & 0xffu); }

}  // namespace emprise
