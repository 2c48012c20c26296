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

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// Block-wide sum for blockDim.x a multiple of 64 (<= 1024). `red` holds >= 16 floats.
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
