// Device-side re-layout of uploaded GGUF weights (the reference repacks on the host,
// cuda.cpp:647-701): raw GGUF rows land in a device staging buffer and one thread per
// weight "unit" writes that unit's bytes of the kernel layout (layout.hpp) straight into
// the weight's allocation. The byte count is kept (210 B per Q6_K block, 144 B per Q4_K).
//
// Q6_K unit u (16 values of block u/16): bytes 4j+k = q[4j+k] | ((q[12+k] >> 2j) & 3) << 6
// for j < 3, k < 4, where q are the unit's 6-bit codes; the block's int8 scales and fp16
// d follow in their own regions. Q4_K unit u (32 values of block u/8): byte 4j+k = code
// 4j+k | code 16+4j+k << 4; the 12-byte scale/min packing is copied (unit-major rows) or
// re-packed to one byte per sub-block (chunked rows). Rows of a multiple of 4096 values
// take the chunked layout, others the unit-major one -- the same split as the host
// routine row_to_device, whose inverse (row_from_device) reads the uploads back in the
// round-trip tests.
#include "common.hpp"
#include "kernels.hpp"
#include "layout.hpp"

namespace emprise {
namespace {

// 6-bit code of element i of a GGUF Q6_K block (quant.cpp:25-40, before the -32).
__device__ __forceinline__ uint32_t q6_code_dev(const uint8_t* blk, int i) {
    const int half = i >> 7, g = (i & 127) >> 5, l = i & 31;
    const uint32_t low = (blk[half * 64 + (g & 1) * 32 + l] >> (g >= 2 ? 4 : 0)) & 15u;
    const uint32_t high = (blk[128 + half * 32 + l] >> (2 * g)) & 3u;
    return low | (high << 4);
}

// 4-bit code of element i of a GGUF Q4_K block (quant.cpp:53-60).
__device__ __forceinline__ uint32_t q4_code_dev(const uint8_t* blk, int i) {
    const int chunk = i >> 6, within = i & 63;
    const uint8_t byte = blk[16 + chunk * 32 + (within & 31)];
    return within < 32 ? (byte & 15u) : (byte >> 4);
}

__device__ __forceinline__ void st32(uint8_t* p, uint32_t v) { *reinterpret_cast<uint32_t*>(p) = v; }

// One thread per Q6_K unit of `rows` rows of `nb` blocks.
__global__ __launch_bounds__(256) void repack_q6k_kernel(const uint8_t* src, uint8_t* dst, uint64_t rows, uint32_t nb) {
    const uint64_t units_per_row = (uint64_t)nb * 16;
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * units_per_row) return;
    const uint64_t r = t / units_per_row;
    const uint32_t u = (uint32_t)(t - r * units_per_row), b = u >> 4, su = u & 15;
    const uint8_t* blk = src + r * (uint64_t)nb * 210 + (uint64_t)b * 210;
    uint8_t* row = dst + r * (uint64_t)nb * 210;
    uint32_t q[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) q[i] = q6_code_dev(blk, su * 16 + i);
    uint32_t d[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) w |= (q[4 * j + k] | (((q[12 + k] >> (2 * j)) & 3u) << 6)) << (8 * k);
        d[j] = w;
    }
    const bool chunked = nb % 16 == 0;
    if (chunked) {
        uint8_t* out = row + (uint64_t)(u >> 8) * 3360;  // chunk of 16 blocks = 256 units
        const uint32_t uc = u & 255;
#pragma unroll
        for (int p = 0; p < 3; ++p) st32(out + p * 1024 + 4 * uc, d[p]);
        out[3072 + uc] = blk[192 + su];
        if (su == 0) {
            out[3328 + 2 * (b & 15)] = blk[208];
            out[3328 + 2 * (b & 15) + 1] = blk[209];
        }
    } else {
        uint8_t* unit = row + (uint64_t)u * 12;
#pragma unroll
        for (int p = 0; p < 3; ++p) {
#pragma unroll
            for (int k = 0; k < 4; ++k) unit[4 * p + k] = (uint8_t)(d[p] >> (8 * k));
        }
        row[(uint64_t)nb * 192 + u] = blk[192 + su];
        if (su == 0) {
            row[(uint64_t)nb * 208 + 2 * b] = blk[208];
            row[(uint64_t)nb * 208 + 2 * b + 1] = blk[209];
        }
    }
}

// One thread per Q4_K unit of `rows` rows of `nb` blocks.
__global__ __launch_bounds__(256) void repack_q4k_kernel(const uint8_t* src, uint8_t* dst, uint64_t rows, uint32_t nb) {
    const uint64_t units_per_row = (uint64_t)nb * 8;
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= rows * units_per_row) return;
    const uint64_t r = t / units_per_row;
    const uint32_t u = (uint32_t)(t - r * units_per_row), b = u >> 3, su = u & 7;
    const uint8_t* blk = src + r * (uint64_t)nb * 144 + (uint64_t)b * 144;
    uint8_t* row = dst + r * (uint64_t)nb * 144;
    uint32_t d[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t w = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w |= (q4_code_dev(blk, su * 32 + 4 * j + k) | (q4_code_dev(blk, su * 32 + 16 + 4 * j + k) << 4)) << (8 * k);
        d[j] = w;
    }
    const bool chunked = nb % 16 == 0;
    if (chunked) {
        uint8_t* out = row + (uint64_t)(u >> 7) * 2304;  // chunk of 16 blocks = 128 units
        const uint32_t uc = u & 127;
        *reinterpret_cast<uint4*>(out + (uc & 1) * 1024 + 16 * (uc >> 1)) = make_uint4(d[0], d[1], d[2], d[3]);
        if (su == 0) {
            // the block's scales and mins as one byte per sub-block (sc | m_hi << 6) plus
            // the low nibbles of the mins in pairs, then d and dmin
            const uint8_t* s = blk + 4;
            uint8_t* o = out + 2048 + 12 * (b & 15);
            int sc[8], mn[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                if (j < 4) {
                    sc[j] = s[j] & 63;
                    mn[j] = s[j + 4] & 63;
                } else {
                    sc[j] = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
                    mn[j] = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = (uint8_t)(sc[j] | ((mn[j] >> 4) << 6));
#pragma unroll
            for (int k = 0; k < 4; ++k) o[8 + k] = (uint8_t)((mn[2 * k] & 15) | ((mn[2 * k + 1] & 15) << 4));
            uint8_t* dd = out + 2240 + 4 * (b & 15);
#pragma unroll
            for (int k = 0; k < 4; ++k) dd[k] = blk[k];
        }
    } else {
        *reinterpret_cast<uint4*>(row + (uint64_t)u * 16) = make_uint4(d[0], d[1], d[2], d[3]);
        if (su == 0) {
            uint8_t* s = row + (uint64_t)nb * 128 + 12 * (uint64_t)b;
#pragma unroll
            for (int k = 0; k < 12; ++k) s[k] = blk[4 + k];
            uint8_t* dd = row + (uint64_t)nb * 140 + 4 * (uint64_t)b;
#pragma unroll
            for (int k = 0; k < 4; ++k) dd[k] = blk[k];
        }
    }
}

}  // namespace

hipError_t launch_repack(uint32_t type, const uint8_t* src, uint8_t* dst, uint64_t rows, uint64_t cols,
                         hipStream_t stream) {
    const uint32_t nb = (uint32_t)(cols / 256);
    const uint64_t units = rows * nb * (type == kQ6K ? 16 : 8);
    if (!units) return hipSuccess;
    const uint64_t blocks = (units + 255) / 256;
    if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
    if (type == kQ6K) launch_kernel(repack_q6k_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, src, dst, rows, nb);
    else if (type == kQ4K) launch_kernel(repack_q4k_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, src, dst, rows, nb);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace emprise
