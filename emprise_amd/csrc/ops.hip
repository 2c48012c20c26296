// Small per-token kernels: fill, RMSNorm, residual add, SwiGLU, embedding row,
// argmax, Q8 activation quantisation, position/token advance.
#include "common.hpp"
#include "decode.hpp"
#include "kernels.hpp"

namespace emprise {
namespace {

__global__ void fill_kernel(float* dst, float value, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = value;
}

__global__ void fill_u64_kernel(unsigned long long* dst, unsigned long long value, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        dst[i] = value;
}

// rmsnorm_kernel (cuda.cpp:533-542) / rms (model.cpp:19-25): out = x * (scale * w);
// workgroup r normalises row r of x (rows of n floats)
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const float* x, const float* w, float* out, int n, float eps) {
    __shared__ float red[16];
    x += (size_t)blockIdx.x * n;
    out += (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    const float total = block_sum(ss, red);
    const float scale = 1.f / sqrtf(total / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * (scale * w[i]);
}

// add_kernel then rmsnorm_kernel on row r in one pass: x += delta, out = rms(x) * w, the
// same values and the same sum order as the two kernels
__global__ __launch_bounds__(1024) void add_rmsnorm_kernel(float* x, const float* delta, const float* w, float* out,
                                                           int n, float eps) {
    __shared__ float red[16];
    x += (size_t)blockIdx.x * n;
    delta += (size_t)blockIdx.x * n;
    out += (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = x[i] + delta[i];
        x[i] = v;
        ss += v * v;
    }
    const float total = block_sum(ss, red);
    const float scale = 1.f / sqrtf(total / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[i] = x[i] * (scale * w[i]);
}

// The same for rows of at most 1024 * KR values, each sum x + delta kept in registers
// for the second pass instead of read back (same element-to-thread assignment, same
// results).
template <int KR>
__global__ __launch_bounds__(1024) void add_rmsnorm_regs_kernel(float* x, const float* delta, const float* w,
                                                                float* out, int n, float eps) {
    __shared__ float red[16];
    x += (size_t)blockIdx.x * n;
    delta += (size_t)blockIdx.x * n;
    out += (size_t)blockIdx.x * n;
    float v[KR], ss = 0.f;
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const int i = threadIdx.x + 1024 * k;
        if (i < n) {
            v[k] = x[i] + delta[i];
            x[i] = v[k];
            ss += v[k] * v[k];
        }
    }
    const float total = block_sum(ss, red);
    const float scale = 1.f / sqrtf(total / (float)n + eps);
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const int i = threadIdx.x + 1024 * k;
        if (i < n) out[i] = v[k] * (scale * w[i]);
    }
}

__global__ void add_kernel(float* x, const float* y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] += y[i];
}

// swiglu (cuda.cpp:560-566; backend.cpp:96-100): g * sigmoid(g) * u
__global__ void swiglu_kernel(float* gate, const float* up, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) gate[i] = siluf_(gate[i]) * up[i];
}
// swiglu over `rows` rows of n: row r of gate at r * ldg, of up at r * ldu
__global__ void swiglu_rows_kernel(float* gate, size_t ldg, const float* up, size_t ldu, int n, int rows) {
    const int r = blockIdx.y;
    if (r >= rows) return;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x)
        gate[(size_t)r * ldg + i] = siluf_(gate[(size_t)r * ldg + i]) * up[(size_t)r * ldu + i];
}

// row blockIdx.y of out = embedding row token[blockIdx.y]
__global__ void embed_kernel(const uint8_t* w, uint32_t type, int cols, int rows, const int* token, float* out) {
    const int t = token[blockIdx.y];
    out += (size_t)blockIdx.y * cols;
    if (t < 0 || t >= rows) return;  // the host validates ids before they reach the device
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < cols; k += gridDim.x * blockDim.x)
        out[k] = decode_element(w, type, cols, (uint64_t)t, k);
}

__device__ __forceinline__ unsigned long long order_key(float v, int index) {
    uint32_t u = __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)(~(uint32_t)index);
}

// First maximum (std::max_element, model.cpp:499): one workgroup scans all logits.
__global__ __launch_bounds__(1024) void argmax_kernel(const float* logits, int n, int* index) {
    __shared__ unsigned long long best;
    if (threadIdx.x == 0) best = 0ull;
    __syncthreads();
    unsigned long long mine = 0ull;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const unsigned long long k = order_key(logits[i], i);
        mine = k > mine ? k : mine;
    }
    atomicMax(&best, mine);
    __syncthreads();
    if (threadIdx.x == 0) *index = (int)~(uint32_t)(best & 0xffffffffull);
}

// Turns the key left by the LM-head epilogue into an index and clears the key for the
// next token.
__global__ void argmax_finish_kernel(unsigned long long* key, int* index) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        *index = (int)~(uint32_t)(*key & 0xffffffffull);
        *key = 0ull;
    }
}

// quantize_x (cuda.cpp:547-559): one 32-value block per thread.
__global__ void quantize_q8_kernel(const float* x, int cols, int8_t* q, float* scales) {
    const int blk = blockIdx.x * blockDim.x + threadIdx.x;
    if (blk >= cols / 32) return;
    float amax = 0.f;
    for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(x[blk * 32 + i]));
    const float s = amax / 127.f;
    for (int h = 0; h < 4; ++h) {
        float v[8];
        int c[8];
        for (int i = 0; i < 8; ++i) v[i] = x[blk * 32 + 8 * h + i];
        q8_codes<8>(v, s, c);
        for (int i = 0; i < 8; ++i) q[blk * 32 + 8 * h + i] = (int8_t)c[i];
    }
    scales[blk] = half_bits_to_float(float_to_half_bits(s));
}

// state = {position, token, prompt_len}
__global__ void advance_kernel(int* state, const int* prompt, int* history, const int* next) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        const int p = state[0];
        const int nxt = next ? *next : 0;
        if (history) history[p] = nxt;
        state[0] = p + 1;
        state[1] = (prompt && p + 1 < state[2]) ? prompt[p + 1] : nxt;
    }
}

// Plain read stream, in the shape that streams fastest on this part (measured with
// standalone read kernels: one workgroup of 8 waves per CU, one 4 KiB piece in flight
// per wave, non-temporal 16-byte loads, reached 7.6 TB/s over 1 GB; 16 and 32 waves per
// CU, or more pieces in flight, read slower): wave w of the grid takes pieces w, w + nw,
// ... and keeps their XOR.
constexpr int kReadWaves = 8;
__global__ __launch_bounds__(kReadWaves * 64) void stream_read_kernel(const uint4* __restrict__ src, size_t pieces,
                                                                      uint32_t* __restrict__ sink) {
    __shared__ uint32_t red;
    if (threadIdx.x == 0) red = 0;
    __syncthreads();
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const size_t nw = (size_t)gridDim.x * kReadWaves;
    uint32_t acc = 0;
    for (size_t p = (size_t)blockIdx.x * kReadWaves + wave; p < pieces; p += nw) {
        const u4v* base = reinterpret_cast<const u4v*>(src + p * 256) + lane;
        u4v v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = __builtin_nontemporal_load(base + 64 * k);
#pragma unroll
        for (int k = 0; k < 4; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    atomicXor(&red, acc);
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = red;
}

unsigned grid_for(size_t n, unsigned block, unsigned cap) {
    size_t g = (n + block - 1) / block;
    if (g > cap) g = cap;
    return g ? (unsigned)g : 1u;
}

}  // namespace

hipError_t launch_fill(float* dst, float value, size_t n, hipStream_t stream) {
    launch_kernel(fill_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, stream, dst, value, n);
    return hipGetLastError();
}
hipError_t launch_fill_u64(unsigned long long* dst, unsigned long long value, size_t n, hipStream_t stream) {
    launch_kernel(fill_u64_kernel, dim3(grid_for(n, 256, 4096)), dim3(256), 0, stream, dst, value, n);
    return hipGetLastError();
}
hipError_t launch_rmsnorm(const float* x, const float* w, float* out, int n, float eps, hipStream_t stream) {
    launch_kernel(rmsnorm_kernel, dim3(1), dim3(1024), 0, stream, x, w, out, n, eps);
    return hipGetLastError();
}
hipError_t launch_rmsnorm_rows(const float* x, const float* w, float* out, int n, int rows, float eps,
                               hipStream_t stream) {
    if (rows < 1) return hipErrorInvalidValue;
    launch_kernel(rmsnorm_kernel, dim3(rows), dim3(1024), 0, stream, x, w, out, n, eps);
    return hipGetLastError();
}
hipError_t launch_add_rmsnorm_rows(float* x, const float* delta, const float* w, float* out, int n, int rows, float eps,
                                  hipStream_t stream) {
    if (rows < 1) return hipErrorInvalidValue;
    if (n <= 1024 * 4)
        launch_kernel(add_rmsnorm_regs_kernel<4>, dim3(rows), dim3(1024), 0, stream, x, delta, w, out, n, eps);
    else if (n <= 1024 * 8)
        launch_kernel(add_rmsnorm_regs_kernel<8>, dim3(rows), dim3(1024), 0, stream, x, delta, w, out, n, eps);
    else
        launch_kernel(add_rmsnorm_kernel, dim3(rows), dim3(1024), 0, stream, x, delta, w, out, n, eps);
    return hipGetLastError();
}
hipError_t launch_add(float* x, const float* y, int n, hipStream_t stream) {
    launch_kernel(add_kernel, dim3(grid_for((size_t)n, 256, 1u << 20)), dim3(256), 0, stream, x, y, n);
    return hipGetLastError();
}
hipError_t launch_swiglu(float* gate, const float* up, int n, hipStream_t stream) {
    launch_kernel(swiglu_kernel, dim3(grid_for((size_t)n, 256, 1u << 20)), dim3(256), 0, stream, gate, up, n);
    return hipGetLastError();
}
hipError_t launch_swiglu_rows(float* gate, size_t ldg, const float* up, size_t ldu, int n, int rows,
                              hipStream_t stream) {
    if (rows < 1 || rows > 65535 || n < 1) return hipErrorInvalidValue;
    launch_kernel(swiglu_rows_kernel, dim3(grid_for((size_t)n, 256, 64), rows), dim3(256), 0, stream, gate, ldg, up,
                  ldu, n, rows);
    return hipGetLastError();
}
hipError_t launch_embed(const uint8_t* w, uint32_t type, int cols, int rows, const int* token, float* out,
                        hipStream_t stream) {
    launch_kernel(embed_kernel, dim3(grid_for((size_t)cols, 256, 64)), dim3(256), 0, stream, w, type, cols, rows,
                       token, out);
    return hipGetLastError();
}
hipError_t launch_embed_rows(const uint8_t* w, uint32_t type, int cols, int rows, const int* tokens, int count,
                             float* out, hipStream_t stream) {
    if (count < 1 || count > 65535) return hipErrorInvalidValue;
    launch_kernel(embed_kernel, dim3(grid_for((size_t)cols, 256, 64), count), dim3(256), 0, stream, w, type, cols,
                  rows, tokens, out);
    return hipGetLastError();
}
hipError_t launch_argmax(const float* logits, int n, unsigned long long*, int* index, hipStream_t stream) {
    launch_kernel(argmax_kernel, dim3(1), dim3(1024), 0, stream, logits, n, index);
    return hipGetLastError();
}
hipError_t launch_argmax_finish(const unsigned long long* key, int* index, hipStream_t stream) {
    launch_kernel(argmax_finish_kernel, dim3(1), dim3(64), 0, stream, const_cast<unsigned long long*>(key), index);
    return hipGetLastError();
}
hipError_t launch_quantize_q8(const float* x, int cols, int8_t* q, float* scales, hipStream_t stream) {
    launch_kernel(quantize_q8_kernel, dim3(grid_for((size_t)cols / 32, 64, 1u << 20)), dim3(64), 0, stream, x,
                       cols, q, scales);
    return hipGetLastError();
}
hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream) {
    const size_t pieces = bytes / 4096;
    if (!pieces || bytes % 4096) return hipErrorInvalidValue;
    int dev = 0, cus = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return e;
    const int grid = std::min(std::max(cus, 1), 4096);
    launch_kernel(stream_read_kernel, dim3(grid), dim3(kReadWaves * 64), 0, stream, static_cast<const uint4*>(src),
                  pieces, sink);
    return hipGetLastError();
}
hipError_t launch_advance(int* state, const int* prompt, int* history, const int* next, hipStream_t stream) {
    launch_kernel(advance_kernel, dim3(1), dim3(64), 0, stream, state, prompt, history, next);
    return hipGetLastError();
}

}  // namespace emprise
