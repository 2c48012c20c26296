// Batched projection Y = X W^T on the matrix cores (Backend::linear_batch, reference
// backend.hpp:20-24 and the CUDA linear_q6_f32_batch, cuda.cpp:350-413, which stops
// at K <= 4 tokens). Prefill runs thousands of tokens through each projection, so the
// matvec becomes a dense GEMM: M = tokens, N = output rows, K = input columns.
//
// Arithmetic is FP32 end to end: the weights are dequantised exactly (the FP32 value
// (d*sc)*q of every element, as the CPU path forms it) and the products run on
// v_mfma_f32_32x32x2_f32, whose inputs are FP32. Only the order of the FP32 additions
// differs from the CPU's sequential row sum.
//
// Tiling: a workgroup of 4 waves computes a 128 x 128 tile of C; each wave owns a
// 64 x 64 quarter as 2 x 2 MFMA tiles of 32 x 32 (16 accumulators per lane each). The
// K loop stages 16-column slices of A and B in LDS, k-major so that a fragment load
// (32 consecutive rows at one k) is one conflict-free LDS read per lane, and the next
// slice is loaded from global memory into registers while the current one feeds the
// matrix cores.
//
// MFMA 32x32x2 f32 operand layout (lane l, 64 lanes): A[i][k] and B[k][j] come from
// lane i + 32k / j + 32k; the result element D[i][j] is accumulator register r of
// lane l with j = l % 32 and i = 8*(r / 4) + 4*(l / 32) + r % 4.
#include "common.hpp"
#include "kernels.hpp"

namespace emprise {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int GM = 128, GN = 128, GK = 16, GPAD = 4;

// Batch z of a launch (blockIdx.z) multiplies A + z*sA by B + (z/bdiv)*sB into C + z*sC
// (the heads of attention, bdiv q heads per kv head). Causal forms, for the attention of
// a chunk whose row m may use keys 0 .. first+m: kCausalKeysN skips the tiles whose keys
// (N) all lie past every row of the tile; kCausalKeysK stops the K loop of a tile after
// the last key any of its rows may use (A is zero beyond it).
enum { kCausalNone = 0, kCausalKeysN = 1, kCausalKeysK = 2 };

__global__ __launch_bounds__(256) void gemm_f32_kernel(const float* __restrict__ A, const float* __restrict__ B,
                                                      float* __restrict__ C, int M, int N, int K, int lda, int ldb,
                                                      int ldc, size_t sA, size_t sB, size_t sC, int bdiv, int causal,
                                                      int first) {
    __shared__ __align__(16) float As[2][GK][GM + GPAD];
    __shared__ __align__(16) float Bs[2][GK][GN + GPAD];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.y * GM, n0 = blockIdx.x * GN;
    if (causal == kCausalKeysN && n0 >= first + m0 + GM) return;  // whole workgroup, before any barrier
    if (causal == kCausalKeysK) K = min(K, (first + m0 + GM + GK - 1) / GK * GK);
    A += blockIdx.z * sA;
    B += (blockIdx.z / bdiv) * sB;
    C += blockIdx.z * sC;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    // global -> register staging of one 128 x 16 slice of A and of B: thread t loads
    // row t/2, columns 8*(t%2) .. +7 (two float4), zero outside the matrix
    const int lr = threadIdx.x >> 1, lc = (threadIdx.x & 1) * 8;
    float4 ra[2], rb[2];
    auto load_slice = [&](int k0) {
        const int am = m0 + lr, bn = n0 + lr;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            ra[h] = am < M ? *reinterpret_cast<const float4*>(A + (size_t)am * lda + k0 + lc + 4 * h)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
            rb[h] = bn < N ? *reinterpret_cast<const float4*>(B + (size_t)bn * ldb + k0 + lc + 4 * h)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store_slice = [&](int buf) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int k = lc + 4 * h;
            As[buf][k + 0][lr] = ra[h].x;
            As[buf][k + 1][lr] = ra[h].y;
            As[buf][k + 2][lr] = ra[h].z;
            As[buf][k + 3][lr] = ra[h].w;
            Bs[buf][k + 0][lr] = rb[h].x;
            Bs[buf][k + 1][lr] = rb[h].y;
            Bs[buf][k + 2][lr] = rb[h].z;
            Bs[buf][k + 3][lr] = rb[h].w;
        }
    };

    floatx16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int steps = K / GK;
    load_slice(0);
    store_slice(0);
    __syncthreads();
    for (int s = 0; s < steps; ++s) {
        const int buf = s & 1;
        if (s + 1 < steps) load_slice((s + 1) * GK);
#pragma unroll
        for (int kk = 0; kk < GK; kk += 2) {
            const int k = kk + (lane >> 5);
            float a[2], b[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                a[t] = As[buf][k][wm + 32 * t + (lane & 31)];
                b[t] = Bs[buf][k][wn + 32 * t + (lane & 31)];
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (s + 1 < steps) store_slice(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int col = n0 + wn + 32 * j + (lane & 31);
                if (row < M && col < N) C[(size_t)row * ldc + col] = acc[i][j][r];
            }
}

}  // namespace

hipError_t launch_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc,
                           hipStream_t stream) {
    if (M < 1 || N < 1 || K < GK || K % GK || lda % 4 || ldb % 4) return hipErrorInvalidValue;
    const dim3 grid((N + GN - 1) / GN, (M + GM - 1) / GM);
    launch_kernel(gemm_f32_kernel, grid, dim3(256), 0, stream, A, B, C, M, N, K, lda, ldb, ldc, (size_t)0, (size_t)0,
                  (size_t)0, 1, (int)kCausalNone, 0);
    return hipGetLastError();
}

hipError_t launch_gemm_f32_heads(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb,
                                 int ldc, int batch, int bdiv, size_t sA, size_t sB, size_t sC, bool causal_keys_n,
                                 bool causal_keys_k, int first, hipStream_t stream) {
    if (M < 1 || N < 1 || K < GK || K % GK || lda % 4 || ldb % 4 || batch < 1 || batch > 65535 || bdiv < 1 ||
        (causal_keys_n && causal_keys_k) || first < 0 || sA % 4 || sB % 4)
        return hipErrorInvalidValue;
    const dim3 grid((N + GN - 1) / GN, (M + GM - 1) / GM, batch);
    const int causal = causal_keys_n ? kCausalKeysN : causal_keys_k ? kCausalKeysK : kCausalNone;
    launch_kernel(gemm_f32_kernel, grid, dim3(256), 0, stream, A, B, C, M, N, K, lda, ldb, ldc, sA, sB, sC, bdiv,
                  causal, first);
    return hipGetLastError();
}

}  // namespace emprise
