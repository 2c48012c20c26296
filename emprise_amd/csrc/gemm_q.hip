// Prefill projections Y = X W^T with chunked Q6_K / Q4_K weights on the fp16 matrix cores
// (Backend::linear_batch, reference backend.hpp:20-24 / the CUDA linear_q6_f32_batch,
// cuda.cpp:350-413), for batches of 8 tokens and more.
//
// Both operands are exact in fp16 pieces, so the products are those of the FP32 path:
//
// - Weights. A Q6_K element is d * sc * (q - 32) with q a 6-bit code and sc an int8 unit
//   scale (quant.cpp:25-40); v = sc * (q - 32) is an integer of at most 13 bits, written
//   as v = vh + vl with vh = v truncated to fp16's 11 significant bits and vl = v - vh
//   (|vl| <= 1): both exact fp16. A Q4_K element is (d * sc) * q - dmin * m
//   (quant.cpp:41-61); v = sc * q is at most 63 * 15 = 945, exact in fp16 as it stands.
//   The block scales d (and dmin) of each 256 columns are applied in FP32 once per block.
// - Activations. Row m of X is scaled by a power of two 2^-e_m (exact) so that its largest
//   magnitude lies in [1, 2) -- no fp16 overflow whatever the activations -- and split
//   into xh = fp16(x) and xl = fp16(x - xh), which carry x to 22 significant bits.
//
// Per 256-column block the matrix cores accumulate, in FP32, sum v*xh + v*xl (+ vl*xh for
// Q6_K; the dropped vl*xl is below 2^-21 of the term) and the block adds d times that to
// the row's FP32 accumulator; for Q4_K the min term -dmin * sum_u m_u * (sum of x over
// unit u) is one more product per block, with the unit sums split the same way. The
// result is scaled back by 2^e_m. Only the rounding of the FP32 sums differs from the CPU
// path's sequential row sum.
//
// Tiling: a workgroup of 8 waves computes 128 tokens x 128 rows; wave w owns tokens
// 32*(w%4) .. +31 and rows 64*(w/4) .. +63 as two 32x32 v_mfma_f32_32x32x16_f16 tiles.
// The K loop takes 64 columns per step (a quarter of a block; in the chunked layout the
// 64 columns of matvec lane s of a chunk): the next step's split activations and raw
// weight words are loaded into registers while the matrix cores work on the current
// step from LDS, and each thread decodes its row's 16 (Q6_K) or 16-of-32 (Q4_K) codes of
// the step into fp16 while storing them.
//
// MFMA 32x32x16 f16 operand layout (lane l): A[i][k] with i = l % 32, k = 8*(l/32) + 0..7;
// B[k][j] with j = l % 32, the same k; D[i][j] in accumulator r with j = l % 32 and
// i = 8*(r/4) + 4*(l/32) + r%4.
#include "common.hpp"
#include "kernels.hpp"
#include "layout.hpp"

namespace emprise {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int QM = 128, QN = 128, QKS = 64, QROW = QKS + 8;  // LDS rows padded to 144 bytes
constexpr int QThreads = 512;

__device__ __forceinline__ uint32_t pack_rtz(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a, b));
}

// Loads through global-address-space pointers (global_load_*, counted by vmcnt only).
#define QGLOBAL __attribute__((address_space(1)))
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 gld16(const void* p) {
    const u32x4v v = *(const QGLOBAL u32x4v*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint32_t gld4(const void* p) { return *(const QGLOBAL uint32_t*)p; }
__device__ __forceinline__ uint32_t gld2(const void* p) { return *(const QGLOBAL uint16_t*)p; }
__device__ __forceinline__ uint32_t gld1(const void* p) { return *(const QGLOBAL uint8_t*)p; }

// ---- activations: fp16 hi/lo pieces of 2^-e_m * x, and (for Q4_K) of its 32-column sums ----

__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ X, int K, int ldx,
                                                         _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                         int* __restrict__ rexp, _Float16* __restrict__ sh,
                                                         _Float16* __restrict__ sl) {
    __shared__ float red[8];
    const int m = blockIdx.x;
    const float* x = X + (size_t)m * ldx;
    float mx = 0.f;
    for (int i = threadIdx.x; i < K; i += blockDim.x) mx = fmaxf(mx, fabsf(x[i]));
    mx = wave_max(mx);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    mx = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) mx = fmaxf(mx, red[w]);
    int e = 0;
    if (mx > 0.f && mx < INFINITY) {
        (void)frexpf(mx, &e);  // mx = f * 2^e with f in [0.5, 1)
        e -= 1;                // mx * 2^-e in [1, 2)
    }
    if (threadIdx.x == 0) rexp[m] = e;
    _Float16* ho = xh + (size_t)m * K;
    _Float16* lo = xl + (size_t)m * K;
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
        const float v = ldexpf(x[i], -e);
        const _Float16 h = (_Float16)v;
        ho[i] = h;
        lo[i] = (_Float16)(v - (float)h);
    }
    if (sh) {
        const int units = K / 32;
        for (int u = threadIdx.x; u < units; u += blockDim.x) {
            float s = 0.f;
            for (int k = 0; k < 32; ++k) s += ldexpf(x[u * 32 + k], -e);
            const _Float16 h = (_Float16)s;
            sh[(size_t)m * units + u] = h;
            sl[(size_t)m * units + u] = (_Float16)(s - (float)h);
        }
    }
}

// ---- the GEMM ------------------------------------------------------------------------

template <int T> struct QRaw;
template <> struct QRaw<kQ6K> {
    uint32_t d0, d1, d2;  // word j of the three code planes
    int32_t sc;           // the unit's int8 scale
    uint32_t d;           // fp16 block scale (read at a block's first step)
};
template <> struct QRaw<kQ4K> {
    uint4 q;      // the unit's 32 nibbles
    uint32_t s2;  // the lane's two scale bytes (low: unit 0)
    uint32_t m4;  // the lane's min nibbles (low: unit 0)
    uint32_t dd;  // fp16 d | fp16 dmin << 16
};

template <int T>
__global__ __launch_bounds__(QThreads) void gemm_q16_kernel(QGemmArgs a) {
    constexpr int NB = T == kQ6K ? 2 : 1;  // weight pieces
    __shared__ __align__(16) _Float16 As[2][QM][QROW];
    __shared__ __align__(16) _Float16 Bs[NB][QN][QROW];
    __shared__ float ds[QN], dms[QN];
    __shared__ __align__(16) _Float16 Ms[QN][8];  // Q4_K: -m of the block's 8 units

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, t = threadIdx.x;
    const int m0 = blockIdx.y * QM, n0 = blockIdx.x * QN;
    const int wm = (wave & 3) * 32, wn = (wave >> 2) * 64;
    const int steps = a.K / QKS, cpr = a.K / kChunkCols;

    // this thread's loads of a step: activations row ar (piece ap), columns ac .. ac+31;
    // weights row bn = n0 + t/4, part bj = t%4 (Q6_K: unit bj; Q4_K: unit bj/2, half bj%2)
    const int ap = t >> 8, ar = (t & 255) >> 1, ac = (t & 1) * 32;
    const bool a_ok = m0 + ar < a.M;
    const uint16_t* asrc = (ap ? a.xl : a.xh) + (size_t)(a_ok ? m0 + ar : 0) * a.K + ac;
    const int bl = t >> 2, bj = t & 3, bn = n0 + bl;
    const bool b_ok = bn < a.N;
    // (rows past N read row 0 and are zeroed)
    const uint8_t* brow;
    {
        const int r = b_ok ? bn : 0;
        int s = 0;
        while (s + 1 < a.nseg && r >= a.row0[s + 1]) ++s;
        constexpr size_t kChunk = T == kQ6K ? 3360 : 2304;
        brow = a.w[s] + (size_t)(r - a.row0[s]) * cpr * kChunk;
    }

    uint4 ra[4];
    QRaw<T> rb;
    auto load_step = [&](int s) {
        const int k0 = s * QKS;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            ra[i] = gld16(asrc + k0 + 8 * i);  // row clamped in range; zeroed past M
            if (!a_ok) ra[i] = make_uint4(0, 0, 0, 0);
        }
        const int c = k0 / kChunkCols, ls = (k0 % kChunkCols) / QKS;  // chunk, matvec lane
        if constexpr (T == kQ6K) {
            const uint8_t* base = brow + (size_t)c * 3360;
            rb.d0 = gld4(base + 16 * ls + 4 * bj);
            rb.d1 = gld4(base + 1024 + 16 * ls + 4 * bj);
            rb.d2 = gld4(base + 2048 + 16 * ls + 4 * bj);
            rb.sc = (int8_t)gld1(base + 3072 + 4 * ls + bj);
            rb.d = gld2(base + 3328 + 2 * (ls >> 2));
            if (!b_ok) rb = {0u, 0u, 0u, 0, 0u};
        } else {
            const uint8_t* base = brow + (size_t)c * 2304;
            const int p = bj >> 1;
            rb.q = gld16(base + 1024 * p + 16 * ls);
            const uint8_t* sb = base + 2048 + 12 * (ls >> 2);
            rb.s2 = gld2(sb + 2 * (ls & 3));
            rb.m4 = gld1(sb + 8 + (ls & 3));
            rb.dd = gld4(base + 2240 + 4 * (ls >> 2));
            if (!b_ok) {
                rb.q = make_uint4(0, 0, 0, 0);
                rb.s2 = rb.m4 = rb.dd = 0u;
            }
        }
    };

    // registers -> LDS: the activation pieces as they are, the weights decoded to fp16
    auto store_step = [&](int s) {
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(&As[ap][ar][ac + 8 * i]) = ra[i];
        const bool block_start = (s & 3) == 0;
        if constexpr (T == kQ6K) {
            // unit bj: codes 0..3 in the low 6 bits of d0, 4..7 of d1, 8..11 of d2, and
            // 12..15 gathered from their top two bits
            const uint32_t w[4] = {rb.d0 & 0x3F3F3F3Fu, rb.d1 & 0x3F3F3F3Fu, rb.d2 & 0x3F3F3F3Fu,
                                   ((rb.d0 >> 6) & 0x03030303u) | ((rb.d1 >> 4) & 0x0C0C0C0Cu) |
                                       ((rb.d2 >> 2) & 0x30303030u)};
            const float scf = (float)rb.sc, zp = -32.f * scf;
            uint32_t hi[8], lo[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    // v = sc * (q - 32), exact in FP32; vh keeps its top 11 significant bits
                    const float v0 = fmaf(ubyte_f(w[k], 2 * h), scf, zp), v1 = fmaf(ubyte_f(w[k], 2 * h + 1), scf, zp);
                    const float h0 = __uint_as_float(__float_as_uint(v0) & 0xFFFFE000u);
                    const float h1 = __uint_as_float(__float_as_uint(v1) & 0xFFFFE000u);
                    hi[2 * k + h] = pack_rtz(h0, h1);
                    lo[2 * k + h] = pack_rtz(v0 - h0, v1 - h1);
                }
            }
            _Float16* dh = &Bs[0][bl][16 * bj];
            _Float16* dl = &Bs[1][bl][16 * bj];
            *reinterpret_cast<uint4*>(dh) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
            *reinterpret_cast<uint4*>(dh + 8) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
            *reinterpret_cast<uint4*>(dl) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            *reinterpret_cast<uint4*>(dl + 8) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
            if (block_start && bj == 0) ds[bl] = half_bits_to_float((uint16_t)rb.d);
        } else {
            // unit p = bj/2 of the step: codes 0..15 in the low nibbles of its four words,
            // 16..31 in the high ones; this thread's half is bj%2
            const int p = bj >> 1, hf = bj & 1;
            const uint32_t b = (rb.s2 >> (8 * p)) & 0xffu;
            const float scf = (float)(b & 63u);
            const uint32_t wv[4] = {rb.q.x, rb.q.y, rb.q.z, rb.q.w};
            uint32_t pk[8];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint32_t nib = (wv[k] >> (4 * hf)) & 0x0F0F0F0Fu;
                pk[2 * k] = pack_rtz(ubyte_f(nib, 0) * scf, ubyte_f(nib, 1) * scf);
                pk[2 * k + 1] = pack_rtz(ubyte_f(nib, 2) * scf, ubyte_f(nib, 3) * scf);
            }
            _Float16* dh = &Bs[0][bl][32 * p + 16 * hf];
            *reinterpret_cast<uint4*>(dh) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            *reinterpret_cast<uint4*>(dh + 8) = make_uint4(pk[4], pk[5], pk[6], pk[7]);
            if (hf == 0) {
                const uint32_t mn = ((b >> 6) << 4) | ((rb.m4 >> (4 * p)) & 15u);
                Ms[bl][2 * (s & 3) + p] = (_Float16)(-(float)mn);
            }
            if (block_start && bj == 0) {
                ds[bl] = half_bits_to_float((uint16_t)(rb.dd & 0xffffu));
                dms[bl] = half_bits_to_float((uint16_t)(rb.dd >> 16));
            }
        }
    };

    floatx16 acc[2], cb[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[nb][r] = cb[nb][r] = 0.f;
    const int fr = lane & 31, fk = 8 * (lane >> 5);  // fragment row/column and k offset

    load_step(0);
    for (int s = 0; s < steps; ++s) {
        __syncthreads();  // the previous step's fragments and block scales have been read
        store_step(s);
        __syncthreads();
        if (s + 1 < steps) load_step(s + 1);
#pragma unroll
        for (int q = 0; q < QKS / 16; ++q) {
            const half8 xh = *reinterpret_cast<const half8*>(&As[0][wm + fr][16 * q + fk]);
            const half8 xl = *reinterpret_cast<const half8*>(&As[1][wm + fr][16 * q + fk]);
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int n = wn + 32 * nb + fr;
                const half8 wh = *reinterpret_cast<const half8*>(&Bs[0][n][16 * q + fk]);
                cb[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, wh, cb[nb], 0, 0, 0);
                cb[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xl, wh, cb[nb], 0, 0, 0);
                if constexpr (T == kQ6K) {
                    const half8 wl = *reinterpret_cast<const half8*>(&Bs[NB - 1][n][16 * q + fk]);
                    cb[nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xh, wl, cb[nb], 0, 0, 0);
                }
            }
        }
        if ((s & 3) == 3) {
            // block end: acc += d * (block products); Q4_K also adds -dmin * sum_u m_u * xsum_u
            half8 sh8 = {}, sl8 = {};
            if constexpr (T == kQ4K) {
                // lanes 0..31: units 0..7 of the block for token m; lanes 32..63: zero (k 8..15)
                const int m = m0 + wm + fr, blk = s >> 2;
                const bool ok = lane < 32 && m < a.M;
                const size_t o = (size_t)(m < a.M ? m : 0) * (a.K / 32) + 8 * blk;
                uint4 hv = gld16(a.sh + o), lv = gld16(a.sl + o);
                if (!ok) hv = lv = make_uint4(0, 0, 0, 0);
                sh8 = __builtin_bit_cast(half8, hv);
                sl8 = __builtin_bit_cast(half8, lv);
            }
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int n = wn + 32 * nb + fr;
                const float d = ds[n];
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    acc[nb][r] = fmaf(d, cb[nb][r], acc[nb][r]);
                    cb[nb][r] = 0.f;
                }
                if constexpr (T == kQ4K) {
                    uint4 mr = *reinterpret_cast<const uint4*>(&Ms[n][0]);
                    if (lane >= 32) mr = make_uint4(0, 0, 0, 0);
                    const half8 mv = __builtin_bit_cast(half8, mr);
                    floatx16 cm = {};
                    cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh8, mv, cm, 0, 0, 0);
                    cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(sl8, mv, cm, 0, 0, 0);
                    const float dm = dms[n];
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[nb][r] = fmaf(dm, cm[r], acc[nb][r]);
                }
            }
        }
    }

    // Y[m][n] = 2^e_m * acc
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int n = n0 + wn + 32 * nb + fr;
        if (n >= a.N) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int m = m0 + wm + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
            if (m < a.M) a.y[(size_t)m * a.ldy + n] = ldexpf(acc[nb][r], a.rexp[m]);
        }
    }
}

}  // namespace

size_t gemm_q16_split_bytes(int M, int K, bool sums) {
    size_t b = (size_t)M * K * 2 * sizeof(_Float16) + (size_t)M * sizeof(int);
    if (sums) b += (size_t)M * (K / 32) * 2 * sizeof(_Float16);
    return (b + 255) / 256 * 256;
}

hipError_t launch_gemm_q16_split(const float* X, int M, int K, int ldx, void* scratch, bool sums, QGemmArgs* a,
                                 hipStream_t stream) {
    if (M < 1 || K < QKS || K % kChunkCols || ldx < K) return hipErrorInvalidValue;
    _Float16* xh = static_cast<_Float16*>(scratch);
    _Float16* xl = xh + (size_t)M * K;
    int* rexp = reinterpret_cast<int*>(xl + (size_t)M * K);
    _Float16* sh = sums ? reinterpret_cast<_Float16*>(rexp + M) : nullptr;
    _Float16* sl = sums ? sh + (size_t)M * (K / 32) : nullptr;
    launch_kernel(split_rows_kernel, dim3(M), dim3(256), 0, stream, X, K, ldx, xh, xl, rexp, sh, sl);
    a->xh = reinterpret_cast<const uint16_t*>(xh);
    a->xl = reinterpret_cast<const uint16_t*>(xl);
    a->rexp = rexp;
    a->sh = reinterpret_cast<const uint16_t*>(sh);
    a->sl = reinterpret_cast<const uint16_t*>(sl);
    a->M = M;
    a->K = K;
    return hipGetLastError();
}

hipError_t launch_gemm_q16(uint32_t type, const QGemmArgs& a, hipStream_t stream) {
    if ((type != kQ6K && type != kQ4K) || a.M < 1 || a.N < 1 || a.K % kChunkCols || a.nseg < 1 || a.nseg > kMaxSeg ||
        a.row0[0] != 0 || a.row0[a.nseg] != a.N || a.ldy < a.N || (type == kQ4K && !a.sh))
        return hipErrorInvalidValue;
    const dim3 grid((a.N + QN - 1) / QN, (a.M + QM - 1) / QM);
    if (grid.y > 65535) return hipErrorInvalidValue;
    if (type == kQ6K) launch_kernel(gemm_q16_kernel<kQ6K>, grid, dim3(QThreads), 0, stream, a);
    else launch_kernel(gemm_q16_kernel<kQ4K>, grid, dim3(QThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace emprise
