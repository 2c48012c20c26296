// Prefill projections Y = X W^T with chunked Q6_K / Q4_K weights on the fp16 matrix cores
// (Backend::linear_batch, reference backend.hpp:20-24 / the CUDA linear_q6_f32_batch,
// cuda.cpp:350-413), for batches of 8 tokens and more.
//
// Both operands are exact in fp16 pieces, so the products are those of the FP32 path:
//
// - Weights. A Q6_K element is d * sc * (q - 32) with q a 6-bit code and sc an int8 unit
//   scale (quant.cpp:25-40); v = sc * (q - 32) is an integer of at most 13 bits, written
//   as v = vh + vl with vh = v rounded to fp16 and vl = v - vh (|vl| <= 1): both exact
//   fp16. A Q4_K element is (d * sc) * q - dmin * m (quant.cpp:41-61); v = sc * q is at
//   most 63 * 15 = 945, exact in fp16 as it stands. The block scales d (and dmin) of each
//   256 columns are applied in FP32 once per block. The staging waves decode in packed
//   fp16 arithmetic, every step exact (below).
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
// Tiling: a workgroup of 8 waves computes 128 tokens x 128 rows. Waves 0..3 multiply:
// wave c owns tokens 64*(c%2) .. +63 and rows 64*(c/2) .. +63 as 2 x 2 tiles of
// v_mfma_f32_32x32x16_f16. Waves 4..7 stage: the K loop takes 64 columns per step (a
// quarter of a block; in the chunked layout the 64 columns of matvec lane s of a chunk)
// from two LDS buffers, and while the multiplying waves run step s from one, the staging
// waves decode step s+1's codes into fp16, store them with the activation pieces into the
// other and issue the global loads of step s+3 (two register sets in turn); one barrier
// per step.
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

// The pieces are stored tile by tile, in the order the GEMM reads them: tile (m/128,
// k/64) is 128 x 64 halves, row-major, so a step's activation tile is one contiguous
// 16 KiB run per piece. Rows from M up to the next multiple of 128 are zero.
__device__ __forceinline__ size_t tiled(int m, int k, int K) {
    return ((size_t)(m >> 7) * (K >> 6) + (k >> 6)) * (128 * 64) + (m & 127) * 64 + (k & 63);
}

__global__ __launch_bounds__(256) void split_rows_kernel(const float* __restrict__ X, int M, int K, int ldx,
                                                         _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                         int* __restrict__ rexp, _Float16* __restrict__ sh,
                                                         _Float16* __restrict__ sl) {
    __shared__ float red[8];
    const int m = blockIdx.x;
    if (m >= M) {  // padding rows of the last tile
        for (int i = threadIdx.x; i < K; i += blockDim.x) xh[tiled(m, i, K)] = xl[tiled(m, i, K)] = (_Float16)0.f;
        return;
    }
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
    for (int i = threadIdx.x; i < K; i += blockDim.x) {
        const float v = ldexpf(x[i], -e);
        const _Float16 h = (_Float16)v;
        xh[tiled(m, i, K)] = h;
        xl[tiled(m, i, K)] = (_Float16)(v - (float)h);
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

// The same split for 16-byte aligned rows of P * 2048 columns: lane t of pass p holds
// columns 8(256p + t) .. +7 in registers from the row maximum to the stores (two 16-byte
// loads, one 16-byte store per piece), and a Q4_K unit's 32 columns are a DPP quad: each
// lane sums its 8 values in column order, the quad adds the pairs (s0 + s1) + (s2 + s3).
template <int P>
__global__ __launch_bounds__(256) void split_rows8_kernel(const float* __restrict__ X, int M, int K, int ldx,
                                                          _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                          int* __restrict__ rexp, _Float16* __restrict__ sh,
                                                          _Float16* __restrict__ sl) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    __shared__ float red[4];
    const int m = blockIdx.x, t = threadIdx.x;
    if (m >= M) {  // padding rows of the last tile
        const half8 z = {};
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const size_t o = tiled(m, 8 * (256 * p + t), K);
            *reinterpret_cast<half8*>(xh + o) = z;
            *reinterpret_cast<half8*>(xl + o) = z;
        }
        return;
    }
    const float* x = X + (size_t)m * ldx;
    f4v v[P][2];
    float mx = 0.f;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const f4v* src = reinterpret_cast<const f4v*>(x + 8 * (256 * p + t));
        v[p][0] = src[0];
        v[p][1] = src[1];
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, fmaxf(fabsf(v[p][0][i]), fabsf(v[p][1][i])));
    }
    mx = wave_max(mx);
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.f && mx < INFINITY) {
        (void)frexpf(mx, &e);  // mx = f * 2^e with f in [0.5, 1)
        e -= 1;                // mx * 2^-e in [1, 2)
    }
    if (t == 0) rexp[m] = e;
    const int units = K / 32;
#pragma unroll
    for (int p = 0; p < P; ++p) {
        half8 h8, l8;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float w = ldexpf(v[p][i >> 2][i & 3], -e);
            const _Float16 h = (_Float16)w;
            h8[i] = h;
            l8[i] = (_Float16)(w - (float)h);
            s += w;
        }
        const size_t o = tiled(m, 8 * (256 * p + t), K);
        *reinterpret_cast<half8*>(xh + o) = h8;
        *reinterpret_cast<half8*>(xl + o) = l8;
        if (sh) {
            s += dpp_f<0xb1, 0xf>(0.f, s);  // quad_perm [1,0,3,2]: s0 + s1, s2 + s3
            s += dpp_f<0x4e, 0xf>(0.f, s);  // quad_perm [2,3,0,1]
            if ((t & 3) == 0) {
                const int u = (256 * p + t) >> 2;
                const _Float16 h = (_Float16)s;
                sh[(size_t)m * units + u] = h;
                sl[(size_t)m * units + u] = (_Float16)(s - (float)h);
            }
        }
    }
}

// ---- the GEMM ------------------------------------------------------------------------

template <int T> struct QRaw;
template <> struct QRaw<kQ6K> {
    uint2 d0, d1, d2;  // words j0, j0+1 of the three code planes (units j0, j0+1)
    uint32_t sc;       // the two units' int8 scales (low byte: unit j0)
    uint32_t d;        // fp16 block scale (used at a block's first step)
};
template <> struct QRaw<kQ4K> {
    uint4 q;      // the unit's 32 nibbles
    uint32_t s2;  // the lane's two scale bytes (low: unit 0)
    uint32_t m4;  // the lane's min nibbles (low: unit 0)
    uint32_t dd;  // fp16 d | fp16 dmin << 16
};

typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Two code bytes (bytes 0, 1 of w, or 2, 3 with hi) as the fp16 pair 1024 + q: each byte
// under an exponent byte 0x64 (v_perm_b32), which makes 1024 + q exact for q < 1024.
__device__ __forceinline__ half2v codes_1024(uint32_t w, bool hi) {
    return __builtin_bit_cast(half2v, __builtin_amdgcn_perm(0x64646464u, w, hi ? 0x04030402u : 0x04010400u));
}

// Q6_K unit -> fp16 pieces: codes 0..3 in the low 6 bits of word d0, 4..7 of d1, 8..11 of
// d2, 12..15 gathered from their top two bits. In packed fp16 arithmetic, each step exact:
// q - 32 = (1024 + q) - 1056; vh = fp16(v), v = sc * (q - 32); vl = fma(q - 32, sc, -vh),
// a small integer (|vl| <= 1). Two weights per instruction, about half the instructions
// of the same split in FP32.
__device__ __forceinline__ void q6_unit_f16(uint32_t d0, uint32_t d1, uint32_t d2, int sc, _Float16* dh,
                                            _Float16* dl) {
    const uint32_t w[4] = {d0 & 0x3F3F3F3Fu, d1 & 0x3F3F3F3Fu, d2 & 0x3F3F3F3Fu,
                           ((d0 >> 6) & 0x03030303u) | ((d1 >> 4) & 0x0C0C0C0Cu) | ((d2 >> 2) & 0x30303030u)};
    const _Float16 s16 = (_Float16)(float)sc;
    const half2v sc2 = {s16, s16}, off = {(_Float16)-1056.f, (_Float16)-1056.f};
    uint32_t hi[8], lo[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const half2v q = codes_1024(w[k], h) + off;
            const half2v vh = q * sc2;
            const half2v vl = __builtin_elementwise_fma(q, sc2, -vh);
            hi[2 * k + h] = __builtin_bit_cast(uint32_t, vh);
            lo[2 * k + h] = __builtin_bit_cast(uint32_t, vl);
        }
    }
    *reinterpret_cast<uint4*>(dh) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
    *reinterpret_cast<uint4*>(dh + 8) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
    *reinterpret_cast<uint4*>(dl) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    *reinterpret_cast<uint4*>(dl + 8) = make_uint4(lo[4], lo[5], lo[6], lo[7]);
}

// Waves 0..3 multiply, waves 4..7 stage: with two LDS buffers and one barrier per step, the
// staging waves decode and store step s+1 (and load step s+2) while the multiplying waves
// run step s, so the weight decode, the LDS traffic and the matrix cores overlap.
template <int T>
__global__ __launch_bounds__(QThreads) void gemm_q16_kernel(QGemmArgs a) {
    constexpr int NB = T == kQ6K ? 2 : 1;   // weight pieces
    constexpr int NQ = T == kQ4K ? QN : 1;  // Q4_K-only arrays
    // step s is read from buffer s%2 while step s+1 is stored into the other; the block
    // scales and Q4_K mins by block parity
    __shared__ __align__(16) _Float16 As[2][2][QM][QROW];
    __shared__ __align__(16) _Float16 Bs[2][NB][QN][QROW];
    __shared__ float ds[2][QN], dms[2][NQ];
    __shared__ __align__(16) _Float16 Ms[2][NQ][8];  // Q4_K: -m of the block's 8 units

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m0 = blockIdx.y * QM, n0 = blockIdx.x * QN;
    const int steps = a.K / QKS, cpr = a.K / kChunkCols;
    const bool stager = wave >= 4;

    if (stager) {
        // ---- staging waves: thread pt loads and stores four 16-byte pieces of each
        // activation tile, and weight row pr, units 2*(pt%2), +1 (Q6_K) or unit pt%2 (Q4_K,
        // both halves)
        const int pt = threadIdx.x - 256, pr = pt >> 1, ph = pt & 1;
        const size_t abase = (size_t)blockIdx.y * steps * (QM * QKS);  // the tile row's first step
        const int bn = n0 + pr;
        const bool b_ok = bn < a.N;
        const uint8_t* brow;  // (rows past N read row 0 and are zeroed)
        {
            const int r = b_ok ? bn : 0;
            constexpr size_t kChunk = T == kQ6K ? 3360 : 2304;
            if (a.pair) {
                brow = a.w[r & 1] + (size_t)(r >> 1) * cpr * kChunk;
            } else {
                int sg = 0;
                while (sg + 1 < a.nseg && r >= a.row0[sg + 1]) ++sg;
                brow = a.w[sg] + (size_t)(r - a.row0[sg]) * cpr * kChunk;
            }
        }
        // two register sets in turn (step k in set k%2): the loads of step k go out two
        // steps before it is stored; every load is issued whatever the step (past the last
        // step it re-reads the last one), so the waits for a set never cover the other's
        struct Regs {
            uint4 rh[4], rl[4];
            QRaw<T> rb;
        } R0, R1;
        auto load_step = [&](int s, Regs& R) {
            uint4* rh = R.rh;
            uint4* rl = R.rl;
            QRaw<T>& rb = R.rb;
            s = min(s, steps - 1);
            const int k0 = s * QKS;
            // the step's 128 x 64 tile of each piece: 16 KiB in a row, 16 bytes per thread
            // and load, a wave's load 1 KiB in a row
            const size_t at = abase + (size_t)s * (QM * QKS);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                rh[i] = gld16(a.xh + at + 8 * (i * 256 + pt));
                rl[i] = gld16(a.xl + at + 8 * (i * 256 + pt));
            }
            const int c = k0 / kChunkCols, ls = (k0 % kChunkCols) / QKS;  // chunk, matvec lane
            if constexpr (T == kQ6K) {
                const uint8_t* base = brow + (size_t)c * 3360 + 16 * ls + 8 * ph;
                const uint32_t x0 = gld4(base), x1 = gld4(base + 4);
                const uint32_t y0 = gld4(base + 1024), y1 = gld4(base + 1028);
                const uint32_t z0 = gld4(base + 2048), z1 = gld4(base + 2052);
                rb.d0 = make_uint2(x0, x1);
                rb.d1 = make_uint2(y0, y1);
                rb.d2 = make_uint2(z0, z1);
                rb.sc = gld2(brow + (size_t)c * 3360 + 3072 + 4 * ls + 2 * ph);
                rb.d = gld2(brow + (size_t)c * 3360 + 3328 + 2 * (ls >> 2));
                if (!b_ok) rb = {make_uint2(0, 0), make_uint2(0, 0), make_uint2(0, 0), 0u, 0u};
            } else {
                const uint8_t* base = brow + (size_t)c * 2304;
                rb.q = gld16(base + 1024 * ph + 16 * ls);
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
        // registers -> LDS buffer `buf`: the activation pieces as they are, the weights
        // decoded to fp16
        auto store_step = [&](int s, int buf, const Regs& R) {
            const uint4* rh = R.rh;
            const uint4* rl = R.rl;
            const QRaw<T>& rb = R.rb;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int e = i * 256 + pt;  // 16-byte piece e: row e/8, columns 8*(e%8) ..
                *reinterpret_cast<uint4*>(&As[buf][0][e >> 3][8 * (e & 7)]) = rh[i];
                *reinterpret_cast<uint4*>(&As[buf][1][e >> 3][8 * (e & 7)]) = rl[i];
            }
            const bool block_start = (s & 3) == 0;
            const int bp = (s >> 2) & 1;
            if constexpr (T == kQ6K) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int j = 2 * ph + u;
                    q6_unit_f16(u ? rb.d0.y : rb.d0.x, u ? rb.d1.y : rb.d1.x, u ? rb.d2.y : rb.d2.x,
                                (int)(int8_t)(rb.sc >> (8 * u)), &Bs[buf][0][pr][16 * j], &Bs[buf][NB - 1][pr][16 * j]);
                }
                if (block_start && ph == 0) ds[bp][pr] = half_bits_to_float((uint16_t)rb.d);
            } else {
                // unit p = ph of the step: codes 0..15 in the low nibbles of its four words,
                // 16..31 in the high ones
                const uint32_t b = (rb.s2 >> (8 * ph)) & 0xffu;
                const float scf = (float)(b & 63u);
                const uint32_t wv[4] = {rb.q.x, rb.q.y, rb.q.z, rb.q.w};
                // v = (1024 + q) * sc - 1024 * sc in one fused step: exact, the product below
                // 1039 * 63 < 65504 and the result at most 945
                const _Float16 s16 = (_Float16)scf;
                const half2v sc2 = {s16, s16}, base = {(_Float16)(-1024.f * scf), (_Float16)(-1024.f * scf)};
#pragma unroll
                for (int hf = 0; hf < 2; ++hf) {
                    uint32_t pk[8];
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t nib = (wv[k] >> (4 * hf)) & 0x0F0F0F0Fu;
#pragma unroll
                        for (int h = 0; h < 2; ++h)
                            pk[2 * k + h] = __builtin_bit_cast(
                                uint32_t, __builtin_elementwise_fma(codes_1024(nib, h), sc2, base));
                    }
                    _Float16* dh = &Bs[buf][0][pr][32 * ph + 16 * hf];
                    *reinterpret_cast<uint4*>(dh) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
                    *reinterpret_cast<uint4*>(dh + 8) = make_uint4(pk[4], pk[5], pk[6], pk[7]);
                }
                const uint32_t mn = ((b >> 6) << 4) | ((rb.m4 >> (4 * ph)) & 15u);
                Ms[bp][pr % NQ][2 * (s & 3) + ph] = (_Float16)(-(float)mn);
                if (block_start && ph == 0) {
                    ds[bp][pr] = half_bits_to_float((uint16_t)(rb.dd & 0xffffu));
                    dms[bp][pr % NQ] = half_bits_to_float((uint16_t)(rb.dd >> 16));
                }
            }
        };
        // (steps is even: K is a multiple of 4096)
        load_step(0, R0);
        load_step(1, R1);
        store_step(0, 0, R0);
        load_step(2, R0);
        __syncthreads();
        for (int s = 0; s < steps; s += 2) {
            if (s + 1 < steps) store_step(s + 1, 1, R1);
            load_step(s + 3, R1);
            __syncthreads();
            if (s + 2 < steps) store_step(s + 2, 0, R0);
            load_step(s + 4, R0);
            __syncthreads();
        }
        return;
    }

    // ---- multiplying waves: wave c owns tokens 64*(c%2) .. +63 and rows 64*(c/2) .. +63
    // as 2 x 2 tiles of 32 x 32
    const int wm = (wave & 1) * 64, wn = (wave >> 1) * 64;
    const int fr = lane & 31, fk = 8 * (lane >> 5);  // fragment row/column and k offset
    floatx16 acc[2][2], cb[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = cb[i][j][r] = 0.f;
    half8 sh8[2] = {}, sl8[2] = {};  // Q4_K: the block's unit sums (lanes 0..31; 32..63 zero)
    __syncthreads();
    for (int s = 0; s < steps; ++s) {
        const int buf = s & 1;
        if (T == kQ4K && (s & 3) == 0) {
#pragma unroll
            for (int mb = 0; mb < 2; ++mb) {
                const int m = m0 + wm + 32 * mb + fr, blk = s >> 2;
                const bool ok = lane < 32 && m < a.M;
                const size_t o = (size_t)(m < a.M ? m : 0) * (a.K / 32) + 8 * blk;
                uint4 hv = gld16(a.sh + o), lv = gld16(a.sl + o);
                if (!ok) hv = lv = make_uint4(0, 0, 0, 0);
                sh8[mb] = __builtin_bit_cast(half8, hv);
                sl8[mb] = __builtin_bit_cast(half8, lv);
            }
        }
        // fragments of 16-column slice q, read one slice ahead of its products; the products
        // go out piece by piece over the four tiles, so consecutive MFMAs never depend on
        // each other
        half8 fx[2][2][2], fw[2][2][NB];  // [slice parity][tile][piece]
        auto frags = [&](int q, int f) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                fx[f][i][0] = *reinterpret_cast<const half8*>(&As[buf][0][wm + 32 * i + fr][16 * q + fk]);
                fx[f][i][1] = *reinterpret_cast<const half8*>(&As[buf][1][wm + 32 * i + fr][16 * q + fk]);
#pragma unroll
                for (int pc = 0; pc < NB; ++pc)
                    fw[f][i][pc] = *reinterpret_cast<const half8*>(&Bs[buf][pc][wn + 32 * i + fr][16 * q + fk]);
            }
        };
        frags(0, 0);
#pragma unroll
        for (int q = 0; q < QKS / 16; ++q) {
            const int f = q & 1;
            if (q + 1 < QKS / 16) frags(q + 1, f ^ 1);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    cb[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fx[f][mb][0], fw[f][nb][0], cb[mb][nb], 0, 0, 0);
#pragma unroll
            for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    cb[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fx[f][mb][1], fw[f][nb][0], cb[mb][nb], 0, 0, 0);
            if constexpr (T == kQ6K) {
#pragma unroll
                for (int mb = 0; mb < 2; ++mb)
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb)
                        cb[mb][nb] =
                            __builtin_amdgcn_mfma_f32_32x32x16_f16(fx[f][mb][0], fw[f][nb][NB - 1], cb[mb][nb], 0, 0, 0);
            }
        }
        if ((s & 3) == 3) {
            // block end: acc += d * (block products); Q4_K also adds -dmin * sum_u m_u * xsum_u
            const int bp = (s >> 2) & 1;
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int n = wn + 32 * nb + fr;
                const float d = ds[bp][n];
                half8 mv = {};
                float dm = 0.f;
                if constexpr (T == kQ4K) {
                    uint4 mr = *reinterpret_cast<const uint4*>(&Ms[bp][n % NQ][0]);
                    if (lane >= 32) mr = make_uint4(0, 0, 0, 0);
                    mv = __builtin_bit_cast(half8, mr);
                    dm = dms[bp][n % NQ];
                }
#pragma unroll
                for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        acc[mb][nb][r] = fmaf(d, cb[mb][nb][r], acc[mb][nb][r]);
                        cb[mb][nb][r] = 0.f;
                    }
                    if constexpr (T == kQ4K) {
                        floatx16 cm = {};
                        cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(sh8[mb], mv, cm, 0, 0, 0);
                        cm = __builtin_amdgcn_mfma_f32_32x32x16_f16(sl8[mb], mv, cm, 0, 0, 0);
#pragma unroll
                        for (int r = 0; r < 16; ++r) acc[mb][nb][r] = fmaf(dm, cm[r], acc[mb][nb][r]);
                    }
                }
            }
        }
        __syncthreads();
    }

    // Y[m][n] = 2^e_m * acc. SwiGLU pairs: the gate (even n) and up (odd n) of one output sit
    // in adjacent lanes; of accumulators r, r+1 (rows m, m+1) the even lane writes row m and
    // the odd lane row m+1, each receiving the one value it lacks through a lane swap, so
    // every lane evaluates one silu(gate) * up (swiglu_kernel's form) per two entries.
    const bool odd = fr & 1;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int n = n0 + wn + 32 * nb + fr;
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const int m = m0 + wm + 32 * mb + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                const float v0 = ldexpf(acc[mb][nb][r], a.rexp[min(m, a.M - 1)]);
                const float v1 = ldexpf(acc[mb][nb][r + 1], a.rexp[min(m + 1, a.M - 1)]);
                if (a.pair) {
                    const float recv = dpp_f<0xb1, 0xf>(0.f, odd ? v0 : v1);  // quad_perm [1,0,3,2]
                    const float gate = odd ? recv : v0, up = odd ? v1 : recv;
                    const int mo = odd ? m + 1 : m;
                    if (mo < a.M && n < a.N) a.y[(size_t)mo * a.ldy + (n >> 1)] = siluf_(gate) * up;
                } else if (n < a.N) {
                    if (m < a.M) a.y[(size_t)m * a.ldy + n] = v0;
                    if (m + 1 < a.M) a.y[(size_t)(m + 1) * a.ldy + n] = v1;
                }
            }
        }
}

}  // namespace

size_t gemm_q16_split_bytes(int M, int K, bool sums) {
    const size_t mp = (size_t)(M + QM - 1) / QM * QM;  // rows padded to whole tiles
    size_t b = mp * K * 2 * sizeof(_Float16) + (size_t)M * sizeof(int);
    if (sums) b += (size_t)M * (K / 32) * 2 * sizeof(_Float16);
    return (b + 255) / 256 * 256;
}

hipError_t launch_gemm_q16_split(const float* X, int M, int K, int ldx, void* scratch, bool sums, QGemmArgs* a,
                                 hipStream_t stream) {
    if (M < 1 || K < QKS || K % kChunkCols || ldx < K) return hipErrorInvalidValue;
    const int mp = (M + QM - 1) / QM * QM;
    _Float16* xh = static_cast<_Float16*>(scratch);
    _Float16* xl = xh + (size_t)mp * K;
    int* rexp = reinterpret_cast<int*>(xl + (size_t)mp * K);
    _Float16* sh = sums ? reinterpret_cast<_Float16*>(rexp + M) : nullptr;
    _Float16* sl = sums ? sh + (size_t)M * (K / 32) : nullptr;
    const bool v16 = reinterpret_cast<uintptr_t>(X) % 16 == 0 && ldx % 4 == 0;
    if (v16 && K == 4096)
        launch_kernel(split_rows8_kernel<2>, dim3(mp), dim3(256), 0, stream, X, M, K, ldx, xh, xl, rexp, sh, sl);
    else if (v16 && K == 8192)
        launch_kernel(split_rows8_kernel<4>, dim3(mp), dim3(256), 0, stream, X, M, K, ldx, xh, xl, rexp, sh, sl);
    else if (v16 && K == 12288)
        launch_kernel(split_rows8_kernel<6>, dim3(mp), dim3(256), 0, stream, X, M, K, ldx, xh, xl, rexp, sh, sl);
    else
        launch_kernel(split_rows_kernel, dim3(mp), dim3(256), 0, stream, X, M, K, ldx, xh, xl, rexp, sh, sl);
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
        a.row0[0] != 0 || a.row0[a.nseg] != a.N || (type == kQ4K && !a.sh))
        return hipErrorInvalidValue;
    if (a.pair ? (a.nseg != 2 || a.N % 2 || a.row0[1] * 2 != a.N || a.ldy < a.N / 2) : a.ldy < a.N)
        return hipErrorInvalidValue;
    const dim3 grid((a.N + QN - 1) / QN, (a.M + QM - 1) / QM);
    if (grid.y > 65535) return hipErrorInvalidValue;
    if (type == kQ6K) launch_kernel(gemm_q16_kernel<kQ6K>, grid, dim3(QThreads), 0, stream, a);
    else launch_kernel(gemm_q16_kernel<kQ4K>, grid, dim3(QThreads), 0, stream, a);
    return hipGetLastError();
}

}  // namespace emprise
