// Dequant-matvec kernels for batch-1 decode on gfx950.
//
// One launch computes up to kMaxSeg projections that share one input vector
// (Backend::linear / linear_many / the gate+up half of feed_forward,
// reference cuda.cpp:199-304, 499-532, 567-596).
//
// Two kernels share this structure. Rows whose width is a multiple of 4096 (every
// projection of the qwen35 shapes) run in matvec_stream_kernel: workgroups of 8 or 16
// waves, items of one row x one 4096-column chunk, one item in flight per wave (see the
// streaming section below). Other widths run in matvec_kernel over the unit-major
// layout: a workgroup of 4 waves stages the input vector once in LDS (with the
// residual add + RMSNorm of the reference's dev_add/dev_rmsnorm fused in, and the
// per-unit input sums the zero-point terms need), then each wave takes groups of R
// rows. In a group, lane l handles units l, l+64, l+128, ... of every row, so one
// vector load instruction covers 64 consecutive units: 768 contiguous bytes of Q6_K
// codes, 1 KiB of Q4_K nibbles. Each lane keeps one FP32 accumulator per row; the 64
// partials are summed with cross-lane shuffles at the end of the group.
//
// Arithmetic (FP32 path): weight = (d*sc)*(q-32) for Q6_K (quant.cpp:25-40) and
// (d*sc)*q - dmin*m for Q4_K (quant.cpp:41-61). A unit's contribution is computed as
// (d*sc) * (sum q*x - 32*sum x) and (d*sc)*(sum q*x) - (dmin*m)*(sum x): the same
// products as the CPU path, grouped per unit. Only the order of FP32 additions
// differs from the reference's sequential row sum.
#include <mutex>

#include "common.hpp"
#include "kernels.hpp"
#include "decode.hpp"
#include "layout.hpp"
#include "stream.hpp"

namespace emprise {

namespace {

// ---- input staging ------------------------------------------------------------------

// xs[i] = rms(x + delta) * norm (or the plain input), usum[u] = sum of unit u of xs.
__device__ void stage_input(const MvArgs& a, float* xs, float* usum, int unit, float* red) {
    const int n = a.cols;
    const bool writer = a.x_out && blockIdx.x == 0;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float v = a.x[i];
        if (a.delta) v += a.delta[i];
        if (writer) a.x_out[i] = v;
        xs[i] = v;
        ss += v * v;
    }
    if (a.norm) {
        const float total = block_sum(ss, red);
        const float scale = 1.f / sqrtf(total / (float)n + a.eps);
        for (int i = threadIdx.x; i < n; i += blockDim.x) xs[i] = xs[i] * (scale * a.norm[i]);
    }
    __syncthreads();
    const int units = n / unit;
    for (int u = threadIdx.x; u < units; u += blockDim.x) {
        float s = 0.f;
        for (int i = 0; i < unit; ++i) s += xs[u * unit + i];
        usum[u] = s;
    }
}

// Q8 activations (quantize_x, cuda.cpp:547-559) computed in the prologue from the
// staged FP32 input: per 32 values s = amax/127, q = round(v/s) with the unrounded s,
// kept scale = fp16_rne(s). xq: n int8, xscale: n/32 floats, qsum: per 16-unit sum of q.
__device__ void stage_q8(int n, const float* xs, int8_t* xq, float* xscale, int* qsum) {
    for (int blk = threadIdx.x; blk < n / 32; blk += blockDim.x) {
        float amax = 0.f;
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(xs[blk * 32 + i]));
        const float s = amax / 127.f;
        int s0 = 0, s1 = 0;
        for (int h = 0; h < 4; ++h) {
            float v[8];
            int q[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = xs[blk * 32 + 8 * h + i];
            q8_codes<8>(v, s, q);
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                xq[blk * 32 + 8 * h + i] = (int8_t)q[i];
                if (h < 2) s0 += q[i]; else s1 += q[i];
            }
        }
        xscale[blk] = half_bits_to_float(float_to_half_bits(s));
        qsum[blk * 2] = s0;
        qsum[blk * 2 + 1] = s1;
    }
}

// ---- per-unit dot products --------------------------------------------------------

__device__ __forceinline__ uint32_t ld_u32(const uint8_t* p) { return *reinterpret_cast<const uint32_t*>(p); }

// Contribution of unit u of one Q6_K row (FP32 activations).
__device__ __forceinline__ float q6_row_unit(const uint8_t* row, int nb, int u, const float4* xv, float xsum) {
    const uint8_t* q = row + (size_t)u * 12;
    const uint32_t d0 = ld_u32(q), d1 = ld_u32(q + 4), d2 = ld_u32(q + 8);
    const float sc = (float)(int8_t)row[(size_t)nb * 192 + u];
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(row + (size_t)nb * 208 + 2 * (u >> 4)));
    const float s = q6_unit(d0, d1, d2, xv);
    return (d * sc) * fmaf(-32.f, xsum, s);
}

__device__ __forceinline__ float q4_row_unit(const uint8_t* row, int nb, int u, const float4* xv, float xsum) {
    const uint4 d = *reinterpret_cast<const uint4*>(row + (size_t)u * 16);
    const uint8_t* sp = row + (size_t)nb * 128 + (size_t)(u >> 3) * 12;
    int sc, mn;
    q4_scale_min(sp, u & 7, sc, mn);
    const uint8_t* dp = row + (size_t)nb * 140 + (size_t)(u >> 3) * 4;
    const float dd = half_bits_to_float(*reinterpret_cast<const uint16_t*>(dp));
    const float dm = half_bits_to_float(*reinterpret_cast<const uint16_t*>(dp + 2));
    const float s = q4_unit(d, xv);
    return (dd * (float)sc) * s - (dm * (float)mn) * xsum;
}

// Q6_K unit with int8 activations (linear_q8, cuda.cpp:567-596): integer dot of the
// codes with q8, minus 32*sum(q8), scaled by (d*sc) and the activation scale.
__device__ __forceinline__ float q6_row_unit_q8(const uint8_t* row, int nb, int u, const int8_t* xq,
                                                const float* xscale, const int* qsum) {
    const uint8_t* q = row + (size_t)u * 12;
    const uint32_t d0 = ld_u32(q), d1 = ld_u32(q + 4), d2 = ld_u32(q + 8);
    const uint32_t a = d0 & 0x3F3F3F3Fu, b = d1 & 0x3F3F3F3Fu, c = d2 & 0x3F3F3F3Fu;
    const uint32_t e = ((d0 >> 6) & 0x03030303u) | ((d1 >> 4) & 0x0C0C0C0Cu) | ((d2 >> 2) & 0x30303030u);
    const int* xv = reinterpret_cast<const int*>(xq + (size_t)u * 16);
    int dot = __builtin_amdgcn_sdot4((int)a, xv[0], 0, false);
    dot = __builtin_amdgcn_sdot4((int)b, xv[1], dot, false);
    dot = __builtin_amdgcn_sdot4((int)c, xv[2], dot, false);
    dot = __builtin_amdgcn_sdot4((int)e, xv[3], dot, false);
    dot -= 32 * qsum[u];
    const float sc = (float)(int8_t)row[(size_t)nb * 192 + u];
    const float d = half_bits_to_float(*reinterpret_cast<const uint16_t*>(row + (size_t)nb * 208 + 2 * (u >> 4)));
    return ((float)dot * (d * sc)) * xscale[u >> 1];
}

// ---- the kernel -------------------------------------------------------------------

// Causal conv1d step of channel c (backend.cpp:22-29): shift the history left, append
// the new value, dot with the taps in history order, SiLU.
__device__ __forceinline__ float conv_step(const float* w, float* hist, int cw, int c, float v) {
    float* h = hist + (size_t)c * cw;
    const float* k = w + (size_t)c * cw;
    float sum = 0.f;
    for (int j = 0; j < cw - 1; ++j) {
        const float hv = h[j + 1];
        h[j] = hv;
        sum += hv * k[j];
    }
    h[cw - 1] = v;
    sum += v * k[cw - 1];
    return siluf_(sum);
}

template <int T, int R, bool Q8, bool PAIR>
__global__ __launch_bounds__(256) void matvec_kernel(MvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float red[16];
    __shared__ unsigned long long block_best;
    constexpr int UW = Fmt<T>::unit;
    float* xs = reinterpret_cast<float*>(smem);
    float* usum = xs + a.cols;
    const int units = a.cols / UW;
    int8_t* xq = reinterpret_cast<int8_t*>(usum + units);
    float* xscale = reinterpret_cast<float*>(xq + a.cols);
    int* qsum = reinterpret_cast<int*>(xscale + a.cols / 32);

    stage_input(a, xs, usum, UW, red);
    if constexpr (Q8) {
        __syncthreads();
        stage_q8(a.cols, xs, xq, xscale, qsum);
    }
    if (a.mode == kMvArgmax && threadIdx.x == 0) block_best = 0ull;
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nb = a.cols / 256;
    const size_t row_bytes = (size_t)nb * Fmt<T>::block;
    constexpr int NA = PAIR ? R * 2 : R;  // accumulators (pair mode: R gate + R up rows)
    unsigned long long best = 0ull;

    for (int g = blockIdx.x * 4 + wave; g < a.groups; g += gridDim.x * 4) {
        int s = 0;
        while (s + 1 < a.nseg && g >= a.seg[s + 1].g0) ++s;
        const MvSeg seg = a.seg[s];
        const int row0 = (g - seg.g0) * R;
        const uint8_t* rp[NA];
#pragma unroll
        for (int r = 0; r < NA; ++r) {
            const int rr = r < R ? row0 + r : row0 + r - R;
            const int rc = rr < seg.rows ? rr : seg.rows - 1;
            const uint8_t* base = r < R ? seg.w : a.seg[1].w;
            rp[r] = base + (size_t)rc * row_bytes;
        }
        float acc[NA];
#pragma unroll
        for (int r = 0; r < NA; ++r) acc[r] = 0.f;

        for (int u = lane; u < units; u += 64) {
            if constexpr (Q8) {
#pragma unroll
                for (int r = 0; r < NA; ++r) acc[r] += q6_row_unit_q8(rp[r], nb, u, xq, xscale, qsum);
            } else {
                float4 xv[UW / 4];
                const float4* xp = reinterpret_cast<const float4*>(xs + (size_t)u * UW);
#pragma unroll
                for (int i = 0; i < UW / 4; ++i) xv[i] = xp[i];
                const float xsum = usum[u];
#pragma unroll
                for (int r = 0; r < NA; ++r) {
                    if constexpr (T == kQ6K) acc[r] += q6_row_unit(rp[r], nb, u, xv, xsum);
                    else acc[r] += q4_row_unit(rp[r], nb, u, xv, xsum);
                }
            }
        }
#pragma unroll
        for (int r = 0; r < NA; ++r) acc[r] = wave_sum(acc[r]);
        if (lane == 0) {
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = row0 + r;
                if (row < seg.rows) {
                    if constexpr (PAIR) {
                        seg.y[row] = siluf_(acc[r]) * acc[(R + r) % NA];
                    } else if (a.conv_w && s == 0) {
                        seg.y[row] = conv_step(a.conv_w, a.conv_state, a.conv_width, row, acc[r]);
                    } else {
                        seg.y[row] = (a.silu_mask >> s) & 1 ? siluf_(acc[r]) : acc[r];
                        if (a.mode == kMvArgmax) {
                            const unsigned long long k = argmax_key(acc[r], row);
                            best = k > best ? k : best;
                        }
                    }
                }
            }
        }
    }
    if (a.mode == kMvArgmax) {
        if (lane == 0 && best) atomicMax(&block_best, best);
        __syncthreads();
        if (threadIdx.x == 0 && block_best) atomicMax(a.argmax, block_best);
    }
}

// ---- streaming kernel for rows in the chunked layout (cols % 4096 == 0) --------------
//
// A wave walks a sequence of items (R rows, or R gate/up row pairs, x one 4096-column
// chunk; R = kMvStreamRows / kMvStreamPairRows), with kStreamDepth items in flight: it
// issues the loads of the item kStreamDepth ahead as soon as it has computed one, and
// the first items' loads go out before the workgroup stages its input. One item in
// flight measured fastest in the 9B-shape decode (543.0 tok/s, against 510.0 with two
// and 464.1 with three): the other waves of the CU hide a wave's load latency, and the
// fewer requests in flight the better the memory system streams them. Issuing the next
// item as soon as the current one has arrived (two buffers, still one item in flight,
// the loads overlapping the arithmetic) measured 2% slower than issuing it after. Lane l owns 64
// consecutive weights of every chunk row: per row and chunk it issues three (Q6_K) or
// two (Q4_K) 16-byte loads that each cover 1 KiB contiguous across the wave, plus one
// scale load and one d load. Row pointers are wave-uniform (scalar registers).

// Q8 activations (Q6_K only): int8 input in LDS, unit granules of 16 B at
// ((c*4 + j)*64 + l)*16 for unit 4l+j of chunk c.
template <int NA>
__device__ __forceinline__ void scompute_q8(const SChunk<kQ6K, NA>& ch, float* acc, const int8_t* xq,
                                            const float* xscale, const int* qsum, int c, int lane) {
    const int4 qs = reinterpret_cast<const int4*>(qsum)[c * 64 + lane];
    const float2 s8 = reinterpret_cast<const float2*>(xscale)[c * 64 + lane];
    const int qsv[4] = {qs.x, qs.y, qs.z, qs.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int4 xv = reinterpret_cast<const int4*>(xq)[(c * 4 + j) * 64 + lane];
        const float s8j = j < 2 ? s8.x : s8.y;
#pragma unroll
        for (int r = 0; r < NA; ++r) {
            const uint32_t d0 = lane_word(ch.q[r][0], j), d1 = lane_word(ch.q[r][1], j), d2 = lane_word(ch.q[r][2], j);
            const uint32_t e = ((d0 >> 6) & 0x03030303u) | ((d1 >> 4) & 0x0C0C0C0Cu) | ((d2 >> 2) & 0x30303030u);
            int dot = __builtin_amdgcn_sdot4((int)(d0 & 0x3F3F3F3Fu), xv.x, 0, false);
            dot = __builtin_amdgcn_sdot4((int)(d1 & 0x3F3F3F3Fu), xv.y, dot, false);
            dot = __builtin_amdgcn_sdot4((int)(d2 & 0x3F3F3F3Fu), xv.z, dot, false);
            dot = __builtin_amdgcn_sdot4((int)e, xv.w, dot, false);
            const float d = half_bits_to_float((uint16_t)ch.d[r]);
            const float sc = (float)(int)(int8_t)(ch.sc[r] >> (8 * j));
            acc[r] += ((float)(dot - 32 * qsv[j]) * (d * sc)) * s8j;
        }
    }
}

// Input staging for the streaming kernels: 16-byte loads, four in flight per thread;
// FP32 input goes to chunk_slot order, per-unit sums in natural order.
//
// Inputs of up to 4 floats per thread with a norm take one pass: x, delta and the norm
// weights are loaded together and the normalised input is written to LDS once.
template <bool Q8>
__device__ void sstage_normed(const MvArgs& a, float4* xs4, float* red) {
    const int n4 = a.cols / 4;
    const bool writer = a.x_out && blockIdx.x == 0;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    const float4* d4 = reinterpret_cast<const float4*>(a.delta);
    const float4* n4p = reinterpret_cast<const float4*>(a.norm);
    float4 v[4], w[4], dv[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        if (i < n4) {
            v[k] = x4[i];
            if (d4) dv[k] = d4[i];
            w[k] = n4p[i];
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        if (i < n4) {
            if (d4) {
                v[k].x += dv[k].x;
                v[k].y += dv[k].y;
                v[k].z += dv[k].z;
                v[k].w += dv[k].w;
            }
            if (writer) reinterpret_cast<float4*>(a.x_out)[i] = v[k];
            ss += v[k].x * v[k].x + v[k].y * v[k].y + v[k].z * v[k].z + v[k].w * v[k].w;
        }
    }
    const float total = block_sum(ss, red);
    const float scale = 1.f / sqrtf(total / (float)a.cols + a.eps);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        if (i < n4) {
            float4 o;
            o.x = v[k].x * (scale * w[k].x);
            o.y = v[k].y * (scale * w[k].y);
            o.z = v[k].z * (scale * w[k].z);
            o.w = v[k].w * (scale * w[k].w);
            xs4[Q8 ? i : chunk_slot(i)] = o;
        }
    }
}

// B float4 per thread per batch. Every load of a batch is issued before any is used
// (indices are clamped to the last float4, so no load sits under a branch): one memory
// round trip per batch.
template <bool Q8, int B>
__device__ float sstage_batch(const MvArgs& a, float4* xs4, int i0) {
    const int n4 = a.cols / 4;
    const bool writer = a.x_out && blockIdx.x == 0;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
    const float4* d4 = reinterpret_cast<const float4*>(a.delta);
    float4 v[B];
#pragma unroll
    for (int k = 0; k < B; ++k) v[k] = x4[min(i0 + k * (int)blockDim.x, n4 - 1)];
    if (d4) {
        float4 dv[B];
#pragma unroll
        for (int k = 0; k < B; ++k) dv[k] = d4[min(i0 + k * (int)blockDim.x, n4 - 1)];
#pragma unroll
        for (int k = 0; k < B; ++k) {
            v[k].x += dv[k].x;
            v[k].y += dv[k].y;
            v[k].z += dv[k].z;
            v[k].w += dv[k].w;
        }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < B; ++k) {
        const int i = i0 + k * blockDim.x;
        if (i < n4) {
            if (writer) reinterpret_cast<float4*>(a.x_out)[i] = v[k];
            xs4[Q8 ? i : chunk_slot(i)] = v[k];
            ss += v[k].x * v[k].x + v[k].y * v[k].y + v[k].z * v[k].z + v[k].w * v[k].w;
        }
    }
    return ss;
}

template <bool Q8>
__device__ void sstage_general(const MvArgs& a, float4* xs4, float* red) {
    const int n4 = a.cols / 4;
    float ss = 0.f;
    if (!a.delta && n4 <= 6 * (int)blockDim.x) {
        ss = sstage_batch<Q8, 6>(a, xs4, threadIdx.x);  // up to 6144 columns in one round trip
    } else if (!a.delta && n4 <= 12 * (int)blockDim.x) {
        ss = sstage_batch<Q8, 6>(a, xs4, threadIdx.x);  // up to 12288 columns in two
        ss += sstage_batch<Q8, 6>(a, xs4, threadIdx.x + 6 * blockDim.x);
    } else {
        for (int i0 = threadIdx.x; i0 < n4; i0 += 4 * blockDim.x) ss += sstage_batch<Q8, 4>(a, xs4, i0);
    }
    if (!a.norm) return;
    const float total = block_sum(ss, red);
    const float scale = 1.f / sqrtf(total / (float)a.cols + a.eps);
    const float4* n4p = reinterpret_cast<const float4*>(a.norm);
    for (int i0 = threadIdx.x; i0 < n4; i0 += 4 * blockDim.x) {
        float4 w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) w[k] = n4p[min(i0 + k * (int)blockDim.x, n4 - 1)];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = i0 + k * blockDim.x;
            if (i < n4) {
                const int sl = Q8 ? i : chunk_slot(i);
                float4 v = xs4[sl];
                v.x = v.x * (scale * w[k].x);
                v.y = v.y * (scale * w[k].y);
                v.z = v.z * (scale * w[k].z);
                v.w = v.w * (scale * w[k].w);
                xs4[sl] = v;
            }
        }
    }
}

template <int UNIT, bool Q8>
__device__ void sstage(const MvArgs& a, float* xs, float* usum, float* red) {
    float4* xs4 = reinterpret_cast<float4*>(xs);
    if (a.norm && a.cols <= 16 * (int)blockDim.x) sstage_normed<Q8>(a, xs4, red);
    else sstage_general<Q8>(a, xs4, red);
    __syncthreads();
    if constexpr (!Q8) {
        constexpr int U4 = UNIT / 4;
        const int units = a.cols / UNIT;
        for (int u = threadIdx.x; u < units; u += blockDim.x) {
            float s = 0.f;
#pragma unroll
            for (int j = 0; j < U4; ++j) {
                const float4 v = xs4[chunk_slot(u * U4 + j)];
                s += (v.x + v.y) + (v.z + v.w);
            }
            usum[u] = stored_unit_sum<UNIT>(s);
        }
    }
}

// Q8 quantisation of the staged input (natural order) into unit granules at
// ((c*4 + j)*64 + l)*16 for unit u = c*256 + 4l + j; 8 values per thread.
__device__ void sstage_q8(int n, const float* xs, int8_t* xq, float* xscale, int* qsum) {
    for (int e = threadIdx.x; e < n / 8; e += blockDim.x) {
        const float4 v0 = reinterpret_cast<const float4*>(xs)[2 * e];
        const float4 v1 = reinterpret_cast<const float4*>(xs)[2 * e + 1];
        const float v[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        const float s = amax / 127.f;
        int q[8], part = 0;
        q8_codes<8>(v, s, q);
#pragma unroll
        for (int i = 0; i < 8; ++i) part += q[i];
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo |= (uint32_t)(q[i] & 0xff) << (8 * i);
            hi |= (uint32_t)(q[4 + i] & 0xff) << (8 * i);
        }
        const int u = e >> 1, c = u >> 8, w = u & 255;
        reinterpret_cast<uint2*>(xq)[(((c * 4 + (w & 3)) * 64 + (w >> 2)) << 1) + (e & 1)] = make_uint2(lo, hi);
        part += __shfl_xor(part, 1, 64);
        if ((e & 1) == 0) qsum[u] = part;
        if ((e & 3) == 0) xscale[e >> 2] = half_bits_to_float(float_to_half_bits(s));
    }
}

// Input registers of the one-shot staging: SB float4 per thread of x, and with DN of
// the residual delta and the norm weights.
template <int SB, bool DN> struct SInput {
    float4 x[SB];
    float4 d[DN ? SB : 1], w[DN ? SB : 1];  // delta, or the gate in the per-head mode
};

template <int SB, bool DN>
__device__ __forceinline__ void sinput_issue(const MvArgs& a, SInput<SB, DN>& s) {
    const int n4 = a.cols / 4;
    const float4* x4 = reinterpret_cast<const float4*>(a.x);
#pragma unroll
    for (int k = 0; k < SB; ++k) s.x[k] = x4[min((int)threadIdx.x + k * (int)blockDim.x, n4 - 1)];
    if constexpr (DN) {
        if (a.delta || a.gate) {
            const float4* d4 = reinterpret_cast<const float4*>(a.gate ? a.gate : a.delta);
#pragma unroll
            for (int k = 0; k < SB; ++k) s.d[k] = d4[min((int)threadIdx.x + k * (int)blockDim.x, n4 - 1)];
        }
        if (a.norm) {
            const float4* w4 = reinterpret_cast<const float4*>(a.norm);
            const int wn4 = a.gate ? a.head_dim / 4 : n4;  // per-head weights repeat every head
#pragma unroll
            for (int k = 0; k < SB; ++k) s.w[k] = w4[min((int)threadIdx.x + k * (int)blockDim.x, n4 - 1) % wn4];
        }
    }
}

// Finishes the one-shot staging from registers: residual add (workgroup 0 writes
// x_out), RMSNorm, the LDS store (chunk_slot order; natural order for Q8) and the
// per-unit input sums, reduced across the UNIT/4 consecutive threads that hold a unit.
template <int UNIT, bool Q8, int SB, bool DN>
__device__ __forceinline__ void sinput_finish(const MvArgs& a, SInput<SB, DN>& s, float* xs, float* usum, float* red,
                                              int8_t* xq, float* xscale, int* qsum) {
    const int n4 = a.cols / 4;
    const bool writer = a.x_out && blockIdx.x == 0;
    float4* xs4 = reinterpret_cast<float4*>(xs);
    if (DN && a.gate) {
        // per-head RMSNorm x SiLU(gate): a head is head_dim/4 consecutive float4, held
        // by as many consecutive lanes of one wave, so its sum of squares is a
        // butterfly over those lanes
        const int h4 = a.head_dim / 4;
#pragma unroll
        for (int k = 0; k < SB; ++k) {
            float ss = s.x[k].x * s.x[k].x + s.x[k].y * s.x[k].y + s.x[k].z * s.x[k].z + s.x[k].w * s.x[k].w;
            for (int m = 1; m < h4; m <<= 1) ss += __shfl_xor(ss, m, 64);
            const float scale = 1.f / sqrtf(ss / (float)a.head_dim + a.eps);
            s.x[k].x = s.x[k].x * (scale * s.w[k].x) * s.d[k].x;
            s.x[k].y = s.x[k].y * (scale * s.w[k].y) * s.d[k].y;
            s.x[k].z = s.x[k].z * (scale * s.w[k].z) * s.d[k].z;
            s.x[k].w = s.x[k].w * (scale * s.w[k].w) * s.d[k].w;
        }
    } else if constexpr (DN) {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < SB; ++k) {
            const int i = threadIdx.x + k * blockDim.x;
            if (a.delta) {
                s.x[k].x += s.d[k].x;
                s.x[k].y += s.d[k].y;
                s.x[k].z += s.d[k].z;
                s.x[k].w += s.d[k].w;
            }
            if (i < n4) {
                if (writer) reinterpret_cast<float4*>(a.x_out)[i] = s.x[k];
                ss += s.x[k].x * s.x[k].x + s.x[k].y * s.x[k].y + s.x[k].z * s.x[k].z + s.x[k].w * s.x[k].w;
            }
        }
        if (a.norm) {
            const float total = block_sum(ss, red);
            const float scale = 1.f / sqrtf(total / (float)a.cols + a.eps);
#pragma unroll
            for (int k = 0; k < SB; ++k) {
                s.x[k].x = s.x[k].x * (scale * s.w[k].x);
                s.x[k].y = s.x[k].y * (scale * s.w[k].y);
                s.x[k].z = s.x[k].z * (scale * s.w[k].z);
                s.x[k].w = s.x[k].w * (scale * s.w[k].w);
            }
        }
    }
    constexpr int U4 = UNIT / 4;
#pragma unroll
    for (int k = 0; k < SB; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        if constexpr (Q8) {
            // quantised straight from registers, sstage_q8's rule and layout: a 32-value
            // block is the float4 of 8 consecutive threads (amax over them), a 16-value
            // unit those of 4 (its code sum), 4 codes per thread in one 32-bit store
            const float4 v = s.x[k];
            float amax = 0.f;
            amax = fmaxf(amax, fabsf(v.x));
            amax = fmaxf(amax, fabsf(v.y));
            amax = fmaxf(amax, fabsf(v.z));
            amax = fmaxf(amax, fabsf(v.w));
            amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
            amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
            const float sc = amax / 127.f;
            const float vv[4] = {v.x, v.y, v.z, v.w};
            int qq[4];
            q8_codes<4>(vv, sc, qq);
            int part = 0;
            uint32_t packed = 0;
#pragma unroll
            for (int c4 = 0; c4 < 4; ++c4) {
                const int q = qq[c4];
                part += q;
                packed |= (uint32_t)(q & 0xff) << (8 * c4);
            }
            part += __shfl_xor(part, 1, 64);
            part += __shfl_xor(part, 2, 64);
            if (i < n4) {
                const int e = i >> 1, u = i >> 2, c = u >> 8, w = u & 255;
                reinterpret_cast<uint32_t*>(xq)[(((((c * 4 + (w & 3)) * 64 + (w >> 2)) << 1) + (e & 1)) << 1) + (i & 1)] =
                    packed;
                if ((i & 3) == 0) qsum[u] = part;
                if ((i & 7) == 0) xscale[i >> 3] = half_bits_to_float(float_to_half_bits(sc));
            }
        } else {
            if (i < n4) xs4[chunk_slot(i)] = s.x[k];
            float t = (s.x[k].x + s.x[k].y) + (s.x[k].z + s.x[k].w);
            t += __shfl_xor(t, 1, 64);
            t += __shfl_xor(t, 2, 64);
            if constexpr (U4 == 8) t += __shfl_xor(t, 4, 64);
            if (i < n4 && (i & (U4 - 1)) == 0) usum[i / U4] = stored_unit_sum<UNIT>(t);
        }
    }
}

// Staging modes of a launch: 0 generic (sstage, after the first items' loads),
// 1 up to 4096 columns with residual add and norm, 2 up to 12288 columns, plain input.
// W: waves per workgroup (8 or 16; see launch_stream_mode).
constexpr int kStreamWavesPerCU = 16;  // resident waves per CU the grid is sized for
constexpr int kStreamDepth = 1;        // items in flight per wave
template <int W, int SM> struct StageMode;
template <int W> struct StageMode<W, 0> { static constexpr int sb = 1; static constexpr bool dn = false; };
template <int W> struct StageMode<W, 1> { static constexpr int sb = 1024 / (W * 64); static constexpr bool dn = true; };
template <int W> struct StageMode<W, 2> { static constexpr int sb = 3072 / (W * 64); static constexpr bool dn = false; };

template <int T, bool Q8, bool PAIR, bool CONV, int SM, int W>
__global__ __launch_bounds__(W * 64) void matvec_stream_kernel(MvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float red[W];
    __shared__ unsigned long long block_best;
    constexpr int R = PAIR ? kMvStreamPairRows : kMvStreamRows;
    constexpr int UW = Fmt<T>::unit;
    constexpr int NA = PAIR ? R * 2 : R;
    constexpr int SB = StageMode<W, SM>::sb;
    constexpr bool DN = StageMode<W, SM>::dn;
    float* xs = reinterpret_cast<float*>(smem);
    float* usum = xs + a.cols;
    const int units = a.cols / UW;
    int8_t* xq = reinterpret_cast<int8_t*>(usum + units);
    float* xscale = reinterpret_cast<float*>(xq + a.cols);
    int* qsum = reinterpret_cast<int*>(xscale + a.cols / 32);

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int cpr = a.cols / kChunkCols;
    const size_t row_bytes = (size_t)(a.cols / 256) * Fmt<T>::block;
    const int stride = gridDim.x * W;
    const uint8_t* dummy = reinterpret_cast<const uint8_t*>(a.x);

    // row pointers of item `it`'s row group
    auto rows_of = [&](SItem<NA>& it) {
        int s = 0;
        while (s + 1 < a.nseg && it.g >= a.seg[s + 1].g0) ++s;
        it.seg = s;
        it.row0 = (it.g - a.seg[s].g0) * R;
        const int nrows = a.seg[s].rows;
#pragma unroll
        for (int r = 0; r < NA; ++r) {
            const int rr = r < R ? it.row0 + r : it.row0 + r - R;
            const int rc = rr < nrows ? rr : nrows - 1;
            it.rp[r] = (r < R ? a.seg[s].w : a.seg[1].w) + (size_t)rc * row_bytes;
        }
    };
    // Item order. Round-robin (wave v takes groups v, v + nw, v + 2nw, ... with nw waves
    // in the grid), except for the SwiGLU pair launches with two workgroups per CU: the
    // second workgroup on a CU finishes its input staging ~3 us after the first (its
    // input loads queue behind the first one's weight loads), and its waves end that much
    // later. There the second round goes to the first workgroups only (nw/2 groups) and
    // the full rounds follow, so a first-workgroup wave takes one group more (two more when
    // the last, partial round reaches only them: 4 against 2 in the 9B FFN gate+up, which
    // then takes 16.6 instead of 17.1 us).
    const bool tilt = PAIR && W == 8 && kStreamDepth == 1 && gridDim.x % 2 == 0;
    const int vw = blockIdx.x * W + wave, half_nw = stride / 2;
    const bool first_wg = (int)blockIdx.x < (int)gridDim.x / 2;
    int later = 0;  // groups taken after the first round
    // moves `it` n items ahead in this wave's sequence
    auto skip = [&](SItem<NA>& it, int n) {
        const int c = it.c + n, hop = c / cpr;
        it.c = c - hop * cpr;
        if (hop) {
            if (tilt && hop == 1) {
                // rounds after the first: [stride, stride + nw/2) for the first workgroups,
                // then full rounds of nw groups from stride + nw/2
                const int k = ++later, full = first_wg ? k - 2 : k - 1;
                it.g = full < 0 ? stride + vw : stride + half_nw + full * stride + vw;
            } else {
                it.g += hop * stride;
            }
            if (it.g < a.groups) rows_of(it);
        }
    };
    // Issues the loads of item `it` into `buf`. The same instructions run for every
    // item -- one past the end reads the input vector instead (L2-resident, never
    // used) -- so the compiler's wait counts stay exact and a wave never waits for
    // more than the buffer it is about to compute.
    auto iload = [&](SChunk<T, NA>& buf, SItem<NA>& it) {
        const bool valid = it.g < a.groups;
        const uint8_t* p[NA];
#pragma unroll
        for (int r = 0; r < NA; ++r) p[r] = valid ? it.rp[r] : dummy;
        sload<T, NA>(buf, p, valid ? it.c : 0, lane);
        if constexpr (CONV) {
            const int cw = a.conv_width, r = lane / cw, j = lane - r * cw, row = it.row0 + r;
            const bool on = valid && it.seg == 0 && r < R && row < a.seg[0].rows;
            const size_t o = on ? (size_t)row * cw + j : 0;
            const float h = *(on ? a.conv_state + o : a.x), k = *(on ? a.conv_w + o : a.x);
            it.conv_h = on ? h : 0.f;
            it.conv_k = on ? k : 0.f;
        }
    };

    // Input loads first, then the weights of the wave's first D items, then the
    // staging arithmetic: the loads return in issue order, so the staging waits only
    // for its own (L2-resident) data while the weight streams are in flight.
    // (sched_barrier keeps the groups of loads in this order: the wait for one buffer
    // must not cover the loads of the next.)
    SInput<SB, DN> sin;
    if constexpr (SM != 0) sinput_issue<SB, DN>(a, sin);
    constexpr int D = kStreamDepth;
    SItem<NA> its[D];
    its[0].g = blockIdx.x * W + wave;
    its[0].c = 0;
    if (its[0].g < a.groups) rows_of(its[0]);
#pragma unroll
    for (int k = 1; k < D; ++k) {
        its[k] = its[k - 1];
        skip(its[k], 1);
    }
    SChunk<T, NA> bufs[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        __builtin_amdgcn_sched_barrier(0);
        iload(bufs[k], its[k]);
    }
    __builtin_amdgcn_sched_barrier(0);

    if constexpr (SM != 0) sinput_finish<UW, Q8, SB, DN>(a, sin, xs, usum, red, xq, xscale, qsum);
    else sstage<UW, Q8>(a, xs, usum, red);
    if constexpr (Q8 && SM == 0) {
        __syncthreads();
        sstage_q8(a.cols, xs, xq, xscale, qsum);
    }
    if (a.mode == kMvArgmax && threadIdx.x == 0) block_best = 0ull;
    __syncthreads();

    unsigned long long best = 0ull;
    float acc[NA];
#pragma unroll
    for (int r = 0; r < NA; ++r) acc[r] = 0.f;

    // Computes the item held in `buf`, runs the row epilogue after a row group's last
    // chunk, then refills `buf` with the item D ahead (the other buffers hold the next).
    auto finish = [&](SChunk<T, NA>& buf, SItem<NA>& it) {
        if constexpr (Q8) scompute_q8<NA>(buf, acc, xq, xscale, qsum, it.c, lane);
        else scompute<T, NA>(buf, acc, xs, usum, it.c, lane);
        if (it.c == cpr - 1) {
#pragma unroll
            for (int r = 0; r < NA; ++r) acc[r] = wave_sum(acc[r]);
            if (CONV && it.seg == 0) {
                // causal conv1d + SiLU of the rows (backend.cpp:22-29): the history
                // shifts left by one slot, the new value enters the last slot, and the
                // taps are summed in slot order
                const int cw = a.conv_width, r = lane / cw, j = lane - r * cw, row = it.row0 + r;
                float v = 0.f;
#pragma unroll
                for (int rr = 0; rr < R; ++rr) v = r == rr ? acc[rr] : v;
                const float shifted = __shfl_down(it.conv_h, 1, 64);
                const float hn = j == cw - 1 ? v : shifted;
                const float p = hn * it.conv_k;
                float sum = 0.f;
                for (int jj = 0; jj < cw; ++jj) sum += __shfl(p, lane - j + jj, 64);
                if (r < R && row < a.seg[0].rows) {
                    a.conv_state[(size_t)row * cw + j] = hn;
                    if (j == 0) a.seg[0].y[row] = siluf_(sum);
                }
            } else if (lane == 0) {
                const MvSeg sg = a.seg[it.seg];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int row = it.row0 + r;
                    if (row < sg.rows) {
                        if constexpr (PAIR) {
                            sg.y[row] = siluf_(acc[r]) * acc[(R + r) % NA];
                        } else {
                            float v = acc[r];
                            // only the conv variant (the GDN in-projection) carries SiLU'd
                            // segments; the empty volatile asm keeps SiLU behind the
                            // (wave-uniform) branch instead of evaluated for every row
                            if constexpr (CONV)
                                if ((a.silu_mask >> it.seg) & 1) {
                                    asm volatile("" : "+v"(v));
                                    v = siluf_(v);
                                }
                            sg.y[row] = v;
                            if (a.mode == kMvArgmax) {
                                const unsigned long long k = argmax_key(acc[r], row);
                                best = k > best ? k : best;
                            }
                        }
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < NA; ++r) acc[r] = 0.f;
        }
    };
    // items are visited in sequence order, so once one is past the end so are the rest
    bool live = its[0].g < a.groups;
    while (live) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            if (live) {
                finish(bufs[k], its[k]);
                skip(its[k], D);
                iload(bufs[k], its[k]);
                live = its[(k + 1) % D].g < a.groups;
            }
        }
    }
    if (a.mode == kMvArgmax) {
        if (lane == 0 && best) atomicMax(&block_best, best);
        __syncthreads();
        if (threadIdx.x == 0 && block_best) atomicMax(a.argmax, block_best);
    }
}

// Workgroups of a streaming launch: one full round of resident workgroups (occupancy x
// CUs, at most kStreamWavesPerCU waves per CU), so no wave waits for a second dispatch
// round. Occupancy differs per kernel instantiation (registers) and per LDS size, so
// the cache is keyed by both. The cap: every workgroup stages the whole input, and 32
// waves per CU (four 8-wave or two 16-wave workgroups, which the one-item kernels have
// room for) measured slower than 16 in the 9B-shape decode (526.0 and 540.7 vs 543.0
// tok/s with 8-wave workgroups).
int resident_blocks(const void* kernel, size_t lds, int waves) {
    struct Entry {
        const void* kernel;
        size_t lds;
        int blocks;
    };
    static Entry cache[64];
    static int used = 0;
    static std::mutex mu;
    std::lock_guard<std::mutex> lock(mu);
    for (int i = 0; i < used; ++i)
        if (cache[i].kernel == kernel && cache[i].lds == lds) return cache[i].blocks;
    int dev = 0, per_cu = 0;
    hipDeviceProp_t prop;
    (void)hipGetDevice(&dev);
    (void)hipGetDeviceProperties(&prop, dev);
    (void)hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, waves * 64, lds);
    const int cap = kStreamWavesPerCU / waves;
    const int blocks = (per_cu > 0 ? (per_cu < cap ? per_cu : cap) : 1) * prop.multiProcessorCount;
    if (used < 64) cache[used++] = {kernel, lds, blocks};
    return blocks;
}

template <int W, class K> hipError_t launch_stream(K kernel, const MvArgs& a, size_t lds, hipStream_t stream) {
    int blocks = (a.groups + W - 1) / W;
    const int cap = resident_blocks(reinterpret_cast<const void*>(kernel), lds, W);
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    launch_kernel(kernel, dim3(blocks), dim3(W * 64), lds, stream, a);
    return hipGetLastError();
}

// Workgroup size per staging mode, both sized to 16 resident waves per CU. Measured in
// the 9B-shape decode (one item in flight per wave): 8-wave workgroups (two per CU) are
// faster for the launches whose staging has a residual add + RMSNorm (FFN gate+up 17.2 vs
// 18.0 µs, GDN in-projection 12.1 vs 13.3 µs), one 16-wave workgroup per CU for the plain
// 12288-wide input (ffn_down 9.3 vs 10.5 µs) and the per-head gated staging (GDN
// out-projection 5.5 vs 6.8 µs). The mode sets which block reduction runs, and the two
// 16-wave modes have none, so results do not depend on the workgroup size.
template <int T, bool Q8, bool PAIR, bool CONV>
hipError_t launch_stream_mode(const MvArgs& a, size_t lds, hipStream_t stream) {
    const int n4 = a.cols / 4;
    if (n4 <= StageMode<8, 1>::sb * 8 * 64) {
        if constexpr (!PAIR && !CONV)
            if (a.gate) return launch_stream<16>(matvec_stream_kernel<T, Q8, false, false, 1, 16>, a, lds, stream);
        return launch_stream<8>(matvec_stream_kernel<T, Q8, PAIR, CONV, 1, 8>, a, lds, stream);
    }
    if (a.gate) return hipErrorInvalidValue;  // the per-head transform stages in one pass only
    if constexpr (!CONV) {
        if (!a.delta && !a.norm && n4 <= StageMode<16, 2>::sb * 16 * 64)
            return launch_stream<16>(matvec_stream_kernel<T, Q8, PAIR, false, 2, 16>, a, lds, stream);
    }
    return launch_stream<8>(matvec_stream_kernel<T, Q8, PAIR, CONV, 0, 8>, a, lds, stream);
}

template <int T, bool Q8> hipError_t launch_stream_kind(const MvArgs& a, size_t lds, hipStream_t stream) {
    if (a.mode == kMvSwiglu) return launch_stream_mode<T, Q8, true, false>(a, lds, stream);
    if (a.conv_w) return launch_stream_mode<T, Q8, false, true>(a, lds, stream);
    return launch_stream_mode<T, Q8, false, false>(a, lds, stream);
}

}  // namespace

// Rows per item of the streaming kernel: one row (one gate/up pair). Measured in the
// 9B-shape decode (per-op graph): 1 row 510.6 tok/s, 2 rows 492.0, 4 rows 426.5 -- most
// launches give a wave only a few items, and single-row items spread them over more
// waves and cut the registers (66-85 VGPRs: 5-7 waves per SIMD instead of 4).
int matvec_rows_per_group(uint32_t type, uint64_t cols, int mode, uint64_t total_rows) {
    (void)total_rows;
    if ((type == kQ6K || type == kQ4K) && cols % kChunkCols == 0)
        return mode == kMvSwiglu ? kMvStreamPairRows : kMvStreamRows;
    return (type == kQ6K || type == kQ4K) ? kMvRows : 1;
}

hipError_t launch_matvec_stream(uint32_t type, bool q8, const MvArgs& a, hipStream_t stream) {
    const size_t lds = matvec_lds_bytes(type, a.cols, q8);
    // per-head transform: whole heads of a power-of-two number of float4 within a wave
    if (a.gate && (a.delta || a.x_out || !a.norm || a.head_dim < 4 || a.head_dim > 256 || a.head_dim % 4 ||
                   ((a.head_dim / 4) & (a.head_dim / 4 - 1)) || a.cols % a.head_dim))
        return hipErrorInvalidValue;
    if (a.rows_per_group != (a.mode == kMvSwiglu ? kMvStreamPairRows : kMvStreamRows)) return hipErrorInvalidValue;
    if (a.silu_mask && !a.conv_w) return hipErrorInvalidValue;  // SiLU'd segments ride with the conv epilogue
    // the conv epilogue holds an item's rows x taps in the lanes of one wave
    if (a.conv_w && (a.mode == kMvSwiglu || a.conv_width < 1 || a.conv_width * a.rows_per_group > 64))
        return hipErrorInvalidValue;
    if (type == kQ6K) return q8 ? launch_stream_kind<kQ6K, true>(a, lds, stream) : launch_stream_kind<kQ6K, false>(a, lds, stream);
    return launch_stream_kind<kQ4K, false>(a, lds, stream);
}

namespace {


// Plain-layout (F32 / F16 / BF16) matvec: one wave per row, lanes stride the columns.
template <int T>
__device__ __forceinline__ float raw_elem(const uint8_t* row, int k) {
    if constexpr (T == kF32) return reinterpret_cast<const float*>(row)[k];
    else if constexpr (T == kF16) return half_bits_to_float(reinterpret_cast<const uint16_t*>(row)[k]);
    else return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(row)[k] << 16);
}

template <int T>
__global__ __launch_bounds__(256) void matvec_raw_kernel(MvArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ float red[16];
    __shared__ unsigned long long block_best;
    float* xs = reinterpret_cast<float*>(smem);
    float* usum = xs + a.cols;
    stage_input(a, xs, usum, 1 << 30, red);  // no unit sums needed
    if (a.mode == kMvArgmax && threadIdx.x == 0) block_best = 0ull;
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const size_t row_bytes = (size_t)a.cols * (T == kF32 ? 4 : 2);
    const bool pair = a.mode == kMvSwiglu;
    unsigned long long best = 0ull;
    for (int g = blockIdx.x * 4 + wave; g < a.groups; g += gridDim.x * 4) {
        int s = 0;
        while (s + 1 < a.nseg && g >= a.seg[s + 1].g0) ++s;
        const MvSeg seg = a.seg[s];
        const int row = g - seg.g0;
        const uint8_t* r0 = seg.w + (size_t)row * row_bytes;
        const uint8_t* r1 = pair ? a.seg[1].w + (size_t)row * row_bytes : r0;
        float acc0 = 0.f, acc1 = 0.f;
        for (int k = lane; k < a.cols; k += 64) {
            acc0 = fmaf(raw_elem<T>(r0, k), xs[k], acc0);
            if (pair) acc1 = fmaf(raw_elem<T>(r1, k), xs[k], acc1);
        }
        acc0 = wave_sum(acc0);
        if (pair) acc1 = wave_sum(acc1);
        if (lane == 0) {
            if (pair) seg.y[row] = siluf_(acc0) * acc1;
            else {
                seg.y[row] = acc0;
                if (a.mode == kMvArgmax) {
                    const unsigned long long k = argmax_key(acc0, row);
                    best = k > best ? k : best;
                }
            }
        }
    }
    if (a.mode == kMvArgmax) {
        if (lane == 0 && best) atomicMax(&block_best, best);
        __syncthreads();
        if (threadIdx.x == 0 && block_best) atomicMax(a.argmax, block_best);
    }
}

// ---- dequantisation of whole rows (dequantize(), quant.cpp:64-78) -------------------

__global__ void dequant_rows_kernel(const uint8_t* w, uint32_t type, int cols, uint64_t row0, uint64_t n,
                                    float* out) {
    const uint64_t total = n * (uint64_t)cols;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = decode_element(w, type, cols, row0 + i / cols, (int)(i % cols));
}

// The same values for the chunked Q6_K / Q4_K layouts, a 4096-column chunk per wave and
// work item: the streaming matvec's lane loads (lane l holds columns 64l .. 64l+63 of the
// chunk; the next item's loads are in flight while one is decoded) and the shared element
// formulas. The decoded chunk passes through LDS so that each store instruction writes 1
// KiB of consecutive floats (stored from the lanes' own columns, a store would cover 16
// bytes of each of 64 lines). Lane rows are padded to 17 float4, which keeps both the
// row-wise writes and the column-wise reads free of bank conflicts.
constexpr int kDequantGrid = 512;

template <int T> __device__ __forceinline__ void dequant_chunk_values(const SChunk<T, 1>& ch, float4* v) {
    if constexpr (T == kQ6K) {
        // unit 4l+j: codes 0..11 are the low 6 bits of plane (t/4)'s word j, codes 12..15
        // the top 2 bits of the three planes' bytes
        const float d = half_bits_to_float((uint16_t)ch.d[0]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int8_t sc = (int8_t)(ch.sc[0] >> (8 * j));
            const uint32_t pw[3] = {lane_word(ch.q[0][0], j), lane_word(ch.q[0][1], j), lane_word(ch.q[0][2], j)};
#pragma unroll
            for (int p = 0; p < 3; ++p)
                v[4 * j + p] = make_float4(q6k_weight(d, sc, pw[p] & 63), q6k_weight(d, sc, (pw[p] >> 8) & 63),
                                           q6k_weight(d, sc, (pw[p] >> 16) & 63), q6k_weight(d, sc, (pw[p] >> 24) & 63));
            float hi[4];
#pragma unroll
            for (int b = 0; b < 4; ++b)
                hi[b] = q6k_weight(d, sc, (int)(((pw[0] >> (8 * b + 6)) & 3) | (((pw[1] >> (8 * b + 6)) & 3) << 2) |
                                                (((pw[2] >> (8 * b + 6)) & 3) << 4)));
            v[4 * j + 3] = make_float4(hi[0], hi[1], hi[2], hi[3]);
        }
    } else {
        // unit 2l+p: codes 0..15 the low nibbles of its 16 bytes, 16..31 the high nibbles
        const float dd = half_bits_to_float((uint16_t)(ch.dd[0] & 0xffff));
        const float dm = half_bits_to_float((uint16_t)(ch.dd[0] >> 16));
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint32_t b = (ch.s2[0] >> (8 * p)) & 0xff;
            const int sc = b & 63, mn = ((b >> 6) << 4) | ((ch.m4[0] >> (4 * p)) & 15);
#pragma unroll
            for (int wd = 0; wd < 4; ++wd) {
                const uint32_t q = lane_word(ch.q[0][p], wd);
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    v[8 * p + 4 * h + wd] = make_float4(
                        q4k_weight(dd, dm, sc, mn, (q >> (4 * h)) & 15), q4k_weight(dd, dm, sc, mn, (q >> (8 + 4 * h)) & 15),
                        q4k_weight(dd, dm, sc, mn, (q >> (16 + 4 * h)) & 15),
                        q4k_weight(dd, dm, sc, mn, (q >> (24 + 4 * h)) & 15));
            }
        }
    }
}

template <int T>
__global__ __launch_bounds__(256) void dequant_chunks_kernel(const uint8_t* w, int cols, uint64_t row0, uint64_t n,
                                                             float* out) {
    __shared__ float4 tile[4][64 * 17];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, chunks = cols / kChunkCols;
    const uint64_t items = n * (uint64_t)chunks, stride = (uint64_t)gridDim.x * 4;
    const uint64_t row_bytes = (uint64_t)(cols / 256) * Fmt<T>::block;
    float4* t = tile[wave];
    auto load = [&](SChunk<T, 1>& ch, uint64_t item) {
        const uint64_t r = item / (uint64_t)chunks;
        const uint8_t* rp = w + (row0 + r) * row_bytes;
        sload<T, 1>(ch, &rp, (int)(item - r * (uint64_t)chunks), lane);
    };
    uint64_t it = (uint64_t)blockIdx.x * 4 + wave;
    SChunk<T, 1> cur, nxt;
    if (it < items) load(cur, it);
    for (; it < items; it += stride) {
        if (it + stride < items) load(nxt, it + stride);
        float4 v[16];
        dequant_chunk_values<T>(cur, v);
#pragma unroll
        for (int i = 0; i < 16; ++i) t[lane * 17 + i] = v[i];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // float4 q = 64i + lane of the chunk comes from lane q/16, its float4 q%16; the item
        // is row r, chunk c, so the chunk starts at r*cols + c*4096 = item*4096
        float4* o = reinterpret_cast<float4*>(out + it * (uint64_t)kChunkCols);
#pragma unroll
        for (int i = 0; i < 16; ++i) o[64 * i + lane] = t[(4 * i + (lane >> 4)) * 17 + (lane & 15)];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        cur = nxt;
    }
}

// The same values for rows whose width is a multiple of 1024 (the GEMM path's weights):
// workgroup = (row, 1024-column segment) by 32-bit block index, each thread four
// consecutive columns and one 16-byte store.
__global__ __launch_bounds__(256) void dequant_rows_1k_kernel(const uint8_t* w, uint32_t type, int cols, uint64_t row0,
                                                              float* out) {
    const int segs = cols >> 10;
    const uint32_t r = blockIdx.x / segs;
    const int k = (blockIdx.x - r * segs) * 1024 + 4 * threadIdx.x;
    float4 v;
    v.x = decode_element(w, type, cols, row0 + r, k);
    v.y = decode_element(w, type, cols, row0 + r, k + 1);
    v.z = decode_element(w, type, cols, row0 + r, k + 2);
    v.w = decode_element(w, type, cols, row0 + r, k + 3);
    *reinterpret_cast<float4*>(out + (size_t)r * cols + k) = v;
}

// ---- small batches: K inputs through one chunked matrix, its weights read once ----------
//
// linear_batch for 2 <= K <= kBatchMax rows of X (the reference's chunked prefill and
// draft verification batch up to 4 positions, cuda.cpp:350-413, model.cpp:355-366). A
// wave takes whole rows (rows v, v + waves, ...), loads each 4096-column chunk of its row
// once -- the next chunk's loads in flight while the current one is computed -- decodes
// it once and runs the single-input arithmetic (scompute's product chains) on it for every
// staged input, so the K outputs of a row are K single-input dot products over the same
// decoded weights. The inputs sit
// in LDS side by side, each in the streaming kernels' lane layout with its unit sums;
// one 16-wave workgroup per CU.
constexpr int kBatchWaves = 16;

// The codes of a chunk's unit as floats, converted once for all K inputs (the
// conversions are exact, so every product and sum below is scompute's for that input).
__device__ __forceinline__ void codes4(uint32_t q, float* w) {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = ubyte_f(q, i);
}
__device__ __forceinline__ float dot4f(const float* w, const float4& x, float acc) {
    acc = fmaf(w[0], x.x, acc);
    acc = fmaf(w[1], x.y, acc);
    acc = fmaf(w[2], x.z, acc);
    acc = fmaf(w[3], x.w, acc);
    return acc;
}

// scompute<T, 1> of one weight item for K staged inputs (input k at xs + k * xstride,
// its unit sums at usum + k * ustride): the weights are decoded once, then each input
// runs scompute's product chains in scompute's order.
template <int T, int K>
__device__ __forceinline__ void scompute_k(const SChunk<T, 1>& ch, float* acc, const float* xs, size_t xstride,
                                           const float* usum, size_t ustride, int c, int lane) {
    if constexpr (T == kQ6K) {
        const float dv = half_bits_to_float((uint16_t)ch.d[0]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d0 = lane_word(ch.q[0][0], j), d1 = lane_word(ch.q[0][1], j), d2 = lane_word(ch.q[0][2], j);
            float wa[4], wb[4], wc[4], we[4];
            codes4(opaque(d0 & 0x3F3F3F3Fu), wa);
            codes4(opaque(d1 & 0x3F3F3F3Fu), wb);
            codes4(opaque(d2 & 0x3F3F3F3Fu), wc);
            codes4(opaque(((d0 >> 6) & 0x03030303u) | ((d1 >> 4) & 0x0C0C0C0Cu) | ((d2 >> 2) & 0x30303030u)), we);
            const float scale = dv * (float)(int)(int8_t)(ch.sc[0] >> (8 * j));
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const float4* x4 = reinterpret_cast<const float4*>(xs + k * xstride) + (size_t)c * 1024 + lane;
                const float4 off4 = reinterpret_cast<const float4*>(usum + k * ustride)[c * 64 + lane];
                const float off = j == 0 ? off4.x : j == 1 ? off4.y : j == 2 ? off4.z : off4.w;
                float4 xv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) xv[i] = x4[(j * 4 + i) * 64];
                float s0 = dot4f(wa, xv[0], off);
                float s1 = dot4f(wb, xv[1], 0.f);
                s0 = dot4f(wc, xv[2], s0);
                s1 = dot4f(we, xv[3], s1);
                acc[k] = fmaf(scale, s0 + s1, acc[k]);
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const uint4 d = ch.q[0][p];
            float w[8][4];
            codes4(opaque(d.x & 0x0F0F0F0Fu), w[0]);
            codes4(opaque(d.y & 0x0F0F0F0Fu), w[1]);
            codes4(opaque(d.z & 0x0F0F0F0Fu), w[2]);
            codes4(opaque(d.w & 0x0F0F0F0Fu), w[3]);
            codes4(opaque((d.x >> 4) & 0x0F0F0F0Fu), w[4]);
            codes4(opaque((d.y >> 4) & 0x0F0F0F0Fu), w[5]);
            codes4(opaque((d.z >> 4) & 0x0F0F0F0Fu), w[6]);
            codes4(opaque((d.w >> 4) & 0x0F0F0F0Fu), w[7]);
            const uint32_t b = (ch.s2[0] >> (8 * p)) & 0xff;
            const int sc = b & 63;
            const int mn = ((b >> 6) << 4) | ((ch.m4[0] >> (4 * p)) & 15);
            const float dd = half_bits_to_float((uint16_t)(ch.dd[0] & 0xffff));
            const float dm = half_bits_to_float((uint16_t)(ch.dd[0] >> 16));
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const float4* x4 = reinterpret_cast<const float4*>(xs + k * xstride) + (size_t)c * 1024 + lane;
                const float2 xsum = reinterpret_cast<const float2*>(usum + k * ustride)[c * 64 + lane];
                float4 xv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) xv[i] = x4[(p * 8 + i) * 64];
                float s0 = dot4f(w[0], xv[0], 0.f);
                float s1 = dot4f(w[1], xv[1], 0.f);
                s0 = dot4f(w[2], xv[2], s0);
                s1 = dot4f(w[3], xv[3], s1);
                s0 = dot4f(w[4], xv[4], s0);
                s1 = dot4f(w[5], xv[5], s1);
                s0 = dot4f(w[6], xv[6], s0);
                s1 = dot4f(w[7], xv[7], s1);
                acc[k] += (dd * (float)sc) * (s0 + s1) - (dm * (float)mn) * (p == 0 ? xsum.x : xsum.y);
            }
        }
    }
}

template <int T, int K>
__global__ __launch_bounds__(kBatchWaves * 64) void matvec_batch_kernel(MvBatchArgs a) {
    extern __shared__ __align__(16) unsigned char smem[];
    constexpr int UW = Fmt<T>::unit, U4 = UW / 4;
    const int cols = a.cols, units = cols / UW, n4 = cols / 4, cpr = cols / kChunkCols;
    float* xs = reinterpret_cast<float*>(smem);
    float* usum = xs + (size_t)K * cols;
    float4* xs4 = reinterpret_cast<float4*>(xs);
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const float4* x4 = reinterpret_cast<const float4*>(a.x + (size_t)k * a.ldx);
        for (int i = threadIdx.x; i < n4; i += blockDim.x) xs4[(size_t)k * n4 + chunk_slot(i)] = x4[i];
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < K; ++k)
        for (int u = threadIdx.x; u < units; u += blockDim.x) {
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < U4; ++j) {
                const float4 v = xs4[(size_t)k * n4 + chunk_slot(u * U4 + j)];
                sum += (v.x + v.y) + (v.z + v.w);
            }
            usum[(size_t)k * units + u] = stored_unit_sum<UW>(sum);
        }
    __syncthreads();

    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int waves = gridDim.x * kBatchWaves;
    const size_t row_bytes = (size_t)(cols / 256) * Fmt<T>::block;
    for (int row = blockIdx.x * kBatchWaves + wave; row < a.rows; row += waves) {
        const uint8_t* rp[1] = {a.w + (size_t)row * row_bytes};
        float acc[K];
#pragma unroll
        for (int k = 0; k < K; ++k) acc[k] = 0.f;
        SChunk<T, 1> cur, next;
        sload<T, 1>(cur, rp, 0, lane);
        for (int c = 0; c < cpr; ++c) {
            if (c + 1 < cpr) sload<T, 1>(next, rp, c + 1, lane);
            scompute_k<T, K>(cur, acc, xs, (size_t)cols, usum, (size_t)units, c, lane);
            cur = next;
        }
#pragma unroll
        for (int k = 0; k < K; ++k) acc[k] = wave_sum(acc[k]);
        if (lane == 0)
#pragma unroll
            for (int k = 0; k < K; ++k) a.y[(size_t)k * a.ldy + row] = acc[k];
    }
}

}  // namespace

// ---- host launchers ------------------------------------------------------------------

size_t matvec_batch_lds_bytes(uint32_t type, int cols, int k) {
    const int unit = type == kQ6K ? 16 : 32;
    return (size_t)k * ((size_t)cols * 4 + (size_t)(cols / unit) * 4);
}

template <int T, int K> hipError_t launch_batch_k(const MvBatchArgs& a, size_t lds, hipStream_t stream) {
    const void* fn = reinterpret_cast<const void*>(matvec_batch_kernel<T, K>);
    const int cap = resident_blocks(fn, lds, kBatchWaves);
    int blocks = (a.rows + kBatchWaves - 1) / kBatchWaves;
    if (blocks > cap) blocks = cap;
    if (blocks < 1) blocks = 1;
    launch_kernel(matvec_batch_kernel<T, K>, dim3(blocks), dim3(kBatchWaves * 64), lds, stream, a);
    return hipGetLastError();
}

template <int T> hipError_t launch_batch_t(const MvBatchArgs& a, int k, size_t lds, hipStream_t stream) {
    switch (k) {
    case 1: return launch_batch_k<T, 1>(a, lds, stream);
    case 2: return launch_batch_k<T, 2>(a, lds, stream);
    case 3: return launch_batch_k<T, 3>(a, lds, stream);
    case 4: return launch_batch_k<T, 4>(a, lds, stream);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_matvec_batch(uint32_t type, const MvBatchArgs& a, int k, hipStream_t stream) {
    if ((type != kQ6K && type != kQ4K) || a.cols % kChunkCols || k < 1 || k > kBatchMax || a.ldx % 4 ||
        reinterpret_cast<uintptr_t>(a.x) % 16)
        return hipErrorInvalidValue;
    const size_t lds = matvec_batch_lds_bytes(type, a.cols, k);
    if (lds > kBatchLdsMax) return hipErrorInvalidValue;
    return type == kQ6K ? launch_batch_t<kQ6K>(a, k, lds, stream) : launch_batch_t<kQ4K>(a, k, lds, stream);
}

size_t matvec_lds_bytes(uint32_t type, int cols, bool q8) {
    if (type == kQ6K || type == kQ4K) {
        const int unit = type == kQ6K ? 16 : 32;
        size_t b = (size_t)cols * 4 + (size_t)(cols / unit) * 4;
        if (q8) b += (size_t)cols + (size_t)(cols / 32) * 4 + (size_t)(cols / 16) * 4;
        return b;
    }
    return (size_t)cols * 4 + 16;
}

hipError_t launch_matvec(uint32_t type, bool q8, const MvArgs& a, int grid_cap, hipStream_t stream) {
    const size_t lds = matvec_lds_bytes(type, a.cols, q8);
    int blocks = (a.groups + 3) / 4;
    if (blocks > grid_cap) blocks = grid_cap;
    if (blocks < 1) blocks = 1;
    const dim3 grid(blocks), block(256);
    const bool pair = a.mode == kMvSwiglu;
    if ((type == kQ6K || type == kQ4K) && a.cols % kChunkCols == 0) return launch_matvec_stream(type, q8, a, stream);
    if (a.gate) return hipErrorInvalidValue;  // the per-head input transform is a streaming-kernel feature
    switch (type) {
    case kQ6K:
        if (q8) {
            if (pair) launch_kernel((matvec_kernel<kQ6K, kMvRows, true, true>), grid, block, lds, stream, a);
            else launch_kernel((matvec_kernel<kQ6K, kMvRows, true, false>), grid, block, lds, stream, a);
        } else {
            if (pair) launch_kernel((matvec_kernel<kQ6K, kMvRows, false, true>), grid, block, lds, stream, a);
            else launch_kernel((matvec_kernel<kQ6K, kMvRows, false, false>), grid, block, lds, stream, a);
        }
        break;
    case kQ4K:
        if (pair) launch_kernel((matvec_kernel<kQ4K, kMvRows, false, true>), grid, block, lds, stream, a);
        else launch_kernel((matvec_kernel<kQ4K, kMvRows, false, false>), grid, block, lds, stream, a);
        break;
    case kF32: launch_kernel((matvec_raw_kernel<kF32>), grid, block, lds, stream, a); break;
    case kF16: launch_kernel((matvec_raw_kernel<kF16>), grid, block, lds, stream, a); break;
    case kBF16: launch_kernel((matvec_raw_kernel<kBF16>), grid, block, lds, stream, a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_dequant_rows(const uint8_t* w, uint32_t type, int cols, uint64_t row0, uint64_t n, float* out,
                               hipStream_t stream) {
    const uint64_t total = n * (uint64_t)cols;
    const bool aligned = reinterpret_cast<uintptr_t>(out) % 16 == 0;
    if ((type == kQ6K || type == kQ4K) && cols % kChunkCols == 0 && n > 0 && aligned) {
        const uint64_t blocks = std::min<uint64_t>((n * (uint64_t)(cols / kChunkCols) + 3) / 4, kDequantGrid);
        {
            if (type == kQ6K) launch_kernel(dequant_chunks_kernel<kQ6K>, dim3((unsigned)blocks), dim3(256), 0, stream, w, cols, row0, n, out);
            else launch_kernel(dequant_chunks_kernel<kQ4K>, dim3((unsigned)blocks), dim3(256), 0, stream, w, cols, row0, n, out);
            return hipGetLastError();
        }
    }
    if (cols % 1024 == 0 && total > 0 && total / 1024 < (1ull << 31) && reinterpret_cast<uintptr_t>(out) % 16 == 0) {
        launch_kernel(dequant_rows_1k_kernel, dim3((unsigned)(total / 1024)), dim3(256), 0, stream, w, type, cols, row0,
                      out);
        return hipGetLastError();
    }
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks < 1) blocks = 1;
    launch_kernel(dequant_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, w, type, cols, row0, n, out);
    return hipGetLastError();
}

}  // namespace emprise
