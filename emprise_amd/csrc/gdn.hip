// Gated DeltaNet decode step on gfx950 (Backend::delta_net, reference
// backend.cpp:19-60; the CUDA delta_conv/delta_scan/delta_norm_gate, cuda.cpp:417-479).
//
// Two forms. gdn_rows_kernel (the recurrent block's path when the out-projection is in
// the chunked layout) splits each head's rows over SPLIT workgroups and writes the raw
// outputs S.q; the per-head RMSNorm x gate then runs in the out-projection's input
// staging, and the gate rows arrive already SiLU'd from the in-projection. gdn_kernel
// (Backend::delta_net, and the other out-projection widths) does the whole head:
// one workgroup per value head (8 waves). The head's q/k are L2-normalised inside the
// workgroup (every wave redundantly; 2*state_dim values), the 64 KiB state of the head
// is streamed once -- each wave loads all of its rows before any arithmetic so the
// reads overlap -- updated in registers and written back, and the per-head RMSNorm x
// SiLU(gate) is applied before the single write of the head's output. Lane l of a wave
// holds state columns l, l+64 (state_dim = 64*E), so every row access is one coalesced
// 256-byte (E=1) or 512-byte (E=2) transfer.
#include "common.hpp"
#include "kernels.hpp"

namespace emprise {
namespace {

constexpr int kGdnWaves = 8;

__global__ void delta_conv_kernel(const float* qkv, const float* w, float* hist, float* out, int channels, int cw) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= channels) return;
    float* h = hist + (size_t)c * cw;
    const float* k = w + (size_t)c * cw;
    float sum = 0.f;
    for (int j = 0; j < cw - 1; ++j) {
        const float hv = h[j + 1];
        h[j] = hv;
        sum += hv * k[j];
    }
    const float v = qkv[c];
    h[cw - 1] = v;
    sum += v * k[cw - 1];
    out[c] = siluf_(sum);
}

template <int E>
__global__ __launch_bounds__(kGdnWaves * 64) void gdn_kernel(GdnArgs a) {
    constexpr int SD = 64 * E, RPW = SD / kGdnWaves;  // rows per wave
    __shared__ float o_row[SD];
    const int h = blockIdx.x, kh = h % a.key_heads;  // tiled V-head order (backend.cpp:37)
    const int key_dim = a.key_heads * SD;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const float* q = a.qkv + (size_t)kh * SD;
    const float* k = a.qkv + key_dim + (size_t)kh * SD;
    const float* v = a.qkv + 2 * (size_t)key_dim + (size_t)h * SD;
    float* S = a.state + (size_t)h * SD * SD;

    // issue the state reads of this wave's rows first; lane r also fetches v of row r
    // (read back with readlane, so no load waits behind the state stores of the loop)
    const float v_lane = lane < RPW ? v[wave * RPW + lane] : 0.f;
    float s[RPW][E];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int e = 0; e < E; ++e) s[r][e] = S[(size_t)(wave * RPW + r) * SD + lane + 64 * e];

    // q/k L2 normalisation (backend.cpp:30-35): qscale = 1/sqrt(sum q^2 + eps)/sqrt(SD)
    float qv[E], kv[E], qs = 0.f, ks = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        qv[e] = q[lane + 64 * e];
        kv[e] = k[lane + 64 * e];
        qs += qv[e] * qv[e];
        ks += kv[e] * kv[e];
    }
    qs = wave_sum(qs);
    ks = wave_sum(ks);
    const float qscale = 1.f / sqrtf(qs + a.eps) / sqrtf((float)SD), kscale = 1.f / sqrtf(ks + a.eps);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        qv[e] *= qscale;
        kv[e] *= kscale;
    }
    const float decay = expf(a.ssm_a[h] * softplusf_(a.alpha[h] + a.dt[h]));
    const float b = sigmoidf_(a.beta[h]);

#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int d = wave * RPW + r;
        float mem = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            s[r][e] *= decay;
            mem += s[r][e] * kv[e];
        }
        mem = wave_sum(mem);
        const float vd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_lane), r));
        const float delta = (vd - mem) * b;
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            s[r][e] += kv[e] * delta;
            sum += s[r][e] * qv[e];
        }
        sum = wave_sum(sum);
#pragma unroll
        for (int e = 0; e < E; ++e) S[(size_t)d * SD + lane + 64 * e] = s[r][e];
        if (lane == 0) o_row[d] = sum;
    }
    __syncthreads();
    // per-head RMSNorm with ssm_norm, then SiLU(gate) (backend.cpp:57-58)
    if (wave == 0) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) ss += o_row[lane + 64 * e] * o_row[lane + 64 * e];
        ss = wave_sum(ss);
        const float scale = 1.f / sqrtf(ss / (float)SD + a.eps);
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int j = lane + 64 * e;
            a.out[(size_t)h * SD + j] = o_row[j] * (scale * a.norm[j]) * siluf_(a.gate[(size_t)h * SD + j]);
        }
    }
}

// The state update of rows [part*SD/SPLIT, (part+1)*SD/SPLIT) of value head h, with
// workgroup blockIdx = h*SPLIT + part; each of the 8 waves owns RPW rows and writes their
// raw outputs o[d] = S[d,:].q straight to global memory (no cross-wave step). q and k
// are L2-normalised by every workgroup of the head (2*SD values).
template <int E, int SPLIT>
__global__ __launch_bounds__(kGdnWaves * 64) void gdn_rows_kernel(GdnArgs a) {
    constexpr int SD = 64 * E, RPW = SD / SPLIT / kGdnWaves;
    static_assert(RPW >= 1 && RPW <= 64, "rows per wave");
    const int h = blockIdx.x / SPLIT, part = blockIdx.x - h * SPLIT, kh = h % a.key_heads;
    const int key_dim = a.key_heads * SD;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int d0 = part * (SD / SPLIT) + wave * RPW;
    const float* q = a.qkv + (size_t)kh * SD;
    const float* k = a.qkv + key_dim + (size_t)kh * SD;
    const float* v = a.qkv + 2 * (size_t)key_dim + (size_t)h * SD;
    float* S = a.state + (size_t)h * SD * SD;

    // all loads first: the wave's state rows, v of its rows (lane r holds row d0 + r),
    // q and k
    float s[RPW][E];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int e = 0; e < E; ++e) s[r][e] = S[(size_t)(d0 + r) * SD + lane + 64 * e];
    const float v_lane = v[d0 + min(lane, RPW - 1)];
    float qv[E], kv[E], qs = 0.f, ks = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        qv[e] = q[lane + 64 * e];
        kv[e] = k[lane + 64 * e];
        qs += qv[e] * qv[e];
        ks += kv[e] * kv[e];
    }
    qs = wave_sum(qs);
    ks = wave_sum(ks);
    const float qscale = 1.f / sqrtf(qs + a.eps) / sqrtf((float)SD), kscale = 1.f / sqrtf(ks + a.eps);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        qv[e] *= qscale;
        kv[e] *= kscale;
    }
    const float decay = expf(a.ssm_a[h] * softplusf_(a.alpha[h] + a.dt[h]));
    const float b = sigmoidf_(a.beta[h]);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        float mem = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            s[r][e] *= decay;
            mem += s[r][e] * kv[e];
        }
        mem = wave_sum(mem);
        const float vd = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v_lane), r));
        const float delta = (vd - mem) * b;
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            s[r][e] += kv[e] * delta;
            sum += s[r][e] * qv[e];
        }
        sum = wave_sum(sum);
#pragma unroll
        for (int e = 0; e < E; ++e) S[(size_t)(d0 + r) * SD + lane + 64 * e] = s[r][e];
        if (lane == 0) a.out[(size_t)h * SD + d0 + r] = sum;
    }
}

// ---- batched form: `count` consecutive positions (the prompt prefill) -------------------
//
// Position by position, the decode kernels above pay two launches and two dependent
// memory round trips per position and layer. Over a prompt the three stages separate:
// the conv1d is a scan per channel (one thread keeps a channel's history in registers
// over all positions), the delta rule a scan per state row (one wave keeps its row in
// registers over all positions) after a parallel pass that normalises q/k and forms the
// decay and beta gate of every position, and the per-head RMSNorm x SiLU(gate) is
// independent per position. Each step does the arithmetic of delta_conv_kernel and gdn_kernel in the
// same order, so the outputs and the final states are those of `count` calls of the
// per-position path.

// conv1d + SiLU of every (position, channel). Output t reads only inputs t-CW+1 .. t
// (the ones before the prompt from the history), so the positions are independent:
// thread = (channel, kConvSpan consecutive positions), channels across the threads of a
// workgroup for coalesced rows. The sum runs in delta_conv_kernel's order, so the outputs
// are its outputs bit for bit; the history moves on in delta_conv_history_kernel, once
// every read of the old one is done.
constexpr int kConvSpan = 8;

template <int CW>
__global__ __launch_bounds__(256) void delta_conv_batch_kernel(GdnBatchArgs a) {
    constexpr int U = kConvSpan;
    const int c = blockIdx.x * 256 + threadIdx.x, t0 = blockIdx.y * U;
    const int ch = 2 * a.key_heads * a.state_dim + a.value_heads * a.state_dim;
    if (c >= ch) return;
    const float* hist = a.conv_state + (size_t)c * CW;
    float k[CW], y[CW - 1 + U];  // y[i]: input of position t0 - (CW-1) + i
#pragma unroll
    for (int j = 0; j < CW; ++j) k[j] = a.conv_w[(size_t)c * CW + j];
#pragma unroll
    for (int i = 0; i < CW - 1; ++i) {
        const int m = t0 - (CW - 1) + i;
        y[i] = m >= 0 ? a.qkv[(size_t)m * a.stride + c] : hist[CW + m];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) y[CW - 1 + u] = a.qkv[(size_t)min(t0 + u, a.count - 1) * a.stride + c];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (t0 + u < a.count) {
            float sum = 0.f;
#pragma unroll
            for (int j = 0; j < CW - 1; ++j) sum += y[u + j] * k[j];
            sum += y[u + CW - 1] * k[CW - 1];
            a.conv_out[(size_t)(t0 + u) * ch + c] = siluf_(sum);
        }
    }
}

// The history after the prompt: the last CW inputs of (old history, prompt). One thread
// per channel, ascending, so each old entry is read before its slot is overwritten.
template <int CW>
__global__ __launch_bounds__(256) void delta_conv_history_kernel(GdnBatchArgs a) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int ch = 2 * a.key_heads * a.state_dim + a.value_heads * a.state_dim;
    if (c >= ch) return;
    float* hist = a.conv_state + (size_t)c * CW;
#pragma unroll
    for (int i = 0; i < CW; ++i) {
        const int m = a.count - CW + i;
        hist[i] = m >= 0 ? a.qkv[(size_t)m * a.stride + c] : hist[CW + m];
    }
}

// The per-position inputs of the delta rule that every row of a head shares, computed
// once per position instead of once per row: the L2-normalised q and k of each key head
// (a wave per (position, key head), lane l keeping columns l, l+64 as gdn_kernel does, so
// the sums and scales are gdn_kernel's bit for bit), stored lane-interleaved -- lane l's
// q[l], q[l+64], k[l], k[l+64] are consecutive, one 16-byte load in the scan -- and the
// decay and beta gate of each value head.
template <int E>
__global__ __launch_bounds__(256) void gdn_prep_batch_kernel(GdnBatchArgs a) {
    constexpr int SD = 64 * E;
    const int lane = threadIdx.x & 63;
    const int pair = blockIdx.x * 4 + (threadIdx.x >> 6);  // position * key_heads + key head
    const int key_dim = a.key_heads * SD, ch = 2 * key_dim + a.value_heads * SD;
    if (pair < a.count * a.key_heads) {
        const int t = pair / a.key_heads, kh = pair - t * a.key_heads;
        const float* row = a.conv_out + (size_t)t * ch;
        // q/k L2 normalisation (backend.cpp:30-35), as gdn_kernel
        float qv[E], kv[E], qs = 0.f, ks = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            qv[e] = row[(size_t)kh * SD + lane + 64 * e];
            kv[e] = row[key_dim + (size_t)kh * SD + lane + 64 * e];
            qs += qv[e] * qv[e];
            ks += kv[e] * kv[e];
        }
        qs = wave_sum(qs);
        ks = wave_sum(ks);
        const float qscale = 1.f / sqrtf(qs + a.eps) / sqrtf((float)SD), kscale = 1.f / sqrtf(ks + a.eps);
        float* dst = a.qk + ((size_t)pair * 64 + lane) * 2 * E;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            dst[e] = qv[e] * qscale;
            dst[E + e] = kv[e] * kscale;
        }
    }
    const int i = blockIdx.x * 256 + threadIdx.x;  // position * value_heads + value head
    if (i < a.count * a.value_heads) {
        const int t = i / a.value_heads, h = i - t * a.value_heads;
        a.gates[2 * (size_t)i] = expf(a.ssm_a[h] * softplusf_(a.alpha[(size_t)t * a.stride + h] + a.dt[h]));
        a.gates[2 * (size_t)i + 1] = sigmoidf_(a.beta[(size_t)t * a.stride + h]);
    }
}

template <int E> __device__ __forceinline__ void load_qk(const float* p, float (&q)[E], float (&k)[E]) {
    if constexpr (E == 2) {
        const float4 v = *reinterpret_cast<const float4*>(p);
        q[0] = v.x, q[1] = v.y, k[0] = v.z, k[1] = v.w;
    } else {
        const float2 v = *reinterpret_cast<const float2*>(p);
        q[0] = v.x, k[0] = v.y;
    }
}

constexpr int kScanAhead = 8;  // positions whose q/k are in flight ahead of the one in use
// workgroups per value head of the scan at state_dim 64 / 128: one row per wave (two
// rows per wave measured the same, 15.9 ms per 2048-token 9B prefill: the chain of wave
// reductions bounds it, not the loads)
constexpr int kScanSplit1 = 8, kScanSplit2 = 16;

// Rows [part*SD/SPLIT, (part+1)*SD/SPLIT) of value head h over all positions; RPW
// consecutive rows per wave, their states in registers throughout. The chain per
// position is the update itself -- two wave reductions per row, the rows' chains
// interleaved -- with the inputs already in registers: q/k of the next kScanAhead
// positions are in flight, and each row's v and the head's decay and beta gate of 64
// positions arrive in one load each (lane u holds position t0 + u; the next 64 load while
// these are used). The raw outputs S.q of 64 positions are collected the same way (lane
// u) and written with one store per row.
template <int E, int SPLIT>
__global__ __launch_bounds__(kGdnWaves * 64) void gdn_scan_kernel(GdnBatchArgs a) {
    constexpr int SD = 64 * E, RPW = SD / SPLIT / kGdnWaves, P = kScanAhead;
    static_assert(RPW >= 1 && RPW <= 4, "rows per wave");
    static_assert(64 % P == 0, "prefetch depth divides the 64-position block");
    const int h = blockIdx.x / SPLIT, part = blockIdx.x - h * SPLIT, kh = h % a.key_heads;
    const int key_dim = a.key_heads * SD, ch = 2 * key_dim + a.value_heads * SD;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int d0 = part * (SD / SPLIT) + wave * RPW, last = a.count - 1;
    float* S = a.state + (size_t)h * SD * SD + (size_t)d0 * SD;
    float s[RPW][E];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int e = 0; e < E; ++e) s[r][e] = S[(size_t)r * SD + lane + 64 * e];

    const size_t qk_step = (size_t)a.key_heads * 64 * 2 * E;  // floats per position
    const float* qk = a.qk + ((size_t)kh * 64 + lane) * 2 * E;
    const float* v_col = a.conv_out + 2 * (size_t)key_dim + (size_t)h * SD + d0;
    const size_t o_step = (size_t)a.value_heads * SD;
    float* o_col = a.o + (size_t)h * SD + d0;

    float rq[P][E], rk[P][E];  // position t's q/k sit in slot t % P
#pragma unroll
    for (int u = 0; u < P; ++u) load_qk<E>(qk + (size_t)min(u, last) * qk_step, rq[u], rk[u]);
    // lane u: the rows' v and the head's decay and beta gate of position t0 + u
    struct Lanes {
        float v[RPW], dec, b;
    };
    auto lane_inputs = [&](int t0, Lanes& l) {
        const int t = min(t0 + lane, last);
#pragma unroll
        for (int r = 0; r < RPW; ++r) l.v[r] = v_col[(size_t)t * ch + r];
        const float2 g = *reinterpret_cast<const float2*>(a.gates + 2 * ((size_t)t * a.value_heads + h));
        l.dec = g.x, l.b = g.y;
    };
    // positions t0 .. t0+63 with their lane inputs in `cur`, while those of the next 64
    // load into `nxt`
    auto block = [&](int t0, const Lanes& cur, Lanes& nxt) {
        lane_inputs(t0 + 64, nxt);
        const int n = min(64, a.count - t0);
        float ol[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) ol[r] = 0.f;
        for (int u0 = 0; u0 < n; u0 += P) {
#pragma unroll
            for (int j = 0; j < P; ++j) {
                const int u = u0 + j, t = t0 + u;
                if (u < n) {
                    const float(&qv)[E] = rq[j];
                    const float(&kv)[E] = rk[j];
                    const float decay = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.dec), u));
                    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.b), u));
                    float mem[RPW], sum[RPW];
#pragma unroll
                    for (int r = 0; r < RPW; ++r) {
                        mem[r] = 0.f;
#pragma unroll
                        for (int e = 0; e < E; ++e) {
                            s[r][e] *= decay;
                            mem[r] += s[r][e] * kv[e];
                        }
                    }
#pragma unroll
                    for (int r = 0; r < RPW; ++r) mem[r] = wave_sum(mem[r]);
#pragma unroll
                    for (int r = 0; r < RPW; ++r) {
                        const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.v[r]), u));
                        const float delta = (v - mem[r]) * b;
                        sum[r] = 0.f;
#pragma unroll
                        for (int e = 0; e < E; ++e) {
                            s[r][e] += kv[e] * delta;
                            sum[r] += s[r][e] * qv[e];
                        }
                    }
#pragma unroll
                    for (int r = 0; r < RPW; ++r) {
                        sum[r] = wave_sum(sum[r]);
                        ol[r] = lane == u ? sum[r] : ol[r];
                    }
                }
                // refill the slot once its position is done, so the load lands in the same
                // registers (a refill issued while the slot is still read needs a copy at
                // the loop's back edge, and with it a wait for the load)
                load_qk<E>(qk + (size_t)min(t + P, last) * qk_step, rq[j], rk[j]);
            }
        }
        if (lane < n)
#pragma unroll
            for (int r = 0; r < RPW; ++r) o_col[(size_t)(t0 + lane) * o_step + r] = ol[r];
    };
    // two register sets in turn, so no copy (and no wait for the next block's loads) sits
    // between blocks
    Lanes la, lb;
    lane_inputs(0, la);
    // Everything above has arrived before the loop starts, so the wait the compiler
    // places before each slot's use is the steady state's (the loads of the following
    // slots stay in flight), not one shaped by the order of these first loads.
    __builtin_amdgcn_s_waitcnt(0);
    for (int t0 = 0; t0 < a.count; t0 += 128) {
        block(t0, la, lb);
        if (t0 + 64 < a.count) block(t0 + 64, lb, la);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int e = 0; e < E; ++e) S[(size_t)r * SD + lane + 64 * e] = s[r][e];
}

// Per-head RMSNorm with ssm_norm, then SiLU(gate) (backend.cpp:57-58), as gdn_kernel's
// epilogue; workgroup (position, head), one wave.
template <int E>
__global__ __launch_bounds__(64) void gdn_norm_gate_batch_kernel(GdnBatchArgs a) {
    constexpr int SD = 64 * E;
    const int t = blockIdx.x / a.value_heads, h = blockIdx.x - t * a.value_heads, lane = threadIdx.x;
    const float* o = a.o + (size_t)t * a.value_heads * SD + (size_t)h * SD;
    const float* gate = a.gate + (size_t)t * a.stride + (size_t)h * SD;
    float ov[E], ss = 0.f;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        ov[e] = o[lane + 64 * e];
        ss += ov[e] * ov[e];
    }
    ss = wave_sum(ss);
    const float scale = 1.f / sqrtf(ss / (float)SD + a.eps);
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const int j = lane + 64 * e;
        a.out[(size_t)t * a.out_stride + (size_t)h * SD + j] = ov[e] * (scale * a.norm[j]) * siluf_(gate[j]);
    }
}

}  // namespace

hipError_t launch_gdn_batch(const GdnBatchArgs& a, hipStream_t stream) {
    if (a.count < 1 || a.count > 65535 * kConvSpan || (a.state_dim != 64 && a.state_dim != 128))
        return hipErrorInvalidValue;
    const int ch = 2 * a.key_heads * a.state_dim + a.value_heads * a.state_dim;
    const dim3 cgrid((ch + 255) / 256, (a.count + kConvSpan - 1) / kConvSpan), hgrid((ch + 255) / 256), cblock(256);
#define EMPRISE_CONV_CASE(W)                                                              \
    case W:                                                                               \
        launch_kernel(delta_conv_batch_kernel<W>, cgrid, cblock, 0, stream, a);           \
        launch_kernel(delta_conv_history_kernel<W>, hgrid, cblock, 0, stream, a);         \
        break;
    switch (a.conv_width) {
        EMPRISE_CONV_CASE(1)
        EMPRISE_CONV_CASE(2)
        EMPRISE_CONV_CASE(3)
        EMPRISE_CONV_CASE(4)
        EMPRISE_CONV_CASE(5)
        EMPRISE_CONV_CASE(6)
        EMPRISE_CONV_CASE(7)
        EMPRISE_CONV_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef EMPRISE_CONV_CASE
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 block(kGdnWaves * 64);
    const int pgrid = std::max((a.count * a.key_heads + 3) / 4, (a.count * a.value_heads + 255) / 256);
    if (a.state_dim == 64) {
        launch_kernel(gdn_prep_batch_kernel<1>, dim3(pgrid), dim3(256), 0, stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        launch_kernel(gdn_scan_kernel<1, kScanSplit1>, dim3(a.value_heads * kScanSplit1), block, 0, stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        launch_kernel(gdn_norm_gate_batch_kernel<1>, dim3(a.count * a.value_heads), dim3(64), 0, stream, a);
    } else {
        launch_kernel(gdn_prep_batch_kernel<2>, dim3(pgrid), dim3(256), 0, stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        launch_kernel(gdn_scan_kernel<2, kScanSplit2>, dim3(a.value_heads * kScanSplit2), block, 0, stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        launch_kernel(gdn_norm_gate_batch_kernel<2>, dim3(a.count * a.value_heads), dim3(64), 0, stream, a);
    }
    return hipGetLastError();
}

hipError_t launch_gdn_rows(const GdnArgs& a, hipStream_t stream) {
    const dim3 block(kGdnWaves * 64);
    if (a.state_dim == 64) launch_kernel(gdn_rows_kernel<1, 2>, dim3(a.value_heads * 2), block, 0, stream, a);
    else if (a.state_dim == 128) launch_kernel(gdn_rows_kernel<2, 4>, dim3(a.value_heads * 4), block, 0, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_delta_conv(const float* qkv, const float* conv_w, float* conv_state, float* out, int channels,
                             int conv_width, hipStream_t stream) {
    launch_kernel(delta_conv_kernel, dim3((channels + 255) / 256), dim3(256), 0, stream, qkv, conv_w, conv_state,
                       out, channels, conv_width);
    return hipGetLastError();
}

hipError_t launch_gdn(const GdnArgs& a, hipStream_t stream) {
    const dim3 grid(a.value_heads), block(kGdnWaves * 64);
    if (a.state_dim == 64) launch_kernel(gdn_kernel<1>, grid, block, 0, stream, a);
    else if (a.state_dim == 128) launch_kernel(gdn_kernel<2>, grid, block, 0, stream, a);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace emprise
