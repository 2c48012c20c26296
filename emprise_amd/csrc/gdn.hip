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
// over all positions), the delta rule a scan per state row (one wave keeps its rows in
// registers over all positions, the next position's q/k/v/alpha/beta loading while the
// current one is used), and the per-head RMSNorm x SiLU(gate) is independent per
// position. Each step does the arithmetic of delta_conv_kernel and gdn_kernel in the
// same order, so the outputs and the final states are those of `count` calls of the
// per-position path.

template <int CW>
__global__ __launch_bounds__(256) void delta_conv_batch_kernel(GdnBatchArgs a) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    const int ch = 2 * a.key_heads * a.state_dim + a.value_heads * a.state_dim;
    if (c >= ch) return;
    float* hist = a.conv_state + (size_t)c * CW;
    float k[CW], h[CW];
#pragma unroll
    for (int j = 0; j < CW; ++j) {
        k[j] = a.conv_w[(size_t)c * CW + j];
        h[j] = hist[j];
    }
    constexpr int U = 8;  // positions whose inputs are loaded together
    for (int t0 = 0; t0 < a.count; t0 += U) {
        float x[U];
#pragma unroll
        for (int u = 0; u < U; ++u) x[u] = a.qkv[(size_t)min(t0 + u, a.count - 1) * a.stride + c];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (t0 + u < a.count) {
                float sum = 0.f;
#pragma unroll
                for (int j = 0; j < CW - 1; ++j) {
                    const float hv = h[j + 1];
                    h[j] = hv;
                    sum += hv * k[j];
                }
                h[CW - 1] = x[u];
                sum += x[u] * k[CW - 1];
                a.conv_out[(size_t)(t0 + u) * ch + c] = siluf_(sum);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < CW; ++j) hist[j] = h[j];
}

// Rows [part*SD/SPLIT, (part+1)*SD/SPLIT) of value head h over all positions; one row
// per wave. Writes the raw outputs S.q of every position.
template <int E, int SPLIT>
__global__ __launch_bounds__(kGdnWaves * 64) void gdn_scan_kernel(GdnBatchArgs a) {
    constexpr int SD = 64 * E, RPW = SD / SPLIT / kGdnWaves;
    static_assert(RPW == 1, "one row per wave");
    const int h = blockIdx.x / SPLIT, part = blockIdx.x - h * SPLIT, kh = h % a.key_heads;
    const int key_dim = a.key_heads * SD, ch = 2 * key_dim + a.value_heads * SD;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int d = part * (SD / SPLIT) + wave;
    float* S = a.state + (size_t)h * SD * SD + (size_t)d * SD;
    float s[E];
#pragma unroll
    for (int e = 0; e < E; ++e) s[e] = S[lane + 64 * e];
    const float A = a.ssm_a[h], DT = a.dt[h];

    // inputs of position t: q and k of the key head, v of the row, alpha and beta
    struct In {
        float q[E], k[E], v, al, be;
    };
    auto load = [&](In& in, int t) {
        const float* row = a.conv_out + (size_t)t * ch;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            in.q[e] = row[(size_t)kh * SD + lane + 64 * e];
            in.k[e] = row[key_dim + (size_t)kh * SD + lane + 64 * e];
        }
        in.v = row[2 * (size_t)key_dim + (size_t)h * SD + d];
        in.al = a.alpha[(size_t)t * a.stride + h];
        in.be = a.beta[(size_t)t * a.stride + h];
    };
    In cur, nxt;
    load(cur, 0);
    for (int t = 0; t < a.count; ++t) {
        load(nxt, min(t + 1, a.count - 1));
        // q/k L2 normalisation (backend.cpp:30-35), as gdn_kernel
        float qv[E], kv[E], qs = 0.f, ks = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            qv[e] = cur.q[e];
            kv[e] = cur.k[e];
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
        const float decay = expf(A * softplusf_(cur.al + DT));
        const float b = sigmoidf_(cur.be);
        float mem = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            s[e] *= decay;
            mem += s[e] * kv[e];
        }
        mem = wave_sum(mem);
        const float delta = (cur.v - mem) * b;
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            s[e] += kv[e] * delta;
            sum += s[e] * qv[e];
        }
        sum = wave_sum(sum);
        if (lane == 0) a.o[(size_t)t * a.value_heads * SD + (size_t)h * SD + d] = sum;
        cur = nxt;
    }
#pragma unroll
    for (int e = 0; e < E; ++e) S[lane + 64 * e] = s[e];
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
    if (a.count < 1 || (a.state_dim != 64 && a.state_dim != 128)) return hipErrorInvalidValue;
    const int ch = 2 * a.key_heads * a.state_dim + a.value_heads * a.state_dim;
    const dim3 cgrid((ch + 255) / 256), cblock(256);
    switch (a.conv_width) {
    case 1: launch_kernel(delta_conv_batch_kernel<1>, cgrid, cblock, 0, stream, a); break;
    case 2: launch_kernel(delta_conv_batch_kernel<2>, cgrid, cblock, 0, stream, a); break;
    case 3: launch_kernel(delta_conv_batch_kernel<3>, cgrid, cblock, 0, stream, a); break;
    case 4: launch_kernel(delta_conv_batch_kernel<4>, cgrid, cblock, 0, stream, a); break;
    case 5: launch_kernel(delta_conv_batch_kernel<5>, cgrid, cblock, 0, stream, a); break;
    case 6: launch_kernel(delta_conv_batch_kernel<6>, cgrid, cblock, 0, stream, a); break;
    case 7: launch_kernel(delta_conv_batch_kernel<7>, cgrid, cblock, 0, stream, a); break;
    case 8: launch_kernel(delta_conv_batch_kernel<8>, cgrid, cblock, 0, stream, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 block(kGdnWaves * 64);
    if (a.state_dim == 64) {
        launch_kernel(gdn_scan_kernel<1, 8>, dim3(a.value_heads * 8), block, 0, stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        launch_kernel(gdn_norm_gate_batch_kernel<1>, dim3(a.count * a.value_heads), dim3(64), 0, stream, a);
    } else {
        launch_kernel(gdn_scan_kernel<2, 16>, dim3(a.value_heads * 16), block, 0, stream, a);
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
