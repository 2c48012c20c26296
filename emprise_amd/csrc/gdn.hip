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

}  // namespace

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
