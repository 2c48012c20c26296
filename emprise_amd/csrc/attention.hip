// Gated GQA attention decode on gfx950 (Model::Impl::attention_preout, reference
// model.cpp:129-157, which the reference runs on the host even on its device path).
//
// Split-KV ("flash decoding"): workgroup (kv head, chunk of kAttnChunk positions)
// serves the `group` = heads/kv_heads query heads that share the KV head, so each K/V
// row is read once for all of them. Every workgroup recomputes the RMSNorm + RoPE of
// its query heads and of the new key (a few KiB of work); the workgroup whose chunk
// holds the current position also appends the new k/v to the caches and uses them
// straight from LDS. Each workgroup writes an unnormalised partial (o, running max,
// sum of exponentials); a second small kernel merges the partials, divides, and applies
// the sigmoid output gate. (A last-workgroup merge inside the first kernel would need
// device-scope fences, which write back and invalidate a whole L2 on this part.)
//
// The grid covers the whole context so the launch can be replayed from a hipGraph:
// the position is read from device memory and chunks past it return at once.
#include "common.hpp"
#include "kernels.hpp"

namespace emprise {
namespace {

constexpr int kAttnWaves = 4;
constexpr int kMaxGroup = 8;

template <int E>  // head_dim = 64 * E
__global__ __launch_bounds__(kAttnWaves * 64) void attention_kernel(AttnArgs a) {
    constexpr int HD = 64 * E, CH = kAttnChunk;
    __shared__ float qs[kMaxGroup][HD];
    __shared__ float knew[HD], vnew[HD];
    __shared__ float sc[kMaxGroup][CH];
    __shared__ float acc_lds[kAttnWaves][kMaxGroup][HD];
    __shared__ float mstat[kMaxGroup], lstat[kMaxGroup];

    const int group = a.heads / a.kv_heads;
    const int chunks_max = (a.context + CH - 1) / CH;
    const int kvh = blockIdx.x / chunks_max, chunk = blockIdx.x % chunks_max;
    const int pos = *a.position;
    if (pos < 0 || pos >= a.context) return;  // the host keeps positions inside the caches
    const int len = pos + 1;
    const int nchunks = (len + CH - 1) / CH;
    if (chunk >= nchunks) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qd = a.heads * HD * 2, kvd = a.kv_heads * HD;
    const float* kin = a.qkv + qd + (size_t)kvh * HD;
    const float* vin = a.qkv + qd + kvd + (size_t)kvh * HD;

    // Wave w owns positions t0 + w, t0 + w + 4, ...: all of its K and V rows are loaded
    // here, before any arithmetic, so their latency overlaps the norms and RoPE below.
    // (The row at `pos` is not written yet; its value is replaced by the new k/v.)
    constexpr int PW = CH / kAttnWaves;
    const int t0 = chunk * CH;
    const int tn = min(CH, len - t0);
    const size_t row_stride = (size_t)a.kv_heads * HD;
    const float* kb = a.keys + ((size_t)t0 * a.kv_heads + kvh) * HD + lane;
    const float* vb = a.values + ((size_t)t0 * a.kv_heads + kvh) * HD + lane;
    float kr[PW][E], vr[PW][E];
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const int tt = wave + kAttnWaves * i;
        if (tt < tn) {
#pragma unroll
            for (int e = 0; e < E; ++e) kr[i][e] = kb[(size_t)tt * row_stride + 64 * e];
#pragma unroll
            for (int e = 0; e < E; ++e) vr[i][e] = vb[(size_t)tt * row_stride + 64 * e];
        }
    }

    // RMSNorm of the query heads (wave g handles heads g, g+4, ...) and of the new key.
    for (int g = wave; g <= group; g += kAttnWaves) {
        const float* src = g < group ? a.qkv + (size_t)(kvh * group + g) * HD * 2 : kin;
        const float* nw = g < group ? a.q_norm : a.k_norm;
        float x[E], ss = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
            x[e] = src[lane + 64 * e];
            ss += x[e] * x[e];
        }
        ss = wave_sum(ss);
        const float scale = 1.f / sqrtf(ss / (float)HD + a.eps);
        float* dst = g < group ? qs[g] : knew;
#pragma unroll
        for (int e = 0; e < E; ++e) dst[lane + 64 * e] = x[e] * (scale * nw[lane + 64 * e]);
    }
    for (int d = threadIdx.x; d < HD; d += blockDim.x) vnew[d] = vin[d];
    __syncthreads();
    // NEOX RoPE over the first `rotary` dims (model.cpp:121-127); one thread per pair.
    const int half = a.rotary / 2;
    for (int idx = threadIdx.x; idx < (group + 1) * half; idx += blockDim.x) {
        const int g = idx / half, i = idx % half;
        float* row = g < group ? qs[g] : knew;
        const float angle = (float)pos / powf(a.rope_base, 2.f * (float)i / (float)a.rotary);
        const float c = cosf(angle), s = sinf(angle);
        const float x0 = row[i], x1 = row[i + half];
        row[i] = x0 * c - x1 * s;
        row[i + half] = x0 * s + x1 * c;
    }
    __syncthreads();
    if (chunk == nchunks - 1) {  // this chunk holds `pos`: append k/v to the caches
        for (int d = threadIdx.x; d < HD; d += blockDim.x) {
            a.keys[((size_t)pos * a.kv_heads + kvh) * HD + d] = knew[d];
            a.values[((size_t)pos * a.kv_heads + kvh) * HD + d] = vnew[d];
        }
    }

    // scores s[g][t] = q_g . k_t / sqrt(HD); the wave's K rows were loaded up front
    const float inv_root = 1.f / sqrtf((float)HD);
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const int tt = wave + kAttnWaves * i;
        if (tt < tn) {
            if (t0 + tt == pos)
#pragma unroll
                for (int e = 0; e < E; ++e) kr[i][e] = knew[lane + 64 * e];
            for (int g = 0; g < group; ++g) {
                float dot = 0.f;
#pragma unroll
                for (int e = 0; e < E; ++e) dot += qs[g][lane + 64 * e] * kr[i][e];
                dot = wave_sum(dot);
                if (lane == 0) sc[g][tt] = dot * inv_root;
            }
        }
    }
    __syncthreads();
    // chunk-local softmax statistics (CH == 64: one score per lane)
    for (int g = wave; g < group; g += kAttnWaves) {
        const float sv = lane < tn ? sc[g][lane] : -INFINITY;
        const float m = wave_max(sv);
        const float p = lane < tn ? expf(sv - m) : 0.f;
        const float l = wave_sum(p);
        sc[g][lane] = p;
        if (lane == 0) {
            mstat[g] = m;
            lstat[g] = l;
        }
    }
    __syncthreads();
    // o[g] = sum_t p[g][t] v_t over this wave's positions
    float acc[kMaxGroup][E];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[g][e] = 0.f;
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const int tt = wave + kAttnWaves * i;
        if (tt < tn) {
            if (t0 + tt == pos)
#pragma unroll
                for (int e = 0; e < E; ++e) vr[i][e] = vnew[lane + 64 * e];
#pragma unroll
            for (int g = 0; g < kMaxGroup; ++g) {
                if (g < group) {
                    const float p = sc[g][tt];
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[g][e] = fmaf(p, vr[i][e], acc[g][e]);
                }
            }
        }
    }
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
        if (g < group)
#pragma unroll
            for (int e = 0; e < E; ++e) acc_lds[wave][g][lane + 64 * e] = acc[g][e];
    __syncthreads();
    const int stride = HD + 2;
    float* part = a.partial + ((size_t)kvh * chunks_max + chunk) * group * stride;
    for (int idx = threadIdx.x; idx < group * HD; idx += blockDim.x) {
        const int g = idx / HD, d = idx % HD;
        float o = 0.f;
        for (int w = 0; w < kAttnWaves; ++w) o += acc_lds[w][g][d];
        part[g * stride + d] = o;
    }
    if (threadIdx.x < group) {
        part[threadIdx.x * stride + HD] = mstat[threadIdx.x];
        part[threadIdx.x * stride + HD + 1] = lstat[threadIdx.x];
    }
}

// Merges the chunk partials of every query head: o = sum_c e^(m_c - M) o_c /
// sum_c e^(m_c - M) l_c, then the sigmoid output gate (model.cpp:153). One thread per
// output value; the grid covers heads * head_dim.
__global__ void attention_combine_kernel(AttnArgs a) {
    const int hd = a.head_dim, group = a.heads / a.kv_heads;
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= a.heads * hd) return;
    const int pos = *a.position;
    if (pos < 0 || pos >= a.context) return;
    const int head = idx / hd, d = idx % hd, kvh = head / group, g = head % group;
    const int chunks_max = (a.context + kAttnChunk - 1) / kAttnChunk;
    const int nchunks = (pos + kAttnChunk) / kAttnChunk;
    const int stride = hd + 2;
    const float* base = a.partial + (size_t)kvh * chunks_max * group * stride + (size_t)g * stride;
    float M = -INFINITY;
    for (int c = 0; c < nchunks; ++c) M = fmaxf(M, base[(size_t)c * group * stride + hd]);
    float num = 0.f, den = 0.f;
    for (int c = 0; c < nchunks; ++c) {
        const float* p = base + (size_t)c * group * stride;
        const float wgt = expf(p[hd] - M);
        num = fmaf(wgt, p[d], num);
        den = fmaf(wgt, p[hd + 1], den);
    }
    const float gate = a.qkv[(size_t)head * hd * 2 + hd + d];
    a.out[(size_t)head * hd + d] = (num / den) * sigmoidf_(gate);
}

}  // namespace

size_t attention_partial_floats(int heads, int kv_heads, int head_dim, int context) {
    const int chunks = (context + kAttnChunk - 1) / kAttnChunk;
    return (size_t)kv_heads * chunks * (heads / kv_heads) * (head_dim + 2);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t stream) {
    if (a.heads % a.kv_heads || a.heads / a.kv_heads > kMaxGroup || a.rotary > a.head_dim || a.rotary % 2)
        return hipErrorInvalidValue;
    const int chunks = (a.context + kAttnChunk - 1) / kAttnChunk;
    const dim3 grid(a.kv_heads * chunks), block(kAttnWaves * 64);
    switch (a.head_dim) {
    case 64: launch_kernel(attention_kernel<1>, grid, block, 0, stream, a); break;
    case 128: launch_kernel(attention_kernel<2>, grid, block, 0, stream, a); break;
    case 256: launch_kernel(attention_kernel<4>, grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_kernel(attention_combine_kernel, dim3((a.heads * a.head_dim + 255) / 256), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace emprise
