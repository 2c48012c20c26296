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
// Inside a workgroup no output needs a cross-lane reduction chain: the chunk's keys
// are copied to LDS and lane t of wave w computes the score of position t for query
// head w (a 256-long dot product with the query broadcast from LDS), so the softmax
// statistics are one wave max and one wave sum per head; for P.V, lane l of every wave
// accumulates output dims E*l .. E*l+E-1 (head_dim = 64*E) over the wave's own value
// rows, and the four waves' sums are added through LDS. Rows move as one 16-byte
// (E = 4) access per lane.
//
// The grid covers the whole context so the launch can be replayed from a hipGraph:
// the position is read from device memory and chunks past it return at once. Barriers
// order LDS only (lds_barrier), so none of them waits for the K/V rows in flight.
#include "common.hpp"
#include "kernels.hpp"

namespace emprise {
namespace {

constexpr int kAttnWaves = 4;
constexpr int kMaxGroup = 8;
constexpr int kCombineMaxChunks = 1024;  // contexts up to 65536 positions

// E consecutive floats (lane l of a wave owns dims E*l .. E*l+E-1 of a head): one
// 16-, 8- or 4-byte access.
template <int E> __device__ __forceinline__ void ldv(float (&v)[E], const float* p) {
    if constexpr (E == 4) {
        const float4 t = *reinterpret_cast<const float4*>(p);
        v[0] = t.x, v[1] = t.y, v[2] = t.z, v[3] = t.w;
    } else if constexpr (E == 2) {
        const float2 t = *reinterpret_cast<const float2*>(p);
        v[0] = t.x, v[1] = t.y;
    } else {
        v[0] = *p;
    }
}
template <int E> __device__ __forceinline__ void stv(float* p, const float (&v)[E]) {
    if constexpr (E == 4) *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    else if constexpr (E == 2) *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
    else *p = v[0];
}

template <int E>  // head_dim = 64 * E
__global__ __launch_bounds__(kAttnWaves * 64) void attention_kernel(AttnArgs a) {
    constexpr int HD = 64 * E, CH = kAttnChunk, KS = HD + 4;  // padded key rows in LDS
    constexpr int PW = CH / kAttnWaves;                       // rows per wave
    __shared__ __align__(16) float qs[kMaxGroup][HD];
    __shared__ __align__(16) float knew[HD], vnew[HD];
    __shared__ float sc[kMaxGroup][CH];
    __shared__ float mstat[kMaxGroup], lstat[kMaxGroup];
    // the chunk's keys during the scores, then the waves' P.V sums
    constexpr int KBYTES = CH * KS * 4, ABYTES = kAttnWaves * kMaxGroup * HD * 4;
    __shared__ __align__(16) unsigned char kv_lds[KBYTES > ABYTES ? KBYTES : ABYTES];
    float (*ks)[KS] = reinterpret_cast<float (*)[KS]>(kv_lds);
    float (*acc_lds)[kMaxGroup][HD] = reinterpret_cast<float (*)[kMaxGroup][HD]>(kv_lds);

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

    // Loads, in the order they are needed: the inputs of the q/k RMSNorms (wave w
    // normalises heads w, w+4, ... and, as head `group`, the new key), then all of the
    // wave's K and V rows. The norm inputs are loaded unconditionally (clamped heads) so
    // waiting for them never waits for the K/V rows, whose latency overlaps the norms
    // and RoPE. (Wave w owns positions t0 + w, t0 + w + 4, ...; the row at `pos` is not
    // written yet and is replaced by the new k/v.)
    constexpr int NJ = (kMaxGroup + kAttnWaves) / kAttnWaves;  // heads per wave, incl. the key
    float xin[NJ][E], qn[E], kn[E];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int g = min(wave + kAttnWaves * j, group);
        const float* src = g < group ? a.qkv + (size_t)(kvh * group + g) * HD * 2 : kin;
        ldv<E>(xin[j], src + E * lane);
    }
    ldv<E>(qn, a.q_norm + E * lane);
    ldv<E>(kn, a.k_norm + E * lane);
    const float vin_d = vin[min((int)threadIdx.x, HD - 1)];

    const int t0 = chunk * CH;
    const int tn = min(CH, len - t0);
    const size_t row_stride = (size_t)a.kv_heads * HD;
    const float* kb = a.keys + ((size_t)t0 * a.kv_heads + kvh) * HD + E * lane;
    const float* vb = a.values + ((size_t)t0 * a.kv_heads + kvh) * HD + E * lane;
    float kr[PW][E], vr[PW][E];
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const int tt = wave + kAttnWaves * i;
        if (tt < tn) {
            ldv<E>(kr[i], kb + (size_t)tt * row_stride);
            ldv<E>(vr[i], vb + (size_t)tt * row_stride);
        }
    }

    // RMSNorm of the query heads and of the new key (model.cpp:133-134)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int g = wave + kAttnWaves * j;
        if (g <= group) {
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) ss += xin[j][e] * xin[j][e];
            ss = wave_sum(ss);
            const float scale = 1.f / sqrtf(ss / (float)HD + a.eps);
            float y[E];
#pragma unroll
            for (int e = 0; e < E; ++e) y[e] = xin[j][e] * (scale * (g < group ? qn[e] : kn[e]));
            stv<E>((g < group ? qs[g] : knew) + E * lane, y);
        }
    }
    if (threadIdx.x < HD) vnew[threadIdx.x] = vin_d;
    lds_barrier();
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
    lds_barrier();
    if (chunk == nchunks - 1) {  // this chunk holds `pos`: append k/v to the caches
        for (int d = threadIdx.x; d < HD; d += blockDim.x) {
            a.keys[((size_t)pos * a.kv_heads + kvh) * HD + d] = knew[d];
            a.values[((size_t)pos * a.kv_heads + kvh) * HD + d] = vnew[d];
        }
    }
    // the chunk's keys to LDS, row-major (the new key from LDS)
#pragma unroll
    for (int i = 0; i < PW; ++i) {
        const int tt = wave + kAttnWaves * i;
        if (tt < tn) {
            if (t0 + tt == pos) ldv<E>(kr[i], knew + E * lane);
            stv<E>(ks[tt] + E * lane, kr[i]);
        }
    }
    lds_barrier();

    // scores and chunk-local softmax: wave w takes query heads w, w+4, ...; lane t is
    // position t0 + t (model.cpp:143-150)
    const float inv_root = 1.f / sqrtf((float)HD);
    for (int g = wave; g < group; g += kAttnWaves) {
        float s = -INFINITY;
        if (lane < tn) {
            const float4* k4 = reinterpret_cast<const float4*>(ks[lane]);
            const float4* q4 = reinterpret_cast<const float4*>(qs[g]);
            float dx = 0.f, dy = 0.f, dz = 0.f, dw = 0.f;  // four chains, not one long one
#pragma unroll 16
            for (int i = 0; i < HD / 4; ++i) {
                const float4 k = k4[i], q = q4[i];
                dx = fmaf(q.x, k.x, dx);
                dy = fmaf(q.y, k.y, dy);
                dz = fmaf(q.z, k.z, dz);
                dw = fmaf(q.w, k.w, dw);
            }
            s = ((dx + dy) + (dz + dw)) * inv_root;
        }
        const float m = wave_max(s);
        const float p = lane < tn ? expf(s - m) : 0.f;
        const float l = wave_sum(p);
        sc[g][lane] = p;
        if (lane == 0) {
            mstat[g] = m;
            lstat[g] = l;
        }
    }
    lds_barrier();  // scores done: the key tile's LDS now takes the P.V sums

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
            if (t0 + tt == pos) ldv<E>(vr[i], vnew + E * lane);
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
        if (g < group) stv<E>(acc_lds[wave][g] + E * lane, acc[g]);
    lds_barrier();
    const int stride = HD + 2;
    float* part = a.partial + ((size_t)kvh * chunks_max + chunk) * group * stride;
    for (int idx = threadIdx.x; idx < group * HD; idx += blockDim.x) {
        const int g = idx / HD, d = idx % HD;
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) o += acc_lds[w][g][d];
        part[g * stride + d] = o;
    }
    if (threadIdx.x < group) {
        part[threadIdx.x * stride + HD] = mstat[threadIdx.x];
        part[threadIdx.x * stride + HD + 1] = lstat[threadIdx.x];
    }
}

// Merges the chunk partials of one query head and 64 of its output dims:
// o = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c, then the sigmoid output gate
// (model.cpp:153). Every load (chunk statistics and the wave's share of the chunks'
// o values) is issued once the position is known, before any arithmetic; wave w sums
// chunks w, w+4, ... and the four waves' sums are added through LDS.
constexpr int kCombineBatch = 16;  // chunks per wave held in registers per pass
__global__ __launch_bounds__(256) void attention_combine_kernel(AttnArgs a) {
    __shared__ float wts[kCombineMaxChunks];
    __shared__ float red[8];
    __shared__ float part[4][64];
    const int hd = a.head_dim, group = a.heads / a.kv_heads, dblocks = hd / 64;
    const int head = blockIdx.x / dblocks, db = blockIdx.x - head * dblocks;
    const int pos = *a.position;
    if (pos < 0 || pos >= a.context) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunks_max = (a.context + kAttnChunk - 1) / kAttnChunk;
    const int nchunks = pos / kAttnChunk + 1;
    const int kvh = head / group, g = head - kvh * group, stride = hd + 2;
    const float* base = a.partial + ((size_t)kvh * chunks_max * group + g) * stride;
    const size_t cstride = (size_t)group * stride;
    const int d = db * 64 + lane;

    // the gate, the first pass of o values and the statistics, all in flight together
    const float gate = a.qkv[(size_t)head * hd * 2 + hd + d];
    float ov[kCombineBatch];
#pragma unroll
    for (int i = 0; i < kCombineBatch; ++i) {
        const int c = min(wave + 4 * i, nchunks - 1);
        ov[i] = base[(size_t)c * cstride + d];
    }
    float mloc = -INFINITY;
    for (int c = threadIdx.x; c < nchunks; c += blockDim.x) {
        const float m = base[(size_t)c * cstride + hd];
        wts[c] = m;
        mloc = fmaxf(mloc, m);
    }
    mloc = wave_max(mloc);
    if (lane == 0) red[wave] = mloc;
    lds_barrier();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float dloc = 0.f;
    for (int c = threadIdx.x; c < nchunks; c += blockDim.x) {
        const float w = expf(wts[c] - M);
        wts[c] = w;
        dloc = fmaf(w, base[(size_t)c * cstride + hd + 1], dloc);
    }
    dloc = wave_sum(dloc);
    lds_barrier();  // every weight is in wts; red is free again
    if (lane == 0) red[4 + wave] = dloc;
    float num = 0.f;
#pragma unroll
    for (int i = 0; i < kCombineBatch; ++i) {
        const int c = wave + 4 * i;
        if (c < nchunks) num = fmaf(wts[c], ov[i], num);
    }
    for (int c0 = wave + 4 * kCombineBatch; c0 < nchunks; c0 += 4 * kCombineBatch) {  // long contexts
#pragma unroll
        for (int i = 0; i < kCombineBatch; ++i) ov[i] = base[(size_t)min(c0 + 4 * i, nchunks - 1) * cstride + d];
#pragma unroll
        for (int i = 0; i < kCombineBatch; ++i)
            if (c0 + 4 * i < nchunks) num = fmaf(wts[c0 + 4 * i], ov[i], num);
    }
    part[wave][lane] = num;
    lds_barrier();
    if (wave == 0) {
        const float den = (red[4] + red[5]) + (red[6] + red[7]);
        const float o = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
        a.out[(size_t)head * hd + d] = (o / den) * sigmoidf_(gate);
    }
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
    if (chunks > kCombineMaxChunks) return hipErrorInvalidValue;
    const dim3 grid(a.kv_heads * chunks), block(kAttnWaves * 64);
    switch (a.head_dim) {
    case 64: launch_kernel(attention_kernel<1>, grid, block, 0, stream, a); break;
    case 128: launch_kernel(attention_kernel<2>, grid, block, 0, stream, a); break;
    case 256: launch_kernel(attention_kernel<4>, grid, block, 0, stream, a); break;
    default: return hipErrorInvalidValue;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    launch_kernel(attention_combine_kernel, dim3(a.heads * (a.head_dim / 64)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

}  // namespace emprise
