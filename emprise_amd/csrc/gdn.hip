// Gated DeltaNet decode step on gfx950 (Backend::delta_net, reference
// backend.cpp:19-60; the CUDA delta_conv/delta_scan/delta_norm_gate, cuda.cpp:417-479).
//
// Two forms. gdn_rows_kernel (the recurrent block's path when the out-projection is in
// the chunked layout) splits each head's rows over SPLIT workgroups and writes the raw
// outputs S.q; the per-head RMSNorm x gate then runs in the out-projection's input
// staging, and the gate rows arrive already SiLU'd from the in-projection. gdn_kernel
// (Backend::delta_net, and the other out-projection widths) does the whole head:
// one workgroup per value head (8 waves), the per-head RMSNorm x SiLU(gate) applied
// before the single write of the head's output. Both keep each state row on the 16 lanes
// of a DPP row (common.hpp's gdn16 helpers: lane j holds state_dim/16 consecutive
// columns, 16-byte accesses), four rows per wave side by side; every workgroup
// L2-normalises the head's q/k itself (2*state_dim values), and each wave issues the
// reads of all its state rows before any arithmetic so the reads overlap.
#include <utility>

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
    constexpr int SD = 64 * E, NE = SD / 16, P = SD / kGdnWaves / 4;  // passes of four rows per wave
    __shared__ float o_row[SD];
    const int h = blockIdx.x, kh = h % a.key_heads;  // tiled V-head order (backend.cpp:37)
    const int key_dim = a.key_heads * SD;
    const int lane = threadIdx.x & 63, g = lane >> 4, j = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const float* v = a.qkv + 2 * (size_t)key_dim + (size_t)h * SD;
    float* S = a.state + (size_t)h * SD * SD;

    // the state reads of this wave's rows (wave * 4P + 4p + g) first, then v, q and k
    float s[P][NE];
#pragma unroll
    for (int p = 0; p < P; ++p) ld16v<NE>(s[p], S + (size_t)(wave * 4 * P + 4 * p + g) * SD + NE * j);
    float vd[P];
#pragma unroll
    for (int p = 0; p < P; ++p) vd[p] = v[wave * 4 * P + 4 * p + g];
    float qv[NE], kv[NE];
    ld16v<NE>(qv, a.qkv + (size_t)kh * SD + NE * j);
    ld16v<NE>(kv, a.qkv + key_dim + (size_t)kh * SD + NE * j);
    gdn16_qk_norm<NE>(qv, kv, a.eps);
    const float decay = expf(a.ssm_a[h] * softplusf_(a.alpha[h] + a.dt[h]));
    const float b = sigmoidf_(a.beta[h]);
#pragma unroll
    for (int p = 0; p < P; ++p) {
        const int d = wave * 4 * P + 4 * p + g;
        const float sum = gdn16_row<NE>(s[p], qv, kv, decay, b, vd[p]);
        st16v<NE>(S + (size_t)d * SD + NE * j, s[p]);
        if (j == 0) o_row[d] = sum;
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
            const int c = lane + 64 * e;
            a.out[(size_t)h * SD + c] = o_row[c] * (scale * a.norm[c]) * siluf_(a.gate[(size_t)h * SD + c]);
        }
    }
}

// The state update of rows [part*SD/SPLIT, (part+1)*SD/SPLIT) of value head h, with
// workgroup blockIdx = h*SPLIT + part; each of the 8 waves owns four rows and writes
// their raw outputs o[d] = S[d,:].q straight to global memory (no cross-wave step).
template <int E, int SPLIT>
__global__ __launch_bounds__(kGdnWaves * 64) void gdn_rows_kernel(GdnArgs a) {
    constexpr int SD = 64 * E, NE = SD / 16;
    static_assert(SD / SPLIT == 4 * kGdnWaves, "four rows per wave");
    const int h = blockIdx.x / SPLIT, part = blockIdx.x - h * SPLIT, kh = h % a.key_heads;
    const int key_dim = a.key_heads * SD;
    const int lane = threadIdx.x & 63, g = lane >> 4, j = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int d = part * (SD / SPLIT) + wave * 4 + g;  // this lane's row
    float* Sd = a.state + ((size_t)h * SD + d) * SD + NE * j;

    // all loads first: the row's state, its v, q and k
    float s[NE], qv[NE], kv[NE];
    ld16v<NE>(s, Sd);
    const float vd = a.qkv[2 * (size_t)key_dim + (size_t)h * SD + d];
    ld16v<NE>(qv, a.qkv + (size_t)kh * SD + NE * j);
    ld16v<NE>(kv, a.qkv + key_dim + (size_t)kh * SD + NE * j);
    gdn16_qk_norm<NE>(qv, kv, a.eps);
    const float decay = expf(a.ssm_a[h] * softplusf_(a.alpha[h] + a.dt[h]));
    const float b = sigmoidf_(a.beta[h]);
    const float sum = gdn16_row<NE>(s, qv, kv, decay, b, vd);
    st16v<NE>(Sd, s);
    if (j == 0) a.out[(size_t)h * SD + d] = sum;
}

// ---- batched form: `count` consecutive positions (the prompt prefill) -------------------
//
// Position by position, the decode kernels above pay two launches and two dependent
// memory round trips per position and layer. Over a prompt the three stages separate:
// the conv1d is a scan per channel (one thread keeps a channel's history in registers
// over all positions), the delta rule a scan per state row (a DPP row keeps its state row
// in registers over all positions) after a parallel pass that normalises q/k and forms
// the decay and beta gate of every position, and the per-head RMSNorm x SiLU(gate) is
// independent per position. Each step does the arithmetic of delta_conv_kernel and
// gdn_kernel in the same order, so the outputs and the final states are those of `count`
// calls of the per-position path.

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

// ---- prefill scan ------------------------------------------------------------------------
//
// One wave carries four state rows (one per DPP row, common.hpp's layout) through all
// the positions; per position a lane runs NE multiplies, 3*NE FMAs and two 16-lane
// butterflies, the chain a 64-lane row would run with two full-wave reductions per row
// in about a third of the instructions.
constexpr int kScanWaves = 4;   // waves per workgroup, four state rows each
constexpr int kScanBlock = 64;  // positions per block: q/k staged in LDS, lane inputs in registers

// f(integral_constant<int, I>) for I = 0 .. N-1 in order (row16_bcast's lane is an
// immediate)
template <class F, int... I> __device__ __forceinline__ void static_for_(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, class F> __device__ __forceinline__ void static_for(F&& f) {
    static_for_(f, std::make_integer_sequence<int, N>{});
}

// The per-position inputs of the delta rule that every row of a head shares, computed
// once per position instead of once per row: the L2-normalised q and k of each key head
// (gdn16_qk_norm on a DPP row per (position, key head), so the values are the decode
// kernels' bit for bit), and the decay and beta gate of each value head. q|k are stored
// in the scan's lane order: the list of lane j is its NE q columns then its NE k columns,
// cut into 16-byte chunks, and chunk c of lane j sits at (c * 16 + j) * 4 -- a wave's read
// of one chunk is 256 consecutive bytes.
template <int E>
__global__ __launch_bounds__(256) void gdn_prep_batch_kernel(GdnBatchArgs a) {
    constexpr int SD = 64 * E, NE = SD / 16;
    const int j = threadIdx.x & 15;
    const int pair = blockIdx.x * 16 + (threadIdx.x >> 4);  // position * key_heads + key head
    const int key_dim = a.key_heads * SD, ch = 2 * key_dim + a.value_heads * SD;
    if (pair < a.count * a.key_heads) {  // (whole DPP rows, as the row sums need)
        const int t = pair / a.key_heads, kh = pair - t * a.key_heads;
        const float* row = a.conv_out + (size_t)t * ch;
        float qv[NE], kv[NE];
        ld16v<NE>(qv, row + (size_t)kh * SD + NE * j);
        ld16v<NE>(kv, row + key_dim + (size_t)kh * SD + NE * j);
        gdn16_qk_norm<NE>(qv, kv, a.eps);
        float* dst = a.qk + (size_t)pair * 2 * SD;
#pragma unroll
        for (int c = 0; c < NE / 4; ++c) {
            *reinterpret_cast<float4*>(dst + (c * 16 + j) * 4) =
                make_float4(qv[4 * c], qv[4 * c + 1], qv[4 * c + 2], qv[4 * c + 3]);
            *reinterpret_cast<float4*>(dst + ((NE / 4 + c) * 16 + j) * 4) =
                make_float4(kv[4 * c], kv[4 * c + 1], kv[4 * c + 2], kv[4 * c + 3]);
        }
    }
    const int i = blockIdx.x * 256 + threadIdx.x;  // position * value_heads + value head
    if (i < a.count * a.value_heads) {
        const int t = i / a.value_heads, h = i - t * a.value_heads;
        a.gates[2 * (size_t)i] = expf(a.ssm_a[h] * softplusf_(a.alpha[(size_t)t * a.stride + h] + a.dt[h]));
        a.gates[2 * (size_t)i + 1] = sigmoidf_(a.beta[(size_t)t * a.stride + h]);
    }
}

// The delta rule (backend.cpp:36-56) over all positions for 16 rows of value head h
// (workgroup = h * SD/16 + part, wave w: rows part*16 + 4w .. +3, one per DPP row), the
// states in registers throughout. Per block of 64 positions the workgroup stages the
// block's q|k in LDS (loaded during the block before), and each lane holds its row's v,
// and the head's decay and beta gate, of the block's positions (lane u: position t0 + u
// for the gates; lane 16g + j: position t0 + 16q + j of row g for v); the raw outputs
// S.q of 16 positions are collected in lanes and stored together. The update of a row is
// gdn16_row, as in the decode kernels, with the prep kernel's q/k.
template <int E>
__global__ __launch_bounds__(kScanWaves * 64) void gdn_scan_kernel(GdnBatchArgs a) {
    constexpr int SD = 64 * E, NE = SD / 16, NC = NE / 2, PQK = 2 * SD;  // q|k floats per position
    constexpr int RPB = kScanWaves * 4, F4 = kScanBlock * PQK / 4 / (kScanWaves * 64);
    __shared__ __align__(16) float qks[2][kScanBlock][PQK];
    const int parts = SD / RPB;
    const int h = blockIdx.x / parts, part = blockIdx.x - h * parts, kh = h % a.key_heads;
    const int key_dim = a.key_heads * SD, ch = 2 * key_dim + a.value_heads * SD;
    const int lane = threadIdx.x & 63, g = lane >> 4, j = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row = part * RPB + wave * 4 + g, last = a.count - 1;
    float* S = a.state + ((size_t)h * SD + row) * SD + NE * j;
    float s[NE];
    ld16v<NE>(s, S);

    const float* qk = a.qk + (size_t)kh * PQK;
    const size_t qk_step = (size_t)a.key_heads * PQK;  // floats per position
    const float* v_col = a.conv_out + 2 * (size_t)key_dim + (size_t)h * SD + row;
    const size_t o_step = (size_t)a.value_heads * SD;
    float* o_col = a.o + (size_t)h * SD + row;

    // the block's q|k: thread th moves float4 th + 256m, position (th + 256m) / (PQK/4)
    // (plain loops in the kernel body: the array stays in registers)
    typedef float f4v __attribute__((ext_vector_type(4)));  // (a native vector: HIP's float4 struct
    f4v stage[F4];                                           // copies kept the array in scratch)
#define EMPRISE_QK_LOAD(T0)                                                                                     \
    _Pragma("unroll") for (int m = 0; m < F4; ++m) {                                                            \
        const int f = threadIdx.x + kScanWaves * 64 * m, p = f / (PQK / 4), w = f - p * (PQK / 4);              \
        stage[m] = *reinterpret_cast<const f4v*>(qk + (size_t)min((T0) + p, last) * qk_step + 4 * w);            \
    }
#define EMPRISE_QK_STORE(BUF)                                                                                   \
    _Pragma("unroll") for (int m = 0; m < F4; ++m) {                                                            \
        const int f = threadIdx.x + kScanWaves * 64 * m, p = f / (PQK / 4), w = f - p * (PQK / 4);              \
        *reinterpret_cast<f4v*>(&qks[(BUF)][p][4 * w]) = stage[m];                                              \
    }
    struct Lanes {
        float v[kScanBlock / 16];
        float2 dg;
    };
    auto lane_load = [&](int t0, Lanes& l) {
#pragma unroll
        for (int q = 0; q < kScanBlock / 16; ++q) l.v[q] = v_col[(size_t)min(t0 + 16 * q + j, last) * ch];
        // positions past the end leave the state as it is (decay 1, gate 0: s * 1 + k * 0,
        // at most a zero's sign changes), so no position needs a branch
        const float2 dg = *reinterpret_cast<const float2*>(a.gates + 2 * ((size_t)min(t0 + lane, last) * a.value_heads + h));
        l.dg = t0 + lane <= last ? dg : make_float2(1.f, 0.f);
    };

    Lanes cur, nxt;
    lane_load(0, cur);
    EMPRISE_QK_LOAD(0)
    EMPRISE_QK_STORE(0)
    __syncthreads();
    EMPRISE_QK_LOAD(kScanBlock)
    for (int t0 = 0, buf = 0; t0 < a.count; t0 += kScanBlock, buf ^= 1) {
        lane_load(t0 + kScanBlock, nxt);
        // positions t0 + 16q .. +15
        // a position's q|k from LDS, read one position ahead of its use
        auto lds_qk = [&](int u, float (&qv)[NE], float (&kv)[NE]) {
#pragma unroll
            for (int c = 0; c < NC / 2; ++c) {
                const float4 x = *reinterpret_cast<const float4*>(&qks[buf][u][(c * 16 + j) * 4]);
                const float4 y = *reinterpret_cast<const float4*>(&qks[buf][u][((c + NC / 2) * 16 + j) * 4]);
                qv[4 * c] = x.x, qv[4 * c + 1] = x.y, qv[4 * c + 2] = x.z, qv[4 * c + 3] = x.w;
                kv[4 * c] = y.x, kv[4 * c + 1] = y.y, kv[4 * c + 2] = y.z, kv[4 * c + 3] = y.w;
            }
        };
        auto group = [&](auto qc) {
            constexpr int q = decltype(qc)::value;
            float ol = 0.f;
            float qn[NE], kn[NE];
            lds_qk(16 * q, qn, kn);
            static_for<16>([&](auto uc) {
                constexpr int uu = decltype(uc)::value;
                const int u = 16 * q + uu;
                {
                    float qv[NE], kv[NE];
#pragma unroll
                    for (int e = 0; e < NE; ++e) qv[e] = qn[e], kv[e] = kn[e];
                    if constexpr (uu + 1 < 16) lds_qk(u + 1, qn, kn);
                    const float decay = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.dg.x), u));
                    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cur.dg.y), u));
                    const float vd = row16_bcast<uu>(cur.v[q]);
                    const float sum = gdn16_row<NE>(s, qv, kv, decay, b, vd);
                    ol = j == uu ? sum : ol;
                }
            });
            const int t = t0 + 16 * q + j;
            if (t < a.count) o_col[(size_t)t * o_step] = ol;
        };
        static_assert(kScanBlock == 64, "four groups of 16 positions");
        group(std::integral_constant<int, 0>{});
        // the next block's q|k go into the buffer every wave finished reading before the
        // last barrier, once the first 16 positions are done (their loads had that long)
        EMPRISE_QK_STORE(buf ^ 1)
        group(std::integral_constant<int, 1>{});
        group(std::integral_constant<int, 2>{});
        group(std::integral_constant<int, 3>{});
        cur = nxt;
        __syncthreads();
        EMPRISE_QK_LOAD(t0 + 2 * kScanBlock)
    }
#undef EMPRISE_QK_LOAD
#undef EMPRISE_QK_STORE
    st16v<NE>(S, s);
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
    const int pgrid = std::max((a.count * a.key_heads + 15) / 16, (a.count * a.value_heads + 255) / 256);
    if (a.state_dim == 64) {
        launch_kernel(gdn_prep_batch_kernel<1>, dim3(pgrid), dim3(256), 0, stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        launch_kernel(gdn_scan_kernel<1>, dim3(a.value_heads * 64 / (kScanWaves * 4)), dim3(kScanWaves * 64), 0,
                      stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        launch_kernel(gdn_norm_gate_batch_kernel<1>, dim3(a.count * a.value_heads), dim3(64), 0, stream, a);
    } else {
        launch_kernel(gdn_prep_batch_kernel<2>, dim3(pgrid), dim3(256), 0, stream, a);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        launch_kernel(gdn_scan_kernel<2>, dim3(a.value_heads * 128 / (kScanWaves * 4)), dim3(kScanWaves * 64), 0,
                      stream, a);
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
