// Gated GQA attention decode on gfx950 (Model::Impl::attention_preout, reference
// model.cpp:129-157, which the reference runs on the host even on its device path).
//
// Split-KV ("flash decoding") over a fixed grid: workgroup (kv head, range j of
// kAttnSplit) serves the `group` = heads/kv_heads query heads that share the KV head, so
// each K/V row is read once for all of them, over range j of the positions 0..pos. The
// ranges are whole sub-chunks of kAttnSub positions, as many per range as it takes to
// cover the context with kAttnSplit ranges: one sub-chunk each up to 1024 positions,
// four at 4096. Every workgroup recomputes the RMSNorm + RoPE of its query heads and of
// the new key (a few KiB of work); the workgroup whose range holds the current position
// also appends the new k/v to the caches and uses them straight from LDS. Each
// workgroup writes an unnormalised partial (o, running max, sum of exponentials); a
// second small kernel merges the (at most kAttnSplit) partials, divides, and applies the
// sigmoid output gate. (A last-workgroup merge inside the first kernel needs
// agent-scope fences, which write back and invalidate an L2 on this part: measured
// 29.3 us per call at 512 positions against 9.9 us for the two kernels, and 2.9 us more
// even at 16 positions, where four workgroups take part. Without fences -- partials
// written with agent-scope atomic stores, s_waitcnt 0 and a barrier before a relaxed
// ticket, the last range of each KV head merging with agent-scope loads -- it is
// correct and still slower past a few ranges, one workgroup reading every partial:
// 8.3 / 9.7 / 17.3 / 26.6 / 31.9 us at 16 / 100 / 512 / 1024 / 4096 positions against
// 8.7 / 8.6 / 9.0 / 9.5 / 15.6 us for the two kernels, 569 against 592 tok/s.)
//
// Inside a workgroup (8 waves) every wave owns kAttnSub/8 positions of each sub-chunk
// and keeps their K and V rows in registers, lane l holding dims E*l .. E*l+E-1 (head_dim = 64*E,
// one 16-byte access per row at E = 4). A score is then E products and one wave sum,
// with the query heads in registers too; each wave runs an online softmax (its own
// running maximum and sum) over its rows and accumulates their P.V, and the eight
// waves are merged (max-rescaled) through LDS. Measured on the 9B attention shape
// (16 Q / 4 KV heads x 256; one attention + merge, replayed from a graph): 10.3, 13.4
// and 17.5 µs at 512, 2048 and 4096 positions, against 11.6, 16.2 and 23.0 µs with
// 4-wave workgroups and 14.8, 15.1 and 18.4 µs for the earlier design (64-position
// chunks, one workgroup each, keys staged in LDS, one score per lane); 9.1, 11.4 and
// 15.7 µs for this kernel on a later box. Measured alternatives that did not pay, same
// box each: computing the RoPE angles in the kernel instead of reading the table (9.9
// against 9.2 µs at 512), issuing the norm-input loads before the position read (9.13
// against 9.10), loading each range's first K/V rows before the position is known
// (no gain, and the ranges past the position then read rows they never use).
//
// The grid does not depend on the position, so the launch can be replayed from a
// hipGraph: the position is read from device memory and ranges past it return at once.
// Barriers order LDS only (lds_barrier), so none of them waits for the K/V rows in flight.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace emprise {
namespace {

constexpr int kAttnWaves = 8;
constexpr int kMaxGroup = 8;

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

// Positions [first_sub * CH, end_sub * CH) of the workgroup's range: the `len`
// positions are cut into nsub = ceil(len / CH) sub-chunks, and range j of kAttnSplit
// takes `per` = ceil(nsub / kAttnSplit) consecutive sub-chunks (ranges past the end are
// empty). The combine kernel recomputes the same split to know how many partials exist.
__device__ __forceinline__ int attn_per(int len) {
    const int nsub = (len + kAttnSub - 1) / kAttnSub;
    return (nsub + kAttnSplit - 1) / kAttnSplit;
}

// Eight wave-wide sums at once: halving exchanges across lanes l^32 and l^16
// (v_permlane32_swap / v_permlane16_swap, each pair of values trading the halves the
// other lane keeps) and l^8 (a row rotation) leave lane l with value
// (l>>3 & 1) + 2*(l>>4 & 1) + 4*(l>>5 & 1) summed over 8 lanes, and a three-step butterfly
// inside each group of 8 lanes completes it (the same bits in all 8); value j is then
// read from lane 8j. About half the instructions of eight wave_sum, and a shorter chain.
__device__ __forceinline__ void wave_sum8(const float (&x)[8], float (&out)[8]) {
    float y[4], z[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x[j]), __float_as_uint(x[j + 4]), false, false);
        y[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // lanes 0-31: value j, 32-63: value j+4
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(y[j]), __float_as_uint(y[j + 2]), false, false);
        z[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // even rows of 16: slot j, odd rows: slot j+2
    }
    const bool hi8 = (threadIdx.x & 8) != 0;
    float w = (hi8 ? z[1] : z[0]) + dpp_f<0x128, 0xf>(0.f, hi8 ? z[0] : z[1]);  // row_ror:8
    w += dpp_f<0xb1, 0xf>(0.f, w);   // quad_perm [1,0,3,2]
    w += dpp_f<0x4e, 0xf>(0.f, w);   // quad_perm [2,3,0,1]
    w += dpp_f<0x141, 0xf>(0.f, w);  // row_half_mirror
#pragma unroll
    for (int j = 0; j < 8; ++j) out[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 8 * j));
}

template <int E>  // head_dim = 64 * E
__global__ __launch_bounds__(kAttnWaves * 64) void attention_kernel(AttnArgs a) {
    constexpr int HD = 64 * E, CH = kAttnSub, PW = CH / kAttnWaves;  // rows per wave and sub-chunk
    __shared__ __align__(16) float qs[kMaxGroup][HD];
    __shared__ __align__(16) float knew[HD], vnew[HD];
    __shared__ float wstat[kAttnWaves][kMaxGroup][2];  // per wave and head: max, sum
    __shared__ __align__(16) float acc_lds[kAttnWaves][kMaxGroup][HD];

    const int group = a.heads / a.kv_heads;
    const int kvh = blockIdx.x / kAttnSplit, range = blockIdx.x % kAttnSplit;
    const int pos = *a.position;
    if (pos < 0 || pos >= a.context) return;  // the host keeps positions inside the caches
    const int rpos = a.rope_position ? *a.rope_position : pos;
    if (rpos < 0 || rpos >= a.context) return;  // the RoPE table has `context` rows
    const int len = pos + 1;
    const int nsub = (len + CH - 1) / CH, per = attn_per(len);
    const int sub0 = range * per, sub1 = min(nsub, sub0 + per);
    if (sub0 >= sub1) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qd = a.heads * HD * 2, kvd = a.kv_heads * HD;
    const float* kin = a.qkv + qd + (size_t)kvh * HD;
    const float* vin = a.qkv + qd + kvd + (size_t)kvh * HD;
    const size_t row_stride = (size_t)a.kv_heads * HD;
    const float* kb = a.keys + (size_t)kvh * HD + E * lane;
    const float* vb = a.values + (size_t)kvh * HD + E * lane;

    // The wave's K and V rows of sub-chunk `sub` (positions sub*CH + wave + 8i); rows
    // past `len` are loaded clamped and never used; the row at `pos` is not written yet,
    // may hold anything, NaN included, and is replaced by the new k/v.
    auto load_rows = [&](float (&kr)[PW][E], float (&vr)[PW][E], int sub) {
        const int t0 = sub * CH, tn = min(CH, len - t0);
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const size_t t = (size_t)(t0 + min(wave + kAttnWaves * i, tn - 1));
            ldv<E>(kr[i], kb + t * row_stride);
            ldv<E>(vr[i], vb + t * row_stride);
        }
    };

    // Loads, in the order they are needed: the inputs of the q/k RMSNorms (wave w
    // normalises heads w, w+8, ... and, as head `group`, the new key), then the wave's
    // K and V rows of the first sub-chunk. The norm inputs are loaded unconditionally
    // (clamped heads) so waiting for them never waits for the K/V rows, whose latency
    // overlaps the norms and RoPE.
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
    // this thread's first RoPE pair (idx = threadIdx.x below): its (cos, sin) from the table
    const int half = a.rotary / 2;
    const float2 cs0 = half > 0 ? a.rope[(size_t)rpos * half + min((int)threadIdx.x, (group + 1) * half - 1) % half]
                                : make_float2(1.f, 0.f);
    float kr[PW][E], vr[PW][E];
    load_rows(kr, vr, sub0);

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
    // NEOX RoPE over the first `rotary` dims (model.cpp:121-127); one thread per pair,
    // the angles' cos and sin from the backend's table (rope_table_kernel), which the
    // batched prefill reads as well
    for (int idx = threadIdx.x; idx < (group + 1) * half; idx += blockDim.x) {
        const int g = idx / half, i = idx % half;
        float* row = g < group ? qs[g] : knew;
        const float2 cs = idx == (int)threadIdx.x ? cs0 : a.rope[(size_t)rpos * half + i];
        const float c = cs.x, s = cs.y;
        const float x0 = row[i], x1 = row[i + half];
        row[i] = x0 * c - x1 * s;
        row[i + half] = x0 * s + x1 * c;
    }
    lds_barrier();
    if (sub1 == nsub) {  // this range holds `pos`: append k/v to the caches
        for (int d = threadIdx.x; d < HD; d += blockDim.x) {
            a.keys[((size_t)pos * a.kv_heads + kvh) * HD + d] = knew[d];
            a.values[((size_t)pos * a.kv_heads + kvh) * HD + d] = vnew[d];
        }
    }

    // Lane l holds dims E*l .. E*l+E-1 of every query head and of each row, so a score
    // is E products and one wave sum (model.cpp:143-150). Each wave runs an online
    // softmax over its rows of the range's sub-chunks (running maximum, sum and P.V),
    // with the next sub-chunk's rows loading while the current one is used; the four
    // waves are merged (max-rescaled) through LDS at the end.
    float qv[kMaxGroup][E];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g)
        if (g < group) ldv<E>(qv[g], qs[g] + E * lane);
    const float inv_root = 1.f / sqrtf((float)HD);
    float mw[kMaxGroup], lw[kMaxGroup], acc[kMaxGroup][E];
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
        mw[g] = -INFINITY;
        lw[g] = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[g][e] = 0.f;
    }
    for (int sub = sub0; sub < sub1; ++sub) {
        const int t0 = sub * CH, tn = min(CH, len - t0);
        float kn2[PW][E], vn2[PW][E];
        if (sub + 1 < sub1) load_rows(kn2, vn2, sub + 1);
        float sc[PW][kMaxGroup];
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int tt = wave + kAttnWaves * i;
            if (t0 + tt == pos) {
                ldv<E>(kr[i], knew + E * lane);
                ldv<E>(vr[i], vnew + E * lane);
            }
        }
        if (PW * 4 == 8 && group == 4) {
            // the wave's eight scores (PW rows x 4 heads) reduced together
            float d[8], s8[8];
#pragma unroll
            for (int i = 0; i < PW; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    float p = 0.f;
#pragma unroll
                    for (int e = 0; e < E; ++e) p = fmaf(qv[g][e], kr[i][e], p);
                    d[(4 * i + g) & 7] = p;
                }
            wave_sum8(d, s8);
#pragma unroll
            for (int i = 0; i < PW; ++i)
#pragma unroll
                for (int g = 0; g < 4; ++g) sc[i][g] = s8[(4 * i + g) & 7] * inv_root;
        } else {
#pragma unroll
            for (int i = 0; i < PW; ++i)
#pragma unroll
                for (int g = 0; g < kMaxGroup; ++g) {
                    if (g < group) {
                        float p = 0.f;
#pragma unroll
                        for (int e = 0; e < E; ++e) p = fmaf(qv[g][e], kr[i][e], p);
                        sc[i][g] = wave_sum(p) * inv_root;
                    }
                }
        }
#pragma unroll
        for (int g = 0; g < kMaxGroup; ++g) {
            if (g < group) {
                float m = mw[g];
#pragma unroll
                for (int i = 0; i < PW; ++i)
                    if (wave + kAttnWaves * i < tn) m = fmaxf(m, sc[i][g]);
                if (m != -INFINITY) {  // the wave has rows in this sub-chunk
                    const float r = mw[g] == -INFINITY ? 0.f : expf(mw[g] - m);
                    lw[g] *= r;
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[g][e] *= r;
                    mw[g] = m;
                }
                // (rows past `len` hold a clamped copy of the row at `pos`, which the
                // cache does not have yet: never touched, not even times 0)
#pragma unroll
                for (int i = 0; i < PW; ++i) {
                    if (wave + kAttnWaves * i < tn) {
                        const float p = expf(sc[i][g] - m);
                        lw[g] += p;
#pragma unroll
                        for (int e = 0; e < E; ++e) acc[g][e] = fmaf(p, vr[i][e], acc[g][e]);
                    }
                }
            }
        }
        if (sub + 1 < sub1) {
#pragma unroll
            for (int i = 0; i < PW; ++i)
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    kr[i][e] = kn2[i][e];
                    vr[i][e] = vn2[i][e];
                }
        }
    }
#pragma unroll
    for (int g = 0; g < kMaxGroup; ++g) {
        if (g < group) {
            stv<E>(acc_lds[wave][g] + E * lane, acc[g]);
            if (lane == 0) {
                wstat[wave][g][0] = mw[g];
                wstat[wave][g][1] = lw[g];
            }
        }
    }
    lds_barrier();
    // Merge of the waves into the range's partial: o, max, sum. Lane w*8+g of every
    // wave computes the weight exp(m_w - M_g) of wave w for head g. (Every loop below is
    // uniform per wave: head_dim is a multiple of 64, so a wave's 64 consecutive items
    // share one head, and __shfl never reads an inactive lane.)
    float wgt = 0.f, mg = -INFINITY;
    if (lane < kAttnWaves * kMaxGroup) {
        const int w = lane >> 3, g = lane & 7;
        if (g < group) {
#pragma unroll
            for (int v = 0; v < kAttnWaves; ++v) mg = fmaxf(mg, wstat[v][g][0]);
            const float m = wstat[w][g][0];
            wgt = m == -INFINITY ? 0.f : expf(m - mg);
        }
    }
    const int stride = HD + 2;
    float* part = a.partial + ((size_t)kvh * kAttnSplit + range) * group * stride;
    for (int idx = threadIdx.x; idx < group * HD; idx += blockDim.x) {
        const int g = idx / HD, d = idx % HD;
        float o = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) o = fmaf(__shfl(wgt, w * 8 + g, 64), acc_lds[w][g][d], o);
        part[g * stride + d] = o;
    }
    if (wave == 0) {
        const int g = lane < kMaxGroup ? lane : 0;
        float l = 0.f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) l = fmaf(__shfl(wgt, w * 8 + g, 64), wstat[w][g][1], l);
        const float m = __shfl(mg, g, 64);
        if (lane < group) {
            part[lane * stride + HD] = m;
            part[lane * stride + HD + 1] = l;
        }
    }
}

// Merges the range partials of one query head and 64 of its output dims:
// o = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c, then the sigmoid output gate
// (model.cpp:153). There are at most kAttnSplit partials, so every load -- the gate,
// each wave's share of the o values (ranges w, w+4, ...), the statistics -- goes out
// together with the position's, before it is known which ranges hold positions (the
// slots of the others are loaded but never used); the four waves' sums are added
// through LDS. Loading only the ranges that hold positions makes those loads wait for
// the position read: measured 1.2 us slower per call at 512 positions and 2.3 us at
// 1024-4096 (graph replay), for half the merge's fetched bytes at 512.
constexpr int kCombineBatch = kAttnSplit / 4;  // ranges per wave
__global__ __launch_bounds__(256) void attention_combine_kernel(AttnArgs a) {
    __shared__ float wts[kAttnSplit];
    __shared__ float red[8];
    __shared__ float part[4][64];
    const int hd = a.head_dim, group = a.heads / a.kv_heads, dblocks = hd / 64;
    const int head = blockIdx.x / dblocks, db = blockIdx.x - head * dblocks;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int kvh = head / group, g = head - kvh * group, stride = hd + 2;
    const float* base = a.partial + ((size_t)kvh * kAttnSplit * group + g) * stride;
    const size_t cstride = (size_t)group * stride;
    const int d = db * 64 + lane;
    const int pos = *a.position;
    const float gate = a.qkv[(size_t)head * hd * 2 + hd + d];
    float ov[kCombineBatch];
#pragma unroll
    for (int i = 0; i < kCombineBatch; ++i) ov[i] = base[(size_t)(wave + 4 * i) * cstride + d];
    const int cs = min((int)threadIdx.x, kAttnSplit - 1);
    const float m_c = base[(size_t)cs * cstride + hd], l_c = base[(size_t)cs * cstride + hd + 1];
    if (pos < 0 || pos >= a.context) return;
    const int nsub = pos / kAttnSub + 1, per = attn_per(pos + 1);
    const int nchunks = (nsub + per - 1) / per;  // ranges holding positions
    const bool own = (int)threadIdx.x < nchunks;
    const float mloc = wave_max(own ? m_c : -INFINITY);
    if (lane == 0) red[wave] = mloc;
    lds_barrier();
    const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float w = own ? expf(m_c - M) : 0.f;
    if ((int)threadIdx.x < kAttnSplit) wts[threadIdx.x] = w;
    const float dloc = wave_sum(own ? w * l_c : 0.f);
    lds_barrier();  // every weight is in wts; red is free again
    if (lane == 0) red[4 + wave] = dloc;
    float num = 0.f;
#pragma unroll
    for (int i = 0; i < kCombineBatch; ++i) {
        const int c = wave + 4 * i;
        if (c < nchunks) num = fmaf(wts[c], ov[i], num);
    }
    part[wave][lane] = num;
    lds_barrier();
    if (wave == 0) {
        const float den = (red[4] + red[5]) + (red[6] + red[7]);
        const float o = (part[0][lane] + part[1][lane]) + (part[2][lane] + part[3][lane]);
        a.out[(size_t)head * hd + d] = (o / den) * sigmoidf_(gate);
    }
}

// (cos, sin) of angle = pos / base^(2i / rotary) for every position < context and
// i < rotary / 2 (model.cpp:121-127), with the expressions attention_kernel used inline.
__global__ __launch_bounds__(256) void rope_table_kernel(float2* t, int context, int rotary, float base) {
    const int half = rotary / 2;
    const size_t n = (size_t)context * half;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
        const int pos = (int)(idx / half), i = (int)(idx % half);
        const float angle = (float)pos / powf(base, 2.f * (float)i / (float)rotary);
        t[idx] = make_float2(cosf(angle), sinf(angle));
    }
}

// ---- batched form: `count` consecutive prompt positions (the prefill) --------------------
//
// Position t (absolute p0 + t) attends over 0..p0+t. The dense parts run on the matrix
// cores through the FP32 GEMM (S = Q K^T per head, then O = P V): attn_prep_batch_kernel
// normalises and rotates the queries and new keys exactly as attention_kernel does and
// appends k/v to the caches; attn_softmax_batch_kernel turns a row of S into the
// reference's exp(s - peak) / total with s = dot / sqrt(head_dim) (model.cpp:143-150)
// and zeroes the masked keys; attn_gate_batch_kernel applies the sigmoid gate.

// Workgroup = one position; wave w normalises head vectors w, w+8, ... of the group's
// q heads (all kv heads' groups) and the kv heads' new keys.
template <int E>
__global__ __launch_bounds__(512) void attn_prep_batch_kernel(AttnBatchArgs a) {
    constexpr int HD = 64 * E;
    extern __shared__ __align__(16) float rows[];  // (heads + kv_heads) x HD
    const int t = blockIdx.x, pos = a.first + t;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int nh = a.heads + a.kv_heads, qd = a.heads * HD * 2, kvd = a.kv_heads * HD;
    const float* row = a.qkv + (size_t)t * a.stride;
    for (int v = wave; v < nh; v += waves) {
        const bool is_q = v < a.heads;
        const float* src = is_q ? row + (size_t)v * HD * 2 : row + qd + (size_t)(v - a.heads) * HD;
        const float* w = is_q ? a.q_norm : a.k_norm;
        float x[E], ss = 0.f;
        ldv<E>(x, src + E * lane);
#pragma unroll
        for (int e = 0; e < E; ++e) ss += x[e] * x[e];
        ss = wave_sum(ss);
        const float scale = 1.f / sqrtf(ss / (float)HD + a.eps);
        float wv[E], y[E];
        ldv<E>(wv, w + E * lane);
#pragma unroll
        for (int e = 0; e < E; ++e) y[e] = x[e] * (scale * wv[e]);
        stv<E>(rows + (size_t)v * HD + E * lane, y);
    }
    __syncthreads();
    const int half = a.rotary / 2;
    for (int idx = threadIdx.x; idx < nh * half; idx += blockDim.x) {
        const int v = idx / half, i = idx % half;
        float* r = rows + (size_t)v * HD;
        const float2 cs = a.rope[(size_t)pos * half + i];
        const float c = cs.x, s = cs.y;
        const float x0 = r[i], x1 = r[i + half];
        r[i] = x0 * c - x1 * s;
        r[i + half] = x0 * s + x1 * c;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < a.heads * HD; idx += blockDim.x) a.q[(size_t)t * a.heads * HD + idx] = rows[idx];
    for (int idx = threadIdx.x; idx < kvd; idx += blockDim.x) {
        a.keys[(size_t)pos * kvd + idx] = rows[(size_t)a.heads * HD + idx];
        a.values[(size_t)pos * kvd + idx] = row[qd + kvd + idx];
    }
}

// Row (t, h) of S (keys 0..L-1, padded to lp): p = exp(s - peak) / total over keys
// 0..first+t with s = S / sqrt(head_dim); masked and padding keys get 0.
__global__ __launch_bounds__(256) void attn_softmax_batch_kernel(AttnBatchArgs a) {
    __shared__ float red[8];
    const int row = blockIdx.x;  // h * count + t
    const int t = row % a.count;
    const int n = a.first + t + 1;
    float* s = a.scores + (size_t)row * a.lp;
    const float root = sqrtf((float)a.head_dim);
    float m = -INFINITY;
    for (int j = threadIdx.x; j < n; j += blockDim.x) m = fmaxf(m, s[j] / root);
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float total = 0.f;
    for (int j = threadIdx.x; j < n; j += blockDim.x) {
        const float e = expf(s[j] / root - m);
        s[j] = e;
        total += e;
    }
    total = wave_sum(total);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = total;
    __syncthreads();
    total = (red[0] + red[1]) + (red[2] + red[3]);
    for (int j = threadIdx.x; j < a.lp; j += blockDim.x) s[j] = j < n ? s[j] / total : 0.f;
}

// The same row softmax for rows of at most 256 * KR keys, the row held in registers from
// its one read to its one write (the same thread-to-key assignment and sums as above,
// so the same results).
template <int KR>
__global__ __launch_bounds__(256) void attn_softmax_rows_kernel(AttnBatchArgs a) {
    __shared__ float red[8];
    const int row = blockIdx.x;  // h * count + t
    const int t = row % a.count;
    const int n = a.first + t + 1;
    float* s = a.scores + (size_t)row * a.lp;
    const float root = sqrtf((float)a.head_dim);
    float v[KR];
    float m = -INFINITY;
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const int j = threadIdx.x + 256 * k;
        v[k] = j < n ? s[j] / root : -INFINITY;
        m = fmaxf(m, v[k]);
    }
    m = wave_max(m);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        if ((int)threadIdx.x + 256 * k < n) {
            v[k] = expf(v[k] - m);
            total += v[k];
        }
    }
    total = wave_sum(total);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = total;
    __syncthreads();
    total = (red[0] + red[1]) + (red[2] + red[3]);
#pragma unroll
    for (int k = 0; k < KR; ++k) {
        const int j = threadIdx.x + 256 * k;
        if (j < a.lp) s[j] = j < n ? v[k] / total : 0.f;
    }
}

// vt[kvh][d][j] = values[j][kvh][d] for keys j < L, 0 up to lp: 32 x 32 tiles via LDS.
__global__ __launch_bounds__(256) void attn_vt_batch_kernel(AttnBatchArgs a) {
    __shared__ float tile[32][33];
    const int kvh = blockIdx.z, d0 = blockIdx.y * 32, j0 = blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    const int L = a.first + a.count, kvd = a.kv_heads * a.head_dim;
    for (int r = ty; r < 32; r += 8) {
        const int j = j0 + r;
        tile[r][tx] = j < L ? a.values[(size_t)j * kvd + (size_t)kvh * a.head_dim + d0 + tx] : 0.f;
    }
    __syncthreads();
    for (int r = ty; r < 32; r += 8)
        a.vt[((size_t)kvh * a.head_dim + d0 + r) * a.lp + j0 + tx] = tile[tx][r];
}

// out[t][h*hd + d] = o[t][h*hd + d] * sigmoid(gate) (model.cpp:153)
__global__ __launch_bounds__(256) void attn_gate_batch_kernel(AttnBatchArgs a) {
    const int hdim = a.heads * a.head_dim;
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)a.count * hdim) return;
    const int t = (int)(i / hdim), c = (int)(i % hdim), h = c / a.head_dim, d = c % a.head_dim;
    const float g = a.qkv[(size_t)t * a.stride + (size_t)h * a.head_dim * 2 + a.head_dim + d];
    a.out[(size_t)t * a.out_stride + c] = a.o[i] * sigmoidf_(g);
}

}  // namespace

hipError_t launch_attention_batch(const AttnBatchArgs& a, hipStream_t stream) {
    const int group = a.heads / a.kv_heads, hd = a.head_dim, L = a.first + a.count;
    if (a.count < 1 || a.heads % a.kv_heads || a.lp % 32 || a.lp < L || hd % 32) return hipErrorInvalidValue;
    const size_t prep_lds = (size_t)(a.heads + a.kv_heads) * hd * sizeof(float);
    switch (hd) {
    case 64: launch_kernel(attn_prep_batch_kernel<1>, dim3(a.count), dim3(512), prep_lds, stream, a); break;
    case 128: launch_kernel(attn_prep_batch_kernel<2>, dim3(a.count), dim3(512), prep_lds, stream, a); break;
    case 256: launch_kernel(attn_prep_batch_kernel<4>, dim3(a.count), dim3(512), prep_lds, stream, a); break;
    default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int kvd = a.kv_heads * hd;
    // S_h = Q_h K_kvh^T for every head in one launch; tiles wholly past the causal limit
    // are skipped (the softmax reads keys 0 .. first+t of row t only)
    e = launch_gemm_f32_heads(a.q, a.keys, a.scores, a.count, L, hd, a.heads * hd, kvd, a.lp, a.heads, group,
                              (size_t)hd, (size_t)hd, (size_t)a.count * a.lp, true, false, a.first, stream);
    if (e != hipSuccess) return e;
    if (a.lp <= 256 * 8)
        launch_kernel(attn_softmax_rows_kernel<8>, dim3(a.heads * a.count), dim3(256), 0, stream, a);
    else if (a.lp <= 256 * 16)
        launch_kernel(attn_softmax_rows_kernel<16>, dim3(a.heads * a.count), dim3(256), 0, stream, a);
    else
        launch_kernel(attn_softmax_batch_kernel, dim3(a.heads * a.count), dim3(256), 0, stream, a);
    launch_kernel(attn_vt_batch_kernel, dim3(a.lp / 32, hd / 32, a.kv_heads), dim3(256), 0, stream, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    // O_h = P_h V_kvh for every head in one launch, each tile's K loop ending at its rows'
    // last key (P is zero past it)
    e = launch_gemm_f32_heads(a.scores, a.vt, a.o, a.count, hd, a.lp, a.lp, a.lp, a.heads * hd, a.heads, group,
                              (size_t)a.count * a.lp, (size_t)hd * a.lp, (size_t)hd, false, true, a.first, stream);
    if (e != hipSuccess) return e;
    const size_t n = (size_t)a.count * a.heads * hd;
    launch_kernel(attn_gate_batch_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_rope_table(float2* table, int context, int rotary, float base, hipStream_t stream) {
    const size_t n = (size_t)context * (rotary / 2);
    if (!n) return hipSuccess;
    launch_kernel(rope_table_kernel, dim3((unsigned)std::min<size_t>((n + 255) / 256, 1024)), dim3(256), 0, stream,
                  table, context, rotary, base);
    return hipGetLastError();
}

size_t attention_partial_floats(int heads, int kv_heads, int head_dim, int context) {
    (void)context;  // the grid has kAttnSplit ranges at every context length
    return (size_t)kv_heads * kAttnSplit * (heads / kv_heads) * (head_dim + 2);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t stream) {
    if (a.heads % a.kv_heads || a.heads / a.kv_heads > kMaxGroup || a.rotary > a.head_dim || a.rotary % 2)
        return hipErrorInvalidValue;
    const dim3 grid(a.kv_heads * kAttnSplit), block(kAttnWaves * 64);
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
