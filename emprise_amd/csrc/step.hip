// Persistent decode-step kernel on gfx950: one launch runs a recorded phase program
// (step.hpp) -- the grouped dequant-matvecs, Gated DeltaNet updates and attention of
// one qwen35 decode step -- with tagged activation slots instead of kernel boundaries.
//
// Why: a decode step of the 9B shape is ~170 dependent launches. Between two launches
// the chip drains (the last workgroups of one kernel finish while nothing streams) and
// refills (every wave of the next kernel issues its first weight loads at once, and the
// input staging waits behind that burst). Here a wave that runs out of items in one
// phase issues the weight loads of its first items of the next phase immediately and
// only then waits -- on the input slots it needs, not on a grid barrier.
//
// Memory model: producers store {value, tag} as one 8-byte agent-scope store
// (global_store_dwordx2 sc1, written through to the coherence point shared by all XCDs);
// consumers load the slots with agent-scope 8-byte loads (sc1: never a stale L2 copy)
// until every tag matches. No fence or cache maintenance is involved: the value and
// its tag travel in one single-copy-atomic access. Slots are reused only along
// dependency chains (a later writer of a buffer transitively depends on every reader
// of the previous version), so a reader never sees a newer version; a mismatch that
// outlives the deadline sets the error word and ends the kernel instead of hanging.
//
// All waits are bounded: each poll loop checks the real-time counter against a
// deadline fixed at kernel start and the shared error word, so a kernel whose
// workgroups could not all run (or any logic error) ends with err set.
#include "common.hpp"
#include "decode.hpp"
#include "stream.hpp"
#include "step.hpp"

namespace emprise {
namespace {

constexpr uint64_t kStepDeadlineTicks = 200000000ull;  // 2 s of the 100 MHz real-time counter

// ---- global-memory access ----------------------------------------------------------------
// Pointers read from the program are generic; casting them to the global address space
// makes their accesses global_* instructions, which count against vmcnt only (a flat
// access also counts against lgkmcnt, so every LDS wait would wait for it too).

template <class T> __device__ __forceinline__ const EMPRISE_GLOBAL T* gc(const T* p) {
    return (const EMPRISE_GLOBAL T*)p;
}
template <class T> __device__ __forceinline__ EMPRISE_GLOBAL T* gm(T* p) { return (EMPRISE_GLOBAL T*)p; }
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 gld4(const float* p, size_t i4) {
    const f32x4_t v = ((const EMPRISE_GLOBAL f32x4_t*)p)[i4];
    return make_float4(v.x, v.y, v.z, v.w);
}

// ---- tagged operands -------------------------------------------------------------------

__device__ __forceinline__ uint64_t ld_slot(const void* p, size_t i) {
    return __hip_atomic_load(gm(const_cast<uint64_t*>(reinterpret_cast<const uint64_t*>(p))) + i, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_slot(void* p, size_t i, float v, uint32_t tag) {
    __hip_atomic_store(gm(reinterpret_cast<uint64_t*>(p)) + i, ((uint64_t)tag << 32) | __float_as_uint(v),
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_out(const StepOut& o, size_t i, float v, uint32_t tag) {
    if (o.tagged) st_slot(o.p, i, v, tag);
    else gm(reinterpret_cast<float*>(o.p))[i] = v;
}
// Tag an input must carry; plain inputs are packed with the same value.
__device__ __forceinline__ uint32_t want_of(const StepIn& in, uint32_t base) {
    return in.phase < 0 ? 0xffffffffu : (base | (uint32_t)in.phase);
}
__device__ __forceinline__ uint64_t ld_in(const StepIn& in, size_t i, uint32_t want) {
    if (in.phase < 0) return ((uint64_t)want << 32) | __float_as_uint(gc(reinterpret_cast<const float*>(in.p))[i]);
    return ld_slot(in.p, i);
}
__device__ __forceinline__ bool tag_ok(uint64_t v, uint32_t want) { return (uint32_t)(v >> 32) == want; }
// One more poll of a slot that may not be ready: the load is issued unconditionally
// (no per-lane branch, so poll loops unroll) and kept only where the tag was wrong. Only
// tagged inputs reach a re-poll: a plain input always carries its wanted tag.
__device__ __forceinline__ uint64_t repoll(uint64_t v, uint32_t want, const void* p, size_t i) {
    const uint64_t fresh = ld_slot(p, i);
    return tag_ok(v, want) ? v : fresh;
}
__device__ __forceinline__ float val(uint64_t v) { return __uint_as_float((uint32_t)v); }

// Bounded polling: again() sleeps briefly and says whether another round is allowed.
struct Waiter {
    uint64_t deadline;
    uint32_t* err;
    bool failed;
    int rounds;
    __device__ bool again() {
        if (failed) return false;
        __builtin_amdgcn_s_sleep(2);
        if ((++rounds & 15) == 0) {
            if (__builtin_amdgcn_s_memrealtime() > deadline) {
                __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                failed = true;
            } else if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
                failed = true;
            }
        }
        return !failed;
    }
};

// ---- grouped matvec phase ------------------------------------------------------------------

// Elements k .. k+3 of row `row` of an encoded matrix. Kept out of line: the per-type
// decoder is large, and inlined into the staging loops it stops them from unrolling
// (which would move the staged registers to scratch memory).
__device__ __attribute__((noinline)) float4 decode4(const uint8_t* w, uint32_t type, int cols, int row, int k) {
    return make_float4(decode_element(w, type, cols, (uint64_t)row, k), decode_element(w, type, cols, (uint64_t)row, k + 1),
                       decode_element(w, type, cols, (uint64_t)row, k + 2), decode_element(w, type, cols, (uint64_t)row, k + 3));
}

// Waves of a workgroup that stage a matvec phase's input: half of them for inputs of up
// to 4096 columns (the other half prefetch weights meanwhile); all of them for wider,
// plain inputs (the 12288-wide down projection), whose slots would not fit half the waves'
// registers.
constexpr int step_stagers(int sb) { return sb <= 2 ? kStepWaves / 2 : kStepWaves; }

// Input staging of a matvec phase by the stager waves (sw = 0 .. kStagers-1): float4 i of
// the input is held by stager i / 64 % kStagers, lane i % 64, slot i / (64 * kStagers).
// Polls x (+ delta, or the gate) until every tag matches, forms v = x + delta (workgroup
// 0 also stores v to x_out), then RMSNorm (the stagers' partial sums meet in LDS after
// barrier (1)) or the per-head norm x SiLU(gate) (a head is head_dim/4 consecutive float4,
// held by consecutive lanes of one stager), and writes LDS in chunk_slot order plus the
// per-unit input sums. Ends between barriers (1) and (2): the caller issues (2).
// SB: float4 per thread of a whole workgroup (2 for 4096 columns, 6 for 12288).
template <int UNIT, int SB>
__device__ void step_stage(const StepMatvec& m, uint32_t tag, uint32_t base, float* xs, float* usum, float* red,
                           Waiter& wt, int sw) {
    constexpr bool DN = SB <= 2;                     // residual / norm / gate forms (<= 4096 columns)
    constexpr int NS = step_stagers(SB);             // stager waves
    constexpr int K = SB * kStepWaves / NS;          // float4 per stager lane
    const int lane = threadIdx.x & 63;
    const int n4 = m.cols / 4;
    auto idx = [&](int k) { return min(lane + 64 * (sw + NS * k), n4 - 1); };
    const uint32_t wx = want_of(m.x, base), wd = want_of(m.delta, base), wg = want_of(m.gate, base);
    const StepIn& dsrc = m.gate.p ? m.gate : m.delta;
    const uint32_t wdd = m.gate.p ? wg : wd;
    const bool emb = m.emb != nullptr;
    uint64_t xr[K][4];
    uint64_t dr[DN ? K : 1][4];
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const size_t i = idx(k);
        if (!emb) {
#pragma unroll
            for (int j = 0; j < 4; ++j) xr[k][j] = ld_in(m.x, 4 * i + j, wx);
        }
        if constexpr (DN) {
#pragma unroll
            for (int j = 0; j < 4; ++j) dr[k][j] = dsrc.p ? ld_in(dsrc, 4 * i + j, wdd) : 0ull;
        }
    }
    float4 x[K];
    if (emb) {
        // the embedding row of the current token (get_rows), decoded in place
        const int t = *gc(m.token);
        const bool in_range = t >= 0 && t < m.emb_rows;
#pragma unroll
        for (int k = 0; k < K; ++k)
            x[k] = in_range ? decode4(m.emb, m.emb_type, m.cols, t, 4 * idx(k)) : make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
        while (true) {
            bool ready = true;
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int j = 0; j < 4; ++j) ready &= tag_ok(xr[k][j], wx);
            if (ready || !wt.again()) break;
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int j = 0; j < 4; ++j) xr[k][j] = repoll(xr[k][j], wx, m.x.p, 4 * (size_t)idx(k) + j);
        }
#pragma unroll
        for (int k = 0; k < K; ++k) x[k] = make_float4(val(xr[k][0]), val(xr[k][1]), val(xr[k][2]), val(xr[k][3]));
    }
    if constexpr (DN) {
        if (dsrc.p) {
            while (true) {
                bool ready = true;
#pragma unroll
                for (int k = 0; k < K; ++k)
#pragma unroll
                    for (int j = 0; j < 4; ++j) ready &= tag_ok(dr[k][j], wdd);
                if (ready || !wt.again()) break;
#pragma unroll
                for (int k = 0; k < K; ++k)
#pragma unroll
                    for (int j = 0; j < 4; ++j) dr[k][j] = repoll(dr[k][j], wdd, dsrc.p, 4 * (size_t)idx(k) + j);
            }
        }
        if (m.gate.p) {
            // per-head RMSNorm x SiLU(gate) (backend.cpp:57-58)
            const int h4 = m.head_dim / 4;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const float4 w = gld4(m.norm, idx(k) % h4);
                float q = x[k].x * x[k].x + x[k].y * x[k].y + x[k].z * x[k].z + x[k].w * x[k].w;
                for (int s = 1; s < h4; s <<= 1) q += __shfl_xor(q, s, 64);
                const float scale = 1.f / sqrtf(q / (float)m.head_dim + m.eps);
                x[k].x = x[k].x * (scale * w.x) * val(dr[k][0]);
                x[k].y = x[k].y * (scale * w.y) * val(dr[k][1]);
                x[k].z = x[k].z * (scale * w.z) * val(dr[k][2]);
                x[k].w = x[k].w * (scale * w.w) * val(dr[k][3]);
            }
        } else {
            const bool writer = m.x_out.p && blockIdx.x == 0;
            // The sum of squares is formed in the order of an eight-wave workgroup that holds
            // float4 t and t + 512 in thread t (the per-projection kernels' staging): float4 i
            // belongs to "wave" (i / 64) % 8, so slots k and k + 2 of stager sw make wave sw's
            // share and slots k + 1, k + 3 wave sw + 4's; the eight sums meet in order.
            static_assert(K == 4 && NS == 4, "RMSNorm order assumes 4 stagers x 4 float4");
            float part[2] = {0.f, 0.f};
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int i = lane + 64 * (sw + NS * k);
                if (dsrc.p) {
                    x[k].x += val(dr[k][0]);
                    x[k].y += val(dr[k][1]);
                    x[k].z += val(dr[k][2]);
                    x[k].w += val(dr[k][3]);
                }
                if (i < n4) {
                    if (writer) {
                        st_out(m.x_out, 4 * (size_t)i + 0, x[k].x, tag);
                        st_out(m.x_out, 4 * (size_t)i + 1, x[k].y, tag);
                        st_out(m.x_out, 4 * (size_t)i + 2, x[k].z, tag);
                        st_out(m.x_out, 4 * (size_t)i + 3, x[k].w, tag);
                    }
                    part[k & 1] += x[k].x * x[k].x + x[k].y * x[k].y + x[k].z * x[k].z + x[k].w * x[k].w;
                }
            }
            part[0] = wave_sum(part[0]);
            part[1] = wave_sum(part[1]);
            if (lane == 0) {
                red[sw] = part[0];
                red[sw + NS] = part[1];
            }
        }
    }
    lds_barrier();  // (1) every wave has left the previous phase: LDS is free
    if constexpr (DN) {
        if (!m.gate.p && m.norm) {
            float total = 0.f;
#pragma unroll
            for (int w = 0; w < kStepWaves; ++w) total += red[w];
            const float scale = 1.f / sqrtf(total / (float)m.cols + m.eps);
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const float4 w = gld4(m.norm, idx(k));
                x[k].x = x[k].x * (scale * w.x);
                x[k].y = x[k].y * (scale * w.y);
                x[k].z = x[k].z * (scale * w.z);
                x[k].w = x[k].w * (scale * w.w);
            }
        }
    }
    constexpr int U4 = UNIT / 4;
    float4* xs4 = reinterpret_cast<float4*>(xs);
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int i = lane + 64 * (sw + NS * k);
        if (i < n4) xs4[chunk_slot(i)] = x[k];
        float t = (x[k].x + x[k].y) + (x[k].z + x[k].w);
        t += __shfl_xor(t, 1, 64);
        t += __shfl_xor(t, 2, 64);
        if constexpr (U4 == 8) t += __shfl_xor(t, 4, 64);
        if (i < n4 && (i & (U4 - 1)) == 0) usum[i / U4] = stored_unit_sum<UNIT>(t);
    }
}

// One matvec phase: the streaming kernel's item walk (row group x 4096-column chunk per
// wave, two items in flight) with tagged input staging and tagged outputs.
// SB: float4 of input per thread (2: <= 4096 columns with norm / gate / residual; 6: up to
// 12288 columns, plain input).
template <int T, bool PAIR, bool CONV, int SB>
__device__ void step_matvec(const StepMatvec& m, uint32_t tag, uint32_t base, unsigned char* smem, float* red,
                            unsigned long long* block_best, Waiter& wt) {
    constexpr int R = PAIR ? kMvStreamPairRows : kMvStreamRows;
    constexpr int UW = Fmt<T>::unit;
    constexpr int NA = PAIR ? R * 2 : R;
    float* xs = reinterpret_cast<float*>(smem);
    float* usum = xs + m.cols;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int cols = m.cols, groups = m.groups, nseg = m.nseg;
    const int cpr = cols / kChunkCols;
    const size_t row_bytes = (size_t)(cols / 256) * Fmt<T>::block;
    const int stride = gridDim.x * kStepWaves;
    const uint8_t* dummy = m.seg[0].w;  // row 0 of segment 0: a readable, unused source

    auto rows_of = [&](SItem<NA>& it) {
        int s = 0;
        while (s + 1 < nseg && it.g >= m.seg[s + 1].g0) ++s;
        it.seg = s;
        it.row0 = (it.g - m.seg[s].g0) * R;
        const int nrows = m.seg[s].rows;
#pragma unroll
        for (int r = 0; r < NA; ++r) {
            const int rr = r < R ? it.row0 + r : it.row0 + r - R;
            const int rc = rr < nrows ? rr : nrows - 1;
            it.rp[r] = (r < R ? m.seg[s].w : m.seg[1].w) + (size_t)rc * row_bytes;
        }
    };
    auto skip = [&](SItem<NA>& it, int n) {
        const int c = it.c + n, hop = c / cpr;
        it.c = c - hop * cpr;
        if (hop) {
            it.g += hop * stride;
            if (it.g < groups) rows_of(it);
        }
    };
    auto iload = [&](SChunk<T, NA>& buf, SItem<NA>& it) {
        const bool valid = it.g < groups;
        const uint8_t* p[NA];
#pragma unroll
        for (int r = 0; r < NA; ++r) p[r] = valid ? it.rp[r] : dummy;
        sload<T, NA>(buf, p, valid ? it.c : 0, lane);
        if constexpr (CONV) {
            const int cw = m.conv_width, r = lane / cw, j = lane - r * cw, row = it.row0 + r;
            const bool on = valid && it.seg == 0 && r < R && row < m.seg[0].rows;
            const size_t o = on ? (size_t)row * cw + j : 0;
            const float h = gc(m.conv_state)[o], k = gc(m.conv_w)[o];
            it.conv_h = on ? h : 0.f;
            it.conv_k = on ? k : 0.f;
        }
    };

    // Roles: waves 0 .. kStepWaves-kStagers-1 issue the weight loads of their first two
    // items at once and wait; the stager waves poll the input first (no weight loads of
    // their own ahead of the polls, which return in order), stage it into LDS, and only
    // then load their first items.
    constexpr int NS = step_stagers(SB);
    const bool stager = wave >= kStepWaves - NS;
    SItem<NA> ia, ib;
    ia.g = blockIdx.x * kStepWaves + wave;
    ia.c = 0;
    if (ia.g < groups) rows_of(ia);
    ib = ia;
    skip(ib, 1);
    SChunk<T, NA> A, B;
    if (!stager) {
        __builtin_amdgcn_sched_barrier(0);
        iload(A, ia);
        __builtin_amdgcn_sched_barrier(0);
        iload(B, ib);
        __builtin_amdgcn_sched_barrier(0);
        lds_barrier();  // (1) every wave has left the previous phase: LDS is free
    } else {
        step_stage<UW, SB>(m, tag, base, xs, usum, red, wt, wave - (kStepWaves - NS));  // ends with (1)
    }
    if (m.mode == kMvArgmax && threadIdx.x == 0) *block_best = 0ull;
    lds_barrier();  // (2) the staged input and its unit sums are in LDS
    if (stager) {
        __builtin_amdgcn_sched_barrier(0);
        iload(A, ia);
        __builtin_amdgcn_sched_barrier(0);
        iload(B, ib);
        __builtin_amdgcn_sched_barrier(0);
    }

    unsigned long long best = 0ull;
    float acc[NA];
#pragma unroll
    for (int r = 0; r < NA; ++r) acc[r] = 0.f;
    auto process = [&](SChunk<T, NA>& buf, SItem<NA>& it) {
        scompute<T, NA>(buf, acc, xs, usum, it.c, lane);
        if (it.c == cpr - 1) {
#pragma unroll
            for (int r = 0; r < NA; ++r) acc[r] = wave_sum(acc[r]);
            if (CONV && it.seg == 0) {
                // causal conv1d + SiLU (backend.cpp:22-29), as in the streaming kernel
                const int cw = m.conv_width, r = lane / cw, j = lane - r * cw, row = it.row0 + r;
                float v = 0.f;
#pragma unroll
                for (int rr = 0; rr < R; ++rr) v = r == rr ? acc[rr] : v;
                const float shifted = __shfl_down(it.conv_h, 1, 64);
                const float hn = j == cw - 1 ? v : shifted;
                const float p = hn * it.conv_k;
                float sum = 0.f;
                for (int jj = 0; jj < cw; ++jj) sum += __shfl(p, lane - j + jj, 64);
                if (r < R && row < m.seg[0].rows) {
                    gm(m.conv_state)[(size_t)row * cw + j] = hn;
                    if (j == 0) st_out(m.seg[0].y, row, siluf_(sum), tag);
                }
            } else if (lane == 0) {
                const int s = it.seg;
                const int srows = m.seg[s].rows;
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const int row = it.row0 + r;
                    if (row < srows) {
                        if constexpr (PAIR) {
                            st_out(m.seg[s].y, row, siluf_(acc[r]) * acc[(R + r) % NA], tag);
                        } else {
                            float v = acc[r];
                            if constexpr (CONV)  // (see the streaming kernel)
                                if ((m.silu_mask >> s) & 1) {
                                    asm volatile("" : "+v"(v));
                                    v = siluf_(v);
                                }
                            if (m.seg[s].y.p) st_out(m.seg[s].y, row, v, tag);
                            if (m.mode == kMvArgmax) {
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
        skip(it, 2);
        iload(buf, it);
    };
    while (ia.g < groups) {
        process(A, ia);
        if (ib.g >= groups) break;
        process(B, ib);
    }
    if (m.mode == kMvArgmax) {
        if (lane == 0 && best) atomicMax(block_best, best);
        lds_barrier();
        if (threadIdx.x == 0 && *block_best)
            __hip_atomic_fetch_max(gm(m.argmax), *block_best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---- Gated DeltaNet phase ------------------------------------------------------------------

// gdn_rows_kernel's state update (gdn.hip) with tagged q/k/v/alpha/beta inputs: unit u =
// value head u / SPLIT, rows part*(SD/SPLIT).. of it, four rows per wave on the 16 lanes
// of a DPP row each (common.hpp's gdn16 layout), raw outputs S.q.
template <int E, int SPLIT>
__device__ void step_gdn(const StepGdn& g, uint32_t tag, uint32_t base, Waiter& wt) {
    constexpr int SD = 64 * E, NE = SD / 16;
    static_assert(SD / SPLIT == 4 * kStepWaves, "four rows per wave");
    const int units = g.value_heads * SPLIT;
    const int lane = threadIdx.x & 63, j = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wq = want_of(g.qkv, base), wa = want_of(g.alpha, base), wb = want_of(g.beta, base);
    for (int u = blockIdx.x; u < units; u += gridDim.x) {
        const int h = u / SPLIT, part = u - h * SPLIT, kh = h % g.key_heads;  // tiled V heads (backend.cpp:37)
        const int key_dim = g.key_heads * SD;
        const int d = part * (SD / SPLIT) + wave * 4 + (lane >> 4);  // this lane's row
        EMPRISE_GLOBAL float* Sd = gm(g.state) + ((size_t)h * SD + d) * SD + NE * j;
        float s[NE];
#pragma unroll
        for (int i = 0; i < NE; ++i) s[i] = Sd[i];
        const size_t vo = 2 * (size_t)key_dim + (size_t)h * SD + d;
        uint64_t vr = ld_in(g.qkv, vo, wq);
        uint64_t qr[NE], kr[NE];
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            qr[i] = ld_in(g.qkv, (size_t)kh * SD + NE * j + i, wq);
            kr[i] = ld_in(g.qkv, (size_t)key_dim + (size_t)kh * SD + NE * j + i, wq);
        }
        uint64_t ar = ld_in(g.alpha, h, wa), br = ld_in(g.beta, h, wb);
        while (true) {
            bool ready = tag_ok(vr, wq) && tag_ok(ar, wa) && tag_ok(br, wb);
#pragma unroll
            for (int i = 0; i < NE; ++i) ready = ready && tag_ok(qr[i], wq) && tag_ok(kr[i], wq);
            if (ready || !wt.again()) break;
            vr = repoll(vr, wq, g.qkv.p, vo);
#pragma unroll
            for (int i = 0; i < NE; ++i) {
                qr[i] = repoll(qr[i], wq, g.qkv.p, (size_t)kh * SD + NE * j + i);
                kr[i] = repoll(kr[i], wq, g.qkv.p, (size_t)key_dim + (size_t)kh * SD + NE * j + i);
            }
            ar = repoll(ar, wa, g.alpha.p, h);
            br = repoll(br, wb, g.beta.p, h);
        }
        float qv[NE], kv[NE];
#pragma unroll
        for (int i = 0; i < NE; ++i) {
            qv[i] = val(qr[i]);
            kv[i] = val(kr[i]);
        }
        gdn16_qk_norm<NE>(qv, kv, g.eps);  // q/k L2 normalisation (backend.cpp:30-35)
        const float decay = expf(gc(g.ssm_a)[h] * softplusf_(val(ar) + gc(g.dt)[h]));
        const float b = sigmoidf_(val(br));
        const float sum = gdn16_row<NE>(s, qv, kv, decay, b, val(vr));
#pragma unroll
        for (int i = 0; i < NE; ++i) Sd[i] = s[i];
        if (j == 0) st_out(g.out, (size_t)h * SD + d, sum, tag);
    }
}

// ---- attention phases ------------------------------------------------------------------

constexpr int kMaxGroup = 8;
constexpr int kCombineBatch = 8;    // chunks per wave held in registers per pass
constexpr int kCombineMaxChunks = 1024;

template <int E> struct AttnLds {
    static constexpr int HD = 64 * E, CH = kAttnChunk, KS = HD + 4;
    static constexpr int KBYTES = CH * KS * 4, ABYTES = kStepWaves * kMaxGroup * HD * 4;
    static constexpr int KV = KBYTES > ABYTES ? KBYTES : ABYTES;
    static constexpr int QS = kMaxGroup * HD * 4, NEW = 2 * HD * 4, SC = kMaxGroup * CH * 4, ST = 2 * kMaxGroup * 4;
    static constexpr int bytes = KV + QS + NEW + SC + ST;
};

// Split-KV attention partial of (kv head, chunk) units (attention.hip's
// attention_kernel with eight waves and tagged q/k/v inputs and partial outputs): unit
// u = kvh * nchunks + chunk, chunks of kAttnChunk positions.
template <int E>
__device__ void step_attention(const StepAttention& a, uint32_t tag, uint32_t base, unsigned char* smem, Waiter& wt) {
    using L = AttnLds<E>;
    constexpr int HD = L::HD, CH = L::CH, KS = L::KS, NW = kStepWaves, PW = CH / NW;
    constexpr int NJ = (kMaxGroup + NW) / NW;  // heads per wave, incl. the key
    float (*ks)[KS] = reinterpret_cast<float (*)[KS]>(smem);
    float (*acc_lds)[kMaxGroup][HD] = reinterpret_cast<float (*)[kMaxGroup][HD]>(smem);
    float (*qs)[HD] = reinterpret_cast<float (*)[HD]>(smem + L::KV);
    float* knew = reinterpret_cast<float*>(smem + L::KV + L::QS);
    float* vnew = knew + HD;
    float (*sc)[CH] = reinterpret_cast<float (*)[CH]>(smem + L::KV + L::QS + L::NEW);
    float* mstat = reinterpret_cast<float*>(smem + L::KV + L::QS + L::NEW + L::SC);
    float* lstat = mstat + kMaxGroup;

    const int group = a.heads / a.kv_heads;
    const int chunks_max = (a.context + CH - 1) / CH;
    const int pos = *gc(a.position);
    if (pos < 0 || pos >= a.context) return;  // the host keeps positions inside the caches
    const int len = pos + 1, nchunks = (len + CH - 1) / CH;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qd = a.heads * HD * 2, kvd = a.kv_heads * HD;
    const uint32_t wq = want_of(a.qkv, base);
    const int stride = HD + 2;
    for (int u = blockIdx.x; u < a.kv_heads * nchunks; u += gridDim.x) {
        const int kvh = u / nchunks, chunk = u - kvh * nchunks;
        const size_t kin = (size_t)qd + (size_t)kvh * HD, vin = (size_t)qd + kvd + (size_t)kvh * HD;
        // norm inputs (query heads of the group, the new key as head `group`), then rows
        uint64_t xr[NJ][E];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int gg = min(wave + NW * j, group);
            const size_t src = gg < group ? (size_t)(kvh * group + gg) * HD * 2 : kin;
#pragma unroll
            for (int e = 0; e < E; ++e) xr[j][e] = ld_in(a.qkv, src + E * lane + e, wq);
        }
        uint64_t vr0 = ld_in(a.qkv, vin + min((int)threadIdx.x, HD - 1), wq);
        float qn[E], kn[E];
#pragma unroll
        for (int e = 0; e < E; ++e) {
            qn[e] = gc(a.q_norm)[E * lane + e];
            kn[e] = gc(a.k_norm)[E * lane + e];
        }
        const int t0 = chunk * CH, tn = min(CH, len - t0);
        const size_t row_stride = (size_t)a.kv_heads * HD;
        const EMPRISE_GLOBAL float* kb = gc(a.keys) + ((size_t)t0 * a.kv_heads + kvh) * HD + E * lane;
        const EMPRISE_GLOBAL float* vb = gc(a.values) + ((size_t)t0 * a.kv_heads + kvh) * HD + E * lane;
        float kr[PW][E], vr[PW][E];
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int tt = wave + NW * i;
            if (tt < tn) {
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    kr[i][e] = kb[(size_t)tt * row_stride + e];
                    vr[i][e] = vb[(size_t)tt * row_stride + e];
                }
            }
        }
        while (true) {
            bool ready = tag_ok(vr0, wq);
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int e = 0; e < E; ++e) ready = ready && tag_ok(xr[j][e], wq);
            if (ready || !wt.again()) break;
            vr0 = repoll(vr0, wq, a.qkv.p, vin + min((int)threadIdx.x, HD - 1));
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int gg = min(wave + NW * j, group);
                const size_t src = gg < group ? (size_t)(kvh * group + gg) * HD * 2 : kin;
#pragma unroll
                for (int e = 0; e < E; ++e) xr[j][e] = repoll(xr[j][e], wq, a.qkv.p, src + E * lane + e);
            }
        }
        lds_barrier();  // the previous phase or unit is done with LDS
        // RMSNorm of the query heads and of the new key (model.cpp:133-134)
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int gg = wave + NW * j;
            if (gg <= group) {
                float x[E], ss = 0.f;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    x[e] = val(xr[j][e]);
                    ss += x[e] * x[e];
                }
                ss = wave_sum(ss);
                const float scale = 1.f / sqrtf(ss / (float)HD + a.eps);
                float* dst = (gg < group ? qs[gg] : knew) + E * lane;
#pragma unroll
                for (int e = 0; e < E; ++e) dst[e] = x[e] * (scale * (gg < group ? qn[e] : kn[e]));
            }
        }
        if (threadIdx.x < HD) vnew[threadIdx.x] = val(vr0);
        lds_barrier();
        // NEOX RoPE over the first `rotary` dims (model.cpp:121-127)
        const int half = a.rotary / 2;
        for (int idx = threadIdx.x; idx < (group + 1) * half; idx += blockDim.x) {
            const int gg = idx / half, i = idx % half;
            float* row = gg < group ? qs[gg] : knew;
            const float* cs = reinterpret_cast<const float*>(a.rope) + 2 * ((size_t)pos * half + i);
            const float c = gc(cs)[0], s = gc(cs)[1];
            const float x0 = row[i], x1 = row[i + half];
            row[i] = x0 * c - x1 * s;
            row[i + half] = x0 * s + x1 * c;
        }
        lds_barrier();
        if (chunk == nchunks - 1) {  // this chunk holds `pos`: append k/v to the caches
            for (int d = threadIdx.x; d < HD; d += blockDim.x) {
                gm(a.keys)[((size_t)pos * a.kv_heads + kvh) * HD + d] = knew[d];
                gm(a.values)[((size_t)pos * a.kv_heads + kvh) * HD + d] = vnew[d];
            }
        }
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int tt = wave + NW * i;
            if (tt < tn) {
                if (t0 + tt == pos)
#pragma unroll
                    for (int e = 0; e < E; ++e) kr[i][e] = knew[E * lane + e];
#pragma unroll
                for (int e = 0; e < E; ++e) ks[tt][E * lane + e] = kr[i][e];
            }
        }
        lds_barrier();
        // scores and chunk-local softmax: lane t is position t0 + t (model.cpp:143-150)
        const float inv_root = 1.f / sqrtf((float)HD);
        for (int gg = wave; gg < group; gg += NW) {
            float s = -INFINITY;
            if (lane < tn) {
                const float4* k4 = reinterpret_cast<const float4*>(ks[lane]);
                const float4* q4 = reinterpret_cast<const float4*>(qs[gg]);
                float dx = 0.f, dy = 0.f, dz = 0.f, dw = 0.f;
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
            const float mx = wave_max(s);
            const float p = lane < tn ? expf(s - mx) : 0.f;
            const float l = wave_sum(p);
            sc[gg][lane] = p;
            if (lane == 0) {
                mstat[gg] = mx;
                lstat[gg] = l;
            }
        }
        lds_barrier();
        float acc[kMaxGroup][E];
#pragma unroll
        for (int gg = 0; gg < kMaxGroup; ++gg)
#pragma unroll
            for (int e = 0; e < E; ++e) acc[gg][e] = 0.f;
#pragma unroll
        for (int i = 0; i < PW; ++i) {
            const int tt = wave + NW * i;
            if (tt < tn) {
                if (t0 + tt == pos)
#pragma unroll
                    for (int e = 0; e < E; ++e) vr[i][e] = vnew[E * lane + e];
#pragma unroll
                for (int gg = 0; gg < kMaxGroup; ++gg) {
                    if (gg < group) {
                        const float p = sc[gg][tt];
#pragma unroll
                        for (int e = 0; e < E; ++e) acc[gg][e] = fmaf(p, vr[i][e], acc[gg][e]);
                    }
                }
            }
        }
#pragma unroll
        for (int gg = 0; gg < kMaxGroup; ++gg)
            if (gg < group)
#pragma unroll
                for (int e = 0; e < E; ++e) acc_lds[wave][gg][E * lane + e] = acc[gg][e];
        lds_barrier();
        const size_t part = ((size_t)kvh * chunks_max + chunk) * group * stride;
        for (int idx = threadIdx.x; idx < group * HD; idx += blockDim.x) {
            const int gg = idx / HD, d = idx % HD;
            float o = 0.f;
#pragma unroll
            for (int w = 0; w < NW; ++w) o += acc_lds[w][gg][d];
            st_out(a.partial, part + (size_t)gg * stride + d, o, tag);
        }
        if (threadIdx.x < group) {
            st_out(a.partial, part + (size_t)threadIdx.x * stride + HD, mstat[threadIdx.x], tag);
            st_out(a.partial, part + (size_t)threadIdx.x * stride + HD + 1, lstat[threadIdx.x], tag);
        }
    }
}

// Merge of the chunk partials of one query head and 64 of its output dims, then the
// sigmoid output gate (attention.hip's attention_combine_kernel with eight waves).
__device__ void step_combine(const StepAttention& a, uint32_t tag, uint32_t base, unsigned char* smem, Waiter& wt) {
    float* wts = reinterpret_cast<float*>(smem);
    float* red = wts + kCombineMaxChunks;
    float (*part)[64] = reinterpret_cast<float (*)[64]>(red + 2 * kStepWaves);
    const int hd = a.head_dim, group = a.heads / a.kv_heads, dblocks = hd / 64;
    const int pos = *gc(a.position);
    if (pos < 0 || pos >= a.context) return;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int chunks_max = (a.context + kAttnChunk - 1) / kAttnChunk;
    const int nchunks = pos / kAttnChunk + 1;
    const int stride = hd + 2;
    const uint32_t wp = want_of(a.partial_in, base), wq = want_of(a.qkv, base);
    for (int u = blockIdx.x; u < a.heads * dblocks; u += gridDim.x) {
        const int head = u / dblocks, db = u - head * dblocks;
        const int kvh = head / group, g = head - kvh * group;
        const size_t basei = ((size_t)kvh * chunks_max * group + g) * stride;
        const size_t cstride = (size_t)group * stride;
        const int d = db * 64 + lane;
        const size_t gi = (size_t)head * hd * 2 + hd + d;
        uint64_t gr = ld_in(a.qkv, gi, wq);
        uint64_t ov[kCombineBatch];
#pragma unroll
        for (int i = 0; i < kCombineBatch; ++i) {
            const int c = min(wave + kStepWaves * i, nchunks - 1);
            ov[i] = ld_in(a.partial_in, basei + (size_t)c * cstride + d, wp);
        }
        lds_barrier();  // the previous phase or unit is done with LDS
        // chunk statistics: max, then weights and the denominator
        float mloc = -INFINITY;
        for (int c = threadIdx.x; c < nchunks; c += blockDim.x) {
            uint64_t m = ld_in(a.partial_in, basei + (size_t)c * cstride + hd, wp);
            while (!tag_ok(m, wp) && wt.again()) m = ld_in(a.partial_in, basei + (size_t)c * cstride + hd, wp);
            wts[c] = val(m);
            mloc = fmaxf(mloc, val(m));
        }
        mloc = wave_max(mloc);
        if (lane == 0) red[wave] = mloc;
        lds_barrier();
        float M = red[0];
        for (int w = 1; w < kStepWaves; ++w) M = fmaxf(M, red[w]);
        float dloc = 0.f;
        for (int c = threadIdx.x; c < nchunks; c += blockDim.x) {
            const float w = expf(wts[c] - M);
            wts[c] = w;
            uint64_t l = ld_in(a.partial_in, basei + (size_t)c * cstride + hd + 1, wp);
            while (!tag_ok(l, wp) && wt.again()) l = ld_in(a.partial_in, basei + (size_t)c * cstride + hd + 1, wp);
            dloc = fmaf(w, val(l), dloc);
        }
        dloc = wave_sum(dloc);
        lds_barrier();  // every weight is in wts
        if (lane == 0) red[kStepWaves + wave] = dloc;
        float num = 0.f;
        for (int c0 = wave; c0 < nchunks; c0 += kStepWaves * kCombineBatch) {
            if (c0 != wave) {
#pragma unroll
                for (int i = 0; i < kCombineBatch; ++i)
                    ov[i] = ld_in(a.partial_in, basei + (size_t)min(c0 + kStepWaves * i, nchunks - 1) * cstride + d, wp);
            }
#pragma unroll
            for (int i = 0; i < kCombineBatch; ++i) {
                const int c = min(c0 + kStepWaves * i, nchunks - 1);
                while (!tag_ok(ov[i], wp) && wt.again()) ov[i] = ld_in(a.partial_in, basei + (size_t)c * cstride + d, wp);
                if (c0 + kStepWaves * i < nchunks) num = fmaf(wts[c0 + kStepWaves * i], val(ov[i]), num);
            }
        }
        part[wave][lane] = num;
        while (!tag_ok(gr, wq) && wt.again()) gr = ld_in(a.qkv, gi, wq);
        lds_barrier();
        if (wave == 0) {
            float den = 0.f, o = 0.f;
            for (int w = 0; w < kStepWaves; ++w) {
                den += red[kStepWaves + w];
                o += part[w][lane];
            }
            st_out(a.out, (size_t)head * hd + d, (o / den) * sigmoidf_(val(gr)), tag);
        }
    }
}

// ---- the kernel ---------------------------------------------------------------------------

template <int T>
__device__ void step_matvec_dispatch(const StepMatvec& m, uint32_t tag, uint32_t base, unsigned char* smem, float* red,
                                     unsigned long long* best, Waiter& wt) {
    if (m.mode == kMvSwiglu) step_matvec<T, true, false, 2>(m, tag, base, smem, red, best, wt);
    else if (m.conv_w) step_matvec<T, false, true, 2>(m, tag, base, smem, red, best, wt);
    else if (m.cols <= 4 * 2 * kStepWaves * 64) step_matvec<T, false, false, 2>(m, tag, base, smem, red, best, wt);
    else step_matvec<T, false, false, 6>(m, tag, base, smem, red, best, wt);
}

__global__ __launch_bounds__(kStepWaves * 64) void step_kernel(const StepPhase* __restrict__ prog, int n,
                                                               const uint32_t* epoch, uint32_t* err) {
    extern __shared__ __align__(16) unsigned char smem[];
    // matvec staging's cross-wave sums and the argmax of a workgroup: static LDS, apart
    // from the dynamic LDS every phase reuses, so a wave may write them before the
    // workgroup has left the previous phase
    __shared__ float red[kStepWaves];
    __shared__ unsigned long long best;
    const uint32_t base = *epoch << kStepPhaseBits;
    Waiter wt{__builtin_amdgcn_s_memrealtime() + kStepDeadlineTicks, err, false, 0};
    for (int p = 0; p < n; ++p) {
        const StepPhase& ph = prog[p];
        const uint32_t tag = base | (uint32_t)ph.tag_phase;
        switch (ph.kind) {
        case kStepMatvec:
            if (ph.mv.type == kQ6K) step_matvec_dispatch<kQ6K>(ph.mv, tag, base, smem, red, &best, wt);
            else step_matvec_dispatch<kQ4K>(ph.mv, tag, base, smem, red, &best, wt);
            break;
        case kStepGdn:
            if (ph.gdn.state_dim == 128) step_gdn<2, 4>(ph.gdn, tag, base, wt);
            else step_gdn<1, 2>(ph.gdn, tag, base, wt);
            break;
        case kStepAttention:
            if (ph.attn.head_dim == 256) step_attention<4>(ph.attn, tag, base, smem, wt);
            else step_attention<2>(ph.attn, tag, base, smem, wt);
            break;
        case kStepCombine:
            step_combine(ph.attn, tag, base, smem, wt);
            break;
        default:
            break;
        }
        if (wt.failed) return;
    }
}

// state = {position, token, prompt_len} (launch_advance), key -> index first
__global__ void step_finish_kernel(unsigned long long* key, int* index, int* state, const int* prompt, int* history,
                                   const int* next, uint32_t* epoch) {
    if (threadIdx.x == 0 && blockIdx.x == 0) {
        if (key) {
            *index = (int)~(uint32_t)(*key & 0xffffffffull);
            *key = 0ull;
        }
        if (state) {
            const int p = state[0];
            const int nxt = next ? *next : 0;
            if (history) history[p] = nxt;
            state[0] = p + 1;
            state[1] = (prompt && p + 1 < state[2]) ? prompt[p + 1] : nxt;
        }
        *epoch += 1;
    }
}

}  // namespace

size_t step_phase_lds(const StepPhase& ph) {
    switch (ph.kind) {
    case kStepMatvec: {
        const int unit = ph.mv.type == kQ6K ? 16 : 32;
        return (size_t)ph.mv.cols * 4 + (size_t)(ph.mv.cols / unit) * 4;
    }
    case kStepAttention: return ph.attn.head_dim == 256 ? AttnLds<4>::bytes : AttnLds<2>::bytes;
    case kStepCombine: return (kCombineMaxChunks + 2 * kStepWaves + kStepWaves * 64) * 4;
    default: return 0;
    }
}

int step_resident_workgroups(size_t lds) {
    int dev = 0, per_cu = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(step_kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
        return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(step_kernel),
                                                     kStepWaves * 64, lds) != hipSuccess)
        return 0;
    return per_cu * prop.multiProcessorCount;
}

hipError_t launch_step(const StepPhase* prog, int n, const uint32_t* epoch, uint32_t* err, int grid, size_t lds,
                       hipStream_t stream) {
    if (n < 1 || n > kStepMaxPhases || grid < 1) return hipErrorInvalidValue;
    launch_kernel(step_kernel, dim3(grid), dim3(kStepWaves * 64), lds, stream, prog, n, epoch, err);
    return hipGetLastError();
}

hipError_t launch_step_finish(unsigned long long* key, int* index, int* state, const int* prompt, int* history,
                              const int* next, uint32_t* epoch, hipStream_t stream) {
    launch_kernel(step_finish_kernel, dim3(1), dim3(64), 0, stream, key, index, state, prompt, history, next, epoch);
    return hipGetLastError();
}

}  // namespace emprise
