// Phase program of the persistent decode-step kernel (step.hip), shared with the
// backend that records it (backend.hip).
//
// One decode step of the fused qwen35 graph (reference model.cpp:210-260 in the order
// of Backend::recurrent / linear / attention / feed_forward) becomes one kernel launch
// that walks a list of phases: grouped matvecs, the Gated DeltaNet state update, the
// split-KV attention partials and their merge. Workgroups do not wait for each other
// at phase boundaries. Every activation a phase writes for a later phase is a tagged
// 8-byte slot {float bits, tag} with tag = epoch << kStepPhaseBits | phase, stored and
// loaded with agent-scope (cross-XCD coherent) 8-byte accesses; a consumer polls the
// slots it needs until they carry the producer phase's tag of the current step. A
// wave that finishes its share of a phase therefore starts on the next phase at once
// -- its first weight loads go out while other workgroups are still finishing -- and
// no barrier spans more than one workgroup.
#pragma once
#include "kernels.hpp"

namespace emprise {

constexpr int kStepPhaseBits = 10;  // phases per program (tag low bits)
constexpr int kStepMaxPhases = 1 << kStepPhaseBits;
constexpr int kStepWaves = 8;       // waves per workgroup
constexpr int kStepMaxCols = 12288; // widest staged matvec input

// An input operand: plain floats (phase < 0) or tagged slots written by `phase`.
struct StepIn {
    const void* p;
    int phase;
};
// An output operand: tagged slots (written with the running phase's tag) or plain floats.
struct StepOut {
    void* p;
    int tagged;
};

enum StepKind : int { kStepMatvec = 1, kStepGdn = 2, kStepAttention = 3, kStepCombine = 4 };

struct StepSeg {
    const uint8_t* w;  // chunked-layout weight rows
    StepOut y;
    int rows;
    int g0;
};

struct StepMatvec {
    uint32_t type;  // kQ6K or kQ4K, cols % 4096 == 0
    int mode;       // MvMode
    int cols, groups, rows_per_group, nseg;
    StepSeg seg[kMaxSeg];
    // input: v = x + delta (workgroup 0 stores v to x_out), then rms(v) * norm; or, with
    // gate set (already SiLU'd by its producer), the per-head rms(x) * norm * gate; or the
    // embedding row *token of emb instead of x
    StepIn x, delta, gate;
    StepOut x_out;
    const float* norm;
    float eps;
    int head_dim;
    int silu_mask;  // bit s: segment s stores SiLU(row)
    const uint8_t* emb;
    uint32_t emb_type;
    int emb_rows;
    const int* token;
    // causal conv1d + SiLU epilogue on segment 0 (plain per-row history, owned by the row)
    const float* conv_w;
    float* conv_state;
    int conv_width;
    unsigned long long* argmax;  // kMvArgmax: running maximum key
};

struct StepGdn {
    int key_heads, value_heads, state_dim;
    float eps;
    StepIn qkv, alpha, beta;  // conv'd q/k/v channels, per-head alpha and beta
    const float* ssm_a;
    const float* dt;
    float* state;  // [value_heads][state_dim][state_dim], rows owned by their workgroup
    StepOut out;   // raw per-row outputs S.q
};

struct StepAttention {
    int heads, kv_heads, head_dim, rotary, context;
    float eps, rope_base;
    const float2* rope;  // [context][rotary / 2] (cos, sin)
    const float* q_norm;
    const float* k_norm;
    StepIn qkv;        // [q+gate interleaved per head | k | v]
    float* keys;       // caches (plain; the new row is appended by its chunk's workgroup)
    float* values;
    const int* position;
    StepOut partial;   // kStepAttention: [kv_heads][chunks][group][head_dim + 2]
    StepIn partial_in; // kStepCombine
    StepOut out;       // kStepCombine: gated attention output [heads * head_dim]
};

struct StepPhase {
    int kind;
    // phase index carried in the tags of this phase's outputs: its own, or that of the
    // first phase recorded from the same call (a projection group split into runs of
    // equal weight type hands over one version of its outputs)
    int tag_phase;
    union {
        StepMatvec mv;
        StepGdn gdn;
        StepAttention attn;
    };
};

// Dynamic LDS a phase needs (bytes).
size_t step_phase_lds(const StepPhase& ph);
// Workgroups of the step kernel that are resident at once with `lds` bytes each (the
// launch uses exactly this many, so every workgroup runs from the start), or 0.
int step_resident_workgroups(size_t lds);
// Runs phases [0, n) of `prog` (device memory) as one kernel. epoch: device word read at
// the start (the tag base of the step); err: device word set to nonzero if a wait ran
// out of time, in which case the step's outputs are undefined.
hipError_t launch_step(const StepPhase* prog, int n, const uint32_t* epoch, uint32_t* err, int grid, size_t lds,
                       hipStream_t stream);
// After the step kernel: argmax key -> index (key cleared), the position/token advance
// of launch_advance, and epoch += 1. key/index/state may be null (skipped).
hipError_t launch_step_finish(unsigned long long* key, int* index, int* state, const int* prompt, int* history,
                              const int* next, uint32_t* epoch, hipStream_t stream);

}  // namespace emprise
