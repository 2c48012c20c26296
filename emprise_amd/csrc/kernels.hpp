// Host-side launch interface of the gfx950 kernels (internal to libemprise_hip.so).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stddef.h>
#include <stdint.h>

namespace emprise {

// Kernel timing bracket of the launch trace. While `stop` is set, launch_kernel puts the
// events on the dispatch packets themselves (hipExtLaunchKernelGGL): the first launch
// records `start` as it begins and every launch records `stop` as it ends, so a traced
// span is the kernels' own execution time, with no extra packets in the queue.
struct TraceBracket {
    hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local TraceBracket g_trace_bracket;

template <typename F, typename... Args>
inline void launch_kernel(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, Args... args) {
    TraceBracket& t = g_trace_bracket;
    if (t.stop) {
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, stream, t.start, t.stop, 0, args...);
        t.start = nullptr;
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, stream, args...);
    }
}

constexpr int kMaxSeg = 8;
constexpr int kMvRows = 2;            // rows per wave iteration (unit-major rows)
constexpr int kMvStreamRows = 1;      // rows per item of the streaming kernel (chunked rows)
constexpr int kMvStreamPairRows = 1;  // gate/up row pairs per item of the SwiGLU variant

enum MvMode : int { kMvPlain = 0, kMvSwiglu = 1, kMvArgmax = 2 };

// One projection of a grouped matvec launch.
struct MvSeg {
    const uint8_t* w;  // device layout of the weight
    float* y;          // output (rows floats)
    int rows;
    int g0;  // first global row-group index of this segment
};

struct MvArgs {
    MvSeg seg[kMaxSeg];
    int nseg;
    int groups;  // total row groups
    int cols;
    int mode;
    // input transform: v = x + delta; x_out = v; input = rms(v) * norm
    const float* x;
    const float* delta;
    float* x_out;
    const float* norm;
    float eps;
    // per-head transform instead (the GDN output gate, backend.cpp:57-58): when gate is
    // set, input = rms over each head_dim slice of x (weights norm[0..head_dim)) * gate,
    // where gate already holds SiLU(gate rows) (see silu_mask); delta and x_out must be null
    const float* gate;
    int head_dim;
    // bit s: the epilogue stores SiLU(row) for segment s (the GDN gate rows, activated once
    // by their producer instead of in every consumer workgroup)
    int silu_mask;
    // kMvArgmax: running maximum key (value, -index), see argmax_key()
    unsigned long long* argmax;
    // causal conv1d + SiLU epilogue on segment 0 (the GDN qkv projection), or null
    const float* conv_w;  // [rows][conv_width]
    float* conv_state;    // [rows][conv_width]
    int conv_width;
    int rows_per_group;   // R of the launch (matvec_rows_per_group)
};

size_t matvec_lds_bytes(uint32_t type, int cols, bool q8);
// y[k * ldy + r] = row r of w . x[k * ldx ...] for k < K, a chunked Q6_K/Q4_K matrix read
// once for all K inputs (matvec_batch_kernel)
struct MvBatchArgs {
    const uint8_t* w;
    int rows, cols;
    const float* x;
    size_t ldx;
    float* y;
    size_t ldy;
};
constexpr int kBatchMax = 4;                    // inputs per batched launch
constexpr size_t kBatchLdsMax = 160 * 1024;     // LDS of one workgroup (one per CU)
size_t matvec_batch_lds_bytes(uint32_t type, int cols, int k);
hipError_t launch_matvec_batch(uint32_t type, const MvBatchArgs& a, int k, hipStream_t stream);
// rows each row-group of MvArgs covers for this weight shape, mode and the launch's
// total output rows (small launches use one row per wave to spread their arithmetic)
int matvec_rows_per_group(uint32_t type, uint64_t cols, int mode, uint64_t total_rows);
hipError_t launch_matvec(uint32_t type, bool q8, const MvArgs& a, int grid_cap, hipStream_t stream);
hipError_t launch_matvec_stream(uint32_t type, bool q8, const MvArgs& a, hipStream_t stream);
// Raw GGUF Q6_K / Q4_K rows (device) -> the kernel layout of layout.hpp (device).
hipError_t launch_repack(uint32_t type, const uint8_t* src, uint8_t* dst, uint64_t rows, uint64_t cols,
                         hipStream_t stream);
hipError_t launch_dequant_rows(const uint8_t* w, uint32_t type, int cols, uint64_t row0, uint64_t n, float* out,
                               hipStream_t stream);

// Y[M][N] (row stride ldc) = A[M][K] (lda) . B[N][K]^T (ldb), FP32 on the matrix cores.
// K must be a multiple of 16; lda and ldb multiples of 4 (16-byte rows).
hipError_t launch_gemm_f32(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb, int ldc,
                           hipStream_t stream);
// `batch` products in one launch (grid z): C + z*sC = (A + z*sA) (B + (z/bdiv)*sB)^T.
// causal_keys_n: N indexes keys and row m of a chunk uses keys <= first + m, so tiles
// past every row's last key are skipped (their C is left unwritten); causal_keys_k: the
// same with K indexing keys, each tile's K loop ending after its rows' last key (A must
// be zero beyond it).
hipError_t launch_gemm_f32_heads(const float* A, const float* B, float* C, int M, int N, int K, int lda, int ldb,
                                 int ldc, int batch, int bdiv, size_t sA, size_t sB, size_t sC, bool causal_keys_n,
                                 bool causal_keys_k, int first, hipStream_t stream);

// Batched projection on the fp16 matrix cores over chunked Q6_K / Q4_K weights
// (gemm_q.hip): Y[m][n] = row n of the stacked weights . X[m], for up to kMaxSeg weights of
// one type whose rows follow each other in Y. launch_gemm_q16_split fills the activation
// fields from X (fp16 hi/lo pieces of 2^-e_m x, e_m per row, and with `sums` the pieces of
// its 32-column sums) in `scratch` (gemm_q16_split_bytes); the caller fills the weights.
struct QGemmArgs {
    const uint16_t *xh, *xl, *sh, *sl;  // fp16 bits: x in 128 x 64 tiles (gemm_q.hip), sums [M][K/32]
    const int* rexp;                    // [M]
    int M, K;
    const uint8_t* w[kMaxSeg];
    int row0[kMaxSeg + 1];  // weight s holds rows [row0[s], row0[s+1])
    int nseg, N;
    float* y;
    int ldy;
    // SwiGLU pairs: two segments of N/2 rows each (gate, up), interleaved -- GEMM row n is
    // row n/2 of segment n%2 -- and y[m][n/2] = silu(gate) * up in place of both rows
    int pair;
};
size_t gemm_q16_split_bytes(int M, int K, bool sums);
hipError_t launch_gemm_q16_split(const float* X, int M, int K, int ldx, void* scratch, bool sums, QGemmArgs* a,
                                 hipStream_t stream);
hipError_t launch_gemm_q16(uint32_t type, const QGemmArgs& a, hipStream_t stream);

// ---- Gated DeltaNet ----
struct GdnArgs {
    int key_heads, value_heads, state_dim, conv_width;
    float eps;
    const float* qkv;  // conv'd + SiLU'd channels (2*key_dim + value_dim)
    const float* gate;
    const float* alpha;
    const float* beta;
    const float* ssm_a;
    const float* dt;
    const float* norm;
    float* state;  // [value_heads][state_dim][state_dim]
    float* out;    // [value_dim]
};
// `count` consecutive positions of Backend::delta_net: row t of qkv/gate/alpha/beta at
// t * stride floats from the pointers; conv_out: count * channels floats (scratch), o:
// count * value_dim floats (scratch, the raw S.q), out: row t at t * out_stride.
struct GdnBatchArgs {
    int key_heads, value_heads, state_dim, conv_width, count;
    float eps;
    const float* qkv;
    const float* gate;
    const float* alpha;
    const float* beta;
    size_t stride;
    const float* conv_w;
    const float* ssm_a;
    const float* dt;
    const float* norm;
    float* conv_state;
    float* state;
    float* conv_out;
    float* qk;     // count x key_heads x 2*state_dim: normalised q|k in the scan's lane order
    float* gates;  // count x value_heads x {decay, sigmoid(beta)}
    float* o;
    float* out;
    size_t out_stride;
};
hipError_t launch_gdn_batch(const GdnBatchArgs& a, hipStream_t stream);
// conv1d + SiLU over raw channels (delta_conv): out[c] = silu(conv(shifted history)).
hipError_t launch_delta_conv(const float* qkv, const float* conv_w, float* conv_state, float* out, int channels,
                             int conv_width, hipStream_t stream);
hipError_t launch_gdn(const GdnArgs& a, hipStream_t stream);
// The state update alone, each value head split over several workgroups: out gets the
// raw per-row outputs S.q (the per-head RMSNorm x SiLU(gate) is left to the consumer,
// the output projection's input transform).
hipError_t launch_gdn_rows(const GdnArgs& a, hipStream_t stream);

// ---- attention ----
struct AttnArgs {
    int heads, kv_heads, head_dim, rotary, context;
    float eps, rope_base;
    const float* q_norm;
    const float* k_norm;
    const float* qkv;
    float* keys;
    float* values;
    const int* position;
    const int* rope_position;  // rotary position when it differs from *position, or null
    float* out;
    float* partial;  // scratch: [kv_heads][chunks][group][head_dim + 2]
    const float2* rope;  // [context][rotary / 2]: (cos, sin) of pos / base^(2i / rotary)
};
constexpr int kAttnSub = 16;     // positions per step of attention_kernel's online softmax
constexpr int kAttnSplit = 64;   // position ranges (workgroups) per KV head of attention_kernel
// `count` consecutive prompt positions from absolute position `first`: qkv row t at
// t * stride floats; q (count x heads x hd), scores (heads x count x lp), vt (kv_heads x
// hd x lp) and o (count x heads x hd) are scratch, lp = first + count rounded up to 32;
// out row t at t * out_stride.
struct AttnBatchArgs {
    int heads, kv_heads, head_dim, rotary, count, first, lp;
    float eps, rope_base;
    const float2* rope;  // [context][rotary / 2] (cos, sin), as AttnArgs::rope
    const float* q_norm;
    const float* k_norm;
    const float* qkv;
    size_t stride;
    float* keys;
    float* values;
    float* q;
    float* scores;
    float* vt;
    float* o;
    float* out;
    size_t out_stride;
};
hipError_t launch_attention_batch(const AttnBatchArgs& a, hipStream_t stream);
size_t attention_partial_floats(int heads, int kv_heads, int head_dim, int context);
hipError_t launch_attention(const AttnArgs& a, hipStream_t stream);
// The RoPE table of attention_kernel: (cos, sin) of every position's angles.
hipError_t launch_rope_table(float2* table, int context, int rotary, float base, hipStream_t stream);

// ---- small ops ----
hipError_t launch_fill(float* dst, float value, size_t n, hipStream_t stream);
hipError_t launch_stream_read(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream);
hipError_t launch_fill_u64(unsigned long long* dst, unsigned long long value, size_t n, hipStream_t stream);
hipError_t launch_rmsnorm(const float* x, const float* w, float* out, int n, float eps, hipStream_t stream);
hipError_t launch_rmsnorm_rows(const float* x, const float* w, float* out, int n, int rows, float eps,
                               hipStream_t stream);
hipError_t launch_add_rmsnorm_rows(float* x, const float* delta, const float* w, float* out, int n, int rows, float eps,
                                  hipStream_t stream);
hipError_t launch_add(float* x, const float* y, int n, hipStream_t stream);
hipError_t launch_swiglu(float* gate, const float* up, int n, hipStream_t stream);
hipError_t launch_swiglu_rows(float* gate, size_t ldg, const float* up, size_t ldu, int n, int rows,
                              hipStream_t stream);
hipError_t launch_embed(const uint8_t* w, uint32_t type, int cols, int rows, const int* token, float* out,
                        hipStream_t stream);
hipError_t launch_embed_rows(const uint8_t* w, uint32_t type, int cols, int rows, const int* tokens, int count,
                             float* out, hipStream_t stream);
hipError_t launch_argmax(const float* logits, int n, unsigned long long* key, int* index, hipStream_t stream);
hipError_t launch_argmax_finish(const unsigned long long* key, int* index, hipStream_t stream);
hipError_t launch_quantize_q8(const float* x, int cols, int8_t* q, float* scales, hipStream_t stream);
hipError_t launch_advance(int* state, const int* prompt, int* history, const int* next, hipStream_t stream);

}  // namespace emprise
