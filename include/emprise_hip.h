/*
 * emprise_hip.h -- C ABI of the MI355X (gfx950) decode backend.
 *
 * This library replaces the reference's CUDA/NVRTC backend (`cuda_backend()` and the
 * `class Cuda` behind it, reference v1.1 src/cuda.cpp:599-1130) behind the abstract
 * `emprise::Backend` interface (include/emprise/backend.hpp:11-73). Every entry point
 * below names the Backend method or CUDA-backend routine it stands in for.
 *
 * Conventions
 *   - Plain C: no exceptions cross the ABI. Every call returns an emprise_status;
 *     emprise_hip_last_error() holds the message of the last failure on this thread
 *     (the reference throws invalid_argument for shapes and runtime_error for the
 *     device, cuda.cpp:49-51; the status codes keep that split).
 *   - Device buffers and resident weights are opaque uint64_t handles, like the
 *     reference's dev_alloc() handles (backend.hpp:60-63). A buffer handle is the
 *     device address, so handle + byte offset addresses a sub-range.
 *   - Matrices use GGUF order: a weight has `cols` inputs (shape[0]) and `rows`
 *     outputs (shape[1]); y[rows] = W x[cols].
 *   - All work is queued in order on the backend's own HIP stream. Calls return
 *     after queueing; emprise_hip_sync() waits. Downloads are synchronous, like
 *     the reference's cuMemcpyDtoH.
 *   - Not thread-safe per handle, like the reference (README "not thread-safe").
 */
#ifndef EMPRISE_HIP_H
#define EMPRISE_HIP_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct emprise_hip emprise_hip;
typedef uint64_t emprise_dev;    /* device buffer (device address) */
typedef uint64_t emprise_weight; /* resident weight */
typedef uint64_t emprise_graph;  /* instantiated decode graph */

typedef enum {
    EMPRISE_OK = 0,
    EMPRISE_EINVAL = 1,  /* bad argument or shape  (reference: std::invalid_argument) */
    EMPRISE_EDEVICE = 2, /* HIP runtime failure     (reference: runtime_error from check()) */
    EMPRISE_ENOMEM = 3,  /* over the weight budget or out of device memory */
    EMPRISE_ESTATE = 4   /* call not allowed in the current state (e.g. during capture) */
} emprise_status;

/* GGUF tensor encodings (gguf.hpp:12 WeightType). */
enum { EMPRISE_F32 = 0, EMPRISE_F16 = 1, EMPRISE_Q4_K = 12, EMPRISE_Q6_K = 14, EMPRISE_BF16 = 30 };

const char* emprise_hip_last_error(void);

/* ---- lifetime ------------------------------------------------------------------ */

/* cuda_backend(weight_budget, quantize_activations), backend.hpp:72 / Cuda::Cuda
 * cuda.cpp:725-800. budget 0 = free device memory minus a 512 MiB reserve
 * (cuda.cpp:742-744). quantize_activations selects the --fast-q8 path: Q6_K
 * projections then run on int8 activations (cuda.cpp:709-712). */
emprise_status emprise_hip_create(int device, uint64_t weight_budget, int quantize_activations, emprise_hip** out);
void emprise_hip_destroy(emprise_hip* h);
/* Backend::name(), backend.hpp:14. */
const char* emprise_hip_name(const emprise_hip* h);
/* Backend::device_capacity(), backend.hpp:59: the weight budget in bytes. */
uint64_t emprise_hip_capacity(const emprise_hip* h);
/* Bytes of weights resident so far (Cuda::used, cuda.cpp:624). */
uint64_t emprise_hip_weight_bytes(const emprise_hip* h);

/* ---- device buffers (backend.hpp:60-63) ------------------------------------------ */
emprise_status emprise_hip_alloc(emprise_hip* h, size_t bytes, emprise_dev* out);     /* dev_alloc    */
emprise_status emprise_hip_free(emprise_hip* h, emprise_dev buffer);                  /* dev_free     */
emprise_status emprise_hip_upload(emprise_hip* h, emprise_dev dst, const void* src, size_t bytes);  /* dev_upload   */
emprise_status emprise_hip_download(emprise_hip* h, void* dst, emprise_dev src, size_t bytes);      /* dev_download */
/* Fills n floats with value on the stream (graph-safe: a kernel, not a memset). */
emprise_status emprise_hip_fill(emprise_hip* h, emprise_dev dst, float value, size_t n);
/* Measurement aid; no counterpart in the reference. Reads `bytes` (a multiple of 4 KiB)
 * from src with non-temporal 16-byte loads (one 8-wave workgroup per CU, each wave one
 * 4 KiB piece at a time) and writes one word per workgroup (the XOR of what it read) to
 * sink (4096 uint32). Its rate is the achievable HBM read bandwidth bench.py reports the
 * decode against. */
emprise_status emprise_hip_stream_read(emprise_hip* h, emprise_dev src, uint64_t bytes, emprise_dev sink);

/* ---- weights ---------------------------------------------------------------------- */

/* Cuda::resident, cuda.cpp:647-701: uploads one GGUF tensor (raw GGUF bytes, len must
 * equal the encoded size of rows*cols elements) and re-lays it out for the kernels.
 * The device copy keeps the GGUF byte count exactly (210 B per Q6_K super-block, 144 B
 * per Q4_K super-block): blocks are rearranged, never padded. Vectors (norm weights)
 * are uploaded with rows = 1. Returns EMPRISE_ENOMEM when over the budget. */
emprise_status emprise_hip_upload_weight(emprise_hip* h, uint32_t type, uint64_t cols, uint64_t rows,
                                         const void* data, size_t len, emprise_weight* out);
emprise_status emprise_hip_weight_free(emprise_hip* h, emprise_weight w);
/* Device address of a weight's bytes in the device layout (F32 weights: the floats). */
emprise_dev emprise_hip_weight_data(const emprise_hip* h, emprise_weight w);
/* Decodes rows [row0, row0+n) of a resident weight back to FP32 on the device
 * (the GPU counterpart of dequantize(), quant.cpp:64-78). out holds n*cols floats. */
emprise_status emprise_hip_dequantize_rows(emprise_hip* h, emprise_weight w, uint64_t row0, uint64_t n, emprise_dev out);
/* Reads the device layout back and restores the GGUF byte order (test hook for the
 * lossless re-layout). out holds len bytes, len as given at upload. */
emprise_status emprise_hip_weight_download_gguf(emprise_hip* h, emprise_weight w, void* out, size_t len);

/* ---- projections ------------------------------------------------------------------- */

/* Backend::dev_linear (backend.hpp:66) and Backend::linear (backend.hpp:15) on device
 * buffers: y = W x with FP32 activations (exact dequantised weights, FP32 products and
 * sums; only the summation order differs from the CPU), or with Q8 activations for
 * Q6_K weights when the backend was created with quantize_activations. */
emprise_status emprise_hip_linear(emprise_hip* h, emprise_weight w, emprise_dev x, emprise_dev y);

/* Backend::linear_many (backend.hpp:19), the CUDA fused_q6_proj (cuda.cpp:254-304):
 * up to 8 projections with the same input, one launch. */
emprise_status emprise_hip_linear_many(emprise_hip* h, int n, const emprise_weight* w, emprise_dev x,
                                       const emprise_dev* y);

/* Backend::linear_batch (backend.hpp:23-24), linear_q6_f32_batch (cuda.cpp:350-413):
 * Y[k] = W X[k] for k < K; X is K rows of cols floats, Y K rows of rows floats. */
emprise_status emprise_hip_linear_batch(emprise_hip* h, emprise_weight w, emprise_dev X, emprise_dev Y, int K);
/* linear_batch with row strides (floats): X[k] at X + k*ldx, Y[k] at Y + k*ldy, so one
 * call can write its output into a slice of wider rows (e.g. the q|k|v rows that the
 * attention op reads). Batched prefill support; no reference counterpart (the
 * reference prefills in chunks of 4 positions, model.cpp:355-366). */
emprise_status emprise_hip_linear_batch_strided(emprise_hip* h, emprise_weight w, emprise_dev X, uint64_t ldx,
                                                emprise_dev Y, uint64_t ldy, int K);
/* linear_batch_strided over n <= 8 weights of one input width, their outputs side by
 * side: Y[k] = [W_0; W_1; ...] X[k], weight i's rows in the columns that follow weight
 * i-1's. The stacked rows run as one GEMM (e.g. the q|k|v or recurrent in-projections of
 * the prefill). Batched prefill support, like linear_batch_strided. */
emprise_status emprise_hip_linear_batch_many(emprise_hip* h, int n, const emprise_weight* w, emprise_dev X,
                                             uint64_t ldx, emprise_dev Y, uint64_t ldy, int K);
/* The gate/up half of Backend::feed_forward (backend.hpp:27-28; the reference's fused FFN,
 * model.cpp:230-236, swiglu at cuda.cpp:560-566) over K inputs: Y[k] = silu(G X[k]) * (U X[k]),
 * F = rows of G = rows of U floats per row, strides in floats. Chunked Q6_K/Q4_K gate and
 * up of one type run as one GEMM whose epilogue forms the SwiGLU; the values are those of
 * linear_batch_strided for G and U followed by swiglu, bit for bit. Batched prefill
 * support, like linear_batch_strided. */
emprise_status emprise_hip_ffn_gate_up_batch(emprise_hip* h, emprise_weight gate, emprise_weight up, emprise_dev X,
                                             uint64_t ldx, emprise_dev Y, uint64_t ldy, int K);

/* Input transform fused into a projection's prologue. It stands for the reference's
 * dev_add + dev_rmsnorm pair in front of every projection group (model.cpp:429,
 * :454-455, :457, :461):  v = x + delta;  x_out = v;  input = rms(v) * norm.
 * delta, x_out and norm may each be 0 (absent). x_out must not alias x or delta. */
typedef struct {
    emprise_dev x;
    emprise_dev delta;
    emprise_dev x_out;
    emprise_weight norm; /* F32 vector weight of length cols, or 0 */
    float eps;
} emprise_hip_input;

/* linear_many with the input transform above. */
emprise_status emprise_hip_linear_norm(emprise_hip* h, const emprise_hip_input* in, int n,
                                       const emprise_weight* w, const emprise_dev* y);

/* Backend::dev_ffn / feed_forward (backend.hpp:27-28, cuda.cpp:1068-1080):
 * y = down(silu(gate x) * up x). in may be NULL for a plain input x. */
emprise_status emprise_hip_feed_forward(emprise_hip* h, const emprise_hip_input* in, emprise_dev x,
                                        emprise_weight gate, emprise_weight up, emprise_weight down,
                                        emprise_dev y);

/* The gate/up half of the FFN alone: hidden = silu(gate x) * up x (swiglu,
 * cuda.cpp:560-566, fused into the projection epilogue). */
emprise_status emprise_hip_ffn_gate_up(emprise_hip* h, const emprise_hip_input* in, emprise_dev x,
                                       emprise_weight gate, emprise_weight up, emprise_dev hidden);

/* ---- small ops ----------------------------------------------------------------------- */
/* Backend::dev_rmsnorm (backend.hpp:64), rmsnorm_kernel cuda.cpp:533-542. */
emprise_status emprise_hip_rmsnorm(emprise_hip* h, emprise_dev x, emprise_weight w, emprise_dev out, int n, float eps);
/* dev_rmsnorm over `rows` consecutive rows of n floats (batched prefill). */
emprise_status emprise_hip_rmsnorm_rows(emprise_hip* h, emprise_dev x, emprise_weight w, emprise_dev out, int n,
                                       int rows, float eps);
/* dev_add then dev_rmsnorm (backend.hpp:64-65; model.cpp:226-228, :243-249) over `rows`
 * rows in one pass: x += delta, out = rms(x) * w; the results of emprise_hip_add followed
 * by emprise_hip_rmsnorm_rows, bit for bit. out must not alias x or delta. Batched
 * prefill support. */
emprise_status emprise_hip_add_rmsnorm_rows(emprise_hip* h, emprise_dev x, emprise_dev delta, emprise_weight w,
                                           emprise_dev out, int n, int rows, float eps);
/* Backend::dev_add (backend.hpp:65), add_inplace cuda.cpp:543-546: x += y. */
emprise_status emprise_hip_add(emprise_hip* h, emprise_dev x, emprise_dev y, int n);
/* swiglu, cuda.cpp:560-566: gate = silu(gate) * up. */
emprise_status emprise_hip_swiglu(emprise_hip* h, emprise_dev gate, emprise_dev up, int n);
/* Model::Impl::embed (model.cpp:367-375) on device: out = dequantised row `*token` of
 * the embedding. token is a device int32 (graph-replayable). */
emprise_status emprise_hip_embed(emprise_hip* h, emprise_weight embedding, emprise_dev token, emprise_dev out);
/* embed for `count` device token ids (int32): out[i] = dequantised row tokens[i]. */
emprise_status emprise_hip_embed_rows(emprise_hip* h, emprise_weight embedding, emprise_dev tokens, int count,
                                      emprise_dev out);
/* Greedy pick, model.cpp:499 (std::max_element: the first maximum wins): writes the
 * int32 index of the largest of n logits to *index (device). */
emprise_status emprise_hip_argmax(emprise_hip* h, emprise_dev logits, int n, emprise_dev index);
/* quantize_x, cuda.cpp:547-559: per 32 inputs s = amax/127, q = round(x/s) (ties away
 * from zero, unrounded s), stored scale = fp16_rne(s) as float. q: cols int8,
 * scales: cols/32 floats. */
emprise_status emprise_hip_quantize_q8(emprise_hip* h, emprise_dev x, int cols, emprise_dev q, emprise_dev scales);

/* ---- Gated DeltaNet ---------------------------------------------------------------- */

/* Backend::DeltaNet (backend.hpp:32-39) with device buffers. conv/ssm_a/dt/norm are
 * F32 vector weights; conv_state (channels*conv_width floats) and rec_state
 * (value_heads*state_dim*state_dim floats, 16-byte aligned: its rows move as 16-byte
 * accesses) are caller-owned device buffers that persist across tokens. */
typedef struct {
    int key_heads, value_heads, state_dim, conv_width;
    float eps;
    emprise_dev qkv, gate, alpha, beta;
    emprise_weight conv, ssm_a, dt, norm;
    emprise_dev conv_state, rec_state, out;
} emprise_hip_delta_net_params;
/* Backend::delta_net (backend.hpp:40), delta_conv + delta_scan + delta_norm_gate
 * (cuda.cpp:417-479): causal conv1d + SiLU, q/k L2 norm, gated delta-rule update,
 * per-head RMSNorm x SiLU(gate). qkv is not modified. */
emprise_status emprise_hip_delta_net(emprise_hip* h, const emprise_hip_delta_net_params* p);
/* No counterpart in the reference: emprise_hip_delta_net for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). It allocates nothing: the conv'd channels of the step go to a
 * fixed device array of 65536 floats (256 KiB) that each GPU the library runs on holds
 * until the process ends, so (2*key_heads + value_heads)*state_dim may not exceed 65536
 * (EMPRISE_EINVAL otherwise). The caller passes every input, output and state buffer as
 * for emprise_hip_delta_net, and gets the same results bit for bit. Every call on one
 * GPU shares that array: calls that overlap on one GPU (several streams or handles)
 * race. Each call writes all the channels it reads before reading them, so nothing
 * needs clearing between calls. */
emprise_status emprise_hip_delta_net_noalloc(emprise_hip* h, const emprise_hip_delta_net_params* p);
/* Backend::delta_net over `count` consecutive positions, for the batched prompt prefill
 * (the reference runs it position by position inside its 4-position prefill batches,
 * model.cpp:355-366): qkv, gate, alpha and beta are the rows of position 0, the rows of
 * position t are `stride` floats further; out receives `count` rows `out_stride` floats
 * apart. Per position the same arithmetic, in the same order, as emprise_hip_delta_net,
 * so outputs and final states equal `count` calls of it. qkv is not modified.
 * 1 <= count <= 524288. */
emprise_status emprise_hip_delta_net_batch(emprise_hip* h, const emprise_hip_delta_net_params* p, int count,
                                           uint64_t stride, uint64_t out_stride);

/* Backend::RecurrentBlock (backend.hpp:44-51) on device. */
typedef struct {
    emprise_weight qkv_w, gate_w, alpha_w, beta_w, out_w;
    emprise_weight conv, ssm_a, dt, norm;
    int key_heads, value_heads, state_dim, conv_width;
    float eps;
    emprise_dev conv_state, rec_state;
} emprise_hip_recurrent_params;
/* Backend::dev_recurrent (backend.hpp:68), cuda.cpp:1081-1127: projections, delta_net,
 * output projection. in may be NULL for a plain input x; y gets hidden floats. */
emprise_status emprise_hip_recurrent(emprise_hip* h, const emprise_hip_recurrent_params* p,
                                     const emprise_hip_input* in, emprise_dev x, emprise_dev y);

/* ---- gated GQA attention ------------------------------------------------------------ */

/* Model::Impl::attention_preout (model.cpp:129-157), which the reference runs on the
 * host even on its device path (model.cpp:441-452). qkv holds the three projections
 * back to back: q|gate interleaved per head (heads*head_dim*2), then k and v
 * (kv_heads*head_dim each). The new k (after RMSNorm + RoPE) and v are stored at
 * *position (device int32) of the caches keys/values (context*kv_heads*head_dim floats
 * each), then every head attends over positions 0..*position. out = heads*head_dim.
 * rope_position (device int32, or 0 for *position) is the rotary position when it differs
 * from the cache row: the MTP block's own cache grows by one row per draft while it
 * rotates at the caller's position (model.cpp:383-385, attention_preout's pos). */
typedef struct {
    int heads, kv_heads, head_dim, rotary, context;
    float eps, rope_base;
    emprise_weight q_norm, k_norm;
    emprise_dev keys, values;
    emprise_dev position;
    emprise_dev rope_position;
} emprise_hip_attention_params;
emprise_status emprise_hip_attention(emprise_hip* h, const emprise_hip_attention_params* p, emprise_dev qkv,
                                     emprise_dev out);
/* attention_preout over `count` consecutive prompt positions first_position .. +count-1
 * (the reference attends position by position inside its 4-position prefill batches,
 * model.cpp:355-366): qkv is the row of the first position, the rows of later positions
 * `stride` floats further; their k/v are appended to the caches at their positions and
 * position t attends over 0..first_position+t; out receives `count` rows `out_stride`
 * floats apart. p->position is not used. The dot products and P.V run as FP32 GEMMs on
 * the matrix cores, so the outputs equal those of `count` emprise_hip_attention calls
 * up to summation order. */
emprise_status emprise_hip_attention_batch(emprise_hip* h, const emprise_hip_attention_params* p, emprise_dev qkv,
                                           int count, uint64_t stride, int first_position, emprise_dev out,
                                           uint64_t out_stride);

/* ---- state, sync, graphs ---------------------------------------------------------- */
/* Backend::reset_state (backend.hpp:53). The caller owns recurrent and KV state buffers
 * here, so this only clears backend-internal scratch; kept for interface parity. */
emprise_status emprise_hip_reset_state(emprise_hip* h);
emprise_status emprise_hip_sync(emprise_hip* h);
/* Device-side greedy loop step for replayed decode graphs (the host loop of
 * Model::generate, model.cpp:497-502, kept on the device). state is a device int32[3]
 * {position, token, prompt_len}: position feeds attention, token feeds emprise_hip_embed.
 * With p = position: history[p] = *next (when history is non-zero), position = p + 1,
 * token = prompt[p + 1] while p + 1 < prompt_len (prompt non-zero), else *next. */
emprise_status emprise_hip_advance(emprise_hip* h, emprise_dev state, emprise_dev prompt, emprise_dev history,
                                   emprise_dev next);

/* The output head with the greedy pick fused (model.cpp:461-467 then :499):
 * logits = W * rms(x + delta) * norm (the input transform of emprise_hip_linear_norm),
 * and *index (device int32) = the first index of the largest logit. */
emprise_status emprise_hip_lm_head(emprise_hip* h, const emprise_hip_input* in, emprise_weight w, emprise_dev logits,
                                   emprise_dev index);

/* hipGraph capture of the calls queued between begin and end (no reference
 * counterpart: the reference launches each kernel from the host). Calls made while
 * capturing must not download, allocate or upload weights. */
emprise_status emprise_hip_graph_begin(emprise_hip* h);
emprise_status emprise_hip_graph_end(emprise_hip* h, emprise_graph* out);
emprise_status emprise_hip_graph_launch(emprise_hip* h, emprise_graph g);
emprise_status emprise_hip_graph_destroy(emprise_hip* h, emprise_graph g);

/* ---- timing (HIP events on the backend stream) ----------------------------------- */
/* Records event `slot` (0 <= slot < 65536, created on first use) on the backend
 * stream; emprise_hip_event_elapsed waits for end_slot and returns the milliseconds
 * between the two. */
emprise_status emprise_hip_event_record(emprise_hip* h, int slot);
emprise_status emprise_hip_event_elapsed(emprise_hip* h, int start_slot, int end_slot, float* ms);

/* ---- kernel trace (eager launches only) -----------------------------------------
 * Between trace_begin and trace_end every kernel the backend launches is bracketed by
 * two HIP events on the backend stream and recorded with the algorithmic HBM bytes
 * of that launch: encoded weight bytes + activations read and written for
 * projections, state read + written for the GDN step, K/V rows read for attention. */
typedef struct {
    const char* kernel; /* static string: "matvec_q6_k", "gdn_step", "attention", ... */
    uint64_t bytes;
    float ms;
} emprise_hip_trace_record;
emprise_status emprise_hip_trace_begin(emprise_hip* h);
/* Waits for the traced work, copies up to cap records, *n = number recorded. */
emprise_status emprise_hip_trace_end(emprise_hip* h, emprise_hip_trace_record* out, size_t cap, size_t* n);

#ifdef __cplusplus
}
#endif
#endif
