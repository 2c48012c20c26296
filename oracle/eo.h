/*
 * CPU oracle for the qwen35 per-token decode path: a plain-C restatement of the
 * reference's OpenMP CPU path (v1.1 src/quant.cpp, src/backend.cpp, src/model.cpp,
 * src/gguf.cpp).
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or as the timed
 * CPU baseline. The product (emprise_amd/) never links or calls it.
 *
 * Exactness: built with -O3 -fopenmp -ffp-contract=off and no -ffast-math, like the
 * reference's Release build (CMakeLists.txt: -O3, no -march, so no FMA). Sequential
 * FP32 sums follow the reference's loop order, so dequantisation, matvec, RMSNorm,
 * attention and the SwiGLU FFN match the reference CPU build bit for bit; the GDN
 * scan keeps the reference's `omp simd` reductions, whose lane order is GCC's.
 *
 * Pinning (how each function is checked; see tests/test_oracle_*.py):
 *   eo_half_to_float   core.cpp:42-47 known answers + all 65536 inputs vs closed form
 *   eo_dequantize      core.cpp:51-72 independently encoded Q6_K block; Q4_K against an
 *                      independent per-element decoder and the reference build (_ref)
 *   eo_matvec          core.cpp:92-94 2x2 F32 case, exact small-integer dots, fp64
 *                      brute force, and bit-exact agreement with _ref
 *   eo_delta_net       _ref (backend.cpp Backend::delta_net) + closed-form invariants
 *   eo_feed_forward    _ref (backend.cpp Backend::feed_forward)
 *   eo_rms, eo_rope    closed forms (unit vectors, pos=0 identity, rotation norm)
 *   eo_attention       invariants: L=1 gives v*sigmoid(gate), equal keys give the mean
 *                      of v, fp64 brute force
 *   eo_model_*         composition of the above; teacher-forced token agreement
 *                      with a step-by-step composition of _ref ops; bit-equal to the
 *                      reference's own compiled Model (_ref/libemprise_refmodel.so) on
 *                      every traced tensor, logits, hidden vectors, evaluate_block, prefill
 *   eo_quantize_q8     core.cpp:119-125's construction of the checked input; fp16(s) by
 *                      the test's monotone search (core.cpp:14-21), tested against numpy's
 *                      float16 rounding and the GPU's standalone quantiser bit for bit
 *   eo_model_evaluate_many  bit-equal to eo_model_evaluate position by position (logits,
 *                      last residual, the state left behind), plain and Q8
 *   eo_model_mtp_*     bit-equal to the reference's Model::mtp_draft/mtp_hidden; and
 *                      closed forms on F32 models built for them: each half of the
 *                      [enorm(e) | hnorm(h)] input, the one-row attention (v times the
 *                      sigmoid gate), the FFN, the head; cache growth and reset
 *   eo_model_last_hidden_normed  the output norm of eo_model_last_hidden
 */
#ifndef EMPRISE_ORACLE_H
#define EMPRISE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { EO_F32 = 0, EO_F16 = 1, EO_Q4_K = 12, EO_Q6_K = 14, EO_BF16 = 30 };

float eo_half_to_float(uint16_t h);
/* Bytes of `n` elements of `type`; 0 when the count is invalid for the type. */
uint64_t eo_encoded_bytes(uint32_t type, uint64_t n);
/* Returns 0, or -1 when in_len does not match n elements of type. */
int eo_dequantize(uint32_t type, const uint8_t* in, size_t in_len, float* out, size_t n);
/* y[rows] = W x; W is rows x cols in `type` (row-major, rows of whole blocks). */
int eo_matvec(uint32_t type, const uint8_t* w, size_t w_len, const float* x, size_t cols,
              float* y, size_t rows);

void eo_rms(float* x, size_t n, const float* weight, float eps);
void eo_rope(float* x, int rotary, int pos, float base);
float eo_sigmoid(float x);
float eo_silu(float x);
float eo_softplus(float x);

/* Gated GQA attention for one position (model.cpp:129-157). qg is heads*head_dim*2
 * (per head [q | gate]), k and v are kv_heads*head_dim. keys/values are the caches
 * with room for length positions; the new k/v (after norm + RoPE on k) are appended
 * at index length-1. out is heads*head_dim. */
void eo_attention(int heads, int kv_heads, int head_dim, int rotary, float rope_base, float eps,
                  const float* q_norm, const float* k_norm, float* qg, float* k, const float* v,
                  float* keys, float* values, size_t length, int pos, float* out);

/* Backend::delta_net (backend.cpp:19-60). qkv is modified in place like the
 * reference's working copy is not: the caller's qkv stays untouched. */
void eo_delta_net(int key_heads, int value_heads, int state_dim, int conv_width, float eps,
                  const float* qkv, const float* gate, const float* alpha, const float* beta,
                  const float* conv, const float* ssm_a, const float* dt, const float* norm,
                  float* conv_state, float* rec_state, float* out);

/* Backend::feed_forward (backend.cpp:91-104) over raw weight bytes. */
int eo_feed_forward(uint32_t gate_type, const uint8_t* gate_w, uint32_t up_type, const uint8_t* up_w,
                    uint32_t down_type, const uint8_t* down_w, size_t hidden, size_t ffn,
                    const float* x, float* y);

/* --fast-q8 input rule (cuda.cpp:547-559 as checked in core.cpp:119-125): per 32 values
 * s = max|x|/127, out = round(x/s) * fp16(s). */
void eo_quantize_q8(const float* x, size_t n, float* out);

/* ---- whole model (GGUF file in, logits out) ---- */
typedef struct eo_model eo_model;
/* threads = 0 keeps the OpenMP default. Returns NULL and fills err on failure. */
eo_model* eo_model_load(const char* path, size_t context, int threads, char* err, size_t err_len);
void eo_model_free(eo_model* m);
int eo_model_vocab(const eo_model* m);
int eo_model_hidden(const eo_model* m);
void eo_model_reset(eo_model* m);
/* --fast-q8: every Q6_K projection (output head included) sees eo_quantize_q8 of its
 * input, the CPU statement of the reference's device_linear in fast mode (cuda.cpp:707-712). */
void eo_model_set_quantize_activations(eo_model* m, int on);
/* Model::Impl::evaluate (model.cpp:206-259). logits may be NULL. Returns 0 or -1. */
int eo_model_evaluate(eo_model* m, int token, float* logits);
/* ModelOptions::trace (model.hpp:18-19, model.cpp:118-120): eo_model_evaluate calls fn
 * with the position, the tensor's name and the tensor at the reference's points
 * (model.cpp:219, :227, :244, :250, :253): "attn_norm-L", "attn_residual-L", "l_out-L"
 * per layer, then "result_norm" and "logits" when logits are asked for. NULL removes it. */
typedef void (*eo_trace_fn)(void* user, uint64_t position, const char* name, const float* data, uint64_t n);
void eo_model_set_trace(eo_model* m, eo_trace_fn fn, void* user);
/* tokens[0..n) from the current position, bit for bit as n eo_model_evaluate calls, with
 * the projections of all n positions computed together (one weight decode per 64
 * positions). logits (optional) are the last position's. Returns 0 or -1. */
int eo_model_evaluate_many(eo_model* m, const int* tokens, size_t n, float* logits);
/* Timing aid: jump to `position` with zeroed K/V rows (attention then spans position + 1
 * rows, as after a prompt of that length). Returns 0 or -1. */
int eo_model_seek(eo_model* m, size_t position);
/* Model::generate (model.cpp:488-503) with the prompt prefilled position by position.
 * Writes up to count tokens; returns how many were emitted (EOS stops early) or -1.
 * margins (optional) gets the top-1 minus top-2 logit gap for each emitted token. */
int eo_model_generate(eo_model* m, const int* prompt, size_t prompt_len, size_t count,
                      int* tokens, float* margins);
/* The residual stream after the last position evaluated with logits
 * (Model::last_hidden_raw; model.cpp:247-251 updates it only there). */
int eo_model_last_hidden(const eo_model* m, float* out);
/* Model::last_hidden (model.cpp:483): that residual through the output norm. */
int eo_model_last_hidden_normed(const eo_model* m, float* out);
/* The MTP (next-n) draft head, Model::mtp_draft / mtp_hidden / reset_mtp
 * (model.cpp:376-397, :485-487): blk.<layers>.nextn.* + that block's attention and FFN. */
int eo_model_has_mtp(const eo_model* m);
void eo_model_reset_mtp(eo_model* m);
int eo_model_mtp_draft(eo_model* m, const float* hidden, int token, size_t pos, float* logits);
int eo_model_mtp_hidden(const eo_model* m, float* out);
const char* eo_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
