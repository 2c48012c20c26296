/*
 * emprise_host.h -- C ABI of the C++ host (libemprise_host.so): the GGUF loader,
 * the qwen35 decode graph, the greedy loop and the --report numbers of the reference
 * (v1.1 src/gguf.cpp, src/model.cpp, src/chat.cpp), running on the HIP backend of
 * emprise_hip.h. Bindings (Python ctypes, the emprise-chat CLI) go through this header.
 *
 * Every call returns an emprise_status (emprise_hip.h); emprise_host_last_error()
 * holds the message of the last failure on this thread.
 */
#ifndef EMPRISE_HOST_H
#define EMPRISE_HOST_H
#include <stddef.h>
#include <stdint.h>

#include "emprise_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

const char* emprise_host_last_error(void);

/* Gguf::Gguf (gguf.cpp:87-147) without a device: maps and validates a GGUF v2/v3 file
 * (header, metadata, tensor table, the data section's extents) and reports how many
 * tensors and metadata keys it holds. EMPRISE_EINVAL when the file is not a valid GGUF
 * this reader decodes (the reference throws from the same checks). */
emprise_status emprise_gguf_inspect(const char* path, uint64_t* tensors, uint64_t* metadata);

/* ModelOptions (model.hpp:8-20) for the device path. */
typedef struct {
    const char* path;              /* GGUF file */
    size_t context;                /* --context, default 4096 */
    int device;                    /* HIP device ordinal */
    uint64_t weight_vram_budget;   /* --vram-mib in bytes; 0 = free memory - 512 MiB */
    int quantize_activations;      /* --fast-q8 */
    int fused;                     /* 1: fused projection kernels (default); 0: one op per launch like
                                      the reference's evaluate_device (model.cpp:422-472) */
    int graph;                     /* 1: replay the decode step as a hipGraph (default) */
    int batch_prefill;             /* prompts with at least this many tokens before the last one
                                      prefill in batches (GEMM projections); 0 = 64, < 0 = never */
} emprise_model_options;

typedef struct emprise_model emprise_model;

/* Model::Model (model.cpp:47-79, :474): parses the GGUF, checks the qwen35 dimensions,
 * uploads every weight to the device. */
emprise_status emprise_model_open(const emprise_model_options* options, emprise_model** out);
void emprise_model_close(emprise_model* m);
const char* emprise_model_backend_name(const emprise_model* m);

typedef struct {
    int hidden, layers, heads, kv_heads, head_dim, rotary;
    int key_heads, value_heads, state_dim, conv_width, ffn, vocab, eos;
    float eps, rope_base;
    size_t context;
    uint64_t weight_bytes;       /* GGUF bytes of every tensor uploaded */
    uint64_t token_weight_bytes; /* GGUF bytes streamed per decoded token (matrices + one embedding row + vectors) */
    double load_seconds;
} emprise_model_info;
emprise_status emprise_model_get_info(const emprise_model* m, emprise_model_info* info);

/* Model::profile (model.hpp:21-25): the reference times every backend call on its host
 * path (model.cpp:90-115, :216-256) and, on its device path (evaluate_device,
 * model.cpp:422-472), counts evaluated tokens only. Here a decode step is one replayed
 * graph, so its split by kind comes from the per-launch HIP event timing of the last
 * emprise_model_trace_step (one eager step), scaled by the decode steps run since the model
 * was opened (traced steps themselves are measurements and are not counted); with no traced
 * step the times are 0. matrix_* covers the projection kernels
 * (matvec, GEMM), matrix_calls counts projections the reference's way (one per weight:
 * q/k/v/o or qkv/gate/alpha/beta/out, gate/up/down, the output head), norm_* the
 * stand-alone RMSNorm kernels (the fused path folds RMSNorm into the projections' input
 * staging, so 0 there), attention_* / recurrent_* the attention and Gated DeltaNet
 * kernels, and non_matrix_* everything but the projections. Batched prefills add their
 * positions to evaluated_tokens only. */
typedef struct {
    double matrix_seconds, non_matrix_seconds;
    double norm_seconds, attention_seconds, recurrent_seconds;
    uint64_t matrix_calls, evaluated_tokens;
    uint64_t decode_steps;  /* single-position steps with the output head since open */
    uint64_t traced_steps;  /* steps the per-kind split was measured on (0: none yet) */
} emprise_model_profile;
emprise_status emprise_model_get_profile(const emprise_model* m, emprise_model_profile* out);

/* Model::reset (model.cpp:479). */
emprise_status emprise_model_reset(emprise_model* m);
/* Model::evaluate (model.cpp:206-259) on the device: one position; logits (vocab
 * floats) may be NULL. */
emprise_status emprise_model_evaluate(emprise_model* m, int token, float* logits);
/* ModelOptions::trace (model.hpp:18-19, model.cpp:118-120): a synchronous diagnostic
 * hook that emprise_model_evaluate calls with the position, a tensor name and the tensor
 * (valid only during the call) at the reference's points, in its order: per layer L
 * "attn_norm-L" (the normalised input of the attention / recurrent block),
 * "attn_residual-L" (the stream after its residual add) and "l_out-L" (after the
 * feed-forward's), then, when logits are wanted, "result_norm" and "logits"
 * (model.cpp:219, :227, :244, :250, :253). While a hook is set, evaluate runs its step as
 * eager launches and copies each tensor to the host at its point (the fused path's
 * normalised inputs, which its projections compute in their input staging, by a
 * stand-alone RMSNorm launch); generate and the batched paths do not call it, as the
 * reference's device path (evaluate_device) does not. fn NULL removes the hook. */
typedef void (*emprise_trace_fn)(void* user, uint64_t position, const char* name, const float* data, uint64_t n);
emprise_status emprise_model_set_trace(emprise_model* m, emprise_trace_fn fn, void* user);
/* Model::prefill (model.cpp:355-366, model.hpp:40-41): evaluates `tokens` from the current
 * position on -- all but the last in batches (GEMM projections, from 64 tokens) or as
 * replayed steps, the last as a decode step -- and writes the last position's logits
 * (vocab floats; may be NULL). The reference prefills in chunks of 4 positions. */
emprise_status emprise_model_prefill(emprise_model* m, const int* tokens, size_t n, float* logits);
/* The residual stream after the last position evaluated with logits (Model::last_hidden_raw;
   model.cpp:247-251 keeps it only there: positions evaluated without logits leave it). */
emprise_status emprise_model_last_hidden(emprise_model* m, float* hidden);
/* Model::last_hidden (model.cpp:483): that residual through the output norm. */
emprise_status emprise_model_last_hidden_normed(emprise_model* m, float* hidden);
/* Model::evaluate_block (model.hpp:37-39, model.cpp:274-354): the n tokens from the
 * current position on, in order, with every position's logits (n rows of vocab floats;
 * the reference's draft-verification call). */
emprise_status emprise_model_evaluate_block(emprise_model* m, const int* tokens, size_t n, float* logits);

/* The MTP (next-n) draft head (model.hpp:42-48; model.cpp:376-397, :485-487), present
 * when the file has blk.<layers>.nextn.* (blk.32 at the 9B shape). */
int emprise_model_has_mtp(const emprise_model* m);
/* Model::mtp_draft: from a hidden vector (hidden floats) and the token that followed it,
 * the logits (vocab floats) of the token after; the block's attention appends one row to
 * its own cache and rotates at `position`. EINVAL without the block. */
emprise_status emprise_model_mtp_draft(emprise_model* m, const float* hidden, int token, size_t position,
                                       float* logits);
/* Model::mtp_hidden: the block's output of the last draft (before the shared head norm). */
emprise_status emprise_model_mtp_hidden(emprise_model* m, float* hidden);
/* Model::reset_mtp: the block's cache emptied. */
emprise_status emprise_model_reset_mtp(emprise_model* m);

/* Model::generate (model.cpp:488-503): prefill, then greedy tokens until count or EOS.
 * tokens receives up to count ids, *emitted the number written, arrivals (optional,
 * count doubles) the completion time of each token in seconds after the first
 * prefill launch, measured with HIP events on the backend stream. */
emprise_status emprise_model_generate(emprise_model* m, const int* prompt, size_t prompt_len, size_t count,
                                      int* tokens, size_t* emitted, double* arrivals);

/* One eager (non-graph) decode step at the current position with every kernel launch
 * bracketed by HIP events (emprise_hip_trace_begin/end): per-launch kernel name,
 * algorithmic bytes and milliseconds. Attention records carry the K/V bytes of the
 * position they ran at. Advances the position like emprise_model_evaluate. */
emprise_status emprise_model_trace_step(emprise_model* m, int token, emprise_hip_trace_record* records, size_t cap,
                                        size_t* n);

/* ---- tokenizer (include/emprise/tokenizer.hpp, src/tokenizer.cpp) ----------------- */
/* The qwen35 GPT-2 byte-level BPE of a GGUF's tokenizer.ggml.* metadata. */
typedef struct emprise_tokenizer emprise_tokenizer;
/* A file's tokenizer without a device (the reference's --tokenize path, chat.cpp:47-52):
 * EINVAL when the file has no qwen35 GPT-2 BPE tokenizer (tokenizer.cpp:62-63). */
emprise_status emprise_tokenizer_open(const char* path, emprise_tokenizer** out);
/* Releases a tokenizer from emprise_tokenizer_open; a model's tokenizer is left alone. */
void emprise_tokenizer_close(emprise_tokenizer* t);
/* Model::tokenizer (model.hpp:33): the model's tokenizer, NULL when its file has none. */
const emprise_tokenizer* emprise_model_tokenizer(const emprise_model* m);
/* Tokenizer::encode (tokenizer.cpp:114-131): len bytes of UTF-8 text; parse_special
 * matches special tokens verbatim. Writes min(cap, count) ids and the count to *n. */
emprise_status emprise_tokenizer_encode(const emprise_tokenizer* t, const char* text, size_t len, int parse_special,
                                        int* ids, size_t cap, size_t* n);
/* Tokenizer::decode (tokenizer.cpp:132-135): the token's bytes (min(cap, count) written,
 * no terminator; the count in *n). EINVAL for an id outside the vocabulary. */
emprise_status emprise_tokenizer_decode(const emprise_tokenizer* t, int token, char* out, size_t cap, size_t* n);
/* Tokenizer::chat_prompt (tokenizer.cpp:136-139): the single-turn template around user. */
emprise_status emprise_tokenizer_chat_prompt(const emprise_tokenizer* t, const char* user, size_t len, char* out,
                                             size_t cap, size_t* n);

/* ---- synthetic qwen35 GGUF (test and benchmark inputs) ----------------------- */
typedef struct {
    uint64_t seed;
    int hidden, layers, ffn, vocab;
    int heads, kv_heads, head_dim, rotary;
    int key_heads, value_heads, state_dim, conv_width;
    int full_attention_interval; /* layer i is attention when (i+1) % interval == 0 */
    int context_length;
    float rope_base, eps;
    int eos;
    uint32_t matrix_type; /* EMPRISE_Q6_K or EMPRISE_Q4_K for every matrix */
    int q4_k_m_mix;       /* 1: attn_v and ffn_down Q6_K, every other matrix Q4_K */
    int mtp;              /* 1: add the MTP (next-n) block blk.<layers> (qwen35.nextn_predict_layers = 1) */
    int tokenizer;        /* 1: add a qwen35 GPT-2 BPE tokenizer: 256 byte tokens, merges trained on a
                             built-in text, the chat template's special tokens, control tokens up to vocab */
} emprise_synth_config;

/* Writes a GGUF v3 file with deterministic weights: counter-based SplitMix64 streams per
 * tensor (so the bytes do not depend on thread count), normals by Irwin-Hall sums of
 * twelve uniforms. Q6_K: codes uniform bytes, int8 sub-scales uniform in [-32, 31],
 * d = fp16(|N|*2e-4). Q4_K: bytes uniform, d and dmin = fp16(|N|*1e-3). Norm weights
 * 1 + N*0.02, ssm_a = -exp(0.5N - 2), ssm_dt.bias = 0.5N - 1, conv taps 0.5N. */
emprise_status emprise_synth_write(const emprise_synth_config* config, const char* path);
/* Seeded prompt ids uniform over [0, vocab). */
emprise_status emprise_synth_prompt(uint64_t seed, int vocab, size_t n, int* ids);

#ifdef __cplusplus
}
#endif
#endif
