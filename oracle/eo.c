/*
 * CPU oracle: plain-C restatement of the reference's CPU decode path.
 * TEST INFRASTRUCTURE ONLY -- see eo.h for who may load it and how each function is
 * pinned. All citations are to the reference's v1.1 tree.
 */
#define _GNU_SOURCE
#include "eo.h"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static __thread char g_err[512];
static void set_err(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
const char* eo_last_error(void) { return g_err; }

/* quant.cpp:8-17 */
float eo_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const uint32_t ex = (h >> 10) & 31, frac = h & 1023;
    if (ex == 0) {
        const float x = ldexpf((float)frac, -24);
        return sign ? -x : x;
    }
    const uint32_t bits = sign | (ex == 31 ? 0x7f800000u : (ex + 112) << 23) | (frac << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* gguf.cpp:72-85 (0 = rejected) */
uint64_t eo_encoded_bytes(uint32_t type, uint64_t n) {
    switch (type) {
    case EO_F32: return n > UINT64_MAX / 4 ? 0 : n * 4;
    case EO_F16:
    case EO_BF16: return n > UINT64_MAX / 2 ? 0 : n * 2;
    case EO_Q6_K: return (n % 256) ? 0 : n / 256 * 210;
    case EO_Q4_K: return (n % 256) ? 0 : n / 256 * 144;
    default: return 0;
    }
}

static uint16_t rd16(const uint8_t* p) { uint16_t v; memcpy(&v, p, 2); return v; }

/* quant.cpp:25-40: 210-byte super-block, ql[128] qh[64] int8 sc[16] fp16 d */
static void q6_block(const uint8_t* b, float* out) {
    const int8_t* scales = (const int8_t*)(b + 192);
    const float d = eo_half_to_float(rd16(b + 208));
    for (int half = 0; half < 2; ++half)
        for (int group = 0; group < 4; ++group)
            for (int lane = 0; lane < 32; ++lane) {
                const int low_index = half * 64 + (group & 1) * 32 + lane;
                const int low = (b[low_index] >> (group >= 2 ? 4 : 0)) & 15;
                const int high = (b[128 + half * 32 + lane] >> (group * 2)) & 3;
                const int q = (low | (high << 4)) - 32;
                /* (d * sc) * q, both products in float */
                out[half * 128 + group * 32 + lane] = d * (float)scales[half * 8 + group * 2 + lane / 16] * (float)q;
            }
}

/* quant.cpp:48-52 */
static void q4_scale_min(const uint8_t* s, int j, uint8_t* sc, uint8_t* mn) {
    if (j < 4) { *sc = s[j] & 63; *mn = s[j + 4] & 63; }
    else { *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
           *mn = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4)); }
}

/* quant.cpp:41-61: 144-byte super-block, fp16 d, fp16 dmin, 12 B scales, qs[128] */
static void q4_k_block(const uint8_t* b, float* out) {
    const float d = eo_half_to_float(rd16(b));
    const float dmin = eo_half_to_float(rd16(b + 2));
    const uint8_t* scales = b + 4;
    const uint8_t* q = b + 16;
    int is = 0;
    for (int j = 0; j < 256; j += 64) {
        uint8_t sc, mn;
        q4_scale_min(scales, is + 0, &sc, &mn);
        const float d1 = d * (float)sc, m1 = dmin * (float)mn;
        q4_scale_min(scales, is + 1, &sc, &mn);
        const float d2 = d * (float)sc, m2 = dmin * (float)mn;
        for (int l = 0; l < 32; ++l) out[j + l] = d1 * (float)(q[l] & 0xF) - m1;
        for (int l = 0; l < 32; ++l) out[j + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
        q += 32;
        is += 2;
    }
}

static float raw_element(uint32_t type, const uint8_t* p) {
    if (type == EO_F32) { float v; memcpy(&v, p, 4); return v; }
    const uint16_t bits = rd16(p);
    if (type == EO_BF16) { uint32_t u = (uint32_t)bits << 16; float v; memcpy(&v, &u, 4); return v; }
    return eo_half_to_float(bits);
}

/* quant.cpp:64-78 */
int eo_dequantize(uint32_t type, const uint8_t* in, size_t in_len, float* out, size_t n) {
    const uint64_t need = eo_encoded_bytes(type, n);
    if (!need || need != in_len) { set_err("Incorrect encoded size"); return -1; }
    if (type == EO_F32) memcpy(out, in, in_len);
    else if (type == EO_Q6_K) for (size_t i = 0; i < n / 256; ++i) q6_block(in + i * 210, out + i * 256);
    else if (type == EO_Q4_K) for (size_t i = 0; i < n / 256; ++i) q4_k_block(in + i * 144, out + i * 256);
    else for (size_t i = 0; i < n; ++i) out[i] = raw_element(type, in + i * 2);
    return 0;
}

/* quant.cpp:80-111: one FP32 accumulator per row, summed in element order. */
int eo_matvec(uint32_t type, const uint8_t* w, size_t w_len, const float* x, size_t cols,
              float* y, size_t rows) {
    if (!cols) { set_err("Empty input vector"); return -1; }
    const uint64_t row_bytes = eo_encoded_bytes(type, cols);
    if (!row_bytes || w_len / row_bytes != rows || w_len % row_bytes) { set_err("Matrix size mismatch"); return -1; }
    #pragma omp parallel for schedule(static)
    for (int64_t row = 0; row < (int64_t)rows; ++row) {
        const uint8_t* ptr = w + (uint64_t)row * row_bytes;
        float sum = 0;
        if (type == EO_Q6_K || type == EO_Q4_K) {
            const size_t block_bytes = type == EO_Q6_K ? 210 : 144;
            float block[256];
            for (size_t k = 0; k < cols; k += 256) {
                if (type == EO_Q6_K) q6_block(ptr + k / 256 * block_bytes, block);
                else q4_k_block(ptr + k / 256 * block_bytes, block);
                for (size_t j = 0; j < 256; ++j) sum += block[j] * x[k + j];
            }
        } else {
            const size_t es = type == EO_F32 ? 4 : 2;
            for (size_t k = 0; k < cols; ++k) sum += raw_element(type, ptr + k * es) * x[k];
        }
        y[row] = sum;
    }
    return 0;
}

/* model.cpp:16-18 (= backend.cpp:10-12) */
float eo_sigmoid(float x) { return x >= 0 ? 1.f / (1.f + expf(-x)) : expf(x) / (1.f + expf(x)); }
float eo_silu(float x) { return x * eo_sigmoid(x); }
float eo_softplus(float x) { return (x < 0.f ? 0.f : x) + log1pf(expf(-fabsf(x))); }

/* model.cpp:19-25 */
void eo_rms(float* x, size_t n, const float* weight, float eps) {
    float sum = 0;
    for (size_t i = 0; i < n; ++i) sum += x[i] * x[i];
    const float scale = 1.f / sqrtf(sum / (float)n + eps);
    for (size_t i = 0; i < n; ++i) x[i] *= scale * weight[i];
}

/* model.cpp:121-127: NEOX half-split rotation of the first `rotary` dims */
void eo_rope(float* x, int rotary, int pos, float base) {
    for (int i = 0; i < rotary / 2; ++i) {
        const float angle = (float)pos / powf(base, 2.f * (float)i / (float)rotary);
        const float a = x[i], b = x[i + rotary / 2], c = cosf(angle), s = sinf(angle);
        x[i] = a * c - b * s;
        x[i + rotary / 2] = a * s + b * c;
    }
}

/* model.cpp:129-157 */
void eo_attention(int heads, int kv_heads, int head_dim, int rotary, float rope_base, float eps,
                  const float* q_norm, const float* k_norm, float* qg, float* k, const float* v,
                  float* keys, float* values, size_t length, int pos, float* out) {
    for (int h = 0; h < heads; ++h) {
        float* q = qg + (size_t)h * head_dim * 2;
        eo_rms(q, (size_t)head_dim, q_norm, eps);
        eo_rope(q, rotary, pos, rope_base);
    }
    for (int h = 0; h < kv_heads; ++h) {
        float* kh = k + (size_t)h * head_dim;
        eo_rms(kh, (size_t)head_dim, k_norm, eps);
        eo_rope(kh, rotary, pos, rope_base);
    }
    const size_t stride = (size_t)kv_heads * head_dim;
    memcpy(keys + (length - 1) * stride, k, stride * sizeof(float));
    memcpy(values + (length - 1) * stride, v, stride * sizeof(float));
    const float root = sqrtf((float)head_dim);
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < heads; ++h) {
        const int kh = h / (heads / kv_heads);
        float* scores = (float*)malloc(length * sizeof(float));
        float peak = -INFINITY;
        for (size_t t = 0; t < length; ++t) {
            float dot = 0;
            for (int d = 0; d < head_dim; ++d)
                dot += qg[(size_t)h * head_dim * 2 + d] * keys[t * stride + (size_t)kh * head_dim + d];
            scores[t] = dot / root;
            peak = peak < scores[t] ? scores[t] : peak;
        }
        float total = 0;
        for (size_t t = 0; t < length; ++t) { scores[t] = expf(scores[t] - peak); total += scores[t]; }
        for (int d = 0; d < head_dim; ++d) {
            float sum = 0;
            for (size_t t = 0; t < length; ++t)
                sum += scores[t] / total * values[t * stride + (size_t)kh * head_dim + d];
            out[(size_t)h * head_dim + d] = sum * eo_sigmoid(qg[(size_t)h * head_dim * 2 + head_dim + d]);
        }
        free(scores);
    }
}

/* backend.cpp:19-60 */
void eo_delta_net(int key_heads, int value_heads, int state_dim, int conv_width, float eps,
                  const float* qkv_in, const float* gate, const float* alpha, const float* beta,
                  const float* conv, const float* ssm_a, const float* dt, const float* norm,
                  float* conv_state, float* rec_state, float* out) {
    const int key_dim = key_heads * state_dim, value_dim = value_heads * state_dim;
    const int channels = 2 * key_dim + value_dim;
    float* qkv = (float*)malloc((size_t)channels * sizeof(float));
    memcpy(qkv, qkv_in, (size_t)channels * sizeof(float));
    /* causal conv1d over the per-channel history, then SiLU (backend.cpp:22-29) */
    for (int c = 0; c < channels; ++c) {
        float* history = conv_state + (size_t)c * conv_width;
        for (int j = 0; j < conv_width - 1; ++j) history[j] = history[j + 1];
        history[conv_width - 1] = qkv[c];
        float sum = 0;
        for (int j = 0; j < conv_width; ++j) sum += history[j] * conv[c * conv_width + j];
        qkv[c] = eo_silu(sum);
    }
    /* q/k L2 normalisation per key head (backend.cpp:30-35) */
    for (int h = 0; h < key_heads; ++h) {
        float qs = 0, ks = 0;
        for (int d = 0; d < state_dim; ++d) {
            const float q = qkv[h * state_dim + d], k = qkv[key_dim + h * state_dim + d];
            qs += q * q;
            ks += k * k;
        }
        const float qscale = 1.f / sqrtf(qs + eps) / sqrtf((float)state_dim), kscale = 1.f / sqrtf(ks + eps);
        for (int d = 0; d < state_dim; ++d) {
            qkv[h * state_dim + d] *= qscale;
            qkv[key_dim + h * state_dim + d] *= kscale;
        }
    }
    /* gated delta-rule scan, one value head per iteration (backend.cpp:36-56) */
    #pragma omp parallel for schedule(static)
    for (int h = 0; h < value_heads; ++h) {
        const int kh = h % key_heads;
        const float* q = qkv + kh * state_dim;
        const float* k = qkv + key_dim + kh * state_dim;
        const float* v = qkv + 2 * key_dim + h * state_dim;
        float* state = rec_state + (size_t)h * state_dim * state_dim;
        const float decay = expf(ssm_a[h] * eo_softplus(alpha[h] + dt[h])), b = eo_sigmoid(beta[h]);
        for (int d = 0; d < state_dim; ++d) {
            float memory = 0;
            #pragma omp simd reduction(+:memory)
            for (int j = 0; j < state_dim; ++j) {
                state[d * state_dim + j] *= decay;
                memory += state[d * state_dim + j] * k[j];
            }
            const float delta = (v[d] - memory) * b;
            float sum = 0;
            #pragma omp simd reduction(+:sum)
            for (int j = 0; j < state_dim; ++j) {
                state[d * state_dim + j] += k[j] * delta;
                sum += state[d * state_dim + j] * q[j];
            }
            out[h * state_dim + d] = sum;
        }
        float* chunk = out + (size_t)h * state_dim;
        eo_rms(chunk, (size_t)state_dim, norm, eps);
        for (int d = 0; d < state_dim; ++d) chunk[d] *= eo_silu(gate[h * state_dim + d]);
    }
    free(qkv);
}

/* backend.cpp:91-104 */
int eo_feed_forward(uint32_t gate_type, const uint8_t* gate_w, uint32_t up_type, const uint8_t* up_w,
                    uint32_t down_type, const uint8_t* down_w, size_t hidden, size_t ffn,
                    const float* x, float* y) {
    float* g = (float*)malloc(ffn * sizeof(float));
    float* u = (float*)malloc(ffn * sizeof(float));
    int rc = eo_matvec(gate_type, gate_w, eo_encoded_bytes(gate_type, hidden * ffn), x, hidden, g, ffn);
    if (!rc) rc = eo_matvec(up_type, up_w, eo_encoded_bytes(up_type, hidden * ffn), x, hidden, u, ffn);
    if (!rc) {
        for (size_t i = 0; i < ffn; ++i) {
            const float e = expf(-fabsf(g[i]));
            const float s = g[i] >= 0 ? 1.f / (1.f + e) : e / (1.f + e);
            g[i] = g[i] * s * u[i];
        }
        rc = eo_matvec(down_type, down_w, eo_encoded_bytes(down_type, hidden * ffn), g, ffn, y, hidden);
    }
    free(g);
    free(u);
    return rc;
}

/* The nearest fp16 value of a positive float, ties to the even code: the reference
 * test's own rule (tests/core.cpp:14-21, a monotone search over the finite positive
 * half codes), used there to form the Q8 check input. */
static float round_positive_half(float value) {
    unsigned lo = 0, hi = 0x7bff;
    while (lo < hi) {
        const unsigned mid = (lo + hi) / 2;
        if (eo_half_to_float((uint16_t)mid) < value) lo = mid + 1;
        else hi = mid;
    }
    if (!lo) return 0;
    const float a = eo_half_to_float((uint16_t)(lo - 1)), b = eo_half_to_float((uint16_t)lo);
    return value - a < b - value || (value - a == b - value && ((lo - 1) & 1) == 0) ? a : b;
}

/* --fast-q8 activations as the CPU sees them (cuda.cpp:547-559, checked against the CPU
 * path in tests/core.cpp:119-125): per 32 inputs s = max|x| / 127, and
 * x' = round(x / s) * fp16(s) (round: ties away from zero, with the unrounded s). */
void eo_quantize_q8(const float* x, size_t n, float* out) {
    for (size_t start = 0; start < n; start += 32) {
        float scale = 0;
        for (size_t j = 0; j < 32 && start + j < n; ++j) scale = fmaxf(scale, fabsf(x[start + j]));
        scale /= 127;
        const float kept = round_positive_half(scale);
        for (size_t j = 0; j < 32 && start + j < n; ++j)
            out[start + j] = scale != 0.f ? roundf(x[start + j] / scale) * kept : 0.f;
    }
}

/* ------------------------------------------------------------------------------ */
/* GGUF reader (gguf.cpp:87-147), resident in RAM like the reference's default.     */

typedef struct {
    char* name;
    uint32_t type;
    uint64_t shape[4];
    uint32_t ndim;
    uint64_t offset, bytes, elements;
} eo_tensor;

typedef struct {
    char* key;
    int is_string, is_number;
    double number;
    char* string;
} eo_kv;

typedef struct {
    FILE* f;
    uint64_t size;
    int ok;
} rdr;

static int rd(rdr* r, void* dst, size_t n) {
    if (!r->ok) return -1;
    if (fread(dst, 1, n, r->f) != n) { r->ok = 0; set_err("Truncated GGUF header"); return -1; }
    return 0;
}
static uint64_t rd_u64(rdr* r) { uint64_t v = 0; rd(r, &v, 8); return v; }
static uint32_t rd_u32(rdr* r) { uint32_t v = 0; rd(r, &v, 4); return v; }
static char* rd_str(rdr* r) {
    const uint64_t n = rd_u64(r);
    if (!r->ok) return NULL;
    const uint64_t pos = (uint64_t)ftello(r->f);
    if (pos > r->size || n > r->size - pos || n > 64ull * 1024 * 1024) { r->ok = 0; set_err("Invalid GGUF string length"); return NULL; }
    char* s = (char*)malloc(n + 1);
    if (rd(r, s, n)) { free(s); return NULL; }
    s[n] = 0;
    return s;
}

/* Reads one metadata value; scalars are kept as numbers, strings as text, arrays skipped. */
static int rd_value(rdr* r, uint32_t type, int depth, eo_kv* kv) {
    if (depth > 4) { r->ok = 0; set_err("Excessive metadata nesting"); return -1; }
    union { uint8_t u8; int8_t i8; uint16_t u16; int16_t i16; uint32_t u32; int32_t i32; float f32;
            uint64_t u64; int64_t i64; double f64; } v;
    double num = 0;
    switch (type) {
    case 0: rd(r, &v.u8, 1); num = v.u8; break;
    case 1: rd(r, &v.i8, 1); num = v.i8; break;
    case 2: rd(r, &v.u16, 2); num = v.u16; break;
    case 3: rd(r, &v.i16, 2); num = v.i16; break;
    case 4: rd(r, &v.u32, 4); num = v.u32; break;
    case 5: rd(r, &v.i32, 4); num = v.i32; break;
    case 6: rd(r, &v.f32, 4); num = v.f32; break;
    case 7: rd(r, &v.u8, 1); if (v.u8 > 1) { r->ok = 0; set_err("Invalid boolean metadata"); return -1; } num = v.u8; break;
    case 8: {
        char* s = rd_str(r);
        if (!s) return -1;
        if (kv) { kv->is_string = 1; kv->string = s; } else free(s);
        return r->ok ? 0 : -1;
    }
    case 9: {
        const uint32_t sub = rd_u32(r);
        const uint64_t count = rd_u64(r);
        if (!r->ok) return -1;
        if (count > r->size || count > 10000000) { r->ok = 0; set_err("Invalid metadata array"); return -1; }
        for (uint64_t i = 0; i < count; ++i)
            if (rd_value(r, sub, depth + 1, NULL)) return -1;
        return 0;
    }
    case 10: rd(r, &v.u64, 8); num = (double)v.u64; break;
    case 11: rd(r, &v.i64, 8); num = (double)v.i64; break;
    case 12: rd(r, &v.f64, 8); num = v.f64; break;
    default: r->ok = 0; set_err("Unknown GGUF metadata type"); return -1;
    }
    if (kv) { kv->is_number = 1; kv->number = num; }
    return r->ok ? 0 : -1;
}

typedef struct {
    float *conv, *rec, *keys, *values;
    size_t length;
} eo_layer_state;

typedef struct {
    const uint8_t *qkv, *gate, *alpha, *beta, *out, *q, *k, *v, *o, *fg, *fu, *fd;
    uint32_t tqkv, tgate, talpha, tbeta, tout, tq, tk, tv, to, tfg, tfu, tfd;
    float *attn_norm, *post_norm, *conv, *ssm_a, *dt, *ssm_norm, *q_norm, *k_norm;
    int recurrent;
} eo_layer;

struct eo_model {
    eo_tensor* tensors;
    size_t n_tensors;
    eo_kv* kvs;
    size_t n_kvs;
    uint8_t* data;
    uint64_t data_bytes;
    int hidden, layers, heads, kv_heads, head_dim, rotary, key_heads, value_heads, state_dim, conv_width, eos;
    int vocab, ffn;
    float eps, rope_base;
    size_t context, position;
    eo_layer* layer;
    eo_layer_state* state;
    const uint8_t *embd, *output;
    uint32_t tembd, toutput;
    float* output_norm;
    float* last_hidden;
    int q8; /* --fast-q8: Q6_K projections see quantised inputs */
    eo_trace_fn trace;
    void* trace_user;
    /* the MTP (next-n) block, blk.<layers> (model.cpp:376-397), when the file has one:
     * an attention layer plus the nextn embedding/hidden norms, eh_proj [2H -> H] and the
     * shared head norm; its own K/V cache (mtp_state) and last output (mtp_hidden) */
    int has_mtp;
    eo_layer mtp;
    const uint8_t* eh;
    uint32_t teh;
    float *enorm, *hnorm, *head_norm;
    eo_layer_state mtp_state;
    float* mtp_hidden;
};

static const eo_kv* find_kv(const eo_model* m, const char* key) {
    for (size_t i = 0; i < m->n_kvs; ++i)
        if (!strcmp(m->kvs[i].key, key)) return &m->kvs[i];
    return NULL;
}
static const eo_tensor* find_tensor(const eo_model* m, const char* name) {
    for (size_t i = 0; i < m->n_tensors; ++i)
        if (!strcmp(m->tensors[i].name, name)) return &m->tensors[i];
    return NULL;
}

void eo_model_free(eo_model* m) {
    if (!m) return;
    for (size_t i = 0; i < m->n_tensors; ++i) free(m->tensors[i].name);
    for (size_t i = 0; i < m->n_kvs; ++i) { free(m->kvs[i].key); free(m->kvs[i].string); }
    free(m->tensors);
    free(m->kvs);
    free(m->data);
    if (m->layer)
        for (int l = 0; l < m->layers; ++l) {
            eo_layer* L = &m->layer[l];
            free(L->attn_norm); free(L->post_norm); free(L->conv); free(L->ssm_a); free(L->dt);
            free(L->ssm_norm); free(L->q_norm); free(L->k_norm);
        }
    if (m->state)
        for (int l = 0; l < m->layers; ++l) {
            free(m->state[l].conv); free(m->state[l].rec); free(m->state[l].keys); free(m->state[l].values);
        }
    free(m->layer);
    free(m->state);
    free(m->output_norm);
    free(m->last_hidden);
    free(m->mtp.attn_norm); free(m->mtp.post_norm); free(m->mtp.q_norm); free(m->mtp.k_norm);
    free(m->enorm); free(m->hnorm); free(m->head_norm);
    free(m->mtp_state.keys); free(m->mtp_state.values);
    free(m->mtp_hidden);
    free(m);
}

static int parse_gguf(eo_model* m, const char* path) {
    FILE* f = fopen(path, "rb");
    if (!f) { set_err("Cannot open model: %s", path); return -1; }
    fseeko(f, 0, SEEK_END);
    rdr r = {f, (uint64_t)ftello(f), 1};
    fseeko(f, 0, SEEK_SET);
    int rc = -1;
    if (rd_u32(&r) != 0x46554747u) { if (r.ok) set_err("Not a GGUF file"); goto done; }
    const uint32_t version = rd_u32(&r);
    if (version != 2 && version != 3) { if (r.ok) set_err("Unsupported GGUF version"); goto done; }
    const uint64_t nt = rd_u64(&r), nkv = rd_u64(&r);
    if (!r.ok) goto done;
    if (nt > 1000000 || nkv > 1000000) { set_err("Excessive header entries"); goto done; }
    m->kvs = (eo_kv*)calloc(nkv ? nkv : 1, sizeof(eo_kv));
    for (uint64_t i = 0; i < nkv; ++i) {
        eo_kv* kv = &m->kvs[i];
        kv->key = rd_str(&r);
        if (!kv->key) goto done;
        m->n_kvs = i + 1;
        for (uint64_t j = 0; j < i; ++j)
            if (!strcmp(m->kvs[j].key, kv->key)) { set_err("Duplicate metadata key"); goto done; }
        const uint32_t type = rd_u32(&r);
        if (!r.ok || rd_value(&r, type, 0, kv)) goto done;
    }
    const eo_kv* al = find_kv(m, "general.alignment");
    const uint64_t alignment = al && al->is_number ? (uint64_t)al->number : 32;
    if (!alignment || alignment > 1024 * 1024 || (alignment & (alignment - 1))) { set_err("Invalid GGUF alignment"); goto done; }
    m->tensors = (eo_tensor*)calloc(nt ? nt : 1, sizeof(eo_tensor));
    for (uint64_t i = 0; i < nt; ++i) {
        eo_tensor* t = &m->tensors[i];
        t->name = rd_str(&r);
        if (!t->name) goto done;
        m->n_tensors = i + 1;
        t->ndim = rd_u32(&r);
        if (!r.ok) goto done;
        if (!t->ndim || t->ndim > 4) { set_err("Unsupported tensor rank"); goto done; }
        t->elements = 1;
        for (uint32_t d = 0; d < t->ndim; ++d) {
            t->shape[d] = rd_u64(&r);
            if (!r.ok) goto done;
            if (!t->shape[d]) { set_err("Zero tensor dimension"); goto done; }
            if (t->elements > UINT64_MAX / t->shape[d]) { set_err("GGUF dimension overflow"); goto done; }
            t->elements *= t->shape[d];
        }
        t->type = rd_u32(&r);
        t->bytes = eo_encoded_bytes(t->type, t->elements);
        if (!t->bytes) { set_err("Unsupported GGUF tensor encoding: %u", t->type); goto done; }
        if ((t->type == EO_Q6_K || t->type == EO_Q4_K) && t->shape[0] % 256) { set_err("Q6_K row must contain whole blocks"); goto done; }
        t->offset = rd_u64(&r);
        if (!r.ok) goto done;
        if (t->offset % alignment) { set_err("Misaligned tensor offset"); goto done; }
        for (uint64_t j = 0; j < i; ++j)
            if (!strcmp(m->tensors[j].name, t->name)) { set_err("Duplicate tensor name"); goto done; }
    }
    const uint64_t header_end = (uint64_t)ftello(f);
    const uint64_t data_offset = (header_end + alignment - 1) / alignment * alignment;
    if (data_offset > r.size) { set_err("Missing tensor data"); goto done; }
    m->data_bytes = r.size - data_offset;
    for (size_t i = 0; i < m->n_tensors; ++i) {
        const eo_tensor* t = &m->tensors[i];
        if (t->offset > m->data_bytes || t->bytes > m->data_bytes - t->offset) { set_err("Truncated tensor: %s", t->name); goto done; }
        for (size_t j = 0; j < i; ++j) {
            const eo_tensor* u = &m->tensors[j];
            if (t->offset < u->offset + u->bytes && u->offset < t->offset + t->bytes) { set_err("Overlapping tensor extents"); goto done; }
        }
    }
    m->data = (uint8_t*)malloc(m->data_bytes ? m->data_bytes : 1);
    if (!m->data) { set_err("Out of memory for resident weights"); goto done; }
    fseeko(f, (off_t)data_offset, SEEK_SET);
    for (uint64_t off = 0; off < m->data_bytes;) {
        const uint64_t n = m->data_bytes - off < (64ull << 20) ? m->data_bytes - off : (64ull << 20);
        if (fread(m->data + off, 1, n, f) != n) { set_err("Failed to load resident weights"); goto done; }
        off += n;
    }
    rc = 0;
done:
    fclose(f);
    return rc;
}

static int meta_int(const eo_model* m, const char* key, int* out) {
    char full[256];
    snprintf(full, sizeof full, "qwen35.%s", key);
    const eo_kv* kv = find_kv(m, full);
    if (!kv || !kv->is_number) { set_err("Missing metadata: %s", full); return -1; }
    *out = (int)kv->number;
    return 0;
}

static const eo_tensor* need(const eo_model* m, const char* name) {
    const eo_tensor* t = find_tensor(m, name);
    if (!t) set_err("Missing tensor: %s", name);
    return t;
}

/* a matrix [cols, rows] whose input is `cols` */
static int matrix(const eo_model* m, const char* name, uint64_t cols, uint64_t rows, const uint8_t** w, uint32_t* type) {
    const eo_tensor* t = need(m, name);
    if (!t) return -1;
    if (t->ndim != 2 || t->shape[0] != cols || (rows && t->shape[1] != rows)) { set_err("Matrix shape mismatch: %s", name); return -1; }
    *w = m->data + t->offset;
    *type = t->type;
    return 0;
}

/* Model::Impl::parameter (model.cpp:80-89): small tensors dequantised once */
static float* param(const eo_model* m, const char* name, uint64_t elements) {
    const eo_tensor* t = need(m, name);
    if (!t) return NULL;
    if (t->elements != elements) { set_err("Parameter size mismatch: %s", name); return NULL; }
    if (t->bytes > 16ull * 1024 * 1024) { set_err("Unexpected non-matrix parameter size"); return NULL; }
    float* v = (float*)malloc(elements * sizeof(float));
    if (eo_dequantize(t->type, m->data + t->offset, t->bytes, v, elements)) { free(v); return NULL; }
    return v;
}

eo_model* eo_model_load(const char* path, size_t context, int threads, char* err, size_t err_len) {
    eo_model* m = (eo_model*)calloc(1, sizeof(eo_model));
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    if (parse_gguf(m, path)) goto fail;
    const eo_kv* arch = find_kv(m, "general.architecture");
    if (!arch || !arch->is_string || strcmp(arch->string, "qwen35")) { set_err("Only qwen35 is implemented"); goto fail; }
    int blocks = 0, ctx_len = 0;
    if (meta_int(m, "embedding_length", &m->hidden) || meta_int(m, "block_count", &blocks) ||
        meta_int(m, "attention.head_count", &m->heads) || meta_int(m, "attention.head_count_kv", &m->kv_heads) ||
        meta_int(m, "attention.key_length", &m->head_dim) || meta_int(m, "rope.dimension_count", &m->rotary) ||
        meta_int(m, "ssm.group_count", &m->key_heads) || meta_int(m, "ssm.time_step_rank", &m->value_heads) ||
        meta_int(m, "ssm.state_size", &m->state_dim) || meta_int(m, "ssm.conv_kernel", &m->conv_width) ||
        meta_int(m, "context_length", &ctx_len))
        goto fail;
    const eo_kv* nextn = find_kv(m, "qwen35.nextn_predict_layers");
    m->layers = blocks - (nextn && nextn->is_number ? (int)nextn->number : 0);
    const eo_kv* eos = find_kv(m, "tokenizer.ggml.eos_token_id");
    const eo_kv* eps = find_kv(m, "qwen35.attention.layer_norm_rms_epsilon");
    const eo_kv* base = find_kv(m, "qwen35.rope.freq_base");
    if (!eos || !eps || !base || !eos->is_number || !eps->is_number || !base->is_number) { set_err("Missing metadata"); goto fail; }
    m->eos = (int)eos->number;
    m->eps = (float)eps->number;
    m->rope_base = (float)base->number;
    m->context = context;
    /* model.cpp:67-70 */
    if (m->hidden <= 0 || m->layers <= 0 || m->heads <= 0 || m->kv_heads <= 0 || m->head_dim <= 0 ||
        m->rotary <= 0 || m->key_heads <= 0 || m->value_heads <= 0 || m->state_dim <= 0 || m->conv_width <= 0 ||
        m->heads % m->kv_heads || m->value_heads % m->key_heads || m->rotary > m->head_dim || m->rotary % 2 ||
        context == 0 || context > (size_t)ctx_len) {
        set_err("Unsupported or invalid Qwen dimensions/context");
        goto fail;
    }
    const eo_tensor* emb = need(m, "token_embd.weight");
    if (!emb || emb->ndim != 2 || emb->shape[0] != (uint64_t)m->hidden) { if (emb) set_err("token_embd shape"); goto fail; }
    m->vocab = (int)emb->shape[1];
    m->embd = m->data + emb->offset;
    m->tembd = emb->type;
    const int H = m->hidden;
    if (matrix(m, "output.weight", (uint64_t)H, 0, &m->output, &m->toutput)) goto fail;
    const eo_tensor* ot = find_tensor(m, "output.weight");
    if ((int)ot->shape[1] != m->vocab) { set_err("output.weight rows"); goto fail; }
    if (!(m->output_norm = param(m, "output_norm.weight", (uint64_t)H))) goto fail;
    m->layer = (eo_layer*)calloc((size_t)m->layers, sizeof(eo_layer));
    m->state = (eo_layer_state*)calloc((size_t)m->layers, sizeof(eo_layer_state));
    const int kd = m->key_heads * m->state_dim, vd = m->value_heads * m->state_dim, ch = 2 * kd + vd;
    const int qd = m->heads * m->head_dim * 2, kvd = m->kv_heads * m->head_dim;
    char name[256];
#define NAME(s) (snprintf(name, sizeof name, "blk.%d.%s", l, s), name)
    for (int l = 0; l < m->layers; ++l) {
        eo_layer* L = &m->layer[l];
        L->recurrent = find_tensor(m, NAME("ssm_a")) != NULL; /* model.cpp:75-78 */
        if (!(L->attn_norm = param(m, NAME("attn_norm.weight"), (uint64_t)H))) goto fail;
        if (!(L->post_norm = param(m, NAME("post_attention_norm.weight"), (uint64_t)H))) goto fail;
        if (matrix(m, NAME("ffn_gate.weight"), (uint64_t)H, 0, &L->fg, &L->tfg)) goto fail;
        const eo_tensor* g = find_tensor(m, name);
        if (l == 0) m->ffn = (int)g->shape[1];
        if ((int)g->shape[1] != m->ffn) { set_err("FFN dimensions"); goto fail; }
        if (matrix(m, NAME("ffn_up.weight"), (uint64_t)H, (uint64_t)m->ffn, &L->fu, &L->tfu)) goto fail;
        if (matrix(m, NAME("ffn_down.weight"), (uint64_t)m->ffn, (uint64_t)H, &L->fd, &L->tfd)) goto fail;
        if (L->recurrent) {
            if (matrix(m, NAME("attn_qkv.weight"), (uint64_t)H, (uint64_t)ch, &L->qkv, &L->tqkv) ||
                matrix(m, NAME("attn_gate.weight"), (uint64_t)H, (uint64_t)vd, &L->gate, &L->tgate) ||
                matrix(m, NAME("ssm_alpha.weight"), (uint64_t)H, (uint64_t)m->value_heads, &L->alpha, &L->talpha) ||
                matrix(m, NAME("ssm_beta.weight"), (uint64_t)H, (uint64_t)m->value_heads, &L->beta, &L->tbeta) ||
                matrix(m, NAME("ssm_out.weight"), (uint64_t)vd, (uint64_t)H, &L->out, &L->tout))
                goto fail;
            if (!(L->conv = param(m, NAME("ssm_conv1d.weight"), (uint64_t)ch * m->conv_width)) ||
                !(L->ssm_a = param(m, NAME("ssm_a"), (uint64_t)m->value_heads)) ||
                !(L->dt = param(m, NAME("ssm_dt.bias"), (uint64_t)m->value_heads)) ||
                !(L->ssm_norm = param(m, NAME("ssm_norm.weight"), (uint64_t)m->state_dim)))
                goto fail;
            m->state[l].conv = (float*)calloc((size_t)ch * m->conv_width, sizeof(float));
            m->state[l].rec = (float*)calloc((size_t)vd * m->state_dim, sizeof(float));
        } else {
            if (matrix(m, NAME("attn_q.weight"), (uint64_t)H, (uint64_t)qd, &L->q, &L->tq) ||
                matrix(m, NAME("attn_k.weight"), (uint64_t)H, (uint64_t)kvd, &L->k, &L->tk) ||
                matrix(m, NAME("attn_v.weight"), (uint64_t)H, (uint64_t)kvd, &L->v, &L->tv) ||
                matrix(m, NAME("attn_output.weight"), (uint64_t)m->heads * m->head_dim, (uint64_t)H, &L->o, &L->to))
                goto fail;
            if (!(L->q_norm = param(m, NAME("attn_q_norm.weight"), (uint64_t)m->head_dim)) ||
                !(L->k_norm = param(m, NAME("attn_k_norm.weight"), (uint64_t)m->head_dim)))
                goto fail;
            m->state[l].keys = (float*)malloc(context * (size_t)kvd * sizeof(float));
            m->state[l].values = (float*)malloc(context * (size_t)kvd * sizeof(float));
            if (!m->state[l].keys || !m->state[l].values) { set_err("Out of memory for KV cache"); goto fail; }
        }
    }
    {
        /* the MTP block, named after the last main layer index + 1 (blk.32 at the 9B
         * shape, the name model.cpp:378-392 uses) */
        const int l = m->layers;
        if (find_tensor(m, NAME("nextn.eh_proj.weight"))) {
            eo_layer* L = &m->mtp;
            if (matrix(m, NAME("nextn.eh_proj.weight"), 2 * (uint64_t)H, (uint64_t)H, &m->eh, &m->teh) ||
                !(m->enorm = param(m, NAME("nextn.enorm.weight"), (uint64_t)H)) ||
                !(m->hnorm = param(m, NAME("nextn.hnorm.weight"), (uint64_t)H)) ||
                !(m->head_norm = param(m, NAME("nextn.shared_head_norm.weight"), (uint64_t)H)) ||
                !(L->attn_norm = param(m, NAME("attn_norm.weight"), (uint64_t)H)) ||
                !(L->post_norm = param(m, NAME("post_attention_norm.weight"), (uint64_t)H)) ||
                !(L->q_norm = param(m, NAME("attn_q_norm.weight"), (uint64_t)m->head_dim)) ||
                !(L->k_norm = param(m, NAME("attn_k_norm.weight"), (uint64_t)m->head_dim)) ||
                matrix(m, NAME("attn_q.weight"), (uint64_t)H, (uint64_t)qd, &L->q, &L->tq) ||
                matrix(m, NAME("attn_k.weight"), (uint64_t)H, (uint64_t)kvd, &L->k, &L->tk) ||
                matrix(m, NAME("attn_v.weight"), (uint64_t)H, (uint64_t)kvd, &L->v, &L->tv) ||
                matrix(m, NAME("attn_output.weight"), (uint64_t)m->heads * m->head_dim, (uint64_t)H, &L->o, &L->to) ||
                matrix(m, NAME("ffn_gate.weight"), (uint64_t)H, (uint64_t)m->ffn, &L->fg, &L->tfg) ||
                matrix(m, NAME("ffn_up.weight"), (uint64_t)H, (uint64_t)m->ffn, &L->fu, &L->tfu) ||
                matrix(m, NAME("ffn_down.weight"), (uint64_t)m->ffn, (uint64_t)H, &L->fd, &L->tfd))
                goto fail;
            m->mtp_state.keys = (float*)malloc(context * (size_t)kvd * sizeof(float));
            m->mtp_state.values = (float*)malloc(context * (size_t)kvd * sizeof(float));
            m->mtp_hidden = (float*)calloc((size_t)H, sizeof(float));
            if (!m->mtp_state.keys || !m->mtp_state.values || !m->mtp_hidden) { set_err("Out of memory for MTP"); goto fail; }
            m->has_mtp = 1;
        }
    }
#undef NAME
    m->last_hidden = (float*)calloc((size_t)H, sizeof(float));
    return m;
fail:
    if (err && err_len) snprintf(err, err_len, "%s", g_err);
    eo_model_free(m);
    return NULL;
}

int eo_model_vocab(const eo_model* m) { return m->vocab; }
int eo_model_hidden(const eo_model* m) { return m->hidden; }

/* Model::reset (model.cpp:479): position 0, states cleared */
void eo_model_reset(eo_model* m) {
    m->position = 0;
    const int kd = m->key_heads * m->state_dim, vd = m->value_heads * m->state_dim, ch = 2 * kd + vd;
    for (int l = 0; l < m->layers; ++l) {
        if (m->state[l].conv) memset(m->state[l].conv, 0, (size_t)ch * m->conv_width * sizeof(float));
        if (m->state[l].rec) memset(m->state[l].rec, 0, (size_t)vd * m->state_dim * sizeof(float));
        m->state[l].length = 0;
    }
}

/* Timing aid (no reference counterpart): moves the model to `position` as if that many
 * positions had been evaluated, with zero K/V rows in the attention caches, so a timed
 * decode sample runs at the positions of a long prompt (attention over position + 1
 * rows) without evaluating the prompt. The recurrent states are left as they are. */
int eo_model_seek(eo_model* m, size_t position) {
    if (position >= m->context) { set_err("Context budget exhausted"); return -1; }
    const size_t kvd = (size_t)m->kv_heads * (size_t)m->head_dim;
    for (int l = 0; l < m->layers; ++l) {
        eo_layer_state* S = &m->state[l];
        if (!S->keys) continue;
        memset(S->keys, 0, position * kvd * sizeof(float));
        memset(S->values, 0, position * kvd * sizeof(float));
        S->length = position;
    }
    m->position = position;
    return 0;
}

static int linear(uint32_t type, const uint8_t* w, const float* x, size_t cols, float* y, size_t rows) {
    return eo_matvec(type, w, eo_encoded_bytes(type, cols * rows), x, cols, y, rows);
}

/* A projection of the model: with --fast-q8, Q6_K weights see the quantised input
 * (device_linear, cuda.cpp:707-712: every Q6_K projection, the output head included). */
static int mlinear(const eo_model* m, uint32_t type, const uint8_t* w, const float* x, size_t cols, float* y,
                   size_t rows) {
    if (!m->q8 || type != EO_Q6_K) return linear(type, w, x, cols, y, rows);
    float* xq = (float*)malloc(cols * sizeof(float));
    eo_quantize_q8(x, cols, xq);
    const int rc = linear(type, w, xq, cols, y, rows);
    free(xq);
    return rc;
}

/* Backend::feed_forward (backend.cpp:91-104) with the projections of mlinear. Without
 * --fast-q8 this is eo_feed_forward exactly. */
static int model_feed_forward(const eo_model* m, const eo_layer* L, const float* x, float* y) {
    const size_t H = (size_t)m->hidden, F = (size_t)m->ffn;
    if (!m->q8) return eo_feed_forward(L->tfg, L->fg, L->tfu, L->fu, L->tfd, L->fd, H, F, x, y);
    float* g = (float*)malloc(F * sizeof(float));
    float* u = (float*)malloc(F * sizeof(float));
    int rc = mlinear(m, L->tfg, L->fg, x, H, g, F);
    if (!rc) rc = mlinear(m, L->tfu, L->fu, x, H, u, F);
    if (!rc) {
        for (size_t i = 0; i < F; ++i) {
            const float e = expf(-fabsf(g[i]));
            const float s = g[i] >= 0 ? 1.f / (1.f + e) : e / (1.f + e);
            g[i] = g[i] * s * u[i];
        }
        rc = mlinear(m, L->tfd, L->fd, g, F, y, H);
    }
    free(g);
    free(u);
    return rc;
}

void eo_model_set_quantize_activations(eo_model* m, int on) { m->q8 = on != 0; }

void eo_model_set_trace(eo_model* m, eo_trace_fn fn, void* user) {
    m->trace = fn;
    m->trace_user = user;
}

/* model.cpp:118-120 */
static void trace_point(const eo_model* m, const char* name, int layer, const float* x, size_t n) {
    if (!m->trace) return;
    char full[64];
    if (layer >= 0) snprintf(full, sizeof full, "%s-%d", name, layer);
    else snprintf(full, sizeof full, "%s", name);
    m->trace(m->trace_user, (uint64_t)m->position, full, x, (uint64_t)n);
}

/* Model::Impl::evaluate (model.cpp:206-259) with the fused feed-forward default. */
int eo_model_evaluate(eo_model* m, int token, float* logits) {
    if (m->position >= m->context) { set_err("Context budget exhausted"); return -1; }
    if (token < 0 || token >= m->vocab) { set_err("Token ID"); return -1; }
    const int H = m->hidden;
    const int kd = m->key_heads * m->state_dim, vd = m->value_heads * m->state_dim, ch = 2 * kd + vd;
    const int qd = m->heads * m->head_dim * 2, kvd = m->kv_heads * m->head_dim;
    const size_t row_bytes = eo_encoded_bytes(m->tembd, (uint64_t)H);
    float* x = (float*)malloc((size_t)H * sizeof(float));
    float* nrm = (float*)malloc((size_t)H * sizeof(float));
    float* attn = (float*)malloc((size_t)H * sizeof(float));
    size_t big = (size_t)(ch > qd ? ch : qd);
    float* b0 = (float*)malloc(big * sizeof(float));
    float* b1 = (float*)malloc((size_t)(vd > kvd ? vd : kvd) * sizeof(float));
    float* b2 = (float*)malloc((size_t)(m->value_heads > kvd ? m->value_heads : kvd) * sizeof(float));
    float* b3 = (float*)malloc((size_t)m->value_heads * sizeof(float));
    float* b4 = (float*)malloc((size_t)(vd > m->heads * m->head_dim ? vd : m->heads * m->head_dim) * sizeof(float));
    int rc = eo_dequantize(m->tembd, m->embd + (size_t)token * row_bytes, row_bytes, x, (size_t)H);
    for (int l = 0; rc == 0 && l < m->layers; ++l) {
        eo_layer* L = &m->layer[l];
        eo_layer_state* S = &m->state[l];
        memcpy(nrm, x, (size_t)H * sizeof(float));
        eo_rms(nrm, (size_t)H, L->attn_norm, m->eps);
        trace_point(m, "attn_norm", l, nrm, (size_t)H);
        if (L->recurrent) {
            /* Backend::recurrent_block (backend.cpp:61-77) */
            if ((rc = mlinear(m, L->tqkv, L->qkv, nrm, (size_t)H, b0, (size_t)ch))) break;
            if ((rc = mlinear(m, L->tgate, L->gate, nrm, (size_t)H, b1, (size_t)vd))) break;
            if ((rc = mlinear(m, L->talpha, L->alpha, nrm, (size_t)H, b2, (size_t)m->value_heads))) break;
            if ((rc = mlinear(m, L->tbeta, L->beta, nrm, (size_t)H, b3, (size_t)m->value_heads))) break;
            eo_delta_net(m->key_heads, m->value_heads, m->state_dim, m->conv_width, m->eps, b0, b1, b2, b3,
                         L->conv, L->ssm_a, L->dt, L->ssm_norm, S->conv, S->rec, b4);
            if ((rc = mlinear(m, L->tout, L->out, b4, (size_t)vd, attn, (size_t)H))) break;
        } else {
            /* attention (model.cpp:161-164) */
            if ((rc = mlinear(m, L->tq, L->q, nrm, (size_t)H, b0, (size_t)qd))) break;
            if ((rc = mlinear(m, L->tk, L->k, nrm, (size_t)H, b1, (size_t)kvd))) break;
            if ((rc = mlinear(m, L->tv, L->v, nrm, (size_t)H, b2, (size_t)kvd))) break;
            S->length += 1;
            eo_attention(m->heads, m->kv_heads, m->head_dim, m->rotary, m->rope_base, m->eps, L->q_norm, L->k_norm,
                         b0, b1, b2, S->keys, S->values, S->length, (int)m->position, b4);
            if ((rc = mlinear(m, L->to, L->o, b4, (size_t)m->heads * m->head_dim, attn, (size_t)H))) break;
        }
        for (int i = 0; i < H; ++i) x[i] += attn[i];
        trace_point(m, "attn_residual", l, x, (size_t)H);
        memcpy(nrm, x, (size_t)H * sizeof(float));
        eo_rms(nrm, (size_t)H, L->post_norm, m->eps);
        if ((rc = model_feed_forward(m, L, nrm, attn))) break;
        for (int i = 0; i < H; ++i) x[i] += attn[i];
        trace_point(m, "l_out", l, x, (size_t)H);
    }
    if (rc == 0) {
        if (logits) {
            /* the hidden vectors are kept from positions with logits only (model.cpp:247-251) */
            memcpy(m->last_hidden, x, (size_t)H * sizeof(float));
            eo_rms(x, (size_t)H, m->output_norm, m->eps);
            trace_point(m, "result_norm", -1, x, (size_t)H);
            rc = mlinear(m, m->toutput, m->output, x, (size_t)H, logits, (size_t)m->vocab);
            if (rc == 0) trace_point(m, "logits", -1, logits, (size_t)m->vocab);
        }
        if (rc == 0) ++m->position;
    }
    free(x); free(nrm); free(attn); free(b0); free(b1); free(b2); free(b3); free(b4);
    return rc;
}

/* Projections of n positions at once: Y[p * rows + r] = row r of the matrix times
 * X[p * cols ...], each output the same single FP32 sum in element order as eo_matvec
 * (no fused multiply-add: -ffp-contract=off), so every value equals eo_matvec's bit for
 * bit. Positions advance together in tiles of EO_TILE: a weight block is decoded once
 * per tile, and the tile's sums are independent lanes the compiler can vectorise. */
#define EO_TILE 64
static int matmul_rows(uint32_t type, const uint8_t* w, const float* X, size_t n, size_t cols, float* Y,
                       size_t rows) {
    const uint64_t row_bytes = eo_encoded_bytes(type, cols);
    if (!cols || !row_bytes) { set_err("Matrix size mismatch"); return -1; }
    float* xt = (float*)malloc(cols * EO_TILE * sizeof(float));
    if (!xt) { set_err("Out of memory"); return -1; }
    const size_t es = type == EO_F32 ? 4 : 2;
    for (size_t p0 = 0; p0 < n; p0 += EO_TILE) {
        const size_t t = n - p0 < EO_TILE ? n - p0 : EO_TILE;
        for (size_t c = 0; c < cols; ++c)
            for (size_t q = 0; q < EO_TILE; ++q) xt[c * EO_TILE + q] = q < t ? X[(p0 + q) * cols + c] : 0.f;
        #pragma omp parallel for schedule(static)
        for (int64_t row = 0; row < (int64_t)rows; ++row) {
            const uint8_t* ptr = w + (uint64_t)row * row_bytes;
            float sum[EO_TILE];
            float block[256];
            for (int q = 0; q < EO_TILE; ++q) sum[q] = 0.f;
            for (size_t k = 0; k < cols; k += 256) {
                const size_t len = cols - k < 256 ? cols - k : 256;
                if (type == EO_Q6_K) q6_block(ptr + k / 256 * 210, block);
                else if (type == EO_Q4_K) q4_k_block(ptr + k / 256 * 144, block);
                else for (size_t j = 0; j < len; ++j) block[j] = raw_element(type, ptr + (k + j) * es);
                for (size_t j = 0; j < len; ++j) {
                    const float wj = block[j];
                    const float* xr = xt + (k + j) * EO_TILE;
                    for (int q = 0; q < EO_TILE; ++q) sum[q] += wj * xr[q];
                }
            }
            for (size_t q = 0; q < t; ++q) Y[(p0 + q) * rows + (size_t)row] = sum[q];
        }
    }
    free(xt);
    return 0;
}

/* matmul_rows with mlinear's --fast-q8 rule applied to each position's input. */
static int model_matmul(const eo_model* m, uint32_t type, const uint8_t* w, const float* X, size_t n, size_t cols,
                        float* Y, size_t rows) {
    if (!m->q8 || type != EO_Q6_K) return matmul_rows(type, w, X, n, cols, Y, rows);
    float* xq = (float*)malloc(n * cols * sizeof(float));
    if (!xq) { set_err("Out of memory"); return -1; }
    for (size_t p = 0; p < n; ++p) eo_quantize_q8(X + p * cols, cols, xq + p * cols);
    const int rc = matmul_rows(type, w, xq, n, cols, Y, rows);
    free(xq);
    return rc;
}

/* n positions from the current one, with the same bits as n calls of eo_model_evaluate
 * (the reference's chunked prefill, model.cpp:355-366, whose CPU-backend projections are
 * per-position loops, backend.cpp:81-90): every projection of the n positions runs as
 * one matmul_rows, the recurrent and attention steps run position by position in order.
 * logits (optional) are the last position's. Test and fixture generation aid. */
int eo_model_evaluate_many(eo_model* m, const int* tokens, size_t n, float* logits) {
    if (!n) { set_err("Empty token list"); return -1; }
    if (m->position >= m->context || n > m->context - m->position) { set_err("Context budget exhausted"); return -1; }
    for (size_t p = 0; p < n; ++p)
        if (tokens[p] < 0 || tokens[p] >= m->vocab) { set_err("Token ID"); return -1; }
    const size_t H = (size_t)m->hidden, F = (size_t)m->ffn, vh = (size_t)m->value_heads;
    const size_t kd = (size_t)m->key_heads * m->state_dim, vd = vh * m->state_dim, ch = 2 * kd + vd;
    const size_t qd = (size_t)m->heads * m->head_dim * 2, kvd = (size_t)m->kv_heads * m->head_dim;
    const size_t ad = (size_t)m->heads * m->head_dim;
    const size_t w0 = ch > qd ? ch : qd, w1 = vd > kvd ? vd : kvd, w2 = vh > kvd ? vh : kvd, w4 = vd > ad ? vd : ad;
    const size_t row_bytes = eo_encoded_bytes(m->tembd, H);
    float* x = (float*)malloc(n * H * sizeof(float));
    float* nrm = (float*)malloc(n * H * sizeof(float));
    float* attn = (float*)malloc(n * H * sizeof(float));
    float* b0 = (float*)malloc(n * w0 * sizeof(float));
    float* b1 = (float*)malloc(n * w1 * sizeof(float));
    float* b2 = (float*)malloc(n * w2 * sizeof(float));
    float* b3 = (float*)malloc(n * vh * sizeof(float));
    float* b4 = (float*)malloc(n * w4 * sizeof(float));
    float* g = (float*)malloc(n * F * sizeof(float));
    float* u = (float*)malloc(n * F * sizeof(float));
    int rc = 0;
    if (!x || !nrm || !attn || !b0 || !b1 || !b2 || !b3 || !b4 || !g || !u) { set_err("Out of memory"); rc = -1; }
    for (size_t p = 0; rc == 0 && p < n; ++p)
        rc = eo_dequantize(m->tembd, m->embd + (size_t)tokens[p] * row_bytes, row_bytes, x + p * H, H);
    for (int l = 0; rc == 0 && l < m->layers; ++l) {
        eo_layer* L = &m->layer[l];
        eo_layer_state* S = &m->state[l];
        memcpy(nrm, x, n * H * sizeof(float));
        for (size_t p = 0; p < n; ++p) eo_rms(nrm + p * H, H, L->attn_norm, m->eps);
        if (L->recurrent) {
            if ((rc = model_matmul(m, L->tqkv, L->qkv, nrm, n, H, b0, ch))) break;
            if ((rc = model_matmul(m, L->tgate, L->gate, nrm, n, H, b1, vd))) break;
            if ((rc = model_matmul(m, L->talpha, L->alpha, nrm, n, H, b2, vh))) break;
            if ((rc = model_matmul(m, L->tbeta, L->beta, nrm, n, H, b3, vh))) break;
            for (size_t p = 0; p < n; ++p)
                eo_delta_net(m->key_heads, m->value_heads, m->state_dim, m->conv_width, m->eps, b0 + p * ch,
                             b1 + p * vd, b2 + p * vh, b3 + p * vh, L->conv, L->ssm_a, L->dt, L->ssm_norm, S->conv,
                             S->rec, b4 + p * vd);
            if ((rc = model_matmul(m, L->tout, L->out, b4, n, vd, attn, H))) break;
        } else {
            if ((rc = model_matmul(m, L->tq, L->q, nrm, n, H, b0, qd))) break;
            if ((rc = model_matmul(m, L->tk, L->k, nrm, n, H, b1, kvd))) break;
            if ((rc = model_matmul(m, L->tv, L->v, nrm, n, H, b2, kvd))) break;
            for (size_t p = 0; p < n; ++p) {
                S->length += 1;
                eo_attention(m->heads, m->kv_heads, m->head_dim, m->rotary, m->rope_base, m->eps, L->q_norm,
                             L->k_norm, b0 + p * qd, b1 + p * kvd, b2 + p * kvd, S->keys, S->values, S->length,
                             (int)(m->position + p), b4 + p * ad);
            }
            if ((rc = model_matmul(m, L->to, L->o, b4, n, ad, attn, H))) break;
        }
        for (size_t i = 0; i < n * H; ++i) x[i] += attn[i];
        memcpy(nrm, x, n * H * sizeof(float));
        for (size_t p = 0; p < n; ++p) eo_rms(nrm + p * H, H, L->post_norm, m->eps);
        /* model_feed_forward / eo_feed_forward over the n positions */
        if ((rc = model_matmul(m, L->tfg, L->fg, nrm, n, H, g, F))) break;
        if ((rc = model_matmul(m, L->tfu, L->fu, nrm, n, H, u, F))) break;
        for (size_t i = 0; i < n * F; ++i) {
            const float e = expf(-fabsf(g[i]));
            const float s = g[i] >= 0 ? 1.f / (1.f + e) : e / (1.f + e);
            g[i] = g[i] * s * u[i];
        }
        if ((rc = model_matmul(m, L->tfd, L->fd, g, n, F, attn, H))) break;
        for (size_t i = 0; i < n * H; ++i) x[i] += attn[i];
    }
    if (rc == 0) {
        float* last = x + (n - 1) * H;
        if (logits) {
            memcpy(m->last_hidden, last, H * sizeof(float));
            eo_rms(last, H, m->output_norm, m->eps);
            rc = mlinear(m, m->toutput, m->output, last, H, logits, (size_t)m->vocab);
        }
        if (rc == 0) m->position += n;
    }
    free(x); free(nrm); free(attn); free(b0); free(b1); free(b2); free(b3); free(b4); free(g); free(u);
    return rc;
}

int eo_model_has_mtp(const eo_model* m) { return m->has_mtp; }

/* Model::reset_mtp (model.cpp:487): the MTP block's attention cache emptied */
void eo_model_reset_mtp(eo_model* m) { m->mtp_state.length = 0; }

/* Model::Impl::mtp_step (model.cpp:376-397): the next-n draft head. From the caller's
 * hidden vector and token: [enorm(embed(token)) | hnorm(hidden)] through eh_proj, one
 * attention block (the main attention's arithmetic at rotary position `pos`, over the
 * block's own cache, which grows by one row per call), the unfused SwiGLU FFN, then the
 * shared head norm and the output head. The block's output before the head norm is kept
 * (Model::mtp_hidden). Projections follow mlinear (--fast-q8 as the main path). */
int eo_model_mtp_draft(eo_model* m, const float* hidden, int token, size_t pos, float* logits) {
    if (!m->has_mtp) { set_err("The model has no MTP (nextn) block"); return -1; }
    if (token < 0 || token >= m->vocab) { set_err("Token ID"); return -1; }
    if (m->mtp_state.length >= m->context) { set_err("MTP context budget exhausted"); return -1; }
    const size_t H = (size_t)m->hidden, F = (size_t)m->ffn, kvd = (size_t)m->kv_heads * m->head_dim;
    const size_t qd = (size_t)m->heads * m->head_dim * 2, ad = (size_t)m->heads * m->head_dim;
    const eo_layer* L = &m->mtp;
    const size_t row_bytes = eo_encoded_bytes(m->tembd, H);
    float* cat = (float*)malloc(2 * H * sizeof(float));
    float* cur = (float*)malloc(H * sizeof(float));
    float* nrm = (float*)malloc(H * sizeof(float));
    float* t = (float*)malloc(H * sizeof(float));
    float* q = (float*)malloc(qd * sizeof(float));
    float* k = (float*)malloc(kvd * sizeof(float));
    float* v = (float*)malloc(kvd * sizeof(float));
    float* ao = (float*)malloc(ad * sizeof(float));
    float* g = (float*)malloc(F * sizeof(float));
    float* u = (float*)malloc(F * sizeof(float));
    int rc = eo_dequantize(m->tembd, m->embd + (size_t)token * row_bytes, row_bytes, cat, H);
    if (!rc) {
        eo_rms(cat, H, m->enorm, m->eps);
        memcpy(cat + H, hidden, H * sizeof(float));
        eo_rms(cat + H, H, m->hnorm, m->eps);
        rc = mlinear(m, m->teh, m->eh, cat, 2 * H, cur, H);
    }
    if (!rc) {
        memcpy(nrm, cur, H * sizeof(float));
        eo_rms(nrm, H, L->attn_norm, m->eps);
        rc = mlinear(m, L->tq, L->q, nrm, H, q, qd);
        if (!rc) rc = mlinear(m, L->tk, L->k, nrm, H, k, kvd);
        if (!rc) rc = mlinear(m, L->tv, L->v, nrm, H, v, kvd);
    }
    if (!rc) {
        m->mtp_state.length += 1;
        eo_attention(m->heads, m->kv_heads, m->head_dim, m->rotary, m->rope_base, m->eps, L->q_norm, L->k_norm, q, k,
                     v, m->mtp_state.keys, m->mtp_state.values, m->mtp_state.length, (int)pos, ao);
        rc = mlinear(m, L->to, L->o, ao, ad, t, H);
    }
    if (!rc) {
        for (size_t i = 0; i < H; ++i) cur[i] += t[i];
        memcpy(nrm, cur, H * sizeof(float));
        eo_rms(nrm, H, L->post_norm, m->eps);
        rc = mlinear(m, L->tfg, L->fg, nrm, H, g, F);
        if (!rc) rc = mlinear(m, L->tfu, L->fu, nrm, H, u, F);
    }
    if (!rc) {
        for (size_t i = 0; i < F; ++i) g[i] = eo_silu(g[i]) * u[i];
        rc = mlinear(m, L->tfd, L->fd, g, F, t, H);
    }
    if (!rc) {
        for (size_t i = 0; i < H; ++i) cur[i] += t[i];
        memcpy(m->mtp_hidden, cur, H * sizeof(float));
        eo_rms(cur, H, m->head_norm, m->eps);
        if (logits) rc = mlinear(m, m->toutput, m->output, cur, H, logits, (size_t)m->vocab);
    }
    free(cat); free(cur); free(nrm); free(t); free(q); free(k); free(v); free(ao); free(g); free(u);
    return rc;
}

int eo_model_mtp_hidden(const eo_model* m, float* out) {
    if (!m->has_mtp) { set_err("The model has no MTP (nextn) block"); return -1; }
    memcpy(out, m->mtp_hidden, (size_t)m->hidden * sizeof(float));
    return 0;
}

/* Model::last_hidden (model.cpp:483): the last residual through the output norm, the
 * vector the output head multiplies (evaluate's hidden_out, model.cpp:248-251). */
int eo_model_last_hidden_normed(const eo_model* m, float* out) {
    memcpy(out, m->last_hidden, (size_t)m->hidden * sizeof(float));
    eo_rms(out, (size_t)m->hidden, m->output_norm, m->eps);
    return 0;
}

int eo_model_last_hidden(const eo_model* m, float* out) {
    memcpy(out, m->last_hidden, (size_t)m->hidden * sizeof(float));
    return 0;
}

/* std::max_element: the first maximum wins (model.cpp:499) */
static int argmax_first(const float* v, int n, float* margin) {
    int best = 0;
    for (int i = 1; i < n; ++i)
        if (v[best] < v[i]) best = i;
    if (margin) {
        float second = -INFINITY;
        for (int i = 0; i < n; ++i)
            if (i != best && v[i] > second) second = v[i];
        *margin = v[best] - second;
    }
    return best;
}

/* Model::generate (model.cpp:488-503). The reference prefills in chunks of four
 * (model.cpp:355-366); on the CPU backend a chunk's batched projection is a loop of
 * single-token projections (backend.cpp:81-90), so position-by-position evaluation
 * produces the same bits. */
int eo_model_generate(eo_model* m, const int* prompt, size_t prompt_len, size_t count, int* tokens, float* margins) {
    if (!prompt_len) { set_err("Empty prompt"); return -1; }
    if (prompt_len > m->context || count > m->context - prompt_len) { set_err("Prompt plus output exceeds context budget"); return -1; }
    eo_model_reset(m);
    if (!count) return 0;
    float* logits = (float*)malloc((size_t)m->vocab * sizeof(float));
    for (size_t i = 0; i < prompt_len; ++i)
        if (eo_model_evaluate(m, prompt[i], i + 1 == prompt_len ? logits : NULL)) { free(logits); return -1; }
    int emitted = 0;
    for (size_t i = 0; i < count; ++i) {
        float margin;
        const int token = argmax_first(logits, m->vocab, &margin);
        if (token == m->eos) break;
        tokens[emitted] = token;
        if (margins) margins[emitted] = margin;
        ++emitted;
        if (i + 1 < count && eo_model_evaluate(m, token, logits)) { free(logits); return -1; }
    }
    free(logits);
    return emitted;
}
