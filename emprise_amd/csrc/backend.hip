// C ABI of the gfx950 decode backend (include/emprise_hip.h). Stands in for the
// reference's CUDA backend (src/cuda.cpp:599-1130) behind emprise::Backend.
#include "../../include/emprise_hip.h"
#include "common.hpp"
#include "kernels.hpp"
#include "layout.hpp"

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <set>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

using namespace emprise;

thread_local TraceBracket emprise::g_trace_bracket;

namespace {

thread_local std::string g_error;

emprise_status fail(emprise_status s, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return s;
}

#define HIP_TRY(expr)                                                                                  \
    do {                                                                                               \
        hipError_t e_ = (expr);                                                                        \
        if (e_ != hipSuccess) return fail(EMPRISE_EDEVICE, "%s: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

#define TRY(expr)                          \
    do {                                   \
        emprise_status s_ = (expr);        \
        if (s_ != EMPRISE_OK) return s_;   \
    } while (0)

struct Weight {
    uint32_t type = 0;
    uint64_t cols = 0, rows = 0;
    uint8_t* dev = nullptr;
    size_t bytes = 0;
};

bool supported_type(uint32_t t) { return t == kF32 || t == kF16 || t == kBF16 || t == kQ6K || t == kQ4K; }

// Runs f(begin, end) over [0, n) on up to `threads` host threads.
template <class F> void parallel_rows(uint64_t n, F f) {
    unsigned threads = std::max(1u, std::min(32u, std::thread::hardware_concurrency()));
    if (n < 64) threads = 1;
    std::vector<std::thread> pool;
    const uint64_t per = (n + threads - 1) / threads;
    for (unsigned t = 0; t < threads; ++t) {
        const uint64_t b = t * per, e = std::min(n, b + per);
        if (b >= e) break;
        pool.emplace_back([=] { f(b, e); });
    }
    for (auto& th : pool) th.join();
}

// Upload slab size: large enough for whole rows of every shape here (a 12288-wide Q6_K row
// is 10 KiB), small enough that copying the next slab into pinned memory overlaps the
// DMA and re-layout of the previous one.
constexpr uint64_t kUploadSlab = 16ull << 20;

// dst <- src, n bytes, on the host threads (the source is the GGUF memory map)
void parallel_copy(uint8_t* dst, const uint8_t* src, uint64_t n) {
    constexpr uint64_t piece = 256 << 10;
    parallel_rows((n + piece - 1) / piece, [&](uint64_t b, uint64_t e) {
        const uint64_t lo = b * piece, hi = std::min(n, e * piece);
        if (lo < hi) std::memcpy(dst + lo, src + lo, hi - lo);
    });
}

}  // namespace

// Scratch of emprise_hip_delta_net_noalloc: the conv'd channels of one GDN step, in a
// fixed device array instead of library-allocated memory. 65536 floats (256 KiB) cover
// (2*key_heads + value_heads)*state_dim up to 65536 (the 9B shape has 8192). Each GPU
// the library runs on holds its own copy until the process ends; host code reaches it
// only through the address hipGetSymbolAddress returns for the current device.
constexpr int kNoAllocScratchFloats = 65536;
static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

struct emprise_hip {
    int device = 0;
    float* noalloc_scratch = nullptr;  // this device's address of `scratch`
    // weight upload pipeline: two pinned host slabs and two device slabs, used in turn;
    // done[k] is recorded after slab k's copy and re-layout, so the host waits on it
    // before filling host slab k again
    struct Upload {
        uint8_t* host[2] = {nullptr, nullptr};
        uint8_t* dev[2] = {nullptr, nullptr};
        hipEvent_t done[2] = {nullptr, nullptr};
        uint64_t next = 0;
    } upload;
    hipStream_t stream = nullptr;
    uint64_t budget = 0, used = 0;
    bool q8 = false;
    bool capturing = false;
    std::string name;
    std::unordered_map<uint64_t, Weight> weights;
    uint64_t next_weight = 1;
    std::unordered_map<uint64_t, hipGraphExec_t> graphs;
    uint64_t next_graph = 1;
    std::vector<hipEvent_t> events;
    // scratch buffers, grown outside graph capture only
    struct Scratch {
        void* ptr = nullptr;
        size_t bytes = 0;
    };
    std::unordered_map<std::string, Scratch> scratch;
    std::set<std::string> rope_ready;  // RoPE tables (scratch keys) already filled
    // kernel trace (emprise_hip_trace_begin/end)
    struct TraceRec {
        const char* kernel;
        uint64_t bytes;
        hipEvent_t a, b;
    };
    bool tracing = false;
    std::vector<TraceRec> trace;
    std::vector<hipEvent_t> trace_pool;
    size_t trace_used = 0;

    hipEvent_t trace_event() {
        if (trace_used == trace_pool.size()) {
            hipEvent_t e = nullptr;
            if (hipEventCreate(&e) != hipSuccess) return nullptr;
            trace_pool.push_back(e);
        }
        return trace_pool[trace_used++];
    }

    const Weight* weight(uint64_t id) const {
        auto it = weights.find(id);
        return it == weights.end() ? nullptr : &it->second;
    }
    emprise_status get_scratch(const char* key, size_t bytes, void** out, bool zero = false) {
        Scratch& s = scratch[key];
        if (s.bytes < bytes) {
            if (capturing) return fail(EMPRISE_ESTATE, "scratch '%s' must be sized before graph capture", key);
            if (s.ptr) HIP_TRY(hipFree(s.ptr));
            s.ptr = nullptr;
            s.bytes = 0;
            HIP_TRY(hipMalloc(&s.ptr, bytes));
            if (zero) HIP_TRY(hipMemset(s.ptr, 0, bytes));
            s.bytes = bytes;
        }
        *out = s.ptr;
        return EMPRISE_OK;
    }
};

namespace {

emprise_status launched(hipError_t e) {
    if (e != hipSuccess) return fail(EMPRISE_EDEVICE, "kernel launch: %s", hipGetErrorString(e));
    return EMPRISE_OK;
}

// Launches through `launch`; while tracing, the launch's kernels carry a start/stop
// event pair on their dispatch packets and the op's algorithmic bytes are recorded.
template <class F> emprise_status traced(emprise_hip* h, const char* kernel, uint64_t bytes, F launch) {
    if (!h->tracing) return launched(launch());
    hipEvent_t a = h->trace_event(), b = h->trace_event();
    if (!a || !b) return fail(EMPRISE_EDEVICE, "trace event");
    g_trace_bracket = {a, b};
    const hipError_t e = launch();
    const bool started = g_trace_bracket.start == nullptr;  // at least one kernel took the bracket
    g_trace_bracket = {};
    TRY(launched(e));
    if (!started) return fail(EMPRISE_EDEVICE, "traced op '%s' launched no kernel", kernel);
    h->trace.push_back({kernel, bytes, a, b});
    return EMPRISE_OK;
}

const char* matvec_name(uint32_t type, bool q8) {
    switch (type) {
    case kQ6K: return q8 ? "matvec_q6_k_q8" : "matvec_q6_k";
    case kQ4K: return "matvec_q4_k";
    case kF32: return "matvec_f32";
    case kF16: return "matvec_f16";
    default: return "matvec_bf16";
    }
}

// GDN step: the state is read and written once; q/k/v, gate, alpha, beta read; output written.
uint64_t gdn_bytes(const GdnArgs& g) {
    const uint64_t sd = (uint64_t)g.state_dim, vh = (uint64_t)g.value_heads, kh = (uint64_t)g.key_heads;
    return 2 * vh * sd * sd * 4 + (2 * kh * sd + vh * sd) * 4 + vh * sd * 4 * 2 + vh * 8;
}

bool is_matrix(const Weight* w) { return w && w->rows >= 1 && w->cols >= 1; }

// Grouped matvec over weights with one input; splits the list into runs of equal type.
struct Proj {
    const Weight* w;
    float* y;
    bool silu = false;  // store SiLU(row) (MvArgs::silu_mask)
};

// Per-head input transform of a projection (the GDN output gate): input = rms over each
// head_dim slice of x, times norm[0..head_dim), times SiLU(gate).
struct HeadGate {
    const float* gate;
    const float* norm;
    int head_dim;
    float eps;
};

emprise_status run_matvec(emprise_hip* h, const Proj* p, int n, int mode, const emprise_hip_input* in,
                          const float* x_plain, const float* conv_w, float* conv_state, int conv_width,
                          unsigned long long* argmax_key, const HeadGate* hg = nullptr) {
    if (n < 1 || n > kMaxSeg) return fail(EMPRISE_EINVAL, "between 1 and %d projections per call", kMaxSeg);
    const uint64_t cols = p[0].w->cols;
    for (int i = 0; i < n; ++i)
        if (p[i].w->cols != cols) return fail(EMPRISE_EINVAL, "projections sharing an input need equal columns");
    if (cols > 12288 + 4096) return fail(EMPRISE_EINVAL, "input width %llu exceeds the staged-input limit", (unsigned long long)cols);
    bool first = true;
    for (int i = 0; i < n;) {
        int j = i + 1;
        if (mode != kMvSwiglu)
            while (j < n && p[j].w->type == p[i].w->type) ++j;
        else
            j = n;
        const uint32_t type = p[i].w->type;
        MvArgs a{};
        a.nseg = j - i;
        a.cols = (int)cols;
        a.mode = mode;
        int g = 0;
        uint64_t total_rows = 0;
        for (int s = 0; s < a.nseg; ++s)
            if (!(mode == kMvSwiglu && s == 1)) total_rows += p[i + s].w->rows;
        const int R = matvec_rows_per_group(type, cols, mode, total_rows);
        a.rows_per_group = R;
        for (int s = 0; s < a.nseg; ++s) {
            const Weight* w = p[i + s].w;
            a.seg[s].w = w->dev;
            a.seg[s].y = p[i + s].y;
            if (p[i + s].silu) a.silu_mask |= 1 << s;
            a.seg[s].rows = (int)w->rows;
            a.seg[s].g0 = g;
            if (mode == kMvSwiglu && s == 1) a.seg[s].g0 = 0x7fffffff;
            else g += (int)((w->rows + R - 1) / R);
        }
        a.groups = g;
        if (in) {
            a.x = reinterpret_cast<const float*>(in->x);
            a.delta = reinterpret_cast<const float*>(in->delta);
            a.x_out = first ? reinterpret_cast<float*>(in->x_out) : nullptr;
            if (in->norm) {
                const Weight* nw = h->weight(in->norm);
                if (!nw || nw->type != kF32 || nw->rows * nw->cols != cols)
                    return fail(EMPRISE_EINVAL, "norm weight must be F32 with %llu elements", (unsigned long long)cols);
                a.norm = reinterpret_cast<const float*>(nw->dev);
            }
            a.eps = in->eps;
        } else {
            a.x = x_plain;
        }
        if (hg) {
            a.gate = hg->gate;
            a.norm = hg->norm;
            a.head_dim = hg->head_dim;
            a.eps = hg->eps;
        }
        if (first && conv_w) {
            a.conv_w = conv_w;
            a.conv_state = conv_state;
            a.conv_width = conv_width;
        }
        a.argmax = argmax_key;
        const bool q8 = h->q8 && type == kQ6K;
        // algorithmic bytes: encoded weights + the input read (x, delta, norm) + outputs
        uint64_t bytes = cols * 4 * (1 + (a.delta ? 1 : 0) + (a.gate ? 1 : 0) + (a.x_out ? 1 : 0)) +
                         (a.norm ? (a.gate ? (uint64_t)a.head_dim : cols) * 4 : 0);
        for (int s = 0; s < a.nseg; ++s) bytes += p[i + s].w->bytes + (uint64_t)a.seg[s].rows * 4;
        if (a.conv_w) bytes += (uint64_t)a.seg[0].rows * a.conv_width * 4 * 3;
        TRY(traced(h, matvec_name(type, q8), bytes, [&] { return launch_matvec(type, q8, a, 2048, h->stream); }));
        first = false;
        i = j;
    }
    return EMPRISE_OK;
}

emprise_status check_weights(emprise_hip* h, int n, const emprise_weight* ids, const Weight** out) {
    for (int i = 0; i < n; ++i) {
        out[i] = h->weight(ids[i]);
        if (!is_matrix(out[i])) return fail(EMPRISE_EINVAL, "unknown weight handle %llu", (unsigned long long)ids[i]);
    }
    return EMPRISE_OK;
}

}  // namespace

extern "C" {

const char* emprise_hip_last_error(void) { return g_error.c_str(); }

emprise_status emprise_hip_create(int device, uint64_t weight_budget, int quantize_activations, emprise_hip** out) {
    if (!out) return fail(EMPRISE_EINVAL, "null output");
    *out = nullptr;
    int count = 0;
    HIP_TRY(hipGetDeviceCount(&count));
    if (device < 0 || device >= count) return fail(EMPRISE_EINVAL, "no HIP device %d (%d present)", device, count);
    HIP_TRY(hipSetDevice(device));
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(EMPRISE_EDEVICE, "built for gfx950, found %s", prop.gcnArchName);
    // the no-alloc entry point's scratch: this device's copy of the array
    void* scratch_addr = nullptr;
    const hipError_t se = hipGetSymbolAddress(&scratch_addr, HIP_SYMBOL(scratch));
    if (se != hipSuccess || !scratch_addr)
        return fail(EMPRISE_EDEVICE, "scratch symbol address: %s", hipGetErrorString(se));
    auto* h = new emprise_hip();
    h->device = device;
    h->noalloc_scratch = static_cast<float*>(scratch_addr);
    h->q8 = quantize_activations != 0;
    hipError_t e = hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete h;
        return fail(EMPRISE_EDEVICE, "stream: %s", hipGetErrorString(e));
    }
    size_t free_b = 0, total_b = 0;
    (void)hipMemGetInfo(&free_b, &total_b);
    const uint64_t reserve = 512ull << 20;
    h->budget = weight_budget ? weight_budget : (free_b > reserve ? free_b - reserve : 0);
    h->name = std::string("HIP ") + prop.gcnArchName + (h->q8 ? " Q8 activations" : " FP32 accumulation");
    const size_t colon = h->name.find(':');
    if (colon != std::string::npos) h->name = h->name.substr(0, colon) + (h->q8 ? " Q8 activations" : " FP32 accumulation");
    *out = h;
    return EMPRISE_OK;
}

void emprise_hip_destroy(emprise_hip* h) {
    if (!h) return;
    (void)hipSetDevice(h->device);
    (void)hipStreamSynchronize(h->stream);
    for (auto& kv : h->graphs) (void)hipGraphExecDestroy(kv.second);
    for (auto& kv : h->weights) (void)hipFree(kv.second.dev);
    for (auto& kv : h->scratch) (void)hipFree(kv.second.ptr);
    for (int k = 0; k < 2; ++k) {
        if (h->upload.host[k]) (void)hipHostFree(h->upload.host[k]);
        if (h->upload.dev[k]) (void)hipFree(h->upload.dev[k]);
        if (h->upload.done[k]) (void)hipEventDestroy(h->upload.done[k]);
    }
    for (auto& ev : h->events) (void)hipEventDestroy(ev);
    (void)hipStreamDestroy(h->stream);
    delete h;
}

const char* emprise_hip_name(const emprise_hip* h) { return h ? h->name.c_str() : ""; }
uint64_t emprise_hip_capacity(const emprise_hip* h) { return h ? h->budget : 0; }
uint64_t emprise_hip_weight_bytes(const emprise_hip* h) { return h ? h->used : 0; }

emprise_status emprise_hip_alloc(emprise_hip* h, size_t bytes, emprise_dev* out) {
    if (!h || !out) return fail(EMPRISE_EINVAL, "null argument");
    if (h->capturing) return fail(EMPRISE_ESTATE, "allocation during graph capture");
    void* p = nullptr;
    HIP_TRY(hipMalloc(&p, bytes ? bytes : 4));
    *out = reinterpret_cast<emprise_dev>(p);
    return EMPRISE_OK;
}

emprise_status emprise_hip_free(emprise_hip* h, emprise_dev buffer) {
    if (!h) return fail(EMPRISE_EINVAL, "null backend");
    if (!buffer) return EMPRISE_OK;
    HIP_TRY(hipStreamSynchronize(h->stream));
    HIP_TRY(hipFree(reinterpret_cast<void*>(buffer)));
    return EMPRISE_OK;
}

emprise_status emprise_hip_upload(emprise_hip* h, emprise_dev dst, const void* src, size_t bytes) {
    if (!h || (!dst && bytes) || (!src && bytes)) return fail(EMPRISE_EINVAL, "null argument");
    if (h->capturing) return fail(EMPRISE_ESTATE, "upload during graph capture");
    HIP_TRY(hipMemcpyAsync(reinterpret_cast<void*>(dst), src, bytes, hipMemcpyHostToDevice, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return EMPRISE_OK;
}

emprise_status emprise_hip_download(emprise_hip* h, void* dst, emprise_dev src, size_t bytes) {
    if (!h || (!dst && bytes) || (!src && bytes)) return fail(EMPRISE_EINVAL, "null argument");
    if (h->capturing) return fail(EMPRISE_ESTATE, "download during graph capture");
    HIP_TRY(hipMemcpyAsync(dst, reinterpret_cast<const void*>(src), bytes, hipMemcpyDeviceToHost, h->stream));
    HIP_TRY(hipStreamSynchronize(h->stream));
    return EMPRISE_OK;
}

emprise_status emprise_hip_fill(emprise_hip* h, emprise_dev dst, float value, size_t n) {
    if (!h || (!dst && n)) return fail(EMPRISE_EINVAL, "null argument");
    if (!n) return EMPRISE_OK;
    return traced(h, "fill", n * 4, [&] { return launch_fill(reinterpret_cast<float*>(dst), value, n, h->stream); });
}

emprise_status emprise_hip_stream_read(emprise_hip* h, emprise_dev src, uint64_t bytes, emprise_dev sink) {
    if (!h || !src || !sink) return fail(EMPRISE_EINVAL, "null argument");
    if (!bytes || bytes % 4096) return fail(EMPRISE_EINVAL, "stream_read: bytes must be a positive multiple of 4 KiB");
    return traced(h, "stream_read", bytes, [&] {
        return launch_stream_read(reinterpret_cast<const void*>(src), bytes, reinterpret_cast<uint32_t*>(sink), h->stream);
    });
}

emprise_status emprise_hip_upload_weight(emprise_hip* h, uint32_t type, uint64_t cols, uint64_t rows, const void* data,
                                         size_t len, emprise_weight* out) {
    if (!h || !data || !out) return fail(EMPRISE_EINVAL, "null argument");
    if (h->capturing) return fail(EMPRISE_ESTATE, "weight upload during graph capture");
    if (!supported_type(type)) return fail(EMPRISE_EINVAL, "unsupported GGUF tensor encoding: %u", type);
    if (!cols || !rows) return fail(EMPRISE_EINVAL, "zero tensor dimension");
    if ((type == kQ6K || type == kQ4K) && cols % 256)
        return fail(EMPRISE_EINVAL, "%s row must contain whole blocks", type == kQ6K ? "Q6_K" : "Q4_K");
    if (rows > UINT64_MAX / cols) return fail(EMPRISE_EINVAL, "dimension overflow");
    const uint64_t bytes = encoded_bytes(type, cols * rows);
    if (!bytes || bytes != len) return fail(EMPRISE_EINVAL, "Incorrect encoded size: %zu for %llu x %llu", len,
                                            (unsigned long long)rows, (unsigned long long)cols);
    if (bytes > h->budget - std::min(h->budget, h->used))
        return fail(EMPRISE_ENOMEM, "weight budget exceeded (%llu + %llu > %llu)", (unsigned long long)h->used,
                    (unsigned long long)bytes, (unsigned long long)h->budget);
    HIP_TRY(hipSetDevice(h->device));
    Weight w;
    w.type = type;
    w.cols = cols;
    w.rows = rows;
    w.bytes = bytes;
    HIP_TRY(hipMalloc(&w.dev, bytes));
    const uint8_t* src = static_cast<const uint8_t*>(data);
    hipError_t err = hipSuccess;
    const bool blocked = type == kQ6K || type == kQ4K;
    const uint64_t row_bytes = blocked ? cols / 256 * type_block_bytes(type) : cols * (type == kF32 ? 4 : 2);
    // Raw GGUF bytes go through two pinned slabs in turn: the host threads copy slab i
    // from the memory map while slab i-1's DMA and re-layout run on the stream. Block
    // encodings are re-laid out on the device (launch_repack), whole rows per slab.
    if (row_bytes <= kUploadSlab) {
        auto& up = h->upload;
        for (int k = 0; k < 2 && err == hipSuccess; ++k) {
            if (!up.host[k]) err = hipHostMalloc(reinterpret_cast<void**>(&up.host[k]), kUploadSlab, hipHostMallocDefault);
            if (err == hipSuccess && !up.dev[k]) err = hipMalloc(&up.dev[k], kUploadSlab);
            if (err == hipSuccess && !up.done[k]) err = hipEventCreateWithFlags(&up.done[k], hipEventDisableTiming);
        }
        const uint64_t slab_rows = kUploadSlab / row_bytes;
        for (uint64_t r0 = 0; r0 < rows && err == hipSuccess; r0 += slab_rows) {
            const uint64_t n = std::min(slab_rows, rows - r0), nbytes = n * row_bytes;
            const int k = (int)(up.next++ & 1);
            err = hipEventSynchronize(up.done[k]);
            if (err != hipSuccess) break;
            parallel_copy(up.host[k], src + r0 * row_bytes, nbytes);
            if (blocked) {
                err = hipMemcpyAsync(up.dev[k], up.host[k], nbytes, hipMemcpyHostToDevice, h->stream);
                if (err == hipSuccess) err = launch_repack(type, up.dev[k], w.dev + r0 * row_bytes, n, cols, h->stream);
            } else {
                err = hipMemcpyAsync(w.dev + r0 * row_bytes, up.host[k], nbytes, hipMemcpyHostToDevice, h->stream);
            }
            if (err == hipSuccess) err = hipEventRecord(up.done[k], h->stream);
        }
    } else if (blocked) {
        // rows wider than a slab (not met by qwen35 shapes): re-laid out on the host
        const uint64_t slab_rows = std::max<uint64_t>(1, (64ull << 20) / row_bytes);
        std::vector<uint8_t> buf((size_t)(std::min(rows, slab_rows) * row_bytes));
        for (uint64_t r0 = 0; r0 < rows && err == hipSuccess; r0 += slab_rows) {
            const uint64_t n = std::min(slab_rows, rows - r0);
            parallel_rows(n, [&](uint64_t b, uint64_t e) {
                std::vector<uint8_t> tmp(row_bytes);
                for (uint64_t r = b; r < e; ++r)
                    row_to_device(type, src + (r0 + r) * row_bytes, buf.data() + r * row_bytes, cols, tmp.data());
            });
            err = hipMemcpy(w.dev + r0 * row_bytes, buf.data(), (size_t)(n * row_bytes), hipMemcpyHostToDevice);
        }
    } else {
        err = hipMemcpy(w.dev, src, bytes, hipMemcpyHostToDevice);
    }
    if (err != hipSuccess) {
        (void)hipStreamSynchronize(h->stream);
        (void)hipFree(w.dev);
        return fail(EMPRISE_EDEVICE, "upload weights: %s", hipGetErrorString(err));
    }
    h->used += bytes;
    const uint64_t id = h->next_weight++;
    h->weights.emplace(id, w);
    *out = id;
    return EMPRISE_OK;
}

emprise_status emprise_hip_weight_free(emprise_hip* h, emprise_weight id) {
    if (!h) return fail(EMPRISE_EINVAL, "null backend");
    auto it = h->weights.find(id);
    if (it == h->weights.end()) return fail(EMPRISE_EINVAL, "unknown weight handle");
    HIP_TRY(hipStreamSynchronize(h->stream));
    HIP_TRY(hipFree(it->second.dev));
    h->used -= it->second.bytes;
    h->weights.erase(it);
    return EMPRISE_OK;
}

emprise_dev emprise_hip_weight_data(const emprise_hip* h, emprise_weight id) {
    const Weight* w = h ? h->weight(id) : nullptr;
    return w ? reinterpret_cast<emprise_dev>(w->dev) : 0;
}

emprise_status emprise_hip_dequantize_rows(emprise_hip* h, emprise_weight id, uint64_t row0, uint64_t n, emprise_dev out) {
    const Weight* w = h ? h->weight(id) : nullptr;
    if (!w || !out) return fail(EMPRISE_EINVAL, "bad weight or output");
    if (row0 > w->rows || n > w->rows - row0) return fail(EMPRISE_EINVAL, "rows out of range");
    if (!n) return EMPRISE_OK;
    return launched(launch_dequant_rows(w->dev, w->type, (int)w->cols, row0, n, reinterpret_cast<float*>(out), h->stream));
}

emprise_status emprise_hip_weight_download_gguf(emprise_hip* h, emprise_weight id, void* out, size_t len) {
    const Weight* w = h ? h->weight(id) : nullptr;
    if (!w || !out) return fail(EMPRISE_EINVAL, "bad weight or output");
    if (len != w->bytes) return fail(EMPRISE_EINVAL, "length mismatch");
    std::vector<uint8_t> buf(w->bytes);
    HIP_TRY(hipStreamSynchronize(h->stream));
    HIP_TRY(hipMemcpy(buf.data(), w->dev, w->bytes, hipMemcpyDeviceToHost));
    if (w->type == kQ6K || w->type == kQ4K) {
        const uint64_t nb = w->cols / 256, row_bytes = nb * type_block_bytes(w->type);
        auto* dst = static_cast<uint8_t*>(out);
        parallel_rows(w->rows, [&](uint64_t b, uint64_t e) {
            std::vector<uint8_t> tmp(row_bytes);
            for (uint64_t r = b; r < e; ++r)
                row_from_device(w->type, buf.data() + r * row_bytes, dst + r * row_bytes, w->cols, tmp.data());
        });
    } else {
        std::memcpy(out, buf.data(), w->bytes);
    }
    return EMPRISE_OK;
}

emprise_status emprise_hip_linear(emprise_hip* h, emprise_weight w, emprise_dev x, emprise_dev y) {
    if (!h || !x || !y) return fail(EMPRISE_EINVAL, "null argument");
    const Weight* wt;
    TRY(check_weights(h, 1, &w, &wt));
    Proj p{wt, reinterpret_cast<float*>(y)};
    return run_matvec(h, &p, 1, kMvPlain, nullptr, reinterpret_cast<const float*>(x), nullptr, nullptr, 0, nullptr);
}

emprise_status emprise_hip_linear_many(emprise_hip* h, int n, const emprise_weight* w, emprise_dev x,
                                       const emprise_dev* y) {
    if (!h || !w || !x || !y || n < 1 || n > kMaxSeg) return fail(EMPRISE_EINVAL, "bad arguments");
    const Weight* wt[kMaxSeg];
    TRY(check_weights(h, n, w, wt));
    Proj p[kMaxSeg];
    for (int i = 0; i < n; ++i) p[i] = {wt[i], reinterpret_cast<float*>(y[i])};
    return run_matvec(h, p, n, kMvPlain, nullptr, reinterpret_cast<const float*>(x), nullptr, nullptr, 0, nullptr);
}

emprise_status emprise_hip_linear_norm(emprise_hip* h, const emprise_hip_input* in, int n, const emprise_weight* w,
                                       const emprise_dev* y) {
    if (!h || !in || !in->x || !w || !y || n < 1 || n > kMaxSeg) return fail(EMPRISE_EINVAL, "bad arguments");
    if (in->x_out && (in->x_out == in->x || in->x_out == in->delta)) return fail(EMPRISE_EINVAL, "x_out aliases an input");
    const Weight* wt[kMaxSeg];
    TRY(check_weights(h, n, w, wt));
    Proj p[kMaxSeg];
    for (int i = 0; i < n; ++i) p[i] = {wt[i], reinterpret_cast<float*>(y[i])};
    return run_matvec(h, p, n, kMvPlain, in, nullptr, nullptr, nullptr, 0, nullptr);
}

// Batches of at least this many tokens run as a GEMM on the matrix cores; smaller ones
// as matvecs, which read the weights once per token at full HBM speed.
constexpr int kGemmMinBatch = 8;
constexpr size_t kGemmScratchBytes = size_t(256) << 20;  // dequantised weight rows per GEMM pass

emprise_status emprise_hip_linear_batch(emprise_hip* h, emprise_weight w, emprise_dev X, emprise_dev Y, int K) {
    const Weight* wt = h ? h->weight(w) : nullptr;
    if (!wt) return fail(EMPRISE_EINVAL, "bad arguments");
    return emprise_hip_linear_batch_strided(h, w, X, wt->cols, Y, wt->rows, K);
}

// Y[k] = [W_0; W_1; ...] X[k]: the weights' rows side by side in Y, for K rows of X. From
// kGemmMinBatch rows up the projections run as GEMMs on the matrix cores -- chunked
// Q6_K/Q4_K weights on exact fp16 pieces, consecutive weights of one type (q|k|v, the
// recurrent in-projections) sharing a launch and its full tiles; other weights
// dequantised exactly to FP32 -- and below that as the streaming matvec per row of X.
static emprise_status linear_batch_rows(emprise_hip* h, int nw, const Weight* const* ws, emprise_dev X, uint64_t ldx,
                                        emprise_dev Y, uint64_t ldy, int K) {
    const int cols = (int)ws[0]->cols;
    uint64_t rows = 0;
    bool all_f32 = true;
    for (int i = 0; i < nw; ++i) rows += ws[i]->rows, all_f32 = all_f32 && ws[i]->type == kF32;
    if (ldx < (uint64_t)cols || ldy < rows || ldx > (1u << 30) || ldy > (1u << 30))
        return fail(EMPRISE_EINVAL, "row strides shorter than the matrix");
    if (K < kGemmMinBatch || cols % 16 != 0 || X % 16 != 0 || ldx % 4 != 0) {
        uint64_t off = 0;
        for (int i = 0; i < nw; ++i) {
            const Weight* wt = ws[i];
            // 2..kGemmMinBatch-1 rows through a chunked Q6_K/Q4_K matrix: up to kBatchMax rows
            // per launch, the weights read once per launch (--fast-q8 keeps Q6_K on the
            // single-input path, which quantises its input)
            const bool batched = K > 1 && (wt->type == kQ6K || wt->type == kQ4K) && chunked_cols(wt->cols) &&
                                 !(h->q8 && wt->type == kQ6K) && X % 16 == 0 && ldx % 4 == 0;
            int per = kBatchMax;
            while (per > 1 && matvec_batch_lds_bytes(wt->type, cols, per) > kBatchLdsMax) --per;
            for (int k0 = 0; k0 < K;) {
                const int n = batched ? std::min(per, K - k0) : 1;
                float* yk = reinterpret_cast<float*>(Y) + (size_t)k0 * ldy + off;
                const float* xk = reinterpret_cast<const float*>(X) + (size_t)k0 * ldx;
                if (n > 1) {
                    MvBatchArgs b{static_cast<const uint8_t*>(wt->dev), (int)wt->rows, cols, xk, (size_t)ldx, yk,
                                  (size_t)ldy};
                    TRY(traced(h, "matvec_batch", wt->bytes + (uint64_t)n * cols * 4,
                               [&] { return launch_matvec_batch(wt->type, b, n, h->stream); }));
                } else {
                    Proj p{wt, yk};
                    TRY(run_matvec(h, &p, 1, kMvPlain, nullptr, xk, nullptr, nullptr, 0, nullptr));
                }
                k0 += n;
            }
            off += wt->rows;
        }
        return EMPRISE_OK;
    }
    const float* A = reinterpret_cast<const float*>(X);
    float* C = reinterpret_cast<float*>(Y);
    const uint64_t flops_per_row = 2ull * (uint64_t)K * (uint64_t)cols;
    if (nw == 1 && all_f32) {
        return traced(h, "gemm_f32", flops_per_row * rows, [&] {
            return launch_gemm_f32(A, reinterpret_cast<const float*>(ws[0]->dev), C, K, (int)rows, cols, (int)ldx,
                                   cols, (int)ldy, h->stream);
        });
    }
    // Chunked Q6_K / Q4_K weights run on the fp16 matrix cores (gemm_q.hip: exact fp16
    // pieces of the weights and of the activations, FP32 sums), consecutive weights of one
    // type in one launch; the others are dequantised (or copied, for F32 rows) exactly into
    // FP32 blocks and multiplied in FP32.
    auto on_q16 = [](const Weight* wt) { return (wt->type == kQ6K || wt->type == kQ4K) && chunked_cols(wt->cols); };
    bool any_q = false, sums = false;
    for (int i = 0; i < nw; ++i)
        if (on_q16(ws[i])) any_q = true, sums = sums || ws[i]->type == kQ4K;
    QGemmArgs qa{};
    if (any_q) {
        void* xs;
        TRY(h->get_scratch("gemm_xs", gemm_q16_split_bytes(K, cols, sums), &xs));
        TRY(traced(h, "split_f16", (uint64_t)K * cols * 8, [&] {
            return launch_gemm_q16_split(A, K, cols, (int)ldx, xs, sums, &qa, h->stream);
        }));
    }
    const uint64_t block = std::max<uint64_t>(128, kGemmScratchBytes / ((uint64_t)cols * 4) / 128 * 128);
    uint64_t first = 0;  // stacked index of weight i's row 0
    for (int i = 0; i < nw;) {
        if (on_q16(ws[i])) {
            const uint32_t type = ws[i]->type;
            int j = i, nr = 0;
            qa.nseg = 0;
            while (j < nw && on_q16(ws[j]) && ws[j]->type == type) {
                qa.w[qa.nseg] = static_cast<const uint8_t*>(ws[j]->dev);
                qa.row0[qa.nseg++] = nr;
                nr += (int)ws[j]->rows;
                ++j;
            }
            qa.row0[qa.nseg] = nr;
            qa.N = nr;
            qa.y = C + first;
            qa.ldy = (int)ldy;
            TRY(traced(h, "gemm_q16", flops_per_row * (uint64_t)nr, [&] { return launch_gemm_q16(type, qa, h->stream); }));
            first += (uint64_t)nr;
            i = j;
            continue;
        }
        const Weight* wt = ws[i];
        const uint64_t nb = std::min<uint64_t>(block, wt->rows);
        void* wf;
        TRY(h->get_scratch("gemm_w", nb * cols * sizeof(float), &wf));
        for (uint64_t r0 = 0; r0 < wt->rows; r0 += nb) {
            const uint64_t n = std::min<uint64_t>(nb, wt->rows - r0);
            TRY(traced(h, "dequant_rows", n * (wt->bytes / wt->rows + (uint64_t)cols * 4), [&] {
                return launch_dequant_rows(wt->dev, wt->type, cols, r0, n, static_cast<float*>(wf), h->stream);
            }));
            TRY(traced(h, "gemm_f32", flops_per_row * n, [&] {
                return launch_gemm_f32(A, static_cast<const float*>(wf), C + first + r0, K, (int)n, cols, (int)ldx, cols,
                                       (int)ldy, h->stream);
            }));
        }
        first += wt->rows;
        ++i;
    }
    return EMPRISE_OK;
}

emprise_status emprise_hip_linear_batch_strided(emprise_hip* h, emprise_weight w, emprise_dev X, uint64_t ldx,
                                                emprise_dev Y, uint64_t ldy, int K) {
    if (!h || !X || !Y || K < 1) return fail(EMPRISE_EINVAL, "bad arguments");
    const Weight* wt;
    TRY(check_weights(h, 1, &w, &wt));
    return linear_batch_rows(h, 1, &wt, X, ldx, Y, ldy, K);
}

emprise_status emprise_hip_linear_batch_many(emprise_hip* h, int n, const emprise_weight* w, emprise_dev X,
                                             uint64_t ldx, emprise_dev Y, uint64_t ldy, int K) {
    if (!h || !w || !X || !Y || K < 1 || n < 1 || n > kMaxSeg) return fail(EMPRISE_EINVAL, "bad arguments");
    const Weight* ws[kMaxSeg];
    TRY(check_weights(h, n, w, ws));
    for (int i = 1; i < n; ++i)
        if (ws[i]->cols != ws[0]->cols) return fail(EMPRISE_EINVAL, "linear_batch_many: input widths differ");
    return linear_batch_rows(h, n, ws, X, ldx, Y, ldy, K);
}

emprise_status emprise_hip_ffn_gate_up_batch(emprise_hip* h, emprise_weight gate, emprise_weight up, emprise_dev X,
                                             uint64_t ldx, emprise_dev Y, uint64_t ldy, int K) {
    if (!h || !X || !Y || K < 1) return fail(EMPRISE_EINVAL, "bad arguments");
    const emprise_weight w[2] = {gate, up};
    const Weight* ws[2];
    TRY(check_weights(h, 2, w, ws));
    const Weight *g = ws[0], *u = ws[1];
    if (g->cols != u->cols || g->rows != u->rows) return fail(EMPRISE_EINVAL, "ffn_gate_up_batch: gate and up differ");
    const int cols = (int)g->cols, F = (int)g->rows;
    if (ldx < (uint64_t)cols || ldy < (uint64_t)F || ldx > (1u << 30) || ldy > (1u << 30) || 2ull * F > (1u << 30))
        return fail(EMPRISE_EINVAL, "row strides shorter than the matrix");
    float* y = reinterpret_cast<float*>(Y);
    // gate and up of one chunked type: one GEMM over their interleaved rows, SwiGLU in its
    // epilogue (gemm_q.hip, QGemmArgs::pair)
    if ((g->type == kQ6K || g->type == kQ4K) && u->type == g->type && chunked_cols(g->cols) && K >= kGemmMinBatch &&
        cols % 16 == 0 && X % 16 == 0 && ldx % 4 == 0) {
        const bool sums = g->type == kQ4K;
        QGemmArgs qa{};
        void* xs;
        TRY(h->get_scratch("gemm_xs", gemm_q16_split_bytes(K, cols, sums), &xs));
        TRY(traced(h, "split_f16", (uint64_t)K * cols * 8, [&] {
            return launch_gemm_q16_split(reinterpret_cast<const float*>(X), K, cols, (int)ldx, xs, sums, &qa, h->stream);
        }));
        qa.nseg = 2;
        qa.w[0] = static_cast<const uint8_t*>(g->dev);
        qa.w[1] = static_cast<const uint8_t*>(u->dev);
        qa.row0[0] = 0;
        qa.row0[1] = F;
        qa.row0[2] = 2 * F;
        qa.N = 2 * F;
        qa.y = y;
        qa.ldy = (int)ldy;
        qa.pair = 1;
        return traced(h, "gemm_q16", 4ull * K * cols * F, [&] { return launch_gemm_q16(g->type, qa, h->stream); });
    }
    // otherwise the two projections (gate into Y, up into scratch), then swiglu per row
    void* ub;
    TRY(h->get_scratch("ffn_up_batch", (size_t)K * F * sizeof(float), &ub));
    TRY(linear_batch_rows(h, 1, &g, X, ldx, Y, ldy, K));
    TRY(linear_batch_rows(h, 1, &u, X, ldx, reinterpret_cast<emprise_dev>(ub), (uint64_t)F, K));
    for (int k0 = 0; k0 < K; k0 += 65535) {
        const int n = std::min(65535, K - k0);
        TRY(traced(h, "swiglu", (uint64_t)n * F * 12, [&] {
            return launch_swiglu_rows(y + (size_t)k0 * ldy, ldy, static_cast<const float*>(ub) + (size_t)k0 * F, F, F, n,
                                      h->stream);
        }));
    }
    return EMPRISE_OK;
}

emprise_status emprise_hip_ffn_gate_up(emprise_hip* h, const emprise_hip_input* in, emprise_dev x, emprise_weight gate,
                                       emprise_weight up, emprise_dev hidden) {
    if (!h || !hidden || (!in && !x)) return fail(EMPRISE_EINVAL, "bad arguments");
    const Weight* g = h->weight(gate);
    const Weight* u = h->weight(up);
    if (!is_matrix(g) || !is_matrix(u) || g->rows != u->rows || g->cols != u->cols)
        return fail(EMPRISE_EINVAL, "Feed-forward shape mismatch");
    if (g->type == u->type) {
        Proj p[2] = {{g, reinterpret_cast<float*>(hidden)}, {u, nullptr}};
        return run_matvec(h, p, 2, kMvSwiglu, in, reinterpret_cast<const float*>(x), nullptr, nullptr, 0, nullptr);
    }
    void* ub;
    TRY(h->get_scratch("ffn_up", g->rows * sizeof(float), &ub));
    Proj p[2] = {{g, reinterpret_cast<float*>(hidden)}, {u, static_cast<float*>(ub)}};
    TRY(run_matvec(h, p, 2, kMvPlain, in, reinterpret_cast<const float*>(x), nullptr, nullptr, 0, nullptr));
    return traced(h, "swiglu", g->rows * 12, [&] { return launch_swiglu(reinterpret_cast<float*>(hidden), static_cast<float*>(ub), (int)g->rows, h->stream); });
}

emprise_status emprise_hip_feed_forward(emprise_hip* h, const emprise_hip_input* in, emprise_dev x, emprise_weight gate,
                                        emprise_weight up, emprise_weight down, emprise_dev y) {
    if (!h || !y) return fail(EMPRISE_EINVAL, "bad arguments");
    const Weight* g = h->weight(gate);
    const Weight* d = h->weight(down);
    if (!is_matrix(g) || !is_matrix(d) || d->cols != g->rows) return fail(EMPRISE_EINVAL, "Feed-forward shape mismatch");
    void* hb;
    TRY(h->get_scratch("ffn_hidden", g->rows * sizeof(float), &hb));
    TRY(emprise_hip_ffn_gate_up(h, in, x, gate, up, reinterpret_cast<emprise_dev>(hb)));
    Proj p{d, reinterpret_cast<float*>(y)};
    return run_matvec(h, &p, 1, kMvPlain, nullptr, static_cast<const float*>(hb), nullptr, nullptr, 0, nullptr);
}

emprise_status emprise_hip_rmsnorm(emprise_hip* h, emprise_dev x, emprise_weight w, emprise_dev out, int n, float eps) {
    const Weight* wt = h ? h->weight(w) : nullptr;
    if (!wt || !x || !out || n < 1) return fail(EMPRISE_EINVAL, "bad arguments");
    if (wt->type != kF32 || wt->rows * wt->cols != (uint64_t)n) return fail(EMPRISE_EINVAL, "RMS normalization dimensions");
    return traced(h, "rmsnorm", (uint64_t)n * 12, [&] { return launch_rmsnorm(reinterpret_cast<const float*>(x), reinterpret_cast<const float*>(wt->dev),
                                   reinterpret_cast<float*>(out), n, eps, h->stream); });
}

emprise_status emprise_hip_rmsnorm_rows(emprise_hip* h, emprise_dev x, emprise_weight w, emprise_dev out, int n,
                                       int rows, float eps) {
    const Weight* wt = h ? h->weight(w) : nullptr;
    if (!wt || !x || !out || n < 1 || rows < 1) return fail(EMPRISE_EINVAL, "bad arguments");
    if (wt->type != kF32 || wt->rows * wt->cols != (uint64_t)n) return fail(EMPRISE_EINVAL, "RMS normalization dimensions");
    return traced(h, "rmsnorm", (uint64_t)n * rows * 8 + (uint64_t)n * 4, [&] {
        return launch_rmsnorm_rows(reinterpret_cast<const float*>(x), reinterpret_cast<const float*>(wt->dev),
                                   reinterpret_cast<float*>(out), n, rows, eps, h->stream);
    });
}

emprise_status emprise_hip_add_rmsnorm_rows(emprise_hip* h, emprise_dev x, emprise_dev delta, emprise_weight w,
                                           emprise_dev out, int n, int rows, float eps) {
    const Weight* wt = h ? h->weight(w) : nullptr;
    if (!wt || !x || !delta || !out || n < 1 || rows < 1) return fail(EMPRISE_EINVAL, "bad arguments");
    if (wt->type != kF32 || wt->rows * wt->cols != (uint64_t)n) return fail(EMPRISE_EINVAL, "RMS normalization dimensions");
    if (out == x || out == delta) return fail(EMPRISE_EINVAL, "out aliases an input");
    return traced(h, "add_rmsnorm", (uint64_t)n * rows * 16 + (uint64_t)n * 4, [&] {
        return launch_add_rmsnorm_rows(reinterpret_cast<float*>(x), reinterpret_cast<const float*>(delta),
                                       reinterpret_cast<const float*>(wt->dev), reinterpret_cast<float*>(out), n, rows,
                                       eps, h->stream);
    });
}

emprise_status emprise_hip_embed_rows(emprise_hip* h, emprise_weight embedding, emprise_dev tokens, int count,
                                      emprise_dev out) {
    const Weight* w = h ? h->weight(embedding) : nullptr;
    if (!w || !tokens || !out || count < 1 || count > 65535) return fail(EMPRISE_EINVAL, "bad arguments");
    return traced(h, "embed", (w->bytes / w->rows + w->cols * 4) * count, [&] {
        return launch_embed_rows(w->dev, w->type, (int)w->cols, (int)w->rows, reinterpret_cast<const int*>(tokens),
                                 count, reinterpret_cast<float*>(out), h->stream);
    });
}

emprise_status emprise_hip_add(emprise_hip* h, emprise_dev x, emprise_dev y, int n) {
    if (!h || !x || !y || n < 0) return fail(EMPRISE_EINVAL, "bad arguments");
    if (!n) return EMPRISE_OK;
    return traced(h, "add", (uint64_t)n * 12, [&] { return launch_add(reinterpret_cast<float*>(x), reinterpret_cast<const float*>(y), n, h->stream); });
}

emprise_status emprise_hip_swiglu(emprise_hip* h, emprise_dev gate, emprise_dev up, int n) {
    if (!h || !gate || !up || n < 0) return fail(EMPRISE_EINVAL, "bad arguments");
    if (!n) return EMPRISE_OK;
    return traced(h, "swiglu", (uint64_t)n * 12, [&] { return launch_swiglu(reinterpret_cast<float*>(gate), reinterpret_cast<const float*>(up), n, h->stream); });
}

emprise_status emprise_hip_embed(emprise_hip* h, emprise_weight embedding, emprise_dev token, emprise_dev out) {
    const Weight* w = h ? h->weight(embedding) : nullptr;
    if (!w || !token || !out) return fail(EMPRISE_EINVAL, "bad arguments");
    return traced(h, "embed", w->bytes / w->rows + w->cols * 4, [&] { return launch_embed(w->dev, w->type, (int)w->cols, (int)w->rows, reinterpret_cast<const int*>(token),
                                 reinterpret_cast<float*>(out), h->stream); });
}

emprise_status emprise_hip_argmax(emprise_hip* h, emprise_dev logits, int n, emprise_dev index) {
    if (!h || !logits || !index || n < 1) return fail(EMPRISE_EINVAL, "bad arguments");
    return traced(h, "argmax", (uint64_t)n * 4, [&] { return launch_argmax(reinterpret_cast<const float*>(logits), n, nullptr, reinterpret_cast<int*>(index), h->stream); });
}

emprise_status emprise_hip_quantize_q8(emprise_hip* h, emprise_dev x, int cols, emprise_dev q, emprise_dev scales) {
    if (!h || !x || !q || !scales || cols < 32 || cols % 32) return fail(EMPRISE_EINVAL, "bad arguments");
    return traced(h, "quantize_q8", (uint64_t)cols * 5, [&] { return launch_quantize_q8(reinterpret_cast<const float*>(x), cols, reinterpret_cast<int8_t*>(q),
                                       reinterpret_cast<float*>(scales), h->stream); });
}

emprise_status emprise_hip_delta_net(emprise_hip* h, const emprise_hip_delta_net_params* p) {
    if (!h || !p) return fail(EMPRISE_EINVAL, "null argument");
    const int kd = p->key_heads * p->state_dim, vd = p->value_heads * p->state_dim, ch = 2 * kd + vd;
    const Weight *conv = h->weight(p->conv), *a = h->weight(p->ssm_a), *dt = h->weight(p->dt), *nw = h->weight(p->norm);
    if (p->key_heads < 1 || p->value_heads % p->key_heads || (p->state_dim != 64 && p->state_dim != 128) ||
        p->conv_width < 1 || !conv || !a || !dt || !nw || conv->rows * conv->cols != (uint64_t)ch * p->conv_width ||
        a->rows * a->cols != (uint64_t)p->value_heads || dt->rows * dt->cols != (uint64_t)p->value_heads ||
        nw->rows * nw->cols != (uint64_t)p->state_dim || conv->type != kF32 || a->type != kF32 || dt->type != kF32 ||
        nw->type != kF32)
        return fail(EMPRISE_EINVAL, "Recurrent projection dimensions");
    if (!p->qkv || !p->gate || !p->alpha || !p->beta || !p->conv_state || !p->rec_state || !p->out)
        return fail(EMPRISE_EINVAL, "null buffer");
    if (p->rec_state % 16) return fail(EMPRISE_EINVAL, "rec_state must be 16-byte aligned");
    void* conv_out;
    TRY(h->get_scratch("gdn_conv", (size_t)ch * sizeof(float), &conv_out));
    TRY(traced(h, "delta_conv", (uint64_t)ch * (p->conv_width * 8 + 8), [&] { return launch_delta_conv(reinterpret_cast<const float*>(p->qkv), reinterpret_cast<const float*>(conv->dev),
                                   reinterpret_cast<float*>(p->conv_state), static_cast<float*>(conv_out), ch,
                                   p->conv_width, h->stream); }));
    GdnArgs g{};
    g.key_heads = p->key_heads;
    g.value_heads = p->value_heads;
    g.state_dim = p->state_dim;
    g.conv_width = p->conv_width;
    g.eps = p->eps;
    g.qkv = static_cast<const float*>(conv_out);
    g.gate = reinterpret_cast<const float*>(p->gate);
    g.alpha = reinterpret_cast<const float*>(p->alpha);
    g.beta = reinterpret_cast<const float*>(p->beta);
    g.ssm_a = reinterpret_cast<const float*>(a->dev);
    g.dt = reinterpret_cast<const float*>(dt->dev);
    g.norm = reinterpret_cast<const float*>(nw->dev);
    g.state = reinterpret_cast<float*>(p->rec_state);
    g.out = reinterpret_cast<float*>(p->out);
    return traced(h, "gdn_step", gdn_bytes(g), [&] { return launch_gdn(g, h->stream); });
}

emprise_status emprise_hip_delta_net_noalloc(emprise_hip* h, const emprise_hip_delta_net_params* p) {
    if (!h || !p) return fail(EMPRISE_EINVAL, "null argument");
    const int kd = p->key_heads * p->state_dim, vd = p->value_heads * p->state_dim, ch = 2 * kd + vd;
    if (p->key_heads < 1 || p->value_heads < 1 || p->state_dim < 1 || ch > kNoAllocScratchFloats)
        return fail(EMPRISE_EINVAL, "delta_net_noalloc: %d channels exceed the %d-float scratch", ch,
                    kNoAllocScratchFloats);
    const Weight *conv = h->weight(p->conv), *a = h->weight(p->ssm_a), *dt = h->weight(p->dt), *nw = h->weight(p->norm);
    if (p->value_heads % p->key_heads || (p->state_dim != 64 && p->state_dim != 128) || p->conv_width < 1 || !conv ||
        !a || !dt || !nw || conv->rows * conv->cols != (uint64_t)ch * p->conv_width ||
        a->rows * a->cols != (uint64_t)p->value_heads || dt->rows * dt->cols != (uint64_t)p->value_heads ||
        nw->rows * nw->cols != (uint64_t)p->state_dim || conv->type != kF32 || a->type != kF32 || dt->type != kF32 ||
        nw->type != kF32)
        return fail(EMPRISE_EINVAL, "Recurrent projection dimensions");
    if (!p->qkv || !p->gate || !p->alpha || !p->beta || !p->conv_state || !p->rec_state || !p->out)
        return fail(EMPRISE_EINVAL, "null buffer");
    if (p->rec_state % 16) return fail(EMPRISE_EINVAL, "rec_state must be 16-byte aligned");
    // the conv kernel writes all ch channels of the scratch before the state update reads
    // them, so nothing carried over from an earlier call is read
    float* conv_out = h->noalloc_scratch;
    TRY(launched(launch_delta_conv(reinterpret_cast<const float*>(p->qkv), reinterpret_cast<const float*>(conv->dev),
                                   reinterpret_cast<float*>(p->conv_state), conv_out, ch, p->conv_width, h->stream)));
    GdnArgs g{};
    g.key_heads = p->key_heads;
    g.value_heads = p->value_heads;
    g.state_dim = p->state_dim;
    g.conv_width = p->conv_width;
    g.eps = p->eps;
    g.qkv = conv_out;
    g.gate = reinterpret_cast<const float*>(p->gate);
    g.alpha = reinterpret_cast<const float*>(p->alpha);
    g.beta = reinterpret_cast<const float*>(p->beta);
    g.ssm_a = reinterpret_cast<const float*>(a->dev);
    g.dt = reinterpret_cast<const float*>(dt->dev);
    g.norm = reinterpret_cast<const float*>(nw->dev);
    g.state = reinterpret_cast<float*>(p->rec_state);
    g.out = reinterpret_cast<float*>(p->out);
    return launched(launch_gdn(g, h->stream));
}

emprise_status emprise_hip_delta_net_batch(emprise_hip* h, const emprise_hip_delta_net_params* p, int count,
                                           uint64_t stride, uint64_t out_stride) {
    if (!h || !p) return fail(EMPRISE_EINVAL, "null argument");
    const int kd = p->key_heads * p->state_dim, vd = p->value_heads * p->state_dim, ch = 2 * kd + vd;
    const Weight *conv = h->weight(p->conv), *a = h->weight(p->ssm_a), *dt = h->weight(p->dt), *nw = h->weight(p->norm);
    if (p->key_heads < 1 || p->value_heads % p->key_heads || (p->state_dim != 64 && p->state_dim != 128) ||
        p->conv_width < 1 || p->conv_width > 8 || !conv || !a || !dt || !nw ||
        conv->rows * conv->cols != (uint64_t)ch * p->conv_width || a->rows * a->cols != (uint64_t)p->value_heads ||
        dt->rows * dt->cols != (uint64_t)p->value_heads || nw->rows * nw->cols != (uint64_t)p->state_dim ||
        conv->type != kF32 || a->type != kF32 || dt->type != kF32 || nw->type != kF32)
        return fail(EMPRISE_EINVAL, "Recurrent projection dimensions");
    if (!p->qkv || !p->gate || !p->alpha || !p->beta || !p->conv_state || !p->rec_state || !p->out)
        return fail(EMPRISE_EINVAL, "null buffer");
    if (p->rec_state % 16) return fail(EMPRISE_EINVAL, "rec_state must be 16-byte aligned");
    if (count < 1 || count > (1 << 19) || stride < (uint64_t)ch || out_stride < (uint64_t)vd)
        return fail(EMPRISE_EINVAL, "delta_net_batch: count %d, stride %llu, out_stride %llu", count,
                    (unsigned long long)stride, (unsigned long long)out_stride);
    void *conv_out, *o, *qk, *gates;
    TRY(h->get_scratch("gdn_conv_batch", (size_t)count * ch * sizeof(float), &conv_out));
    TRY(h->get_scratch("gdn_o_batch", (size_t)count * vd * sizeof(float), &o));
    TRY(h->get_scratch("gdn_qk_batch", (size_t)count * 2 * kd * sizeof(float), &qk));
    TRY(h->get_scratch("gdn_gates_batch", (size_t)count * 2 * p->value_heads * sizeof(float), &gates));
    GdnBatchArgs g{};
    g.key_heads = p->key_heads;
    g.value_heads = p->value_heads;
    g.state_dim = p->state_dim;
    g.conv_width = p->conv_width;
    g.count = count;
    g.eps = p->eps;
    g.qkv = reinterpret_cast<const float*>(p->qkv);
    g.gate = reinterpret_cast<const float*>(p->gate);
    g.alpha = reinterpret_cast<const float*>(p->alpha);
    g.beta = reinterpret_cast<const float*>(p->beta);
    g.stride = stride;
    g.conv_w = reinterpret_cast<const float*>(conv->dev);
    g.ssm_a = reinterpret_cast<const float*>(a->dev);
    g.dt = reinterpret_cast<const float*>(dt->dev);
    g.norm = reinterpret_cast<const float*>(nw->dev);
    g.conv_state = reinterpret_cast<float*>(p->conv_state);
    g.state = reinterpret_cast<float*>(p->rec_state);
    g.conv_out = static_cast<float*>(conv_out);
    g.qk = static_cast<float*>(qk);
    g.gates = static_cast<float*>(gates);
    g.o = static_cast<float*>(o);
    g.out = reinterpret_cast<float*>(p->out);
    g.out_stride = out_stride;
    const uint64_t bytes = (uint64_t)count * (2 * (uint64_t)ch + 2 * vd + 2 * p->value_heads + 2 * vd) * 4 +
                           2 * (uint64_t)p->value_heads * p->state_dim * p->state_dim * 4;
    return traced(h, "gdn_batch", bytes, [&] { return launch_gdn_batch(g, h->stream); });
}

emprise_status emprise_hip_recurrent(emprise_hip* h, const emprise_hip_recurrent_params* p, const emprise_hip_input* in,
                                     emprise_dev x, emprise_dev y) {
    if (!h || !p || !y || (!in && !x)) return fail(EMPRISE_EINVAL, "null argument");
    const int kd = p->key_heads * p->state_dim, vd = p->value_heads * p->state_dim, ch = 2 * kd + vd;
    const emprise_weight ids[5] = {p->qkv_w, p->gate_w, p->alpha_w, p->beta_w, p->out_w};
    const Weight* w[5];
    TRY(check_weights(h, 5, ids, w));
    const Weight *conv = h->weight(p->conv), *a = h->weight(p->ssm_a), *dt = h->weight(p->dt), *nw = h->weight(p->norm);
    if (p->key_heads < 1 || p->value_heads % p->key_heads || (p->state_dim != 64 && p->state_dim != 128) ||
        w[0]->rows != (uint64_t)ch || w[1]->rows != (uint64_t)vd || w[2]->rows != (uint64_t)p->value_heads ||
        w[3]->rows != (uint64_t)p->value_heads || w[4]->cols != (uint64_t)vd || !conv || !a || !dt || !nw ||
        conv->type != kF32 || a->type != kF32 || dt->type != kF32 || nw->type != kF32 ||
        conv->rows * conv->cols != (uint64_t)ch * p->conv_width || a->rows * a->cols != (uint64_t)p->value_heads ||
        dt->rows * dt->cols != (uint64_t)p->value_heads || nw->rows * nw->cols != (uint64_t)p->state_dim)
        return fail(EMPRISE_EINVAL, "Recurrent projection dimensions");
    if (!p->conv_state || !p->rec_state) return fail(EMPRISE_EINVAL, "null state buffer");
    if (p->rec_state % 16) return fail(EMPRISE_EINVAL, "rec_state must be 16-byte aligned");
    void* proj;
    const size_t proj_n = (size_t)ch + vd + 2 * (size_t)p->value_heads + vd;
    TRY(h->get_scratch("gdn_proj", proj_n * sizeof(float), &proj));
    float* qkv = static_cast<float*>(proj);
    float* gate = qkv + ch;
    float* alpha = gate + vd;
    float* beta = alpha + p->value_heads;
    float* dn = beta + p->value_heads;
    // With a chunked out weight whose input fits one staging pass, the per-head RMSNorm x
    // SiLU(gate) moves into the out projection's input staging (the gate rows leave the
    // in-projection already SiLU'd), and the state update splits each head over several
    // workgroups (no cross-wave step left in it).
    const bool split = (w[4]->type == kQ6K || w[4]->type == kQ4K) && vd % kChunkCols == 0 && vd <= kChunkCols;
    Proj pr[4] = {{w[0], qkv}, {w[1], gate, split}, {w[2], alpha}, {w[3], beta}};
    // qkv first, so the conv1d + SiLU epilogue lands on its rows
    TRY(run_matvec(h, pr, 4, kMvPlain, in, reinterpret_cast<const float*>(x), reinterpret_cast<const float*>(conv->dev),
                   reinterpret_cast<float*>(p->conv_state), p->conv_width, nullptr));
    GdnArgs g{};
    g.key_heads = p->key_heads;
    g.value_heads = p->value_heads;
    g.state_dim = p->state_dim;
    g.conv_width = p->conv_width;
    g.eps = p->eps;
    g.qkv = qkv;
    g.gate = gate;
    g.alpha = alpha;
    g.beta = beta;
    g.ssm_a = reinterpret_cast<const float*>(a->dev);
    g.dt = reinterpret_cast<const float*>(dt->dev);
    g.norm = reinterpret_cast<const float*>(nw->dev);
    g.state = reinterpret_cast<float*>(p->rec_state);
    g.out = dn;
    Proj po{w[4], reinterpret_cast<float*>(y)};
    if (split) {
        TRY(traced(h, "gdn_step", gdn_bytes(g) - (uint64_t)vd * 4, [&] { return launch_gdn_rows(g, h->stream); }));
        const HeadGate hg{gate, g.norm, p->state_dim, p->eps};
        return run_matvec(h, &po, 1, kMvPlain, nullptr, dn, nullptr, nullptr, 0, nullptr, &hg);
    }
    TRY(traced(h, "gdn_step", gdn_bytes(g), [&] { return launch_gdn(g, h->stream); }));
    return run_matvec(h, &po, 1, kMvPlain, nullptr, dn, nullptr, nullptr, 0, nullptr);
}

namespace {
// The RoPE table (cos, sin of every position's angles) of this (context, rotary, base),
// shared by the decode and prefill attention so that they rotate with the
// same values; filled by the first eager call (not while a graph is being captured).
emprise_status rope_table(emprise_hip* h, const emprise_hip_attention_params* p, const float2** out) {
    uint32_t bits;
    std::memcpy(&bits, &p->rope_base, 4);
    char key[96];
    std::snprintf(key, sizeof key, "rope:%d:%d:%08x", p->context, p->rotary, bits);
    void* t;
    TRY(h->get_scratch(key, std::max<size_t>((size_t)p->context * (p->rotary / 2) * sizeof(float2), 8), &t));
    if (!h->rope_ready.count(key)) {
        if (h->capturing) return fail(EMPRISE_ESTATE, "the RoPE table must be filled before graph capture");
        TRY(launched(launch_rope_table(static_cast<float2*>(t), p->context, p->rotary, p->rope_base, h->stream)));
        h->rope_ready.insert(key);
    }
    *out = static_cast<const float2*>(t);
    return EMPRISE_OK;
}
}  // namespace

emprise_status emprise_hip_attention_batch(emprise_hip* h, const emprise_hip_attention_params* p, emprise_dev qkv,
                                           int count, uint64_t stride, int first_position, emprise_dev out,
                                           uint64_t out_stride) {
    if (!h || !p || !qkv || !out || !p->keys || !p->values) return fail(EMPRISE_EINVAL, "null argument");
    const Weight *qn = h->weight(p->q_norm), *kn = h->weight(p->k_norm);
    if (p->heads < 1 || p->kv_heads < 1 || p->heads % p->kv_heads ||
        (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256) || p->rotary > p->head_dim || p->rotary % 2 ||
        p->rotary < 0 || p->context < 1 || !qn || !kn || qn->type != kF32 || kn->type != kF32 ||
        qn->rows * qn->cols != (uint64_t)p->head_dim || kn->rows * kn->cols != (uint64_t)p->head_dim)
        return fail(EMPRISE_EINVAL, "Attention projection dimensions");
    const uint64_t qkv_w = (uint64_t)p->heads * p->head_dim * 2 + 2 * (uint64_t)p->kv_heads * p->head_dim;
    if (count < 1 || first_position < 0 || (int64_t)first_position + count > p->context || stride < qkv_w ||
        out_stride < (uint64_t)p->heads * p->head_dim)
        return fail(EMPRISE_EINVAL, "attention_batch: positions %d..%d of a %d-position context, stride %llu",
                    first_position, first_position + count - 1, p->context, (unsigned long long)stride);
    AttnBatchArgs a{};
    TRY(rope_table(h, p, &a.rope));
    a.heads = p->heads;
    a.kv_heads = p->kv_heads;
    a.head_dim = p->head_dim;
    a.rotary = p->rotary;
    a.count = count;
    a.first = first_position;
    a.lp = (first_position + count + 31) / 32 * 32;
    a.eps = p->eps;
    a.rope_base = p->rope_base;
    a.q_norm = reinterpret_cast<const float*>(qn->dev);
    a.k_norm = reinterpret_cast<const float*>(kn->dev);
    a.qkv = reinterpret_cast<const float*>(qkv);
    a.stride = stride;
    a.keys = reinterpret_cast<float*>(p->keys);
    a.values = reinterpret_cast<float*>(p->values);
    a.out = reinterpret_cast<float*>(out);
    a.out_stride = out_stride;
    const size_t hq = (size_t)count * p->heads * p->head_dim;
    void *q, *sc, *vt, *o;
    TRY(h->get_scratch("attnb_q", hq * sizeof(float), &q));
    TRY(h->get_scratch("attnb_s", (size_t)p->heads * count * a.lp * sizeof(float), &sc));
    TRY(h->get_scratch("attnb_vt", (size_t)p->kv_heads * p->head_dim * a.lp * sizeof(float), &vt));
    TRY(h->get_scratch("attnb_o", hq * sizeof(float), &o));
    a.q = static_cast<float*>(q);
    a.scores = static_cast<float*>(sc);
    a.vt = static_cast<float*>(vt);
    a.o = static_cast<float*>(o);
    // K/V rows 0..first+count-1 read twice (scores, transpose), the new rows written
    const uint64_t bytes = 3 * (uint64_t)(first_position + count) * p->kv_heads * p->head_dim * 4 + count * qkv_w * 4;
    return traced(h, "attention_batch", bytes, [&] { return launch_attention_batch(a, h->stream); });
}

emprise_status emprise_hip_attention(emprise_hip* h, const emprise_hip_attention_params* p, emprise_dev qkv,
                                     emprise_dev out) {
    if (!h || !p || !qkv || !out || !p->keys || !p->values || !p->position) return fail(EMPRISE_EINVAL, "null argument");
    const Weight *qn = h->weight(p->q_norm), *kn = h->weight(p->k_norm);
    if (p->heads < 1 || p->kv_heads < 1 || p->heads % p->kv_heads || p->heads / p->kv_heads > 8 ||
        (p->head_dim != 64 && p->head_dim != 128 && p->head_dim != 256) || p->rotary > p->head_dim || p->rotary % 2 ||
        p->rotary < 0 || p->context < 1 || !qn || !kn || qn->type != kF32 || kn->type != kF32 ||
        qn->rows * qn->cols != (uint64_t)p->head_dim || kn->rows * kn->cols != (uint64_t)p->head_dim)
        return fail(EMPRISE_EINVAL, "Attention projection dimensions");
    void* partial;
    TRY(h->get_scratch("attn_partial", attention_partial_floats(p->heads, p->kv_heads, p->head_dim, p->context) * sizeof(float),
                       &partial));
    AttnArgs a{};
    a.heads = p->heads;
    a.kv_heads = p->kv_heads;
    a.head_dim = p->head_dim;
    a.rotary = p->rotary;
    a.context = p->context;
    a.eps = p->eps;
    a.rope_base = p->rope_base;
    a.q_norm = reinterpret_cast<const float*>(qn->dev);
    a.k_norm = reinterpret_cast<const float*>(kn->dev);
    a.qkv = reinterpret_cast<const float*>(qkv);
    a.keys = reinterpret_cast<float*>(p->keys);
    a.values = reinterpret_cast<float*>(p->values);
    a.position = reinterpret_cast<const int*>(p->position);
    a.rope_position = reinterpret_cast<const int*>(p->rope_position);
    a.out = reinterpret_cast<float*>(out);
    a.partial = static_cast<float*>(partial);
    TRY(rope_table(h, p, &a.rope));
    return traced(h, "attention", 0, [&] { return launch_attention(a, h->stream); });
}

emprise_status emprise_hip_reset_state(emprise_hip* h) {
    if (!h) return fail(EMPRISE_EINVAL, "null backend");
    return EMPRISE_OK;
}

emprise_status emprise_hip_sync(emprise_hip* h) {
    if (!h) return fail(EMPRISE_EINVAL, "null backend");
    if (h->capturing) return fail(EMPRISE_ESTATE, "sync during graph capture");
    HIP_TRY(hipStreamSynchronize(h->stream));
    return EMPRISE_OK;
}

emprise_status emprise_hip_advance(emprise_hip* h, emprise_dev state, emprise_dev prompt, emprise_dev history,
                                   emprise_dev next) {
    if (!h || !state) return fail(EMPRISE_EINVAL, "null argument");
    return traced(h, "advance", 16, [&] { return launch_advance(reinterpret_cast<int*>(state), reinterpret_cast<const int*>(prompt),
                                   reinterpret_cast<int*>(history), reinterpret_cast<const int*>(next), h->stream); });
}

emprise_status emprise_hip_lm_head(emprise_hip* h, const emprise_hip_input* in, emprise_weight w, emprise_dev logits,
                                   emprise_dev index) {
    if (!h || !in || !in->x || !logits || !index) return fail(EMPRISE_EINVAL, "null argument");
    if (in->x_out && (in->x_out == in->x || in->x_out == in->delta)) return fail(EMPRISE_EINVAL, "x_out aliases an input");
    const Weight* wt;
    TRY(check_weights(h, 1, &w, &wt));
    void* key;
    TRY(h->get_scratch("argmax_key", sizeof(unsigned long long), &key, true));
    Proj p{wt, reinterpret_cast<float*>(logits)};
    TRY(run_matvec(h, &p, 1, kMvArgmax, in, nullptr, nullptr, nullptr, 0, static_cast<unsigned long long*>(key)));
    return traced(h, "argmax_finish", 16, [&] { return launch_argmax_finish(static_cast<unsigned long long*>(key), reinterpret_cast<int*>(index), h->stream); });
}

emprise_status emprise_hip_graph_begin(emprise_hip* h) {
    if (!h) return fail(EMPRISE_EINVAL, "null backend");
    if (h->capturing) return fail(EMPRISE_ESTATE, "already capturing");
    HIP_TRY(hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal));
    h->capturing = true;
    return EMPRISE_OK;
}

emprise_status emprise_hip_graph_end(emprise_hip* h, emprise_graph* out) {
    if (!h || !out) return fail(EMPRISE_EINVAL, "null argument");
    if (!h->capturing) return fail(EMPRISE_ESTATE, "not capturing");
    h->capturing = false;
    hipGraph_t graph = nullptr;
    HIP_TRY(hipStreamEndCapture(h->stream, &graph));
    hipGraphExec_t exec = nullptr;
    hipError_t e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return fail(EMPRISE_EDEVICE, "graph instantiate: %s", hipGetErrorString(e));
    const uint64_t id = h->next_graph++;
    h->graphs.emplace(id, exec);
    *out = id;
    return EMPRISE_OK;
}

emprise_status emprise_hip_graph_launch(emprise_hip* h, emprise_graph g) {
    if (!h) return fail(EMPRISE_EINVAL, "null backend");
    auto it = h->graphs.find(g);
    if (it == h->graphs.end()) return fail(EMPRISE_EINVAL, "unknown graph");
    HIP_TRY(hipGraphLaunch(it->second, h->stream));
    return EMPRISE_OK;
}

emprise_status emprise_hip_graph_destroy(emprise_hip* h, emprise_graph g) {
    if (!h) return fail(EMPRISE_EINVAL, "null backend");
    auto it = h->graphs.find(g);
    if (it == h->graphs.end()) return fail(EMPRISE_EINVAL, "unknown graph");
    HIP_TRY(hipStreamSynchronize(h->stream));
    HIP_TRY(hipGraphExecDestroy(it->second));
    h->graphs.erase(it);
    return EMPRISE_OK;
}

emprise_status emprise_hip_trace_begin(emprise_hip* h) {
    if (!h) return fail(EMPRISE_EINVAL, "null backend");
    if (h->capturing) return fail(EMPRISE_ESTATE, "trace during graph capture");
    h->tracing = true;
    h->trace.clear();
    h->trace_used = 0;
    return EMPRISE_OK;
}

emprise_status emprise_hip_trace_end(emprise_hip* h, emprise_hip_trace_record* out, size_t cap, size_t* n) {
    if (!h || !n || (!out && cap)) return fail(EMPRISE_EINVAL, "null argument");
    h->tracing = false;
    HIP_TRY(hipStreamSynchronize(h->stream));
    size_t k = 0;
    for (const auto& r : h->trace) {
        if (k >= cap) break;
        float ms = 0.f;
        HIP_TRY(hipEventElapsedTime(&ms, r.a, r.b));
        out[k++] = {r.kernel, r.bytes, ms};
    }
    *n = k;
    h->trace.clear();
    h->trace_used = 0;
    return EMPRISE_OK;
}

emprise_status emprise_hip_event_record(emprise_hip* h, int slot) {
    if (!h || slot < 0 || slot >= 65536) return fail(EMPRISE_EINVAL, "bad event slot");
    if (h->capturing) return fail(EMPRISE_ESTATE, "event during graph capture");
    while ((int)h->events.size() <= slot) {
        hipEvent_t ev;
        HIP_TRY(hipEventCreate(&ev));
        h->events.push_back(ev);
    }
    HIP_TRY(hipEventRecord(h->events[slot], h->stream));
    return EMPRISE_OK;
}

emprise_status emprise_hip_event_elapsed(emprise_hip* h, int start_slot, int end_slot, float* ms) {
    if (!h || !ms || start_slot < 0 || start_slot >= (int)h->events.size() || end_slot < 0 ||
        end_slot >= (int)h->events.size())
        return fail(EMPRISE_EINVAL, "bad event slot");
    HIP_TRY(hipEventSynchronize(h->events[end_slot]));
    HIP_TRY(hipEventElapsedTime(ms, h->events[start_slot], h->events[end_slot]));
    return EMPRISE_OK;
}

}  // extern "C"
