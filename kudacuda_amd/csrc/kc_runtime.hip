// Host side of libkudacuda.so: the C ABI declared in include/kudacuda.h.
//
// Handle lifecycle, error text and the exact-shape guards follow the
// reference runtime (runtime/kudacuda_runtime.cu:228-1226): status 0/1,
// per-handle last_error, "called before kudacuda_freeze" and non-null checks,
// no synchronisation on the launch path, launch errors taken from
// hipGetLastError.  Unlike the reference, every NF4 QKV version and every GQA
// variant maps onto one gfx950 kernel family (kc_nf4.hip, kc_gqa.hip).
#include <hip/hip_runtime.h>

#include <array>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/kudacuda.h"
#include "kc_device.h"
#include "kc_kernels.h"

namespace kc {
namespace {

constexpr int64_t kMaxStandaloneKv = 65536;
// Direct calls (kv_len known on the host) at this many cached tokens or more
// take the matrix-core tactic (MI355X, cold cache, us per call, round path vs
// matrix cores: 4096 8.5 / 9.7, 8192 10.2 / 10.0, 16384 13.1 / 11.1, 32768
// 17.5 / 13.4).
constexpr int64_t kGqaMfmaMinKv = 8192;
constexpr int64_t kMaxModelKv = 32768;

// ------------------------------------------------ allocation-free scratch
// Device scratch of kudacuda_qwen2_gqa_decode_graph_bf16_noalloc: the split
// partials (16 heads x splits x 130 fp32) and the two ticket counters of the
// split-KV attention, in one file-scope device array per GPU (the code object
// holds one copy per device; it lives until the process ends).  Layout:
// bytes [0, 256) counters (uint32 [2], zero between calls), then the partials.
// Host code never passes `scratch` itself to a kernel: its name is a host-side
// stand-in, so every use goes through the device address that
// hipGetSymbolAddress returned on that device (static_scratch_on()).
// Capacity up to the allocating twin's 65536 tokens: every graph-mode plan
// (split cap kGqaSplitCap per KV head, whatever the capacity) fits.
constexpr int64_t kNoAllocMaxKv = kMaxStandaloneKv;
constexpr int64_t kNoAllocMaxSplits = kGqaSplitCap;
static_assert(kNoAllocMaxSplits >= kGqaSplitCap, "the static partials hold the largest graph-mode split plan");
constexpr int64_t kNoAllocCounterBytes = 256;
constexpr int64_t kNoAllocPartialFloats = 16 * kNoAllocMaxSplits * kGqaPartialStride;
constexpr int64_t kNoAllocScratchBytes = kNoAllocCounterBytes + kNoAllocPartialFloats * 4;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// Resolve this device's copy of `scratch` (call with `device` current) and
// zero its counters once; later calls return the recorded address.  Runs in
// kudacuda_create, never under stream capture.
hipError_t setup_static_scratch(int device, void** out) {
    *out = nullptr;
    if (device < 0 || device >= kMaxDevices) {
        return hipErrorInvalidDevice;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[device] == nullptr) {
        void* p = nullptr;
        hipError_t status = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (status != hipSuccess) {
            return status;
        }
        if (p == nullptr) {
            return hipErrorInvalidSymbol;
        }
        status = hipMemset(p, 0, static_cast<size_t>(kNoAllocCounterBytes));
        if (status == hipSuccess) {
            status = hipDeviceSynchronize();
        }
        if (status != hipSuccess) {
            return status;
        }
        g_scratch_ptr[device] = p;
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

struct Handle {
    explicit Handle(int id) : device_id(id) {}
    ~Handle() {
        if (graph_exec != nullptr) {
            (void)hipGraphExecDestroy(graph_exec);
        }
        if (graph != nullptr) {
            (void)hipGraphDestroy(graph);
        }
        if (scratch != nullptr) {
            (void)hipFree(scratch);
        }
        if (scratch_event != nullptr) {
            (void)hipEventDestroy(scratch_event);
        }
    }
    void set_error(const std::string& message) { last_error = message; }
    void set_hip_error(const char* operation, hipError_t status) {
        last_error = std::string(operation) + ": " + hipGetErrorString(status);
    }

    int device_id;
    bool device_ready = false;
    bool frozen = false;
    bool capturing = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    std::string last_error;
    // fixed scratch for the standalone attention / argmax entry points
    void* scratch = nullptr;
    float* gqa_partials = nullptr;
    float* gemm_partials = nullptr;  // kc::kGemmScratchFloats (split-K of the prefill GEMMs)
    float* lm_best = nullptr;
    uint32_t* counters = nullptr;  // [0..1] attention tickets
    int32_t* argmax_slot = nullptr;
    // this device's copy of the file-scope `scratch` array (device address)
    unsigned char* static_scratch = nullptr;
    // the last scratch-using launch: its stream (compared, never queried)
    // and an event recorded behind it (claim_scratch / scratch_launched)
    hipStream_t scratch_stream = nullptr;
    hipEvent_t scratch_event = nullptr;
    bool scratch_used = false;
    // a scratch-using call was recorded into the capture begun by
    // kudacuda_begin_capture / the instantiated graph holds one: its replays
    // take part in the claim like eager calls
    bool capture_uses_scratch = false;
    bool graph_uses_scratch = false;
};

Handle* as_handle(void* raw) { return reinterpret_cast<Handle*>(raw); }

template <typename T>
T* ptr(uint64_t v) {
    return reinterpret_cast<T*>(static_cast<uintptr_t>(v));
}

hipStream_t as_stream(uint64_t v) { return reinterpret_cast<hipStream_t>(static_cast<uintptr_t>(v)); }

// Shared prologue: valid handle, frozen.
bool ready(Handle* h, const char* symbol) {
    if (h == nullptr) {
        return false;
    }
    if (!h->frozen) {
        h->set_error(std::string(symbol) + " called before kudacuda_freeze");
        return false;
    }
    return true;
}

// Calls that use the handle's scratch (split partials, ticket counters,
// argmax winners, GEMM partials) must not overlap on the GPU.  After each
// such launch the handle records its own event on the launch's stream; a
// call on another stream is refused while that event has not completed (the
// previous launch may still be using the scratch).  Only the handle's event
// is queried: the previous stream may have been destroyed since.  A call on
// the same stream is ordered after the previous one.  Launches recorded into
// a stream capture are not checked: they run when the graph is replayed.  A
// graph captured through kudacuda_begin_capture that holds such launches is
// checked at kudacuda_replay_graph instead (claimed on the replay stream, the
// event recorded behind the replay); graphs captured by other means share
// the handle's scratch unchecked, so their replays must not overlap.
bool capturing(hipStream_t s) {
    if (s == nullptr) {
        return false;  // the legacy stream is never captured (and asking it during a global capture is unsafe)
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    const hipError_t q = hipStreamIsCapturing(s, &cs);
    (void)hipGetLastError();
    return q == hipSuccess && cs != hipStreamCaptureStatusNone;
}

bool claim_scratch(Handle* h, const char* symbol, hipStream_t s) {
    if (capturing(s)) {
        h->capture_uses_scratch = true;
        return true;
    }
    if (!h->scratch_used || s == h->scratch_stream) {
        return true;
    }
    const hipError_t q = hipEventQuery(h->scratch_event);
    (void)hipGetLastError();  // "not ready" is an answer, not an error
    if (q == hipErrorNotReady) {
        h->set_error(std::string(symbol) +
                     ": the handle's scratch is in use by work still queued on another stream; "
                     "synchronise that stream first or use one handle per stream");
        return false;
    }
    return true;
}

// Records the handle's event behind a scratch-using launch (not into a
// capture); passes the launch status through.
hipError_t scratch_launched(Handle* h, hipStream_t s, hipError_t launch) {
    if (launch != hipSuccess || capturing(s)) {
        return launch;
    }
    const hipError_t rec = hipEventRecord(h->scratch_event, s);
    if (rec != hipSuccess) {
        return rec;
    }
    h->scratch_stream = s;
    h->scratch_used = true;
    return hipSuccess;
}

int finish(Handle* h, const char* operation, hipError_t status) {
    if (status != hipSuccess) {
        h->set_hip_error(operation, status);
        return 1;
    }
    h->last_error.clear();
    return 0;
}

// split plan of a cache of `capacity` rows into the launch arguments
void set_gqa_plan(GqaArgs& a, int64_t capacity, int64_t split_limit) {
    const GqaPlan p = gqa_plan(capacity, split_limit);
    a.capacity = capacity;
    a.split_cap = p.split_cap;
    a.max_splits = p.max_splits;
}

// splits the decode step's attention leaves for o_proj to merge
int64_t model_defer(int64_t max_splits) { return max_splits < kGqaMaxDefer ? max_splits : kGqaMaxDefer; }

int64_t gqa_workspace(int64_t tokens) { return 16 * gqa_plan(tokens, 0).max_splits * 130; }

const char* const kGfx950Tactics[] = {
    "qwen2_gqa_decode_gfx950_fp16",
    "qwen2_gqa_decode_gfx950_bf16",
    "qwen2_gqa_decode_gfx950_fp16_graph_v1",
    "qwen2_gqa_decode_gfx950_bf16_graph_v1",
    "qwen2_gqa_decode_gfx950_fp16_group_tiled_v2",
    "qwen2_gqa_decode_gfx950_fp16_vectorized_v2",
    "qwen2_gqa_decode_gfx950_fp16_workspace_v3",
    "qwen2_gqa_decode_sm86_fp16",
    "qwen2_gqa_decode_sm89_fp16",
    "qwen2_gqa_decode_sm86_fp16_group_tiled_v2",
    "qwen2_gqa_decode_sm89_fp16_group_tiled_v2",
    "qwen2_gqa_decode_sm86_fp16_vectorized_v2",
    "qwen2_gqa_decode_sm89_fp16_vectorized_v2",
    "qwen2_gqa_decode_sm86_fp16_graph_v1",
    "qwen2_gqa_decode_sm89_fp16_graph_v1",
};

// ------------------------------------------------------------- NF4 QKV
int qkv_common(void* raw, const char* symbol, Act act, uint64_t input, uint64_t norm_weight, uint64_t qw,
               uint64_t qa, uint64_t qb, uint64_t kw, uint64_t ka, uint64_t kb, uint64_t vw, uint64_t va, uint64_t vb,
               uint64_t normalized, bool need_normalized, uint64_t qo, uint64_t ko, uint64_t vo, int64_t rows,
               int64_t hidden, int64_t q_out, int64_t kv_out, int64_t blocksize, float epsilon, uint64_t stream) {
    Handle* h = as_handle(raw);
    const std::string name = std::string("kudacuda_") + symbol;
    if (!ready(h, name.c_str())) {
        return 1;
    }
    if (input == 0 || norm_weight == 0 || qw == 0 || qa == 0 || qb == 0 || kw == 0 || ka == 0 || kb == 0 || vw == 0 ||
        va == 0 || vb == 0 || qo == 0 || ko == 0 || vo == 0 || (need_normalized && normalized == 0)) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (rows != 1 || hidden != 2048 || q_out != 2048 || kv_out != 256 || blocksize != 64 || !(epsilon > 0.0f)) {
        h->set_error(std::string(symbol) +
                     " requires rows=1, hidden=2048, q_out=2048, kv_out=256, blocksize=64, and positive epsilon");
        return 1;
    }
    Nf4RowsArgs a;
    a.x = ptr<const uint16_t>(input);
    a.gamma = ptr<const uint16_t>(norm_weight);
    a.eps = epsilon;
    a.w[0] = ptr<const uint8_t>(qw);
    a.w[1] = ptr<const uint8_t>(kw);
    a.w[2] = ptr<const uint8_t>(vw);
    a.absmax[0] = ptr<const float>(qa);
    a.absmax[1] = ptr<const float>(ka);
    a.absmax[2] = ptr<const float>(va);
    a.bias[0] = ptr<const uint16_t>(qb);
    a.bias[1] = ptr<const uint16_t>(kb);
    a.bias[2] = ptr<const uint16_t>(vb);
    a.out[0] = ptr<uint16_t>(qo);
    a.out[1] = ptr<uint16_t>(ko);
    a.out[2] = ptr<uint16_t>(vo);
    a.rows[0] = q_out;
    a.rows[1] = kv_out;
    a.rows[2] = kv_out;
    a.norm_out = ptr<float>(normalized);
    return finish(h, symbol, launch_nf4_rows2048(RowMode::kQkv, act, a, as_stream(stream)));
}

int swiglu_common(void* raw, const char* symbol, Act act, uint64_t input, uint64_t norm_weight, uint64_t gw,
                  uint64_t ga, uint64_t uw, uint64_t ua, uint64_t output, int64_t rows, int64_t hidden,
                  int64_t intermediate, int64_t blocksize, float epsilon, uint64_t stream, bool clear_error) {
    Handle* h = as_handle(raw);
    const std::string name = std::string("kudacuda_") + symbol;
    if (!ready(h, name.c_str())) {
        return 1;
    }
    if (input == 0 || norm_weight == 0 || gw == 0 || ga == 0 || uw == 0 || ua == 0 || output == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (rows != 1 || hidden != 2048 || intermediate != 11008 || blocksize != 64 || !(epsilon > 0.0f)) {
        h->set_error(std::string(symbol) +
                     " requires rows=1, hidden=2048, intermediate=11008, blocksize=64, and positive epsilon");
        return 1;
    }
    Nf4RowsArgs a;
    a.x = ptr<const uint16_t>(input);
    a.gamma = ptr<const uint16_t>(norm_weight);
    a.eps = epsilon;
    a.w[0] = ptr<const uint8_t>(gw);
    a.w[1] = ptr<const uint8_t>(uw);
    a.absmax[0] = ptr<const float>(ga);
    a.absmax[1] = ptr<const float>(ua);
    a.out[0] = ptr<uint16_t>(output);
    a.rows[0] = intermediate;
    a.rows[1] = intermediate;
    const hipError_t status = launch_nf4_rows2048(RowMode::kSwiGlu, act, a, as_stream(stream));
    if (status != hipSuccess) {
        h->set_hip_error(symbol, status);
        return 1;
    }
    if (clear_error) {
        h->last_error.clear();
    }
    return 0;
}

// ------------------------------------------------------------------ GQA
struct GqaShape {
    int64_t batch, query_len, query_heads, kv_heads, head_dim;
    float scale;
};

bool gqa_shape_ok(Handle* h, const char* symbol, const GqaShape& s, const char* len_name, int64_t len,
                  int64_t len_max) {
    if (s.batch != 1 || s.query_len != 1 || len < 1 || len > len_max || s.query_heads != 16 || s.kv_heads != 2 ||
        s.head_dim != 128) {
        h->set_error(std::string(symbol) + " requires batch=1, query_len=1, " + len_name + "=1.." +
                     std::to_string(len_max) + ", q_heads=16, kv_heads=2, head_dim=128");
        return false;
    }
    if (!(s.scale > 0.0f)) {
        h->set_error(std::string(symbol) + " scale must be positive");
        return false;
    }
    return true;
}

int gqa_direct(void* raw, const char* symbol, Act act, uint64_t q, uint64_t k, uint64_t v, uint64_t out,
               const GqaShape& s, int64_t kv_len, uint64_t stream) {
    Handle* h = as_handle(raw);
    const std::string name = std::string("kudacuda_") + symbol;
    if (!ready(h, name.c_str())) {
        return 1;
    }
    if (q == 0 || k == 0 || v == 0 || out == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (!gqa_shape_ok(h, symbol, s, "kv_len", kv_len, kMaxStandaloneKv)) {
        return 1;
    }
    GqaArgs a;
    a.q = ptr<const uint16_t>(q);
    a.k = ptr<const uint16_t>(k);
    a.v = ptr<const uint16_t>(v);
    a.out = ptr<uint16_t>(out);
    a.partials = h->gqa_partials;
    a.counters = h->counters;
    a.kv_len_host = kv_len;
    set_gqa_plan(a, kv_len, 0);
    a.qk_scale_log2 = s.scale * kLog2e;
    if (!claim_scratch(h, symbol, as_stream(stream))) {
        return 1;
    }
    if (kv_len >= kGqaMfmaMinKv) {
        // long caches: the matrix-core tactic (scores and weighted sum on MFMA)
        a.split_cap = kGqaMfmaSplitCap;
        // 2-wave blocks (64-token units) while one unit per split fits the
        // cap: twice the blocks of 4-wave ones to spread the stream over
        a.mfma_quantum = kv_len <= 64 * kGqaMfmaSplitCap ? 64 : kGqaMfmaQuantum;
        a.max_splits = gqa_mfma_split_count(kv_len, a.split_cap, a.mfma_quantum);
        return finish(h, symbol,
                      scratch_launched(h, as_stream(stream), launch_gqa_decode_mfma(act, a, as_stream(stream))));
    }
    return finish(h, symbol, scratch_launched(h, as_stream(stream), launch_gqa_decode(act, a, as_stream(stream))));
}

// no_alloc: split partials and counters come from this device's copy of the
// file-scope `scratch` array instead of the handle's allocation
int gqa_graph(void* raw, const char* symbol, Act act, uint64_t q, uint64_t k, uint64_t v, uint64_t out,
              const GqaShape& s, int64_t kv_capacity, uint64_t kv_len_device, uint64_t stream,
              bool no_alloc = false) {
    Handle* h = as_handle(raw);
    const std::string name = std::string("kudacuda_") + symbol;
    if (!ready(h, name.c_str())) {
        return 1;
    }
    if (q == 0 || k == 0 || v == 0 || out == 0 || kv_len_device == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (!gqa_shape_ok(h, symbol, s, "kv_capacity", kv_capacity, no_alloc ? kNoAllocMaxKv : kMaxStandaloneKv)) {
        return 1;
    }
    GqaArgs a;
    a.q = ptr<const uint16_t>(q);
    a.k = ptr<const uint16_t>(k);
    a.v = ptr<const uint16_t>(v);
    a.out = ptr<uint16_t>(out);
    a.kv_len_device = ptr<const int32_t>(kv_len_device);
    set_gqa_plan(a, kv_capacity, 0);
    if (no_alloc) {
        if (h->static_scratch == nullptr) {
            h->set_error(std::string(symbol) + ": the static device scratch of this device is not set up");
            return 1;
        }
        if (16 * a.max_splits * kGqaPartialStride > kNoAllocPartialFloats) {
            h->set_error(std::string(symbol) + ": kv_capacity " + std::to_string(kv_capacity) +
                         " needs more split partials than the static scratch holds");
            return 1;
        }
        a.counters = reinterpret_cast<uint32_t*>(h->static_scratch);
        a.partials = reinterpret_cast<float*>(h->static_scratch + kNoAllocCounterBytes);
    } else {
        a.partials = h->gqa_partials;
        a.counters = h->counters;
        if (!claim_scratch(h, symbol, as_stream(stream))) {
            return 1;
        }
    }
    a.qk_scale_log2 = s.scale * kLog2e;
    const hipError_t launched = launch_gqa_decode(act, a, as_stream(stream));
    return finish(h, symbol, no_alloc ? launched : scratch_launched(h, as_stream(stream), launched));
}

// ---------------------------------------------------------------- model
struct Model {
    Handle* handle = nullptr;
    int64_t num_layers = 0;
    int64_t vocab = 0;
    int64_t capacity = 0;
    float eps = 1e-6f;
    std::vector<std::array<uint64_t, KUDACUDA_QWEN2_LAYER_FIELDS>> layers;
    std::array<uint64_t, KUDACUDA_QWEN2_MODEL_FIELDS> g{};
    hipGraph_t graph = nullptr;
    // the captured step in each of its forms (index = form, see model_op);
    // forms 1 .. step_defer_cap always, form 0 when the cache can need it
    std::array<hipGraphExec_t, kGqaMaxDefer + 1> execs{};
    // the step (control[0]) the next launch runs at, as far as the host
    // knows (-1: unknown); only picks among the step forms, which compute
    // the same results
    int64_t host_step = -1;
    ~Model() {
        for (hipGraphExec_t e : execs) {
            if (e != nullptr) {
                (void)hipGraphExecDestroy(e);
            }
        }
        if (graph != nullptr) {
            (void)hipGraphDestroy(graph);
        }
    }
};

// The step's deferral cap: splits attention leaves for o_proj to merge.
int64_t step_defer_cap(const Model& m) {
    GqaArgs plan;
    set_gqa_plan(plan, m.capacity, kGqaStepSplits);
    return model_defer(plan.max_splits);
}

// The form of a step whose position the host does not know: six deferral
// slots (one-round splits up to 192 cached tokens), the plan callers had
// before positions were tracked.
constexpr int64_t kUnknownStepForm = 6;

// form (ops 1 and 2 only): k = 1 .. step_defer_cap -- attention leaves up to
// k splits to o_proj, whose merge prologue requests exactly k split slots,
// and merges more by its own ticket (no merge launch in the graph); -1: the
// unknown-position form, kUnknownStepForm (or the cap, if smaller); 0 -- the
// form for caches whose split count exceeds the cap:
// attention's partials all go to gqa_merge_kernel (one more launch, parallel
// over heads and dims) and o_proj reads the merged vector as a plain GEMV.
// Every form merges by the same rule in the same order: identical results at
// any length, only the time differs.
hipError_t model_op(const Model& m, int op, int64_t layer, bool bookkeeping, hipStream_t stream,
                    int form = -1) {
    const bool long_ctx = form == 0;
    const int64_t cap = step_defer_cap(m);
    const int64_t want = form < 0 ? kUnknownStepForm : form;
    const int64_t defer = want < cap ? want : cap;
    const auto& L = m.layers[static_cast<size_t>(layer)];
    const auto& G = m.g;
    switch (op) {
        case 0: {
            Nf4RowsArgs a;
            a.x = ptr<const uint16_t>(G[KUDACUDA_QWEN2_HIDDEN]);
            a.gamma = ptr<const uint16_t>(L[KUDACUDA_QWEN2_INPUT_NORM]);
            a.eps = m.eps;
            a.w[0] = ptr<const uint8_t>(L[KUDACUDA_QWEN2_Q_PACKED]);
            a.w[1] = ptr<const uint8_t>(L[KUDACUDA_QWEN2_K_PACKED]);
            a.w[2] = ptr<const uint8_t>(L[KUDACUDA_QWEN2_V_PACKED]);
            a.absmax[0] = ptr<const float>(L[KUDACUDA_QWEN2_Q_ABSMAX]);
            a.absmax[1] = ptr<const float>(L[KUDACUDA_QWEN2_K_ABSMAX]);
            a.absmax[2] = ptr<const float>(L[KUDACUDA_QWEN2_V_ABSMAX]);
            a.bias[0] = ptr<const uint16_t>(L[KUDACUDA_QWEN2_Q_BIAS]);
            a.bias[1] = ptr<const uint16_t>(L[KUDACUDA_QWEN2_K_BIAS]);
            a.bias[2] = ptr<const uint16_t>(L[KUDACUDA_QWEN2_V_BIAS]);
            a.out[0] = ptr<uint16_t>(G[KUDACUDA_QWEN2_QUERY]);
            a.rows[0] = 2048;
            a.rows[1] = 256;
            a.rows[2] = 256;
            a.rope_cos = ptr<const float>(G[KUDACUDA_QWEN2_ROPE_COS]);
            a.rope_sin = ptr<const float>(G[KUDACUDA_QWEN2_ROPE_SIN]);
            a.control = ptr<const int32_t>(G[KUDACUDA_QWEN2_CONTROL]);
            a.done = ptr<const int32_t>(G[KUDACUDA_QWEN2_CONTROL]) + 4;
            a.capacity = m.capacity;
            a.kcache = ptr<uint16_t>(L[KUDACUDA_QWEN2_KEY_CACHE]);
            a.vcache = ptr<uint16_t>(L[KUDACUDA_QWEN2_VALUE_CACHE]);
            if (layer == 0) {
                a.embed = ptr<const uint16_t>(G[KUDACUDA_QWEN2_EMBED]);
                a.tokens = ptr<const int32_t>(G[KUDACUDA_QWEN2_TOKENS]);
                a.vocab = m.vocab;
                a.hidden_out = ptr<uint16_t>(G[KUDACUDA_QWEN2_HIDDEN]);
            }
            return launch_nf4_rows2048(RowMode::kQkvRope, Act::kBf16, a, stream);
        }
        case 1: {
            GqaArgs a;
            a.q = ptr<const uint16_t>(G[KUDACUDA_QWEN2_QUERY]);
            a.k = ptr<const uint16_t>(L[KUDACUDA_QWEN2_KEY_CACHE]);
            a.v = ptr<const uint16_t>(L[KUDACUDA_QWEN2_VALUE_CACHE]);
            a.out = ptr<uint16_t>(G[KUDACUDA_QWEN2_ATTN]);
            a.partials = ptr<float>(G[KUDACUDA_QWEN2_ATTN_PARTIALS]);
            a.counters = ptr<uint32_t>(G[KUDACUDA_QWEN2_ATTN_COUNTERS]);
            a.kv_len_device = ptr<const int32_t>(G[KUDACUDA_QWEN2_CONTROL]);
            a.kv_len_offset = 1;
            set_gqa_plan(a, m.capacity, kGqaStepSplits);
            if (long_ctx) {
                a.defer_max = 0;   // gqa_merge_kernel merges every split count above one
                a.ticket_max = 1;
            } else {
                a.defer_max = defer;  // o_proj merges these
                // the rest by ticket: a merge kernel would be one more graph
                // node per layer even at the lengths that never need it
                a.ticket_max = 32;
            }
            a.qk_scale_log2 = static_cast<float>(1.0 / std::sqrt(128.0)) * kLog2e;
            return launch_gqa_decode(Act::kBf16, a, stream);
        }
        case 2: {
            Nf4RowsArgs a;
            a.x = ptr<const uint16_t>(G[KUDACUDA_QWEN2_ATTN]);
            a.w[0] = ptr<const uint8_t>(L[KUDACUDA_QWEN2_O_PACKED]);
            a.absmax[0] = ptr<const float>(L[KUDACUDA_QWEN2_O_ABSMAX]);
            a.out[0] = ptr<uint16_t>(G[KUDACUDA_QWEN2_HIDDEN]);
            a.residual = ptr<const uint16_t>(G[KUDACUDA_QWEN2_HIDDEN]);
            a.rows[0] = 2048;
            if (long_ctx) {
                return launch_nf4_rows2048(RowMode::kGemv, Act::kBf16, a, stream);  // x merged by op 1
            }
            // attention output: merged here from the partials op 1 left
            GqaArgs plan;
            set_gqa_plan(plan, m.capacity, kGqaStepSplits);
            a.attn.partials = ptr<const float>(G[KUDACUDA_QWEN2_ATTN_PARTIALS]);
            a.attn.out = ptr<uint16_t>(G[KUDACUDA_QWEN2_ATTN]);
            a.attn.kv_len_device = ptr<const int32_t>(G[KUDACUDA_QWEN2_CONTROL]);
            a.attn.kv_len_offset = 1;
            a.attn.capacity = plan.capacity;
            a.attn.split_cap = plan.split_cap;
            a.attn.max_splits = plan.max_splits;
            a.attn.defer_max = defer;
            return launch_nf4_rows2048(RowMode::kGemv, Act::kBf16, a, stream);
        }
        case 3: {
            Nf4RowsArgs a;
            a.x = ptr<const uint16_t>(G[KUDACUDA_QWEN2_HIDDEN]);
            a.gamma = ptr<const uint16_t>(L[KUDACUDA_QWEN2_POST_NORM]);
            a.eps = m.eps;
            a.w[0] = ptr<const uint8_t>(L[KUDACUDA_QWEN2_GATE_PACKED]);
            a.w[1] = ptr<const uint8_t>(L[KUDACUDA_QWEN2_UP_PACKED]);
            a.absmax[0] = ptr<const float>(L[KUDACUDA_QWEN2_GATE_ABSMAX]);
            a.absmax[1] = ptr<const float>(L[KUDACUDA_QWEN2_UP_ABSMAX]);
            a.out[0] = ptr<uint16_t>(G[KUDACUDA_QWEN2_MLP]);
            a.rows[0] = 11008;
            a.rows[1] = 11008;
            return launch_nf4_rows2048(RowMode::kSwiGlu, Act::kBf16, a, stream);
        }
        case 4: {
            Nf4DownArgs a;
            a.x = ptr<const uint16_t>(G[KUDACUDA_QWEN2_MLP]);
            a.w = ptr<const uint8_t>(L[KUDACUDA_QWEN2_DOWN_PACKED]);
            a.absmax = ptr<const float>(L[KUDACUDA_QWEN2_DOWN_ABSMAX]);
            a.residual = ptr<const uint16_t>(G[KUDACUDA_QWEN2_HIDDEN]);
            a.out = ptr<uint16_t>(G[KUDACUDA_QWEN2_HIDDEN]);
            a.rows = 2048;
            return launch_nf4_down11008(Act::kBf16, a, stream);
        }
        case 5: {
            LmHeadArgs a;
            a.x = ptr<const uint16_t>(G[KUDACUDA_QWEN2_HIDDEN]);
            a.gamma = ptr<const uint16_t>(G[KUDACUDA_QWEN2_FINAL_NORM]);
            a.eps = m.eps;
            a.weight = ptr<const uint16_t>(G[KUDACUDA_QWEN2_EMBED]);
            a.vocab = m.vocab;
            a.logits = ptr<uint16_t>(G[KUDACUDA_QWEN2_LOGITS]);
            a.block_best = ptr<float>(G[KUDACUDA_QWEN2_LM_BEST]);
            if (bookkeeping) {
                a.control = ptr<int32_t>(G[KUDACUDA_QWEN2_CONTROL]);
                a.tokens = ptr<int32_t>(G[KUDACUDA_QWEN2_TOKENS]);
            }
            return launch_lm_head_argmax(a, stream);
        }
        default:
            return hipErrorInvalidValue;
    }
}

bool gemm_shape_ok(Handle* h, const char* symbol, int64_t tokens, int64_t in_features, int64_t out_features,
                   int64_t blocksize) {
    if (tokens < 1 || in_features < 128 || in_features % 128 != 0 || out_features < 64 || out_features % 64 != 0 ||
        blocksize != 64) {
        h->set_error(std::string(symbol) +
                     " requires tokens>=1, in_features a positive multiple of 128, out_features a positive "
                     "multiple of 64, and blocksize=64");
        return false;
    }
    return true;
}

// tokens in launches of kGemmMaxTokens rows
hipError_t gemm_chunks(GemmEpi epi, Nf4GemmArgs a, int64_t tokens, hipStream_t stream) {
    const uint16_t* x = a.x;
    const uint16_t* res = a.residual;
    uint16_t* out = a.out;
    uint16_t* norm_out = a.norm_out;
    const int64_t start = a.start;
    const int64_t out_stride = epi == GemmEpi::kQkvRope ? a.q_rows : a.n;
    for (int64_t m0 = 0; m0 < tokens; m0 += kGemmMaxTokens) {
        a.m = tokens - m0 < kGemmMaxTokens ? tokens - m0 : kGemmMaxTokens;
        a.x = x + m0 * a.k;
        a.residual = res != nullptr ? res + m0 * a.n : nullptr;
        a.out = out + m0 * out_stride;
        a.norm_out = norm_out != nullptr ? norm_out + m0 * a.n : nullptr;
        a.start = start + m0;
        const hipError_t status = launch_nf4_gemm(epi, a, stream);
        if (status != hipSuccess) {
            return status;
        }
    }
    return hipSuccess;
}

// Prefill of `count` tokens at positions start .. start+count-1 (token ids
// from the device token array) through every layer at once, then the final
// norm + lm_head + argmax of the last row with the decode bookkeeping
// (tokens[start+count] = argmax, step = start+count).  Workspace per token:
// hidden, normalised x, rotated q, attention output (bf16 [2048] each) and
// the SwiGLU output (bf16 [11008]); then the GEMMs' split-K scratch.  k and v
// go straight into the caches.
constexpr int64_t kPrefillBytesPerToken = (4 * 2048 + 11008) * 2;
constexpr int64_t kPrefillFixedBytes = kGemmScratchFloats * 4;

hipError_t model_prefill(const Model& m, uint8_t* ws, int64_t start, int64_t count, hipStream_t stream) {
    const auto& G = m.g;
    uint16_t* hidden = reinterpret_cast<uint16_t*>(ws);
    uint16_t* xn = hidden + count * 2048;
    uint16_t* q = xn + count * 2048;
    uint16_t* attn = q + count * 2048;
    uint16_t* mlp = attn + count * 2048;
    float* gemm_partials = reinterpret_cast<float*>(ws + count * kPrefillBytesPerToken);
    const float qk_scale_log2 = static_cast<float>(1.0 / std::sqrt(128.0)) * kLog2e;
    hipError_t st = hipSuccess;
    // kResidualNorm: out += the product (residual stream in place), then the
    // row RMSNorm with `gamma` (null: none) into xn for the next GEMM
    auto gemm = [&](GemmEpi epi, const uint16_t* x, uint64_t w0, uint64_t a0, uint64_t w1, uint64_t a1,
                    uint16_t* out, int64_t n, int64_t kdim, const uint16_t* gamma) {
        Nf4GemmArgs a;
        a.x = x;
        a.w[0] = ptr<const uint8_t>(w0);
        a.absmax[0] = ptr<const float>(a0);
        a.w[1] = ptr<const uint8_t>(w1);
        a.absmax[1] = ptr<const float>(a1);
        a.residual = epi == GemmEpi::kResidualNorm ? out : nullptr;
        a.out = out;
        a.n = n;
        a.k = kdim;
        a.partials = gemm_partials;
        a.partial_floats = kGemmScratchFloats;
        a.norm_gamma = gamma;
        a.norm_out = gamma != nullptr ? xn : nullptr;
        a.eps = m.eps;
        return gemm_chunks(epi, a, count, stream);
    };
    for (int64_t layer = 0; layer < m.num_layers && st == hipSuccess; ++layer) {
        const auto& L = m.layers[static_cast<size_t>(layer)];
        if (layer == 0) {
            // embedding rows -> hidden, input norm -> xn (later layers get xn
            // from the previous layer's down-projection reduce)
            PrefillNormArgs na;
            na.gamma = ptr<const uint16_t>(L[KUDACUDA_QWEN2_INPUT_NORM]);
            na.eps = m.eps;
            na.out = xn;
            na.m = count;
            na.embed = ptr<const uint16_t>(G[KUDACUDA_QWEN2_EMBED]);
            na.tokens = ptr<const int32_t>(G[KUDACUDA_QWEN2_TOKENS]);
            na.control = ptr<const int32_t>(G[KUDACUDA_QWEN2_CONTROL]);
            na.vocab = m.vocab;
            na.start = start;
            na.hidden_out = hidden;
            st = launch_prefill_norm(na, stream);
        }
        if (st == hipSuccess) {
            // Q, K and V in one GEMM; its split reduce adds the biases, applies
            // RoPE and writes k and v into the caches
            Nf4GemmArgs a;
            a.x = xn;
            a.w[0] = ptr<const uint8_t>(L[KUDACUDA_QWEN2_Q_PACKED]);
            a.w[1] = ptr<const uint8_t>(L[KUDACUDA_QWEN2_K_PACKED]);
            a.w[2] = ptr<const uint8_t>(L[KUDACUDA_QWEN2_V_PACKED]);
            a.absmax[0] = ptr<const float>(L[KUDACUDA_QWEN2_Q_ABSMAX]);
            a.absmax[1] = ptr<const float>(L[KUDACUDA_QWEN2_K_ABSMAX]);
            a.absmax[2] = ptr<const float>(L[KUDACUDA_QWEN2_V_ABSMAX]);
            a.seg_bias[0] = ptr<const uint16_t>(L[KUDACUDA_QWEN2_Q_BIAS]);
            a.seg_bias[1] = ptr<const uint16_t>(L[KUDACUDA_QWEN2_K_BIAS]);
            a.seg_bias[2] = ptr<const uint16_t>(L[KUDACUDA_QWEN2_V_BIAS]);
            a.out = q;
            a.q_rows = 2048;
            a.kv_rows = 256;
            a.n = 2048 + 2 * 256;
            a.k = 2048;
            a.rope_cos = ptr<const float>(G[KUDACUDA_QWEN2_ROPE_COS]);
            a.rope_sin = ptr<const float>(G[KUDACUDA_QWEN2_ROPE_SIN]);
            a.kcache = ptr<uint16_t>(L[KUDACUDA_QWEN2_KEY_CACHE]);
            a.vcache = ptr<uint16_t>(L[KUDACUDA_QWEN2_VALUE_CACHE]);
            a.capacity = m.capacity;
            a.start = start;
            a.partials = gemm_partials;
            a.partial_floats = kGemmScratchFloats;
            st = gemm_chunks(GemmEpi::kQkvRope, a, count, stream);
        }
        if (st == hipSuccess) {
            PrefillAttnArgs aa;
            aa.q = q;
            aa.kcache = ptr<const uint16_t>(L[KUDACUDA_QWEN2_KEY_CACHE]);
            aa.vcache = ptr<const uint16_t>(L[KUDACUDA_QWEN2_VALUE_CACHE]);
            aa.out = attn;
            aa.capacity = m.capacity;
            aa.start = start;
            aa.m = count;
            aa.qk_scale_log2 = qk_scale_log2;
            st = launch_prefill_attention(aa, stream);
        }
        if (st == hipSuccess) {
            st = gemm(GemmEpi::kResidualNorm, attn, L[KUDACUDA_QWEN2_O_PACKED], L[KUDACUDA_QWEN2_O_ABSMAX], 0, 0,
                      hidden, 2048, 2048, ptr<const uint16_t>(L[KUDACUDA_QWEN2_POST_NORM]));
        }
        if (st == hipSuccess) {
            st = gemm(GemmEpi::kSwiGlu, xn, L[KUDACUDA_QWEN2_GATE_PACKED], L[KUDACUDA_QWEN2_GATE_ABSMAX],
                      L[KUDACUDA_QWEN2_UP_PACKED], L[KUDACUDA_QWEN2_UP_ABSMAX], mlp, 11008, 2048, nullptr);
        }
        if (st == hipSuccess) {
            const bool last = layer + 1 == m.num_layers;
            const uint16_t* next_norm =
                last ? nullptr : ptr<const uint16_t>(m.layers[static_cast<size_t>(layer + 1)][KUDACUDA_QWEN2_INPUT_NORM]);
            st = gemm(GemmEpi::kResidualNorm, mlp, L[KUDACUDA_QWEN2_DOWN_PACKED], L[KUDACUDA_QWEN2_DOWN_ABSMAX], 0, 0,
                      hidden, 2048, 11008, next_norm);
        }
    }
    if (st != hipSuccess) {
        return st;
    }
    st = launch_set_step(ptr<int32_t>(G[KUDACUDA_QWEN2_CONTROL]), static_cast<int32_t>(start + count - 1), stream);
    if (st != hipSuccess) {
        return st;
    }
    LmHeadArgs a;
    a.x = hidden + (count - 1) * 2048;
    a.gamma = ptr<const uint16_t>(G[KUDACUDA_QWEN2_FINAL_NORM]);
    a.eps = m.eps;
    a.weight = ptr<const uint16_t>(G[KUDACUDA_QWEN2_EMBED]);
    a.vocab = m.vocab;
    a.logits = ptr<uint16_t>(G[KUDACUDA_QWEN2_LOGITS]);
    a.block_best = ptr<float>(G[KUDACUDA_QWEN2_LM_BEST]);
    a.control = ptr<int32_t>(G[KUDACUDA_QWEN2_CONTROL]);
    a.tokens = ptr<int32_t>(G[KUDACUDA_QWEN2_TOKENS]);
    return launch_lm_head_argmax(a, stream);
}

// The fastest form for the step at `step` (kv_len step + 1): the split
// count itself while o_proj merges it, form 0 past the cap, kUnknownStepForm
// (or the cap, if smaller) when the step is unknown.
int step_form(const Model& m, int64_t step) {
    const int64_t cap = step_defer_cap(m);
    if (step < 0) {
        return static_cast<int>(cap < kUnknownStepForm ? cap : kUnknownStepForm);
    }
    GqaArgs plan;
    set_gqa_plan(plan, m.capacity, kGqaStepSplits);
    const int64_t kv_len = step + 1 < m.capacity ? step + 1 : m.capacity;
    const int64_t nsplit = gqa_split_count(kv_len, plan.split_cap);
    return nsplit > cap ? 0 : static_cast<int>(nsplit < 1 ? 1 : nsplit);
}

// Whether a cache of the model's capacity can need form 0 at all.
bool long_form_possible(const Model& m) { return step_form(m, m.capacity - 1) == 0; }

hipError_t model_step(const Model& m, hipStream_t stream, int form = -1) {
    for (int64_t layer = 0; layer < m.num_layers; ++layer) {
        for (int op = 0; op < 5; ++op) {
            const hipError_t status = model_op(m, op, layer, true, stream, form);
            if (status != hipSuccess) {
                return status;
            }
        }
    }
    return model_op(m, 5, 0, true, stream);
}

}  // namespace
}  // namespace kc

using kc::Act;
using kc::as_handle;
using kc::as_stream;
using kc::finish;
using kc::Handle;
using kc::ptr;
using kc::ready;
using kc::claim_scratch;
using kc::scratch_launched;

extern "C" {

void* kudacuda_create(int device_id) {
    auto* h = new (std::nothrow) Handle(device_id);
    if (h == nullptr) {
        return nullptr;
    }
    hipError_t status = hipSetDevice(device_id);
    if (status != hipSuccess) {
        h->set_hip_error("hipSetDevice", status);
        return h;
    }
    const size_t partial_bytes = static_cast<size_t>(kc::gqa_workspace(kc::kMaxStandaloneKv)) * sizeof(float);
    const size_t best_bytes = static_cast<size_t>(kc::lm_head_workspace_floats()) * sizeof(float);
    const size_t counter_bytes = 64;
    const size_t gemm_bytes = static_cast<size_t>(kc::kGemmScratchFloats) * sizeof(float);
    const size_t total = partial_bytes + best_bytes + counter_bytes + gemm_bytes;
    status = hipMalloc(&h->scratch, total);
    if (status != hipSuccess) {
        h->scratch = nullptr;
        h->set_hip_error("hipMalloc(handle scratch)", status);
        return h;
    }
    char* base = static_cast<char*>(h->scratch);
    h->gqa_partials = reinterpret_cast<float*>(base);
    h->lm_best = reinterpret_cast<float*>(base + partial_bytes);
    h->counters = reinterpret_cast<uint32_t*>(base + partial_bytes + best_bytes);
    h->argmax_slot = reinterpret_cast<int32_t*>(base + partial_bytes + best_bytes + 32);
    h->gemm_partials = reinterpret_cast<float*>(base + partial_bytes + best_bytes + counter_bytes);
    status = hipMemset(h->counters, 0, counter_bytes);
    if (status == hipSuccess) {
        status = hipDeviceSynchronize();
    }
    if (status != hipSuccess) {
        h->set_hip_error("hipMemset(handle counters)", status);
        return h;
    }
    status = hipEventCreateWithFlags(&h->scratch_event, hipEventDisableTiming);
    if (status != hipSuccess) {
        h->scratch_event = nullptr;
        h->set_hip_error("hipEventCreateWithFlags(handle scratch event)", status);
        return h;
    }
    void* static_scratch = nullptr;
    status = kc::setup_static_scratch(device_id, &static_scratch);
    if (status != hipSuccess) {
        h->set_hip_error("hipGetSymbolAddress(scratch)", status);
        return h;
    }
    h->static_scratch = static_cast<unsigned char*>(static_scratch);
    h->device_ready = true;
    return h;
}

int kudacuda_freeze(void* raw) {
    Handle* h = as_handle(raw);
    if (h == nullptr) {
        return 1;
    }
    if (!h->device_ready) {
        if (h->last_error.empty()) {
            h->set_error("HIP device is not ready");
        }
        return 1;
    }
    h->frozen = true;
    h->last_error.clear();
    return 0;
}

int kudacuda_can_dispatch(void* raw, const char* tactic_name, int64_t batch_size, int64_t seq_len) {
    const Handle* h = as_handle(raw);
    if (h == nullptr || !h->frozen || tactic_name == nullptr || batch_size <= 0 || seq_len <= 0) {
        return 0;
    }
    for (const char* name : kc::kGfx950Tactics) {
        if (std::strcmp(tactic_name, name) == 0) {
            return batch_size == 1 && seq_len == 1 ? 1 : 0;
        }
    }
    return std::strcmp(tactic_name, "vector_add") == 0 || std::strcmp(tactic_name, "rmsnorm") == 0 ? 1 : 0;
}

int kudacuda_vector_add(void* raw, uint64_t a, uint64_t b, uint64_t output, int64_t count, uint64_t stream) {
    Handle* h = as_handle(raw);
    if (!ready(h, "kudacuda_vector_add")) {
        return 1;
    }
    if (a == 0 || b == 0 || output == 0) {
        h->set_error("vector_add requires non-null device pointers");
        return 1;
    }
    if (count <= 0) {
        h->set_error("vector_add count must be positive");
        return 1;
    }
    return finish(h, "vector_add_kernel",
                  kc::launch_vector_add(ptr<const float>(a), ptr<const float>(b), ptr<float>(output), count,
                                        as_stream(stream)));
}

int kudacuda_rmsnorm(void* raw, uint64_t input, uint64_t weight, uint64_t output, int64_t rows, int64_t hidden,
                     float epsilon, uint64_t stream) {
    Handle* h = as_handle(raw);
    if (!ready(h, "kudacuda_rmsnorm")) {
        return 1;
    }
    if (input == 0 || weight == 0 || output == 0) {
        h->set_error("rmsnorm requires non-null device pointers");
        return 1;
    }
    if (rows <= 0 || hidden <= 0) {
        h->set_error("rmsnorm rows and hidden must be positive");
        return 1;
    }
    if (!(epsilon > 0.0f)) {
        h->set_error("rmsnorm epsilon must be positive");
        return 1;
    }
    return finish(h, "rmsnorm_kernel",
                  kc::launch_rmsnorm_f32(ptr<const float>(input), ptr<const float>(weight), ptr<float>(output), rows,
                                         hidden, epsilon, as_stream(stream)));
}

int kudacuda_fused_rmsnorm_qkv(void* raw, uint64_t input, uint64_t norm_weight, uint64_t qkv_weight, uint64_t bias,
                               uint64_t output, int64_t rows, int64_t hidden, float epsilon, uint64_t stream) {
    Handle* h = as_handle(raw);
    if (!ready(h, "kudacuda_fused_rmsnorm_qkv")) {
        return 1;
    }
    if (input == 0 || norm_weight == 0 || qkv_weight == 0 || output == 0) {
        h->set_error("fused_rmsnorm_qkv requires non-null input, weights, and output pointers");
        return 1;
    }
    if (rows <= 0 || hidden <= 0 || !(epsilon > 0.0f)) {
        h->set_error("fused_rmsnorm_qkv requires positive rows, hidden, and epsilon");
        return 1;
    }
    return finish(h, "fused_rmsnorm_qkv_kernel",
                  kc::launch_dense_rmsnorm_qkv_f16(ptr<const uint16_t>(input), ptr<const uint16_t>(norm_weight),
                                                   ptr<const uint16_t>(qkv_weight), ptr<const uint16_t>(bias),
                                                   ptr<uint16_t>(output), rows, hidden, epsilon, as_stream(stream)));
}

int kudacuda_qwen2_fused_rmsnorm_qkv_nf4(void* raw, uint64_t input, uint64_t norm_weight, uint64_t q_weight_packed,
                                         uint64_t q_absmax, uint64_t q_bias, uint64_t k_weight_packed,
                                         uint64_t k_absmax, uint64_t k_bias, uint64_t v_weight_packed,
                                         uint64_t v_absmax, uint64_t v_bias, uint64_t q_output, uint64_t k_output,
                                         uint64_t v_output, int64_t rows, int64_t hidden, int64_t q_out,
                                         int64_t kv_out, int64_t blocksize, float epsilon, uint64_t stream) {
    return kc::qkv_common(raw, "qwen2_fused_rmsnorm_qkv_nf4", Act::kF16, input, norm_weight, q_weight_packed, q_absmax,
                          q_bias, k_weight_packed, k_absmax, k_bias, v_weight_packed, v_absmax, v_bias, 0, false,
                          q_output, k_output, v_output, rows, hidden, q_out, kv_out, blocksize, epsilon, stream);
}

int kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v2(void* raw, uint64_t input, uint64_t norm_weight,
                                            uint64_t q_weight_packed, uint64_t q_absmax, uint64_t q_bias,
                                            uint64_t k_weight_packed, uint64_t k_absmax, uint64_t k_bias,
                                            uint64_t v_weight_packed, uint64_t v_absmax, uint64_t v_bias,
                                            uint64_t normalized_workspace, uint64_t q_output, uint64_t k_output,
                                            uint64_t v_output, int64_t rows, int64_t hidden, int64_t q_out,
                                            int64_t kv_out, int64_t blocksize, float epsilon, uint64_t stream) {
    return kc::qkv_common(raw, "qwen2_fused_rmsnorm_qkv_nf4_v2", Act::kF16, input, norm_weight, q_weight_packed,
                          q_absmax, q_bias, k_weight_packed, k_absmax, k_bias, v_weight_packed, v_absmax, v_bias,
                          normalized_workspace, true, q_output, k_output, v_output, rows, hidden, q_out, kv_out,
                          blocksize, epsilon, stream);
}

int kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v3(void* raw, uint64_t input, uint64_t norm_weight,
                                            uint64_t q_weight_packed, uint64_t q_absmax, uint64_t q_bias,
                                            uint64_t k_weight_packed, uint64_t k_absmax, uint64_t k_bias,
                                            uint64_t v_weight_packed, uint64_t v_absmax, uint64_t v_bias,
                                            uint64_t normalized_workspace, uint64_t q_output, uint64_t k_output,
                                            uint64_t v_output, int64_t rows, int64_t hidden, int64_t q_out,
                                            int64_t kv_out, int64_t blocksize, float epsilon, uint64_t stream) {
    return kc::qkv_common(raw, "qwen2_fused_rmsnorm_qkv_nf4_v3", Act::kF16, input, norm_weight, q_weight_packed,
                          q_absmax, q_bias, k_weight_packed, k_absmax, k_bias, v_weight_packed, v_absmax, v_bias,
                          normalized_workspace, true, q_output, k_output, v_output, rows, hidden, q_out, kv_out,
                          blocksize, epsilon, stream);
}

int kudacuda_qwen2_fused_rmsnorm_qkv_nf4_bf16(void* raw, uint64_t input, uint64_t norm_weight,
                                              uint64_t q_weight_packed, uint64_t q_absmax, uint64_t q_bias,
                                              uint64_t k_weight_packed, uint64_t k_absmax, uint64_t k_bias,
                                              uint64_t v_weight_packed, uint64_t v_absmax, uint64_t v_bias,
                                              uint64_t q_output, uint64_t k_output, uint64_t v_output, int64_t rows,
                                              int64_t hidden, int64_t q_out, int64_t kv_out, int64_t blocksize,
                                              float epsilon, uint64_t stream) {
    return kc::qkv_common(raw, "qwen2_fused_rmsnorm_qkv_nf4_bf16", Act::kBf16, input, norm_weight, q_weight_packed,
                          q_absmax, q_bias, k_weight_packed, k_absmax, k_bias, v_weight_packed, v_absmax, v_bias, 0,
                          false, q_output, k_output, v_output, rows, hidden, q_out, kv_out, blocksize, epsilon,
                          stream);
}

int kudacuda_qwen2_qkv_rope_cache_nf4_bf16(void* raw, uint64_t input, uint64_t norm_weight, uint64_t q_weight_packed,
                                           uint64_t q_absmax, uint64_t q_bias, uint64_t k_weight_packed,
                                           uint64_t k_absmax, uint64_t k_bias, uint64_t v_weight_packed,
                                           uint64_t v_absmax, uint64_t v_bias, uint64_t rope_cos, uint64_t rope_sin,
                                           uint64_t position_device, uint64_t q_output, uint64_t key_cache,
                                           uint64_t value_cache, int64_t kv_capacity, int64_t hidden, int64_t q_out,
                                           int64_t kv_out, int64_t blocksize, float epsilon, uint64_t stream) {
    Handle* h = as_handle(raw);
    const char* symbol = "qwen2_qkv_rope_cache_nf4_bf16";
    if (!ready(h, "kudacuda_qwen2_qkv_rope_cache_nf4_bf16")) {
        return 1;
    }
    if (input == 0 || norm_weight == 0 || q_weight_packed == 0 || q_absmax == 0 || q_bias == 0 ||
        k_weight_packed == 0 || k_absmax == 0 || k_bias == 0 || v_weight_packed == 0 || v_absmax == 0 ||
        v_bias == 0 || rope_cos == 0 || rope_sin == 0 || position_device == 0 || q_output == 0 || key_cache == 0 ||
        value_cache == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (hidden != 2048 || q_out != 2048 || kv_out != 256 || blocksize != 64 || kv_capacity < 1 ||
        kv_capacity > kc::kMaxModelKv || !(epsilon > 0.0f)) {
        h->set_error(std::string(symbol) +
                     " requires hidden=2048, q_out=2048, kv_out=256, blocksize=64, kv_capacity=1..32768, and "
                     "positive epsilon");
        return 1;
    }
    kc::Nf4RowsArgs a;
    a.x = ptr<const uint16_t>(input);
    a.gamma = ptr<const uint16_t>(norm_weight);
    a.eps = epsilon;
    a.w[0] = ptr<const uint8_t>(q_weight_packed);
    a.w[1] = ptr<const uint8_t>(k_weight_packed);
    a.w[2] = ptr<const uint8_t>(v_weight_packed);
    a.absmax[0] = ptr<const float>(q_absmax);
    a.absmax[1] = ptr<const float>(k_absmax);
    a.absmax[2] = ptr<const float>(v_absmax);
    a.bias[0] = ptr<const uint16_t>(q_bias);
    a.bias[1] = ptr<const uint16_t>(k_bias);
    a.bias[2] = ptr<const uint16_t>(v_bias);
    a.out[0] = ptr<uint16_t>(q_output);
    a.rows[0] = 2048;
    a.rows[1] = 256;
    a.rows[2] = 256;
    a.rope_cos = ptr<const float>(rope_cos);
    a.rope_sin = ptr<const float>(rope_sin);
    a.control = ptr<const int32_t>(position_device);
    a.capacity = kv_capacity;
    a.kcache = ptr<uint16_t>(key_cache);
    a.vcache = ptr<uint16_t>(value_cache);
    return finish(h, symbol, kc::launch_nf4_rows2048(kc::RowMode::kQkvRope, Act::kBf16, a, as_stream(stream)));
}

int kudacuda_qwen2_swiglu_nf4(void* raw, uint64_t input, uint64_t norm_weight, uint64_t gate_weight_packed,
                              uint64_t gate_absmax, uint64_t up_weight_packed, uint64_t up_absmax, uint64_t output,
                              int64_t rows, int64_t hidden, int64_t intermediate, int64_t blocksize, float epsilon,
                              uint64_t stream) {
    // The reference leaves last_error untouched on success for this symbol
    // (runtime/kudacuda_runtime.cu:750); kept.
    return kc::swiglu_common(raw, "qwen2_swiglu_nf4", Act::kF16, input, norm_weight, gate_weight_packed, gate_absmax,
                             up_weight_packed, up_absmax, output, rows, hidden, intermediate, blocksize, epsilon,
                             stream, false);
}

int kudacuda_qwen2_swiglu_nf4_bf16(void* raw, uint64_t input, uint64_t norm_weight, uint64_t gate_weight_packed,
                                   uint64_t gate_absmax, uint64_t up_weight_packed, uint64_t up_absmax,
                                   uint64_t output, int64_t rows, int64_t hidden, int64_t intermediate,
                                   int64_t blocksize, float epsilon, uint64_t stream) {
    return kc::swiglu_common(raw, "qwen2_swiglu_nf4_bf16", Act::kBf16, input, norm_weight, gate_weight_packed,
                             gate_absmax, up_weight_packed, up_absmax, output, rows, hidden, intermediate, blocksize,
                             epsilon, stream, true);
}

int kudacuda_qwen2_mlp_nf4_bf16(void* raw, uint64_t input, uint64_t norm_weight, uint64_t gate_weight_packed,
                                uint64_t gate_absmax, uint64_t up_weight_packed, uint64_t up_absmax,
                                uint64_t down_weight_packed, uint64_t down_absmax, uint64_t intermediate_workspace,
                                uint64_t residual, uint64_t output, int64_t rows, int64_t hidden,
                                int64_t intermediate, int64_t blocksize, float epsilon, uint64_t stream) {
    Handle* h = as_handle(raw);
    const char* symbol = "qwen2_mlp_nf4_bf16";
    if (!ready(h, "kudacuda_qwen2_mlp_nf4_bf16")) {
        return 1;
    }
    if (input == 0 || gate_weight_packed == 0 || gate_absmax == 0 || up_weight_packed == 0 || up_absmax == 0 ||
        down_weight_packed == 0 || down_absmax == 0 || intermediate_workspace == 0 || output == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (rows != 1 || hidden != 2048 || intermediate != 11008 || blocksize != 64 ||
        (norm_weight != 0 && !(epsilon > 0.0f))) {
        h->set_error(std::string(symbol) +
                     " requires rows=1, hidden=2048, intermediate=11008, blocksize=64, and positive epsilon");
        return 1;
    }
    kc::Nf4RowsArgs a;
    a.x = ptr<const uint16_t>(input);
    a.gamma = ptr<const uint16_t>(norm_weight);
    a.eps = epsilon;
    a.w[0] = ptr<const uint8_t>(gate_weight_packed);
    a.w[1] = ptr<const uint8_t>(up_weight_packed);
    a.absmax[0] = ptr<const float>(gate_absmax);
    a.absmax[1] = ptr<const float>(up_absmax);
    a.out[0] = ptr<uint16_t>(intermediate_workspace);
    a.rows[0] = intermediate;
    a.rows[1] = intermediate;
    hipError_t status = kc::launch_nf4_rows2048(kc::RowMode::kSwiGlu, Act::kBf16, a, as_stream(stream));
    if (status != hipSuccess) {
        return finish(h, "qwen2_mlp_nf4_bf16(gate_up)", status);
    }
    kc::Nf4DownArgs d;
    d.x = ptr<const uint16_t>(intermediate_workspace);
    d.w = ptr<const uint8_t>(down_weight_packed);
    d.absmax = ptr<const float>(down_absmax);
    d.residual = ptr<const uint16_t>(residual);
    d.out = ptr<uint16_t>(output);
    d.rows = hidden;
    return finish(h, "qwen2_mlp_nf4_bf16(down)", kc::launch_nf4_down11008(Act::kBf16, d, as_stream(stream)));
}

int kudacuda_nf4_gemv_bf16(void* raw, uint64_t input, uint64_t weight_packed, uint64_t absmax, uint64_t bias,
                           uint64_t residual, uint64_t output, int64_t rows, int64_t in_features,
                           int64_t out_features, int64_t blocksize, uint64_t stream) {
    Handle* h = as_handle(raw);
    const char* symbol = "nf4_gemv_bf16";
    if (!ready(h, "kudacuda_nf4_gemv_bf16")) {
        return 1;
    }
    if (input == 0 || weight_packed == 0 || absmax == 0 || output == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (rows != 1 || in_features != 2048 || out_features < 1 || blocksize != 64) {
        h->set_error(std::string(symbol) + " requires rows=1, in_features=2048, out_features>=1, blocksize=64");
        return 1;
    }
    kc::Nf4RowsArgs a;
    a.x = ptr<const uint16_t>(input);
    a.w[0] = ptr<const uint8_t>(weight_packed);
    a.absmax[0] = ptr<const float>(absmax);
    a.bias[0] = ptr<const uint16_t>(bias);
    a.residual = ptr<const uint16_t>(residual);
    a.out[0] = ptr<uint16_t>(output);
    a.rows[0] = out_features;
    return finish(h, symbol, kc::launch_nf4_rows2048(kc::RowMode::kGemv, Act::kBf16, a, as_stream(stream)));
}


int kudacuda_nf4_gemm_bf16(void* raw, uint64_t input, uint64_t weight_packed, uint64_t absmax, uint64_t bias,
                           uint64_t residual, uint64_t output, int64_t tokens, int64_t in_features,
                           int64_t out_features, int64_t blocksize, uint64_t stream) {
    Handle* h = as_handle(raw);
    const char* symbol = "nf4_gemm_bf16";
    if (!ready(h, "kudacuda_nf4_gemm_bf16")) {
        return 1;
    }
    if (input == 0 || weight_packed == 0 || absmax == 0 || output == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (!kc::gemm_shape_ok(h, symbol, tokens, in_features, out_features, blocksize)) {
        return 1;
    }
    if (bias != 0 && residual != 0) {
        h->set_error(std::string(symbol) + " takes a bias or a residual, not both");
        return 1;
    }
    kc::Nf4GemmArgs a;
    a.x = ptr<const uint16_t>(input);
    a.w[0] = ptr<const uint8_t>(weight_packed);
    a.absmax[0] = ptr<const float>(absmax);
    a.bias = ptr<const uint16_t>(bias);
    a.residual = ptr<const uint16_t>(residual);
    a.out = ptr<uint16_t>(output);
    a.n = out_features;
    a.k = in_features;
    a.partials = h->gemm_partials;
    a.partial_floats = kc::kGemmScratchFloats;
    const kc::GemmEpi epi = residual != 0 ? kc::GemmEpi::kResidual : kc::GemmEpi::kBias;
    if (!claim_scratch(h, symbol, as_stream(stream))) {
        return 1;
    }
    return finish(h, symbol, scratch_launched(h, as_stream(stream), kc::gemm_chunks(epi, a, tokens, as_stream(stream))));
}

int kudacuda_nf4_gemm_swiglu_bf16(void* raw, uint64_t input, uint64_t gate_weight_packed, uint64_t gate_absmax,
                                  uint64_t up_weight_packed, uint64_t up_absmax, uint64_t output, int64_t tokens,
                                  int64_t in_features, int64_t out_features, int64_t blocksize, uint64_t stream) {
    Handle* h = as_handle(raw);
    const char* symbol = "nf4_gemm_swiglu_bf16";
    if (!ready(h, "kudacuda_nf4_gemm_swiglu_bf16")) {
        return 1;
    }
    if (input == 0 || gate_weight_packed == 0 || gate_absmax == 0 || up_weight_packed == 0 || up_absmax == 0 ||
        output == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (!kc::gemm_shape_ok(h, symbol, tokens, in_features, out_features, blocksize)) {
        return 1;
    }
    kc::Nf4GemmArgs a;
    a.x = ptr<const uint16_t>(input);
    a.w[0] = ptr<const uint8_t>(gate_weight_packed);
    a.absmax[0] = ptr<const float>(gate_absmax);
    a.w[1] = ptr<const uint8_t>(up_weight_packed);
    a.absmax[1] = ptr<const float>(up_absmax);
    a.out = ptr<uint16_t>(output);
    a.n = out_features;
    a.k = in_features;
    a.partials = h->gemm_partials;
    a.partial_floats = kc::kGemmScratchFloats;
    if (!claim_scratch(h, symbol, as_stream(stream))) {
        return 1;
    }
    return finish(h, symbol,
                  scratch_launched(h, as_stream(stream), kc::gemm_chunks(kc::GemmEpi::kSwiGlu, a, tokens, as_stream(stream))));
}

int kudacuda_nf4_quantize(void* raw, uint64_t input, int64_t input_dtype, int64_t count, int64_t blocksize,
                          uint64_t packed_output, uint64_t absmax_output, uint64_t stream) {
    Handle* h = as_handle(raw);
    const char* symbol = "nf4_quantize";
    if (!ready(h, "kudacuda_nf4_quantize")) {
        return 1;
    }
    if (input == 0 || packed_output == 0 || absmax_output == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (blocksize != 64 || count <= 0 || count % 64 != 0 || (input_dtype != 0 && input_dtype != 1)) {
        h->set_error(std::string(symbol) +
                     " requires blocksize=64, a positive count divisible by 64, and input_dtype 0 (fp32) or 1 (bf16)");
        return 1;
    }
    const hipError_t status =
        input_dtype == 0
            ? kc::launch_nf4_quantize_f32(ptr<const float>(input), count, ptr<uint8_t>(packed_output),
                                          ptr<float>(absmax_output), as_stream(stream))
            : kc::launch_nf4_quantize_bf16(ptr<const uint16_t>(input), count, ptr<uint8_t>(packed_output),
                                           ptr<float>(absmax_output), as_stream(stream));
    return finish(h, symbol, status);
}

int kudacuda_nf4_dequantize(void* raw, uint64_t packed, uint64_t absmax, int64_t count, int64_t blocksize,
                            int64_t output_dtype, uint64_t output, uint64_t stream) {
    Handle* h = as_handle(raw);
    const char* symbol = "nf4_dequantize";
    if (!ready(h, "kudacuda_nf4_dequantize")) {
        return 1;
    }
    if (packed == 0 || absmax == 0 || output == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (blocksize <= 0 || count <= 0 || output_dtype < 0 || output_dtype > 2) {
        h->set_error(std::string(symbol) + " requires positive count and blocksize and output_dtype 0, 1 or 2");
        return 1;
    }
    return finish(h, symbol,
                  kc::launch_nf4_dequantize(ptr<const uint8_t>(packed), ptr<const float>(absmax), count, blocksize,
                                            static_cast<int>(output_dtype), ptr<void>(output), as_stream(stream)));
}

int kudacuda_qwen2_gqa_decode_workspace_v3(void* raw, uint64_t query, uint64_t key_cache, uint64_t value_cache,
                                           uint64_t output, uint64_t workspace, uint64_t kv_len_device,
                                           int64_t batch_size, int64_t query_len, int64_t kv_capacity,
                                           int64_t query_heads, int64_t kv_heads, int64_t head_dim, float scale,
                                           uint64_t stream) {
    Handle* h = as_handle(raw);
    const char* symbol = "qwen2_gqa_decode_workspace_v3";
    if (!ready(h, "kudacuda_qwen2_gqa_decode_workspace_v3")) {
        return 1;
    }
    if (query == 0 || key_cache == 0 || value_cache == 0 || output == 0 || workspace == 0 || kv_len_device == 0) {
        h->set_error(std::string(symbol) + " requires non-null device pointers");
        return 1;
    }
    if (batch_size != 1 || query_len != 1 || kv_capacity < 1 || kv_capacity > 512 || query_heads != 16 ||
        kv_heads != 2 || head_dim != 128 || !(scale > 0.0f)) {
        h->set_error(std::string(symbol) +
                     " requires 1x1, capacity=1..512, heads=16/2, head_dim=128, and positive scale");
        return 1;
    }
    kc::GqaArgs a;
    a.q = ptr<const uint16_t>(query);
    a.k = ptr<const uint16_t>(key_cache);
    a.v = ptr<const uint16_t>(value_cache);
    a.out = ptr<uint16_t>(output);
    a.partials = ptr<float>(workspace);
    a.counters = h->counters;
    a.kv_len_device = ptr<const int32_t>(kv_len_device);
    // the caller's workspace holds 16 x 8 x 130 floats (reference contract)
    kc::set_gqa_plan(a, kv_capacity, 8);
    a.qk_scale_log2 = scale * kc::kLog2e;
    if (!claim_scratch(h, symbol, as_stream(stream))) {
        return 1;
    }
    return finish(h, symbol, scratch_launched(h, as_stream(stream), kc::launch_gqa_decode(Act::kF16, a, as_stream(stream))));
}

int kudacuda_qwen2_gqa_decode(void* raw, uint64_t query, uint64_t key_cache, uint64_t value_cache, uint64_t output,
                              int64_t batch_size, int64_t query_len, int64_t kv_len, int64_t query_heads,
                              int64_t kv_heads, int64_t head_dim, float scale, uint64_t stream) {
    return kc::gqa_direct(raw, "qwen2_gqa_decode", Act::kF16, query, key_cache, value_cache, output,
                          {batch_size, query_len, query_heads, kv_heads, head_dim, scale}, kv_len, stream);
}

int kudacuda_qwen2_gqa_decode_bf16(void* raw, uint64_t query, uint64_t key_cache, uint64_t value_cache,
                                   uint64_t output, int64_t batch_size, int64_t query_len, int64_t kv_len,
                                   int64_t query_heads, int64_t kv_heads, int64_t head_dim, float scale,
                                   uint64_t stream) {
    return kc::gqa_direct(raw, "qwen2_gqa_decode_bf16", Act::kBf16, query, key_cache, value_cache, output,
                          {batch_size, query_len, query_heads, kv_heads, head_dim, scale}, kv_len, stream);
}

int kudacuda_qwen2_gqa_decode_graph(void* raw, uint64_t query, uint64_t key_cache, uint64_t value_cache,
                                    uint64_t output, int64_t batch_size, int64_t query_len, int64_t kv_capacity,
                                    int64_t query_heads, int64_t kv_heads, int64_t head_dim, float scale,
                                    uint64_t kv_len_device, uint64_t stream) {
    return kc::gqa_graph(raw, "qwen2_gqa_decode_graph", Act::kF16, query, key_cache, value_cache, output,
                         {batch_size, query_len, query_heads, kv_heads, head_dim, scale}, kv_capacity, kv_len_device,
                         stream);
}

int kudacuda_qwen2_gqa_decode_graph_bf16(void* raw, uint64_t query, uint64_t key_cache, uint64_t value_cache,
                                         uint64_t output, int64_t batch_size, int64_t query_len, int64_t kv_capacity,
                                         int64_t query_heads, int64_t kv_heads, int64_t head_dim, float scale,
                                         uint64_t kv_len_device, uint64_t stream) {
    return kc::gqa_graph(raw, "qwen2_gqa_decode_graph_bf16", Act::kBf16, query, key_cache, value_cache, output,
                         {batch_size, query_len, query_heads, kv_heads, head_dim, scale}, kv_capacity, kv_len_device,
                         stream);
}

int kudacuda_qwen2_gqa_decode_graph_bf16_noalloc(void* raw, uint64_t query, uint64_t key_cache,
                                                 uint64_t value_cache, uint64_t output, int64_t batch_size,
                                                 int64_t query_len, int64_t kv_capacity, int64_t query_heads,
                                                 int64_t kv_heads, int64_t head_dim, float scale,
                                                 uint64_t kv_len_device, uint64_t stream) {
    return kc::gqa_graph(raw, "qwen2_gqa_decode_graph_bf16_noalloc", Act::kBf16, query, key_cache, value_cache,
                         output, {batch_size, query_len, query_heads, kv_heads, head_dim, scale}, kv_capacity,
                         kv_len_device, stream, true);
}

int kudacuda_qwen2_gqa_decode_group_tiled(void* raw, uint64_t query, uint64_t key_cache, uint64_t value_cache,
                                          uint64_t output, int64_t batch_size, int64_t query_len, int64_t kv_len,
                                          int64_t query_heads, int64_t kv_heads, int64_t head_dim, float scale,
                                          uint64_t stream) {
    return kc::gqa_direct(raw, "qwen2_gqa_decode_group_tiled", Act::kF16, query, key_cache, value_cache, output,
                          {batch_size, query_len, query_heads, kv_heads, head_dim, scale}, kv_len, stream);
}

int kudacuda_qwen2_gqa_decode_vectorized(void* raw, uint64_t query, uint64_t key_cache, uint64_t value_cache,
                                         uint64_t output, int64_t batch_size, int64_t query_len, int64_t kv_len,
                                         int64_t query_heads, int64_t kv_heads, int64_t head_dim, float scale,
                                         uint64_t stream) {
    return kc::gqa_direct(raw, "qwen2_gqa_decode_vectorized", Act::kF16, query, key_cache, value_cache, output,
                          {batch_size, query_len, query_heads, kv_heads, head_dim, scale}, kv_len, stream);
}

int64_t kudacuda_gqa_split_chunk(int64_t kv_tokens) {
    return kc::gqa_split_tokens(kv_tokens < 1 ? 1 : kv_tokens, kc::kGqaSplitCap);
}

int64_t kudacuda_gqa_workspace_floats(int64_t kv_tokens) { return kc::gqa_workspace(kv_tokens < 1 ? 1 : kv_tokens); }

int kudacuda_lm_head_argmax_bf16(void* raw, uint64_t input, uint64_t norm_weight, uint64_t weight, uint64_t logits,
                                 uint64_t argmax_out, int64_t vocab, int64_t hidden, float epsilon, uint64_t stream) {
    Handle* h = as_handle(raw);
    const char* symbol = "lm_head_argmax_bf16";
    if (!ready(h, "kudacuda_lm_head_argmax_bf16")) {
        return 1;
    }
    if (input == 0 || weight == 0 || argmax_out == 0) {
        h->set_error(std::string(symbol) + " requires non-null input, weight and argmax pointers");
        return 1;
    }
    if (hidden != 2048 || vocab < 1 || vocab > (int64_t{1} << 30) || (norm_weight != 0 && !(epsilon > 0.0f))) {
        h->set_error(std::string(symbol) + " requires hidden=2048, vocab>=1, and positive epsilon");
        return 1;
    }
    kc::LmHeadArgs a;
    a.x = ptr<const uint16_t>(input);
    a.gamma = ptr<const uint16_t>(norm_weight);
    a.eps = epsilon;
    a.weight = ptr<const uint16_t>(weight);
    a.vocab = vocab;
    a.logits = ptr<uint16_t>(logits);
    a.block_best = h->lm_best;
    a.argmax_out = ptr<int32_t>(argmax_out);
    if (!claim_scratch(h, symbol, as_stream(stream))) {
        return 1;
    }
    return finish(h, symbol, scratch_launched(h, as_stream(stream), kc::launch_lm_head_argmax(a, as_stream(stream))));
}

int64_t kudacuda_lm_head_workspace_floats(void) { return kc::lm_head_workspace_floats(); }

int kudacuda_begin_capture(void* raw, uint64_t stream) {
    Handle* h = as_handle(raw);
    if (h == nullptr || !h->frozen) {
        if (h != nullptr) {
            h->set_error("kudacuda_begin_capture requires a frozen handle");
        }
        return 1;
    }
    if (h->capturing) {
        h->set_error("HIP graph capture is already active");
        return 1;
    }
    const hipError_t status = hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeGlobal);
    if (status != hipSuccess) {
        h->set_hip_error("hipStreamBeginCapture", status);
        return 1;
    }
    h->capturing = true;
    h->capture_uses_scratch = false;
    h->last_error.clear();
    return 0;
}

int kudacuda_end_capture(void* raw, uint64_t stream) {
    Handle* h = as_handle(raw);
    if (h == nullptr || !h->capturing) {
        if (h != nullptr) {
            h->set_error("kudacuda_end_capture called without active capture");
        }
        return 1;
    }
    hipGraph_t graph = nullptr;
    const hipError_t end_status = hipStreamEndCapture(as_stream(stream), &graph);
    h->capturing = false;
    if (end_status != hipSuccess) {
        h->set_hip_error("hipStreamEndCapture", end_status);
        return 1;
    }
    if (h->graph_exec != nullptr) {
        (void)hipGraphExecDestroy(h->graph_exec);
        h->graph_exec = nullptr;
    }
    const hipError_t inst = hipGraphInstantiate(&h->graph_exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (inst != hipSuccess) {
        h->graph_exec = nullptr;
        h->set_hip_error("hipGraphInstantiate", inst);
        return 1;
    }
    h->graph_uses_scratch = h->capture_uses_scratch;
    h->last_error.clear();
    return 0;
}

int kudacuda_replay_graph(void* raw, uint64_t stream) {
    Handle* h = as_handle(raw);
    if (h == nullptr || h->graph_exec == nullptr) {
        if (h != nullptr) {
            h->set_error("kudacuda_replay_graph called before graph instantiation");
        }
        return 1;
    }
    if (!h->graph_uses_scratch) {
        return finish(h, "hipGraphLaunch", hipGraphLaunch(h->graph_exec, as_stream(stream)));
    }
    if (!claim_scratch(h, "kudacuda_replay_graph", as_stream(stream))) {
        return 1;
    }
    return finish(h, "hipGraphLaunch",
                  scratch_launched(h, as_stream(stream), hipGraphLaunch(h->graph_exec, as_stream(stream))));
}

int kudacuda_reset_graph(void* raw) {
    Handle* h = as_handle(raw);
    if (h == nullptr) {
        return 1;
    }
    if (h->capturing) {
        h->set_error("kudacuda_reset_graph called during active capture");
        return 1;
    }
    if (h->graph_exec != nullptr) {
        const hipError_t status = hipGraphExecDestroy(h->graph_exec);
        if (status != hipSuccess) {
            h->set_hip_error("hipGraphExecDestroy", status);
            return 1;
        }
        h->graph_exec = nullptr;
    }
    if (h->graph != nullptr) {
        const hipError_t status = hipGraphDestroy(h->graph);
        if (status != hipSuccess) {
            h->set_hip_error("hipGraphDestroy", status);
            return 1;
        }
        h->graph = nullptr;
    }
    h->graph_uses_scratch = false;
    h->last_error.clear();
    return 0;
}

const char* kudacuda_last_error(void* raw) {
    const Handle* h = as_handle(raw);
    if (h == nullptr) {
        return "invalid KudaCuda handle";
    }
    return h->last_error.c_str();
}

void kudacuda_destroy(void* raw) { delete as_handle(raw); }

void* kudacuda_qwen2_model_create(void* raw, int64_t num_layers, int64_t vocab, int64_t kv_capacity,
                                  float rms_epsilon, const uint64_t* layer_ptrs, const uint64_t* model_ptrs) {
    Handle* h = as_handle(raw);
    if (!ready(h, "kudacuda_qwen2_model_create")) {
        return nullptr;
    }
    if (layer_ptrs == nullptr || model_ptrs == nullptr) {
        h->set_error("qwen2_model_create requires layer and model pointer tables");
        return nullptr;
    }
    if (num_layers < 1 || vocab < 1 || vocab > (int64_t{1} << 30) || kv_capacity < 1 ||
        kv_capacity > kc::kMaxModelKv || !(rms_epsilon > 0.0f)) {
        h->set_error("qwen2_model_create requires num_layers>=1, vocab>=1, kv_capacity=1..32768, positive epsilon");
        return nullptr;
    }
    for (int64_t i = 0; i < num_layers * KUDACUDA_QWEN2_LAYER_FIELDS; ++i) {
        if (layer_ptrs[i] == 0) {
            h->set_error("qwen2_model_create: layer " + std::to_string(i / KUDACUDA_QWEN2_LAYER_FIELDS) + " field " +
                         std::to_string(i % KUDACUDA_QWEN2_LAYER_FIELDS) + " is null");
            return nullptr;
        }
    }
    for (int i = 0; i < KUDACUDA_QWEN2_MODEL_FIELDS; ++i) {
        if (model_ptrs[i] == 0 && i != KUDACUDA_QWEN2_LOGITS && i != KUDACUDA_QWEN2_LM_COUNTER) {
            h->set_error("qwen2_model_create: model field " + std::to_string(i) + " is null");
            return nullptr;
        }
    }
    auto* m = new (std::nothrow) kc::Model();
    if (m == nullptr) {
        h->set_error("qwen2_model_create: out of host memory");
        return nullptr;
    }
    m->handle = h;
    m->num_layers = num_layers;
    m->vocab = vocab;
    m->capacity = kv_capacity;
    m->eps = rms_epsilon;
    m->layers.resize(static_cast<size_t>(num_layers));
    for (int64_t l = 0; l < num_layers; ++l) {
        for (int f = 0; f < KUDACUDA_QWEN2_LAYER_FIELDS; ++f) {
            m->layers[static_cast<size_t>(l)][static_cast<size_t>(f)] =
                layer_ptrs[l * KUDACUDA_QWEN2_LAYER_FIELDS + f];
        }
    }
    for (int f = 0; f < KUDACUDA_QWEN2_MODEL_FIELDS; ++f) {
        m->g[static_cast<size_t>(f)] = model_ptrs[f];
    }
    h->last_error.clear();
    return m;
}

int kudacuda_qwen2_model_step(void* raw_model, uint64_t stream) {
    auto* m = reinterpret_cast<kc::Model*>(raw_model);
    if (m == nullptr) {
        return 1;
    }
    const hipError_t status = kc::model_step(*m, as_stream(stream), kc::step_form(*m, m->host_step));
    if (status == hipSuccess && m->host_step >= 0) {
        ++m->host_step;
    }
    return finish(m->handle, "qwen2_model_step", status);
}

int64_t kudacuda_qwen2_prefill_workspace_bytes(int64_t tokens) {
    return tokens < 1 ? 0 : tokens * kc::kPrefillBytesPerToken + kc::kPrefillFixedBytes;
}

int kudacuda_qwen2_model_prefill(void* raw_model, uint64_t workspace, int64_t workspace_bytes, int64_t start,
                                 int64_t count, uint64_t stream) {
    auto* m = reinterpret_cast<kc::Model*>(raw_model);
    if (m == nullptr) {
        return 1;
    }
    Handle* h = m->handle;
    const char* symbol = "qwen2_model_prefill";
    if (workspace == 0) {
        h->set_error(std::string(symbol) + " requires a non-null workspace");
        return 1;
    }
    if (count < 1 || start < 0 || start + count > m->capacity ||
        workspace_bytes < kudacuda_qwen2_prefill_workspace_bytes(count)) {
        h->set_error(std::string(symbol) +
                     " requires count>=1, 0<=start, start+count<=kv_capacity and a workspace of "
                     "kudacuda_qwen2_prefill_workspace_bytes(count) bytes");
        return 1;
    }
    const hipError_t status = kc::model_prefill(*m, ptr<uint8_t>(workspace), start, count, as_stream(stream));
    if (status == hipSuccess) {
        m->host_step = start + count;  // where the prefill leaves control[0]
    }
    return finish(h, symbol, status);
}

int kudacuda_qwen2_model_capture(void* raw_model, uint64_t stream) {
    auto* m = reinterpret_cast<kc::Model*>(raw_model);
    if (m == nullptr) {
        return 1;
    }
    Handle* h = m->handle;
    auto drop_all = [m]() {
        for (hipGraphExec_t& e : m->execs) {
            if (e != nullptr) {
                (void)hipGraphExecDestroy(e);
                e = nullptr;
            }
        }
    };
    drop_all();
    hipStream_t s = as_stream(stream);
    // forms 1 .. cap always (the split count a step can leave to o_proj),
    // form 0 when this cache can exceed the cap
    const int cap = static_cast<int>(kc::step_defer_cap(*m));
    for (int form = kc::long_form_possible(*m) ? 0 : 1; form <= cap; ++form) {
        hipError_t status = hipStreamBeginCapture(s, hipStreamCaptureModeGlobal);
        if (status != hipSuccess) {
            drop_all();
            return finish(h, "hipStreamBeginCapture", status);
        }
        const hipError_t launch_status = kc::model_step(*m, s, form);
        hipGraph_t graph = nullptr;
        status = hipStreamEndCapture(s, &graph);
        if (launch_status != hipSuccess) {
            if (graph != nullptr) {
                (void)hipGraphDestroy(graph);
            }
            drop_all();
            return finish(h, "qwen2_model_capture(step)", launch_status);
        }
        if (status != hipSuccess) {
            drop_all();
            return finish(h, "hipStreamEndCapture", status);
        }
        status = hipGraphInstantiate(&m->execs[static_cast<size_t>(form)], graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (status != hipSuccess) {
            m->execs[static_cast<size_t>(form)] = nullptr;
            drop_all();  // all or nothing
            return finish(h, "hipGraphInstantiate", status);
        }
    }
    h->last_error.clear();
    return 0;
}

int kudacuda_qwen2_model_replay(void* raw_model, int64_t steps, uint64_t stream) {
    auto* m = reinterpret_cast<kc::Model*>(raw_model);
    if (m == nullptr) {
        return 1;
    }
    const size_t fallback = static_cast<size_t>(kc::step_form(*m, -1));
    if (m->execs[fallback] == nullptr) {
        m->handle->set_error("qwen2_model_replay called before qwen2_model_capture");
        return 1;
    }
    for (int64_t i = 0; i < steps; ++i) {
        hipGraphExec_t e = m->execs[static_cast<size_t>(kc::step_form(*m, m->host_step))];
        const hipError_t status = hipGraphLaunch(e != nullptr ? e : m->execs[fallback], as_stream(stream));
        if (status != hipSuccess) {
            return finish(m->handle, "hipGraphLaunch", status);
        }
        if (m->host_step >= 0) {
            ++m->host_step;
        }
    }
    m->handle->last_error.clear();
    return 0;
}

int kudacuda_qwen2_model_set_position(void* raw_model, int64_t step) {
    auto* m = reinterpret_cast<kc::Model*>(raw_model);
    if (m == nullptr) {
        return 1;
    }
    m->host_step = step < 0 ? -1 : step;
    m->handle->last_error.clear();
    return 0;
}

int kudacuda_qwen2_model_time_op(void* raw_model, int64_t op, int64_t iters, uint64_t stream, float* avg_ms) {
    auto* m = reinterpret_cast<kc::Model*>(raw_model);
    if (m == nullptr) {
        return 1;
    }
    Handle* h = m->handle;
    if (op < 0 || op > 5 || iters < 1 || iters > 4096 || avg_ms == nullptr) {
        h->set_error("qwen2_model_time_op requires op 0..5, iters 1..4096 and an output pointer");
        return 1;
    }
    // The launches are captured into a graph and replayed, so the events see
    // device time back to back rather than host launch gaps.
    hipStream_t s = as_stream(stream);
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    hipError_t status = hipStreamBeginCapture(s, hipStreamCaptureModeGlobal);
    hipError_t launch = hipSuccess;
    for (int64_t i = 0; i < iters && status == hipSuccess && launch == hipSuccess; ++i) {
        launch = kc::model_op(*m, static_cast<int>(op), i % m->num_layers, false, s, kc::step_form(*m, m->host_step));
    }
    if (status == hipSuccess) {
        status = hipStreamEndCapture(s, &graph);
    }
    if (status == hipSuccess && launch != hipSuccess) {
        status = launch;
    }
    if (status == hipSuccess) {
        status = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    }
    if (status == hipSuccess) {
        status = hipGraphLaunch(exec, s);  // warm
    }
    if (status == hipSuccess) {
        status = hipEventCreate(&start);
    }
    if (status == hipSuccess) {
        status = hipEventCreate(&stop);
    }
    if (status == hipSuccess) {
        status = hipEventRecord(start, s);
    }
    if (status == hipSuccess) {
        status = hipGraphLaunch(exec, s);
    }
    if (status == hipSuccess) {
        status = hipEventRecord(stop, s);
    }
    if (status == hipSuccess) {
        status = hipEventSynchronize(stop);
    }
    float ms = 0.0f;
    if (status == hipSuccess) {
        status = hipEventElapsedTime(&ms, start, stop);
    }
    if (start != nullptr) {
        (void)hipEventDestroy(start);
    }
    if (stop != nullptr) {
        (void)hipEventDestroy(stop);
    }
    if (exec != nullptr) {
        (void)hipGraphExecDestroy(exec);
    }
    if (graph != nullptr) {
        (void)hipGraphDestroy(graph);
    }
    if (status == hipSuccess) {
        *avg_ms = ms / static_cast<float>(iters);
    }
    return finish(h, "qwen2_model_time_op", status);
}

void kudacuda_qwen2_model_destroy(void* raw_model) { delete reinterpret_cast<kc::Model*>(raw_model); }

}  // extern "C"
