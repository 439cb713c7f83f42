// Internal launch interface between the C-ABI runtime (kc_runtime.hip) and
// the gfx950 kernels.  Nothing here is exported from libkudacuda.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kc {

enum class Act { kBf16 = 0, kF16 = 1 };

// ------------------------------------------------------------------- NF4 rows
// One launch of the K = 2048 NF4 row kernel.  `mode` selects the row set and
// the epilogue:
//   kGemv      : y[r]   = T(dot_r + bias[r])            (rows 0..n0)
//                with residual: y[r] = T(res[r] + T(dot_r))
//   kQkv       : q/k/v  = T(dot + bias) for Wq, Wk, Wv  (no rotary)
//   kQkvRope   : q = T(rope(dot + bias)); k, v written into the KV cache at
//                the device-resident position control[0]
//   kSwiGlu    : h[r]   = T(silu(gate_r) * up_r)
enum class RowMode { kGemv = 0, kQkv = 1, kQkvRope = 2, kSwiGlu = 3 };

// Split-KV attention partials (per query head h and split s: max, sum and
// acc[128] at (h * max_splits + s) * kGqaPartialStride floats) and the split
// plan they were made with.  The attention kernel leaves them unmerged when
// the split count at this kv_len is <= defer_max; its consumer merges them.
constexpr int kGqaPartialStride = 130;
constexpr int kGqaRoundTokens = 32;      // tokens of one round (one per 16-lane group of a block)
constexpr int64_t kGqaSplitCap = 256;    // most splits per KV head of an uncapped plan
// Most splits a consumer merges.  Each slot costs o_proj ~0.1 us per layer,
// so the decode step is captured once per slot count and a step pays only
// for the splits at its length; 16 covers one-round splits up to 512 cached
// tokens (a consumer's plain split-order sum equals the grouped one only up
// to kGqaMergeGroup splits), past which the merge kernel takes over.
constexpr int kGqaMaxDefer = 16;
constexpr int kGqaMergeGroup = 16;       // merges sum splits in groups of this many, then the groups
static_assert(kGqaMaxDefer <= kGqaMergeGroup, "a deferred merge is one group: its sum is the grouped sum");
// Split cap of the decode step's plan: every split count it can reach is
// merged by o_proj (deferred) or by the in-kernel ticket, so the step's graph
// holds no merge-kernel node.
constexpr int64_t kGqaStepSplits = 32;
struct AttnSplits {
    const float* partials = nullptr;
    uint16_t* out = nullptr;  // optional: receives the merged vector (one block writes it)
    const int32_t* kv_len_device = nullptr;
    int32_t kv_len_offset = 0;
    int64_t capacity = 0;
    int64_t split_cap = 0;
    int64_t max_splits = 0;
    int64_t defer_max = 0;
};

// Tokens per split at kv_len L with at most split_cap splits: the fewest
// whole rounds that keep the split count within the cap.  32-bit unsigned
// arithmetic (kv_len and the cap are far below 2^31; the device has no
// integer divider and a 64-bit quotient costs a long instruction loop).
__host__ __device__ inline int64_t gqa_split_tokens(int64_t L, int64_t split_cap) {
    const uint32_t rounds = (static_cast<uint32_t>(L) + kGqaRoundTokens - 1) / kGqaRoundTokens;
    const uint32_t cap = static_cast<uint32_t>(split_cap);
    const uint32_t per = (rounds + cap - 1) / cap;
    return static_cast<int64_t>(kGqaRoundTokens) * (per > 1 ? per : 1);
}
__host__ __device__ inline int64_t gqa_split_count(int64_t L, int64_t split_cap) {
    const uint32_t c = static_cast<uint32_t>(gqa_split_tokens(L, split_cap));
    return static_cast<int64_t>((static_cast<uint32_t>(L) + c - 1) / c);
}

// Matrix-core tactic for long caches: splits are whole multiples of a
// quantum of 32 tokens per wave of the partial kernel's block (128: 4-wave
// blocks; 64: 2-wave blocks), at most kGqaMfmaSplitCap per KV head, chosen
// by the same fewest-whole-units rule.
constexpr int kGqaMfmaQuantum = 128;
constexpr int64_t kGqaMfmaSplitCap = 128;
__host__ __device__ inline int64_t gqa_mfma_split_tokens(int64_t L, int64_t split_cap,
                                                         int64_t quantum = kGqaMfmaQuantum) {
    const uint32_t q = static_cast<uint32_t>(quantum);
    const uint32_t units = (static_cast<uint32_t>(L) + q - 1) / q;
    const uint32_t cap = static_cast<uint32_t>(split_cap);
    const uint32_t per = (units + cap - 1) / cap;
    return static_cast<int64_t>(q) * (per > 1 ? per : 1);
}
__host__ __device__ inline int64_t gqa_mfma_split_count(int64_t L, int64_t split_cap,
                                                        int64_t quantum = kGqaMfmaQuantum) {
    const uint32_t c = static_cast<uint32_t>(gqa_mfma_split_tokens(L, split_cap, quantum));
    return static_cast<int64_t>((static_cast<uint32_t>(L) + c - 1) / c);
}

struct Nf4RowsArgs {
    const uint16_t* x = nullptr;      // activation [2048], 16-bit
    const uint16_t* gamma = nullptr;  // RMSNorm weight [2048] or null (no norm)
    float eps = 1e-6f;
    const uint8_t* w[3] = {nullptr, nullptr, nullptr};
    const float* absmax[3] = {nullptr, nullptr, nullptr};
    const uint16_t* bias[3] = {nullptr, nullptr, nullptr};
    uint16_t* out[3] = {nullptr, nullptr, nullptr};
    int64_t rows[3] = {0, 0, 0};
    const uint16_t* residual = nullptr;  // kGemv only; may alias out[0]
    float* norm_out = nullptr;           // optional fp32 copy of the normalised x
    // kQkvRope state
    const float* rope_cos = nullptr;  // [capacity, 64]
    const float* rope_sin = nullptr;
    const int32_t* control = nullptr;  // control[0] = position of this token
    // decode step only: the stop flag of the model's control block; when it
    // is set the step writes no KV-cache row
    const int32_t* done = nullptr;
    int64_t capacity = 0;
    uint16_t* kcache = nullptr;  // [2, capacity, 128]
    uint16_t* vcache = nullptr;
    // optional embedding gather for the first layer: x := embed[tokens[pos]]
    const uint16_t* embed = nullptr;
    const int32_t* tokens = nullptr;
    int64_t vocab = 0;
    uint16_t* hidden_out = nullptr;  // receives the gathered row
    // kGemv: with attn.partials set, x is the attention output merged from
    // the partials whenever they were left unmerged (else x is read as is)
    AttnSplits attn;
};

hipError_t launch_nf4_rows2048(RowMode mode, Act act, const Nf4RowsArgs& args, hipStream_t stream);

// K = 11008 NF4 GEMV (Qwen2.5-3B down projection).  y[r] = T(dot_r) or, with
// a residual, y[r] = T(res[r] + T(dot_r)).
struct Nf4DownArgs {
    const uint16_t* x = nullptr;  // [11008]
    const uint8_t* w = nullptr;
    const float* absmax = nullptr;
    const uint16_t* residual = nullptr;
    uint16_t* out = nullptr;
    int64_t rows = 0;
};
hipError_t launch_nf4_down11008(Act act, const Nf4DownArgs& args, hipStream_t stream);

// ------------------------------------------------------- prefill (M tokens)
// NF4 GEMM on MFMA: out[m, n] = epilogue(sum_k x[m, k] * bf16(cb[code] * absmax)),
// x bf16 [m, k] row-major, weights in the bitsandbytes layout ([n, k/2] codes,
// [n, k/64] fp32 absmax), fp32 accumulation.  m <= kGemmMaxTokens per launch,
// n % 64 == 0, k % 128 == 0.
enum class GemmEpi { kBias = 0, kResidual = 1, kSwiGlu = 2, kQkvRope = 3, kResidualNorm = 4 };
constexpr int kGemmMaxTokens = 64;
// split-K scratch: fp32 partial tiles [weights][splits][m][n]
constexpr int64_t kGemmScratchFloats = int64_t{4} << 20;
struct Nf4GemmArgs {
    const uint16_t* x = nullptr;
    const uint8_t* w[3] = {nullptr, nullptr, nullptr};  // kSwiGlu: gate, up; kQkvRope: q, k, v
    const float* absmax[3] = {nullptr, nullptr, nullptr};
    const uint16_t* bias = nullptr;      // kBias: [n] (may be null: no bias)
    const uint16_t* residual = nullptr;  // kResidual: [m, n], may alias out
    uint16_t* out = nullptr;             // [m, n]; kQkvRope: rotated q [m, q_rows]
    int64_t m = 0;
    int64_t n = 0;  // kQkvRope: q_rows + 2 kv_rows
    int64_t k = 0;
    // Split-K scratch (null: one block column per row tile).  With it, K is
    // split so the launch has ~1024 waves; partial tiles are summed in split
    // order by a second kernel that applies the epilogue.  kQkvRope always
    // splits (its epilogue lives in that second kernel).
    float* partials = nullptr;
    int64_t partial_floats = 0;
    // kQkvRope: rows [0, q_rows) of the output come from w[0], the next
    // kv_rows from w[1], the last kv_rows from w[2] (head dim 128, each a
    // multiple of 64); biases per segment; the epilogue adds the bias
    // (bf16 rounding), rotates q and k by RoPE at position start + row
    // (cos/sin tables [position][64]) and writes k and v rows into the caches
    // [kv heads, capacity, 128].
    int64_t q_rows = 0;
    int64_t kv_rows = 0;
    const uint16_t* seg_bias[3] = {nullptr, nullptr, nullptr};
    const float* rope_cos = nullptr;
    const float* rope_sin = nullptr;
    uint16_t* kcache = nullptr;
    uint16_t* vcache = nullptr;
    int64_t capacity = 0;
    int64_t start = 0;
    // kResidualNorm (n = 2048, always split): out = bf16(residual +
    // bf16(sum)) as kResidual, then, with norm_gamma, the row RMSNorm of the
    // new out rows into norm_out (the prefill norm's arithmetic).
    const uint16_t* norm_gamma = nullptr;
    uint16_t* norm_out = nullptr;
    float eps = 1e-6f;
};
hipError_t launch_nf4_gemm(GemmEpi epi, const Nf4GemmArgs& args, hipStream_t stream);

// Row RMSNorm of m rows of 2048: out[r] = bf16((x[r] * inv_rms) * gamma), the
// decode kernels' fp32 order.  With `embed`, row r is embed[tokens[start + r]]
// (token ids clamped to the vocabulary) and is also copied to hidden_out.
struct PrefillNormArgs {
    const uint16_t* x = nullptr;
    const uint16_t* gamma = nullptr;
    float eps = 1e-6f;
    const uint16_t* embed = nullptr;
    const int32_t* tokens = nullptr;
    const int32_t* control = nullptr;  // control[2] = entries of tokens[] (reads stay below it)
    int64_t vocab = 0;
    int64_t start = 0;
    uint16_t* hidden_out = nullptr;
    uint16_t* out = nullptr;
    int64_t m = 0;
};
hipError_t launch_prefill_norm(const PrefillNormArgs& args, hipStream_t stream);

// Causal GQA attention of m query rows (positions start + r) over cache rows
// [0, start + r]: out [m, 2048] bf16.
struct PrefillAttnArgs {
    const uint16_t* q = nullptr;
    const uint16_t* kcache = nullptr;
    const uint16_t* vcache = nullptr;
    uint16_t* out = nullptr;
    int64_t capacity = 0;
    int64_t start = 0;
    int64_t m = 0;
    float qk_scale_log2 = 0.0f;
};
hipError_t launch_prefill_attention(const PrefillAttnArgs& args, hipStream_t stream);
// control[0] = step, stop state cleared (control[4], control[5] = 0); capture-safe
hipError_t launch_set_step(int32_t* control, int32_t step, hipStream_t stream);

// Blockwise NF4 quantisation (blocksize 64) of n elements (n % 64 == 0).
hipError_t launch_nf4_quantize_f32(const float* src, int64_t n, uint8_t* packed, float* absmax, hipStream_t stream);
hipError_t launch_nf4_quantize_bf16(const uint16_t* src, int64_t n, uint8_t* packed, float* absmax, hipStream_t stream);
// out_kind: 0 = fp32, 1 = bf16, 2 = fp16
hipError_t launch_nf4_dequantize(const uint8_t* packed, const float* absmax, int64_t n, int64_t blocksize,
                                 int out_kind, void* out, hipStream_t stream);

// ------------------------------------------------------------------------ GQA
// Split-KV grouped-query decode attention, 16 query heads / 2 KV heads /
// head_dim 128, gqa_split_tokens(kv_len, split_cap) tokens per split.  kv_len
// is read from kv_len_device when non-null, else kv_len_host is used.
struct GqaArgs {
    const uint16_t* q = nullptr;   // [16,128]
    const uint16_t* k = nullptr;   // [2, capacity, 128]
    const uint16_t* v = nullptr;
    uint16_t* out = nullptr;       // [16,128]
    float* partials = nullptr;     // [16, max_splits, 130]
    uint32_t* counters = nullptr;  // [2], zero between calls
    const int32_t* kv_len_device = nullptr;
    int32_t kv_len_offset = 0;     // added to *kv_len_device (decoder: pos + 1)
    int64_t kv_len_host = 0;
    int64_t capacity = 0;          // row stride of the cache
    int64_t max_splits = 0;        // grid size per KV head
    int64_t split_cap = 0;         // most splits at any kv_len (the split rule's parameter)
    int64_t defer_max = 0;         // <= kGqaMaxDefer: partials left for the consumer up to this many splits
    // 1..32: splits the partial kernel merges itself (merge kernel beyond).
    // Measured on standalone calls: the ticket beats the merge kernel up to 16
    // splits (8 splits: 7.5 vs 8.0 us, 16: 8.3 vs 8.5) and loses at 32 (11.1
    // vs 8.9 us).
    int64_t ticket_max = 16;
    float qk_scale_log2 = 0.0f;    // scale * log2(e)
    bool mfma = false;             // split plan of the matrix-core tactic (gqa_mfma_split_tokens)
    int64_t mfma_quantum = kGqaMfmaQuantum;  // its split unit: 64 (2-wave blocks) or 128 (4-wave blocks)
};
hipError_t launch_gqa_decode(Act act, const GqaArgs& args, hipStream_t stream);
// Matrix-core tactic (v_mfma_f32_16x16x32_{bf16,f16} for q.K and P.V, the
// weights P as a hi + lo pair of 16-bit values): partial kernel with
// gqa_mfma_split_tokens(kv_len, split_cap, mfma_quantum) tokens per split,
// then gqa_merge_kernel.  Results agree with the round path to fp32 rounding, not
// bit for bit.  Sets args.mfma itself; max_splits must cover
// gqa_mfma_split_count(capacity, split_cap, mfma_quantum).
hipError_t launch_gqa_decode_mfma(Act act, GqaArgs args, hipStream_t stream);
// Split plan for a cache of `capacity` rows; split_limit > 0 caps the number
// of splits (a caller-sized workspace).  Rule shared with the host oracle.
struct GqaPlan {
    int64_t split_cap = 0;
    int64_t max_splits = 0;  // the most splits any kv_len <= capacity needs: the grid
};
GqaPlan gqa_plan(int64_t capacity, int64_t split_limit);

// ------------------------------------------------------------- lm_head/argmax
struct LmHeadArgs {
    const uint16_t* x = nullptr;      // hidden [2048] bf16
    const uint16_t* gamma = nullptr;  // final norm weight or null
    float eps = 1e-6f;
    const uint16_t* weight = nullptr; // [vocab, 2048] bf16
    int64_t vocab = 0;
    uint16_t* logits = nullptr;       // [vocab] bf16 (may be null)
    float* block_best = nullptr;      // [2 * grid] (value, index-as-bits)
    int32_t* argmax_out = nullptr;    // receives the token id (may be null)
    // decode bookkeeping (null for a plain lm_head call): [0] step, [1]
    // prompt length, [2] token capacity, [3] stop token id (< 0: none),
    // [4] done flag, [5] position of the stop token once emitted
    int32_t* control = nullptr;
    int32_t* tokens = nullptr;
};
hipError_t launch_lm_head_argmax(const LmHeadArgs& args, hipStream_t stream);
int64_t lm_head_workspace_floats();  // size of block_best

// ------------------------------------------------------------------ misc ops
hipError_t launch_vector_add(const float* a, const float* b, float* out, int64_t n, hipStream_t stream);
hipError_t launch_rmsnorm_f32(const float* x, const float* w, float* y, int64_t rows, int64_t hidden, float eps,
                              hipStream_t stream);
hipError_t launch_dense_rmsnorm_qkv_f16(const uint16_t* x, const uint16_t* gamma, const uint16_t* w,
                                        const uint16_t* bias, uint16_t* out, int64_t rows, int64_t hidden,
                                        float eps, hipStream_t stream);

}  // namespace kc
