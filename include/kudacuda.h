/*
 * kudacuda.h — C ABI of libkudacuda.so, the gfx950 (MI355X) decode sidecar.
 *
 * Drop-in boundary: every symbol of the reference's include/kudacuda.h is
 * exported with the same name, argument order and conventions, and is cited
 * below (reference file:line).  Conventions (reference include/kudacuda.h,
 * runtime/kudacuda_runtime.cu:228-256):
 *   - tensors are device addresses passed as uint64_t, sizes are int64_t,
 *     eps/scale are float, the last argument is the caller's stream
 *     (a hipStream_t as uint64_t; PyTorch-ROCm's current_stream().cuda_stream);
 *   - return 0 on success, 1 on failure with the reason in
 *     kudacuda_last_error(handle); launches never synchronise;
 *   - the handle must be frozen; the caller owns every buffer; exact-shape
 *     guards reject anything off-contract (the caller then falls back);
 *   - one handle per host thread / stream: the handle's graph objects and its
 *     attention/argmax/GEMM scratch are not shared safely between concurrent
 *     calls; a call that uses that scratch on another stream than the last
 *     such call returns 1 until that call's launch has completed (an event
 *     the handle records behind it).  Calls recorded into a capture are
 *     checked when the graph runs: kudacuda_replay_graph claims the scratch
 *     for a graph captured by kudacuda_begin_capture that holds such calls;
 *     a graph captured by other means shares the scratch unchecked, so its
 *     replays must not overlap other users of the same handle.
 * Activations named "_bf16" are bfloat16; the reference's un-suffixed NF4 QKV
 * and GQA entry points keep their fp16 activations.
 */
#pragma once

#include <stdint.h>

#define KUDACUDA_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------ lifecycle */

/* reference include/kudacuda.h:19 — select the device, allocate the handle's
 * fixed scratch (attention split partials, argmax workspace, ticket counters). */
KUDACUDA_API void* kudacuda_create(int device_id);

/* reference include/kudacuda.h:21 */
KUDACUDA_API int kudacuda_freeze(void* handle);

/* reference include/kudacuda.h:23 — 1 if the named tactic accepts the shape.
 * Accepts this build's gfx950 tactic names and the reference's sm86/sm89 names. */
KUDACUDA_API int kudacuda_can_dispatch(void* handle, const char* tactic_name, int64_t batch_size, int64_t seq_len);

/* reference include/kudacuda.h:30 — fp32 output = a + b. */
KUDACUDA_API int kudacuda_vector_add(void* handle, uint64_t a, uint64_t b, uint64_t output, int64_t count,
                                     uint64_t stream);

/* reference include/kudacuda.h:39 — fp32 row RMSNorm. */
KUDACUDA_API int kudacuda_rmsnorm(void* handle, uint64_t input, uint64_t weight, uint64_t output, int64_t rows,
                                  int64_t hidden, float epsilon, uint64_t stream);

/* reference include/kudacuda.h:50 — fp16 dense RMSNorm + [3h, h] QKV + bias. */
KUDACUDA_API int kudacuda_fused_rmsnorm_qkv(void* handle, uint64_t input, uint64_t norm_weight, uint64_t qkv_weight,
                                            uint64_t bias, uint64_t output, int64_t rows, int64_t hidden,
                                            float epsilon, uint64_t stream);

/* ------------------------------------------- NF4 fused RMSNorm + QKV + bias */
/* Packed weights are bitsandbytes NF4 (u8 [out*in/2], element 2i in the high
 * nibble of byte i), absmax fp32 [out*in/64], blocksize 64.  Contract:
 * rows=1, hidden=2048, q_out=2048, kv_out=256, blocksize=64, epsilon>0. */

/* reference include/kudacuda.h:63 (fp16 activations) */
KUDACUDA_API int kudacuda_qwen2_fused_rmsnorm_qkv_nf4(
    void* handle, uint64_t input, uint64_t norm_weight, uint64_t q_weight_packed, uint64_t q_absmax, uint64_t q_bias,
    uint64_t k_weight_packed, uint64_t k_absmax, uint64_t k_bias, uint64_t v_weight_packed, uint64_t v_absmax,
    uint64_t v_bias, uint64_t q_output, uint64_t k_output, uint64_t v_output, int64_t rows, int64_t hidden,
    int64_t q_out, int64_t kv_out, int64_t blocksize, float epsilon, uint64_t stream);

/* reference include/kudacuda.h:88 — also writes the fp32 normalised input to
 * normalized_workspace [rows, hidden]. */
KUDACUDA_API int kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v2(
    void* handle, uint64_t input, uint64_t norm_weight, uint64_t q_weight_packed, uint64_t q_absmax, uint64_t q_bias,
    uint64_t k_weight_packed, uint64_t k_absmax, uint64_t k_bias, uint64_t v_weight_packed, uint64_t v_absmax,
    uint64_t v_bias, uint64_t normalized_workspace, uint64_t q_output, uint64_t k_output, uint64_t v_output,
    int64_t rows, int64_t hidden, int64_t q_out, int64_t kv_out, int64_t blocksize, float epsilon, uint64_t stream);

/* reference include/kudacuda.h:114 — same contract as _v2. */
KUDACUDA_API int kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v3(
    void* handle, uint64_t input, uint64_t norm_weight, uint64_t q_weight_packed, uint64_t q_absmax, uint64_t q_bias,
    uint64_t k_weight_packed, uint64_t k_absmax, uint64_t k_bias, uint64_t v_weight_packed, uint64_t v_absmax,
    uint64_t v_bias, uint64_t normalized_workspace, uint64_t q_output, uint64_t k_output, uint64_t v_output,
    int64_t rows, int64_t hidden, int64_t q_out, int64_t kv_out, int64_t blocksize, float epsilon, uint64_t stream);

/* NEW (bf16 twin of reference include/kudacuda.h:63, same argument list). */
KUDACUDA_API int kudacuda_qwen2_fused_rmsnorm_qkv_nf4_bf16(
    void* handle, uint64_t input, uint64_t norm_weight, uint64_t q_weight_packed, uint64_t q_absmax, uint64_t q_bias,
    uint64_t k_weight_packed, uint64_t k_absmax, uint64_t k_bias, uint64_t v_weight_packed, uint64_t v_absmax,
    uint64_t v_bias, uint64_t q_output, uint64_t k_output, uint64_t v_output, int64_t rows, int64_t hidden,
    int64_t q_out, int64_t kv_out, int64_t blocksize, float epsilon, uint64_t stream);

/* NEW — decode-layer front half: RMSNorm + QKV + bias + RoPE (theta table)
 * with q written to q_output and k/v written into the [2, kv_capacity, 128]
 * caches at the device-resident position *position_device (int32).  Replaces
 * the Transformers-side apply_rotary_pos_emb + cache update the reference
 * leaves to the framework (python/kudacuda_sidecar.py:835-855).  rope_cos /
 * rope_sin are fp32 [kv_capacity, 64]. */
KUDACUDA_API int kudacuda_qwen2_qkv_rope_cache_nf4_bf16(
    void* handle, uint64_t input, uint64_t norm_weight, uint64_t q_weight_packed, uint64_t q_absmax, uint64_t q_bias,
    uint64_t k_weight_packed, uint64_t k_absmax, uint64_t k_bias, uint64_t v_weight_packed, uint64_t v_absmax,
    uint64_t v_bias, uint64_t rope_cos, uint64_t rope_sin, uint64_t position_device, uint64_t q_output,
    uint64_t key_cache, uint64_t value_cache, int64_t kv_capacity, int64_t hidden, int64_t q_out, int64_t kv_out,
    int64_t blocksize, float epsilon, uint64_t stream);

/* ------------------------------------------------------------- NF4 SwiGLU */
/* Contract: rows=1, hidden=2048, intermediate=11008, blocksize=64, eps>0.
 * output [1, intermediate] = silu(gate(norm(x))) * up(norm(x)). */

/* reference include/kudacuda.h:140 (fp16) */
KUDACUDA_API int kudacuda_qwen2_swiglu_nf4(void* handle, uint64_t input, uint64_t norm_weight,
                                           uint64_t gate_weight_packed, uint64_t gate_absmax,
                                           uint64_t up_weight_packed, uint64_t up_absmax, uint64_t output,
                                           int64_t rows, int64_t hidden, int64_t intermediate, int64_t blocksize,
                                           float epsilon, uint64_t stream);

/* reference include/kudacuda.h:157 (bf16) */
KUDACUDA_API int kudacuda_qwen2_swiglu_nf4_bf16(void* handle, uint64_t input, uint64_t norm_weight,
                                                uint64_t gate_weight_packed, uint64_t gate_absmax,
                                                uint64_t up_weight_packed, uint64_t up_absmax, uint64_t output,
                                                int64_t rows, int64_t hidden, int64_t intermediate,
                                                int64_t blocksize, float epsilon, uint64_t stream);

/* NEW — whole MLP (the reference keeps down_proj in bitsandbytes,
 * python/kudacuda_sidecar.py:1746): h = silu(gate(n)) * up(n) into
 * intermediate_workspace (bf16 [1, intermediate]), then
 * output = down(h) (+ residual when residual != 0).  n = RMSNorm(input) when
 * norm_weight != 0, else n = input.  Contract: rows=1, hidden=2048,
 * intermediate=11008, blocksize=64. */
KUDACUDA_API int kudacuda_qwen2_mlp_nf4_bf16(void* handle, uint64_t input, uint64_t norm_weight,
                                             uint64_t gate_weight_packed, uint64_t gate_absmax,
                                             uint64_t up_weight_packed, uint64_t up_absmax,
                                             uint64_t down_weight_packed, uint64_t down_absmax,
                                             uint64_t intermediate_workspace, uint64_t residual, uint64_t output,
                                             int64_t rows, int64_t hidden, int64_t intermediate, int64_t blocksize,
                                             float epsilon, uint64_t stream);

/* ------------------------------------------------------------- NF4 GEMV */
/* NEW — standalone NF4 GEMV (the reference has GEMV only inside its fused
 * ops, kernels/common/nf4_tiled_gemv.cuh:15-52).  output[r] =
 * bf16(x . W[r] + bias[r]) or, with residual, bf16(residual[r] + bf16(x . W[r])).
 * bias and residual may be 0.  Contract: rows=1, in_features=2048,
 * out_features>=1, blocksize=64. */
KUDACUDA_API int kudacuda_nf4_gemv_bf16(void* handle, uint64_t input, uint64_t weight_packed, uint64_t absmax,
                                        uint64_t bias, uint64_t residual, uint64_t output, int64_t rows,
                                        int64_t in_features, int64_t out_features, int64_t blocksize,
                                        uint64_t stream);

/* ------------------------------------------------------- NF4 GEMM (prefill) */
/* NEW — multi-token NF4 GEMM on MFMA for prefill (the reference runs prompt
 * tokens through bitsandbytes' dequantize + bf16 matmul in the framework,
 * python/kudacuda_sidecar.py:1719-1738, or as sequential decode steps,
 * README.md:170).  output[m, n] = bf16(x[m] . Wbf16[n] + bias[n]) or, with
 * residual (then bias must be 0), bf16(residual[m, n] + bf16(x[m] . Wbf16[n]))
 * with Wbf16 = bf16(codebook[code] * absmax); fp32 accumulation.  residual may
 * alias output.  Contract: tokens>=1 (any count; processed 64 at a time),
 * out_features a positive multiple of 64, in_features a positive multiple of
 * 128, blocksize=64; x and output row-major [tokens, features] bf16. */
KUDACUDA_API int kudacuda_nf4_gemm_bf16(void* handle, uint64_t input, uint64_t weight_packed, uint64_t absmax,
                                        uint64_t bias, uint64_t residual, uint64_t output, int64_t tokens,
                                        int64_t in_features, int64_t out_features, int64_t blocksize,
                                        uint64_t stream);

/* NEW — gate/up SwiGLU over many tokens on MFMA: output[m, n] =
 * bf16(silu(x[m] . Gbf16[n]) * (x[m] . Ubf16[n])), the multi-token form of
 * kudacuda_qwen2_swiglu_nf4_bf16 (include/kudacuda.h reference :157).  Same
 * contract as kudacuda_nf4_gemm_bf16. */
KUDACUDA_API int kudacuda_nf4_gemm_swiglu_bf16(void* handle, uint64_t input, uint64_t gate_weight_packed,
                                               uint64_t gate_absmax, uint64_t up_weight_packed, uint64_t up_absmax,
                                               uint64_t output, int64_t tokens, int64_t in_features,
                                               int64_t out_features, int64_t blocksize, uint64_t stream);

/* NEW — blockwise NF4 quantisation (blocksize 64) of `count` elements of
 * fp32 (input_dtype 0) or bf16 (input_dtype 1); count % 64 == 0.  Replaces
 * bitsandbytes' quantize_4bit for synthetic models (parity with bitsandbytes
 * itself is not claimed). */
KUDACUDA_API int kudacuda_nf4_quantize(void* handle, uint64_t input, int64_t input_dtype, int64_t count,
                                       int64_t blocksize, uint64_t packed_output, uint64_t absmax_output,
                                       uint64_t stream);

/* NEW — dequantise: output[i] = codebook[code_i] * absmax[i / blocksize]
 * (reference kernels/common/nf4_device.cuh:29-40) as fp32 (output_dtype 0,
 * bit exact), bf16 (1) or fp16 (2). */
KUDACUDA_API int kudacuda_nf4_dequantize(void* handle, uint64_t packed, uint64_t absmax, int64_t count,
                                         int64_t blocksize, int64_t output_dtype, uint64_t output, uint64_t stream);

/* --------------------------------------------------- GQA decode attention */
/* Contract: batch=1, query_len=1, query_heads=16, kv_heads=2, head_dim=128,
 * scale>0; caches are [1, 2, stride, 128] contiguous.  All variants run the
 * same split-KV kernel on gfx950 (one launch, fp32 online softmax). */

/* reference include/kudacuda.h:174 — split partials in the caller's
 * workspace (>= 16*8*130 fp32 for kv_capacity <= 512), kv_len on device. */
KUDACUDA_API int kudacuda_qwen2_gqa_decode_workspace_v3(void* handle, uint64_t query, uint64_t key_cache,
                                                        uint64_t value_cache, uint64_t output, uint64_t workspace,
                                                        uint64_t kv_len_device, int64_t batch_size,
                                                        int64_t query_len, int64_t kv_capacity, int64_t query_heads,
                                                        int64_t kv_heads, int64_t head_dim, float scale,
                                                        uint64_t stream);

/* reference include/kudacuda.h:192 (fp16) — kv_len 1..65536 */
KUDACUDA_API int kudacuda_qwen2_gqa_decode(void* handle, uint64_t query, uint64_t key_cache, uint64_t value_cache,
                                           uint64_t output, int64_t batch_size, int64_t query_len, int64_t kv_len,
                                           int64_t query_heads, int64_t kv_heads, int64_t head_dim, float scale,
                                           uint64_t stream);

/* reference include/kudacuda.h:208 (fp16) — kv_len read from the int32 at
 * kv_len_device (graph-safe), cache stride kv_capacity 1..65536 */
KUDACUDA_API int kudacuda_qwen2_gqa_decode_graph(void* handle, uint64_t query, uint64_t key_cache,
                                                 uint64_t value_cache, uint64_t output, int64_t batch_size,
                                                 int64_t query_len, int64_t kv_capacity, int64_t query_heads,
                                                 int64_t kv_heads, int64_t head_dim, float scale,
                                                 uint64_t kv_len_device, uint64_t stream);

/* reference include/kudacuda.h:225 (fp16) */
KUDACUDA_API int kudacuda_qwen2_gqa_decode_group_tiled(void* handle, uint64_t query, uint64_t key_cache,
                                                       uint64_t value_cache, uint64_t output, int64_t batch_size,
                                                       int64_t query_len, int64_t kv_len, int64_t query_heads,
                                                       int64_t kv_heads, int64_t head_dim, float scale,
                                                       uint64_t stream);

/* reference include/kudacuda.h:241 (fp16) */
KUDACUDA_API int kudacuda_qwen2_gqa_decode_vectorized(void* handle, uint64_t query, uint64_t key_cache,
                                                      uint64_t value_cache, uint64_t output, int64_t batch_size,
                                                      int64_t query_len, int64_t kv_len, int64_t query_heads,
                                                      int64_t kv_heads, int64_t head_dim, float scale,
                                                      uint64_t stream);

/* NEW — bf16 twins of include/kudacuda.h:192 and :208 (same arguments). */
KUDACUDA_API int kudacuda_qwen2_gqa_decode_bf16(void* handle, uint64_t query, uint64_t key_cache,
                                                uint64_t value_cache, uint64_t output, int64_t batch_size,
                                                int64_t query_len, int64_t kv_len, int64_t query_heads,
                                                int64_t kv_heads, int64_t head_dim, float scale, uint64_t stream);
KUDACUDA_API int kudacuda_qwen2_gqa_decode_graph_bf16(void* handle, uint64_t query, uint64_t key_cache,
                                                      uint64_t value_cache, uint64_t output, int64_t batch_size,
                                                      int64_t query_len, int64_t kv_capacity, int64_t query_heads,
                                                      int64_t kv_heads, int64_t head_dim, float scale,
                                                      uint64_t kv_len_device, uint64_t stream);

/* NEW — no counterpart in the reference: the allocation-free twin of
 * kudacuda_qwen2_gqa_decode_graph_bf16 (same arguments, same kernels, same
 * results) for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Its
 * split partials and ticket counters live in a fixed static device array of
 * the library (2,130,176 B per GPU, held until the process ends) instead of
 * the handle's scratch; the call itself allocates nothing.  kv_capacity
 * 1..65536, as for the allocating twin (larger is rejected with status 1).  Every call on one GPU shares that
 * array, so calls that overlap on one GPU (two streams, two handles) race;
 * serialise them. */
KUDACUDA_API int kudacuda_qwen2_gqa_decode_graph_bf16_noalloc(void* handle, uint64_t query, uint64_t key_cache,
                                                              uint64_t value_cache, uint64_t output,
                                                              int64_t batch_size, int64_t query_len,
                                                              int64_t kv_capacity, int64_t query_heads,
                                                              int64_t kv_heads, int64_t head_dim, float scale,
                                                              uint64_t kv_len_device, uint64_t stream);

/* NEW — split-KV chunk (tokens per split) and fp32 workspace size used for a
 * given cache length; the decoder sizes its attention workspace with it. */
KUDACUDA_API int64_t kudacuda_gqa_split_chunk(int64_t kv_tokens);
KUDACUDA_API int64_t kudacuda_gqa_workspace_floats(int64_t kv_tokens);

/* ------------------------------------------------------ lm_head + argmax */
/* NEW — logits = bf16(E . RMSNorm(x)) over a bf16 [vocab, hidden] table
 * (norm skipped when norm_weight == 0), greedy argmax of the bf16 logits
 * (lowest index on ties) into the int32 at argmax_out.  logits may be 0.
 * Contract: hidden=2048, vocab>=1.  Replaces Transformers' lm_head +
 * torch.argmax (tools/benchmark/benchmark_gemma.py:324,350). */
KUDACUDA_API int kudacuda_lm_head_argmax_bf16(void* handle, uint64_t input, uint64_t norm_weight, uint64_t weight,
                                              uint64_t logits, uint64_t argmax_out, int64_t vocab, int64_t hidden,
                                              float epsilon, uint64_t stream);
KUDACUDA_API int64_t kudacuda_lm_head_workspace_floats(void);

/* ------------------------------------------------------------- graphs */
/* reference include/kudacuda.h:257-263 — capture the caller's stream (global
 * mode), instantiate on end, replay with hipGraphLaunch, reset.  A replay of
 * a graph holding scratch-using calls is refused (1) like an eager call while
 * the handle's last scratch user on another stream has work queued. */
KUDACUDA_API int kudacuda_begin_capture(void* handle, uint64_t stream);
KUDACUDA_API int kudacuda_end_capture(void* handle, uint64_t stream);
KUDACUDA_API int kudacuda_replay_graph(void* handle, uint64_t stream);
KUDACUDA_API int kudacuda_reset_graph(void* handle);

/* reference include/kudacuda.h:265,267 */
KUDACUDA_API const char* kudacuda_last_error(void* handle);
KUDACUDA_API void kudacuda_destroy(void* handle);

/* ---------------------------------------------- native Qwen2 decode step */
/* NEW — the whole batch-1 decode step of a Qwen2 (Qwen2.5-3B shape) NF4 model
 * on device: per layer {RMSNorm+QKV+bias+RoPE+cache write, split-KV GQA,
 * O GEMV+residual, RMSNorm+gate/up+SiLU*up, down GEMV+residual}, then final
 * RMSNorm + tied bf16 lm_head + argmax + token bookkeeping.  The reference
 * runs this step through Transformers under a CUDA graph
 * (python/kudacuda_static_decode.py:271-437); here every op is native.
 *
 * All buffers are caller-owned; the model object keeps only the pointer
 * table.  layer_ptrs is [num_layers][KUDACUDA_QWEN2_LAYER_FIELDS], model_ptrs
 * is [KUDACUDA_QWEN2_MODEL_FIELDS] (indices below).  control is int32[8]:
 * [0] step (= position of the current input token tokens[step]), [1] prompt
 * length, [2] token capacity of `tokens`, [3] stop token id (< 0: none),
 * [4] done flag, [5] position of the stop token, [6..7] 0; a step reads
 * tokens[step], writes tokens[step+1] once step+1 >= prompt length, then
 * increments step.  A step that emits the stop token (the reference's EOS
 * stop, tools/benchmark/benchmark_gemma.py:100-112,147, here decided on the
 * device so no host sync per token is needed) keeps it in tokens[], sets
 * [4] = 1 and [5] = its position; every later step is a no-op on the token
 * array, the step counter and the KV cache, so a caller may replay a fixed
 * number of steps and read [4] / [5] afterwards.
 * Counters (attention [2], lm_head [1], uint32) must be zero at creation. */
enum {
    KUDACUDA_QWEN2_INPUT_NORM = 0,
    KUDACUDA_QWEN2_Q_PACKED,
    KUDACUDA_QWEN2_Q_ABSMAX,
    KUDACUDA_QWEN2_Q_BIAS,
    KUDACUDA_QWEN2_K_PACKED,
    KUDACUDA_QWEN2_K_ABSMAX,
    KUDACUDA_QWEN2_K_BIAS,
    KUDACUDA_QWEN2_V_PACKED,
    KUDACUDA_QWEN2_V_ABSMAX,
    KUDACUDA_QWEN2_V_BIAS,
    KUDACUDA_QWEN2_O_PACKED,
    KUDACUDA_QWEN2_O_ABSMAX,
    KUDACUDA_QWEN2_POST_NORM,
    KUDACUDA_QWEN2_GATE_PACKED,
    KUDACUDA_QWEN2_GATE_ABSMAX,
    KUDACUDA_QWEN2_UP_PACKED,
    KUDACUDA_QWEN2_UP_ABSMAX,
    KUDACUDA_QWEN2_DOWN_PACKED,
    KUDACUDA_QWEN2_DOWN_ABSMAX,
    KUDACUDA_QWEN2_KEY_CACHE,
    KUDACUDA_QWEN2_VALUE_CACHE,
    KUDACUDA_QWEN2_LAYER_FIELDS
};
enum {
    KUDACUDA_QWEN2_EMBED = 0,      /* bf16 [vocab, 2048], tied lm_head */
    KUDACUDA_QWEN2_FINAL_NORM,     /* bf16 [2048] */
    KUDACUDA_QWEN2_ROPE_COS,       /* fp32 [kv_capacity, 64] */
    KUDACUDA_QWEN2_ROPE_SIN,
    KUDACUDA_QWEN2_HIDDEN,         /* bf16 [2048] residual stream */
    KUDACUDA_QWEN2_QUERY,          /* bf16 [2048] */
    KUDACUDA_QWEN2_ATTN,           /* bf16 [2048] */
    KUDACUDA_QWEN2_MLP,            /* bf16 [11008] */
    KUDACUDA_QWEN2_LOGITS,         /* bf16 [vocab] or 0 */
    KUDACUDA_QWEN2_TOKENS,         /* int32 [token capacity] */
    KUDACUDA_QWEN2_CONTROL,        /* int32 [8] */
    KUDACUDA_QWEN2_ATTN_PARTIALS,  /* fp32 [kudacuda_gqa_workspace_floats(kv_capacity)] */
    KUDACUDA_QWEN2_ATTN_COUNTERS,  /* uint32 [2] */
    KUDACUDA_QWEN2_LM_BEST,        /* fp32 [kudacuda_lm_head_workspace_floats()] */
    KUDACUDA_QWEN2_LM_COUNTER,     /* reserved, unused: may be 0 (keeps the field numbers stable) */
    KUDACUDA_QWEN2_MODEL_FIELDS
};

/* Contract: hidden 2048, intermediate 11008, 16/2 heads, head_dim 128,
 * blocksize 64, 1 <= kv_capacity <= 32768. Returns null on failure (reason in
 * kudacuda_last_error(handle)). */
KUDACUDA_API void* kudacuda_qwen2_model_create(void* handle, int64_t num_layers, int64_t vocab, int64_t kv_capacity,
                                               float rms_epsilon, const uint64_t* layer_ptrs,
                                               const uint64_t* model_ptrs);
/* Launch one decode step on `stream` (eager). */
KUDACUDA_API int kudacuda_qwen2_model_step(void* model, uint64_t stream);
/* Capture one decode step into the model's own hipGraphs (replaces any
 * previous ones) and instantiate them; the step is not executed.  The step
 * is captured in one form per attention split count o_proj can merge (1..16
 * splits of 32 cached tokens per KV head, o_proj requesting exactly that
 * many) and, when the cache can hold more, in a form for long caches
 * (attention merged by its own kernel, o_proj as a plain GEMV). */
KUDACUDA_API int kudacuda_qwen2_model_capture(void* model, uint64_t stream);
/* Replay the captured step `steps` times back to back on `stream`.  Each
 * replay (and each eager step) takes the form made for the step the host
 * believes it runs at (kudacuda_qwen2_model_set_position, advanced by one
 * per step; set by model_prefill); every form computes identical results at
 * any length, so a wrong or unknown position costs time only. */
KUDACUDA_API int kudacuda_qwen2_model_replay(void* model, int64_t steps, uint64_t stream);
/* NEW (no reference counterpart) -- the step value (control[0]) the next
 * step or replay runs at, or -1 for unknown (then the 6-split form runs).
 * Call it whenever the caller writes control[0] itself. */
KUDACUDA_API int kudacuda_qwen2_model_set_position(void* model, int64_t step);
/* Time one kernel of the step in isolation: op 0 = qkv+rope, 1 = attention,
 * 2 = o_proj, 3 = gate/up, 4 = down, 5 = lm_head; `iters` (1..4096) launches
 * cycling over the layers (so weights are not cache resident) are captured in
 * a hipGraph and replayed between two HIP events on `stream`; *avg_ms
 * receives the mean launch duration. */
KUDACUDA_API int kudacuda_qwen2_model_time_op(void* model, int64_t op, int64_t iters, uint64_t stream,
                                              float* avg_ms);
/* NEW — multi-token prefill (the reference prefills through Transformers or
 * as one decode step per prompt token, python/kudacuda_static_decode.py:
 * 271-437, README.md:170): tokens[start .. start+count-1] (device token array)
 * run through every layer at once (NF4 GEMMs on MFMA with bf16-dequantised
 * weights, causal GQA over the cache), writing KV cache rows start ..
 * start+count-1; then the last row's final norm + lm_head + argmax with the
 * decode bookkeeping (tokens[start+count] = greedy token, step =
 * start+count), so decode steps / replays continue from there.  workspace:
 * device memory of kudacuda_qwen2_prefill_workspace_bytes(count) bytes
 * (activations per token plus 16 MiB of split-K scratch for the GEMMs).
 * Eager (not for capture).  Contract: count>=1, start>=0,
 * start+count<=kv_capacity. */
KUDACUDA_API int64_t kudacuda_qwen2_prefill_workspace_bytes(int64_t tokens);
KUDACUDA_API int kudacuda_qwen2_model_prefill(void* model, uint64_t workspace, int64_t workspace_bytes,
                                              int64_t start, int64_t count, uint64_t stream);
KUDACUDA_API void kudacuda_qwen2_model_destroy(void* model);

#ifdef __cplusplus
}
#endif
