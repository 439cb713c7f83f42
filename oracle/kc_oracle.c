/*
 * CPU ORACLE for the KudaCuda gfx950 decode path — TEST INFRASTRUCTURE ONLY.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the checker (or the timed CPU baseline);
 * the product (kudacuda_amd) never links, imports or calls it.
 *
 * It restates the reference's decode math in plain C, following the exact
 * fp32 operation order the gfx950 kernels are specified to use (lane->chunk
 * mapping, accumulator splits, butterfly stages, exp2 polynomial, rounding
 * points), so a correct kernel agrees with it BIT FOR BIT.  The restatement
 * itself is pinned independently (tests/test_oracle_*.py): against fp64
 * textbook formulas with tolerances, the reference's own known-answer values
 * and smoke-test fixtures, closed forms and invariants.
 *
 * Two GPU paths sum in an order this file does not restate, and are held to
 * the mathematics instead (fp64 references with stated tolerances, closed
 * forms): the multi-token prefill's MFMA GEMM and the matrix-core attention
 * tactic of direct calls from 8192 cached tokens.  gqa() here restates the
 * round path, which serves every other attention call.
 *
 * Reference anchors (paths in lijeuki/KudaCuda):
 *   NF4 codebook / nibble order / dequant  kernels/common/nf4_device.cuh:10-40
 *   RMSNorm (fp32, x*inv_rms*gamma)        kernels/common/nf4_tiled_gemv.cuh:61-100,
 *                                          harness/reference.py:9-31
 *   NF4 row dot, bias in fp32              kernels/common/nf4_tiled_gemv.cuh:15-52,102-168
 *   SwiGLU silu(g)*u                       kernels/common/nf4_swiglu_bf16.cuh:61-164
 *   GQA split-KV + merge                   kernels/common/qwen2_gqa_workspace.cuh:13-120,
 *                                          kernels/common/qwen2_gqa_group_tiled.cuh:122-135
 *   GQA fp32 softmax oracle                tools/correctness/run_qwen2_gqa_check.py:19-28
 *   cache write at device position         python/kudacuda_static_decode.py:147-153
 *   greedy argmax (first max)              tools/benchmark/benchmark_gemma.py:350
 *
 * Build: oracle/build_oracle.sh (gcc -O2 -march=x86-64-v3 -ffp-contract=off
 * -fopenmp); x86 SSE float arithmetic, explicit fmaf only.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define KCO_API __attribute__((visibility("default")))

/* ------------------------------------------------------------ constants */
static const float kCodebook[16] = {
    -0x1.000000p+0f, -0x1.647362p-1f, -0x1.0cd660p-1f, -0x1.946540p-2f,
    -0x1.23449ap-2f, -0x1.7a6a7ep-3f, -0x1.74f0e2p-4f, 0x0.0p+0f,
    0x1.45f5fep-4f,  0x1.4995c6p-3f,  0x1.f809bap-3f,  0x1.5a0674p-2f,
    0x1.c34970p-2f,  0x1.200f56p-1f,  0x1.722766p-1f,  0x1.000000p+0f,
};
/* fp32 of the fp64 midpoints between neighbouring codebook values */
static const float kMid[15] = {
    -0x1.b239b0p-1f, -0x1.38a4e0p-1f, -0x1.d70900p-2f, -0x1.5bd4ecp-2f, -0x1.e079d8p-3f,
    -0x1.1a7178p-3f, -0x1.74f0e2p-5f, 0x1.45f5fep-5f,  0x1.ec90c4p-4f,  0x1.a0cfc0p-3f,
    0x1.2b05a8p-2f,  0x1.8ea7f2p-2f,  0x1.00da08p-1f,  0x1.491b5ep-1f,  0x1.b913b4p-1f,
};
static const float kLog2e = 0x1.715476p+0f;

/* ---------------------------------------------------------- conversions */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

static inline float bf16_to_f32(uint16_t v) { return u2f((uint32_t)v << 16); }
static inline uint16_t f32_to_bf16(float f) {
    uint32_t u = f2u(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static inline float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1fu;
    const uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24, exact in fp32 */
        float v = (float)man * 0x1p-24f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

/* fp32 -> fp16, round to nearest even, subnormals and overflow handled. */
static inline uint16_t f32_to_f16(float f) {
    const uint32_t u = f2u(f);
    const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    const uint32_t au = u & 0x7fffffffu;
    if (au > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((au >> 13) & 0x3ffu));
    if (au >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (au < 0x38800000u) {
        /* result is subnormal (or zero): value / 2^-24 rounded to an integer */
        if (au < 0x33000000u) return sign; /* < 2^-25 rounds to 0 (ties to even 0) */
        const uint32_t e = au >> 23;
        const uint32_t m = (au & 0x7fffffu) | 0x800000u;
        const int shift = (int)(126 - e) ; /* m * 2^(e-150) / 2^-24 = m >> (126 - e) */
        const uint32_t q = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u);
        const uint32_t half = 1u << (shift - 1);
        uint32_t r = q;
        if (rem > half || (rem == half && (q & 1u))) r += 1u;
        return (uint16_t)(sign | r);
    }
    uint32_t v = au - 0x38000000u; /* rebias exponent 127 -> 15 */
    const uint32_t rem = v & 0x1fffu;
    v >>= 13;
    if (rem > 0x1000u || (rem == 0x1000u && (v & 1u))) v += 1u;
    return (uint16_t)(sign | v);
}

static inline float act_load(int act, uint16_t v) { return act == 0 ? bf16_to_f32(v) : f16_to_f32(v); }
static inline uint16_t act_store(int act, float f) { return act == 0 ? f32_to_bf16(f) : f32_to_f16(f); }

/* ------------------------------------------------------------------ exp2 */
static inline float exp2_fixed(float y) {
    if (!(y >= -125.0f)) return (y != y) ? y : 0.0f;
    if (y >= 128.0f) return INFINITY;
    const float n = rintf(y);
    const float f = y - n;
    float p = 0x1.ffcbfcp-17f;
    p = fmaf(p, f, 0x1.430912p-13f);
    p = fmaf(p, f, 0x1.5d87fep-10f);
    p = fmaf(p, f, 0x1.3b2ab6p-7f);
    p = fmaf(p, f, 0x1.c6b08ep-5f);
    p = fmaf(p, f, 0x1.ebfbe0p-3f);
    p = fmaf(p, f, 0x1.62e430p-1f);
    p = fmaf(p, f, 1.0f);
    return ldexpf(p, (int)n);
}

static inline float silu_fixed(float g) {
    const float e = exp2_fixed(g * -kLog2e);
    return g / (1.0f + e);
}

/* ------------------------------------------------------------ reductions */
/* Butterfly over n = 64 (stages 32..1) or n = 16 (stages 8..1) lane values;
 * every lane ends equal, lane 0 is returned. */
static inline float butterfly(float* v, int n) {
    float t[64];
    for (int o = n / 2; o >= 1; o >>= 1) {
        for (int l = 0; l < n; ++l) t[l] = v[l] + v[l ^ o];
        memcpy(v, t, sizeof(float) * (size_t)n);
    }
    return v[0];
}

static inline float chunk_dot_raw(const uint8_t* pk, const float* x) {
    float a[4];
    for (int i = 0; i < 4; ++i) {
        float acc = 0.0f;
        for (int b = 0; b < 4; ++b) {
            const uint32_t byte = pk[4 * i + b];
            acc = fmaf(x[8 * i + 2 * b], kCodebook[byte >> 4], acc);
            acc = fmaf(x[8 * i + 2 * b + 1], kCodebook[byte & 0xfu], acc);
        }
        a[i] = acc;
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

static inline float sumsq32(const float* x) {
    float a[4];
    for (int i = 0; i < 4; ++i) {
        float acc = 0.0f;
        for (int j = 0; j < 8; ++j) acc = fmaf(x[8 * i + j], x[8 * i + j], acc);
        a[i] = acc;
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

static inline float inv_rms(float ss, float n, float eps) { return 1.0f / sqrtf(ss / n + eps); }

/* x (2048, 16-bit) -> xn fp32 laid out lane-major (lane l owns [32l, 32l+32)).
 * Sum of squares in the block-shared order of the GEMV/QKV/SwiGLU kernels:
 * wave w (0..3) covers [512w, 512w + 512), its lane l the 8 elements
 * 512w + 8l .. +7 (one fmaf chain), a 64-lane butterfly per wave, then
 * (w0 + w1) + (w2 + w3). */
static void norm_x2048(int act, const uint16_t* x, const uint16_t* gamma, float eps, float* xn) {
    for (int i = 0; i < 2048; ++i) xn[i] = act_load(act, x[i]);
    if (gamma == NULL) return;
    float ws[4];
    for (int w = 0; w < 4; ++w) {
        float part[64];
        for (int l = 0; l < 64; ++l) {
            float acc = 0.0f;
            for (int j = 0; j < 8; ++j) acc = fmaf(xn[512 * w + 8 * l + j], xn[512 * w + 8 * l + j], acc);
            part[l] = acc;
        }
        ws[w] = butterfly(part, 64);
    }
    const float r = inv_rms((ws[0] + ws[1]) + (ws[2] + ws[3]), 2048.0f, eps);
    for (int i = 0; i < 2048; ++i) xn[i] = (xn[i] * r) * act_load(act, gamma[i]);
}

/* Full dot of one K = 2048 NF4 row with xn. */
static inline float row2048_dot(const uint8_t* w, const float* absmax, int64_t r, const float* xn) {
    float part[64];
    const uint8_t* row = w + r * 1024;
    for (int l = 0; l < 64; ++l) part[l] = chunk_dot_raw(row + 16 * l, xn + 32 * l) * absmax[r * 32 + (l >> 1)];
    return butterfly(part, 64);
}

/* --------------------------------------------------------------- NF4 ops */
static void quantize_block(const float* v, uint8_t* packed, float* absmax) {
    float m = 0.0f;
    for (int i = 0; i < 64; ++i) m = fmaxf(m, fabsf(v[i]));
    int code[64];
    for (int i = 0; i < 64; ++i) {
        int c = 7;
        if (m > 0.0f) {
            const float s = v[i] * (1.0f / m);
            c = 0;
            for (int k = 0; k < 15; ++k) c += s > kMid[k] ? 1 : 0;
        }
        code[i] = c;
    }
    for (int i = 0; i < 32; ++i) packed[i] = (uint8_t)((code[2 * i] << 4) | code[2 * i + 1]);
    *absmax = m;
}

KCO_API void kco_nf4_quantize_f32(const float* src, int64_t n, uint8_t* packed, float* absmax) {
    const int64_t nb = n / 64;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nb; ++b) quantize_block(src + 64 * b, packed + 32 * b, absmax + b);
}

KCO_API void kco_nf4_quantize_bf16(const uint16_t* src, int64_t n, uint8_t* packed, float* absmax) {
    const int64_t nb = n / 64;
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < nb; ++b) {
        float v[64];
        for (int i = 0; i < 64; ++i) v[i] = bf16_to_f32(src[64 * b + i]);
        quantize_block(v, packed + 32 * b, absmax + b);
    }
}

KCO_API void kco_nf4_dequantize_f32(const uint8_t* packed, const float* absmax, int64_t n, int64_t blocksize,
                                    float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const uint32_t byte = packed[i >> 1];
        const uint32_t code = (i & 1) == 0 ? (byte >> 4) : (byte & 0xfu);
        out[i] = kCodebook[code] * absmax[i / blocksize];
    }
}

KCO_API void kco_convert(int from, int to, const void* in, void* out, int64_t n) {
    /* kinds: 0 fp32, 1 bf16, 2 fp16 */
    for (int64_t i = 0; i < n; ++i) {
        float v = from == 0 ? ((const float*)in)[i]
                 : from == 1 ? bf16_to_f32(((const uint16_t*)in)[i])
                             : f16_to_f32(((const uint16_t*)in)[i]);
        if (to == 0) ((float*)out)[i] = v;
        else if (to == 1) ((uint16_t*)out)[i] = f32_to_bf16(v);
        else ((uint16_t*)out)[i] = f32_to_f16(v);
    }
}

KCO_API void kco_exp2_array(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = exp2_fixed(in[i]);
}

KCO_API void kco_silu_array(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = silu_fixed(in[i]);
}

/* GEMV, K = 2048: out[r] = T(dot + bias) / T(res + T(dot)). */
KCO_API void kco_nf4_gemv2048(int act, const uint16_t* x, const uint8_t* w, const float* absmax,
                              const uint16_t* bias, const uint16_t* residual, int64_t rows, uint16_t* out) {
    float xn[2048];
    norm_x2048(act, x, NULL, 0.0f, xn);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        float v = row2048_dot(w, absmax, r, xn);
        if (bias != NULL) v = v + act_load(act, bias[r]);
        if (residual != NULL) v = act_load(act, residual[r]) + act_load(act, act_store(act, v));
        out[r] = act_store(act, v);
    }
}

/* fused RMSNorm + Q/K/V (+bias), optional fp32 normalised copy. */
KCO_API void kco_qkv(int act, const uint16_t* x, const uint16_t* gamma, float eps, const uint8_t* qw,
                     const float* qa, const uint16_t* qb, const uint8_t* kw, const float* ka, const uint16_t* kb,
                     const uint8_t* vw, const float* va, const uint16_t* vb, int64_t q_rows, int64_t kv_rows,
                     uint16_t* qo, uint16_t* ko, uint16_t* vo, float* norm_out) {
    float xn[2048];
    norm_x2048(act, x, gamma, eps, xn);
    if (norm_out != NULL) memcpy(norm_out, xn, sizeof(xn));
    const uint8_t* W[3] = {qw, kw, vw};
    const float* A[3] = {qa, ka, va};
    const uint16_t* B[3] = {qb, kb, vb};
    uint16_t* O[3] = {qo, ko, vo};
    const int64_t R[3] = {q_rows, kv_rows, kv_rows};
    for (int m = 0; m < 3; ++m) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < R[m]; ++r) {
            const float v = row2048_dot(W[m], A[m], r, xn) + act_load(act, B[m][r]);
            O[m][r] = act_store(act, v);
        }
    }
}

/* fused RMSNorm + QKV + bias + RoPE; q -> qo, k/v -> caches at pos. */
KCO_API void kco_qkv_rope_cache(const uint16_t* x, const uint16_t* gamma, float eps, const uint8_t* qw,
                                const float* qa, const uint16_t* qb, const uint8_t* kw, const float* ka,
                                const uint16_t* kb, const uint8_t* vw, const float* va, const uint16_t* vb,
                                const float* rope_cos, const float* rope_sin, int64_t pos, int64_t capacity,
                                uint16_t* qo, uint16_t* kcache, uint16_t* vcache) {
    float xn[2048];
    norm_x2048(0, x, gamma, eps, xn);
    if (pos < 0) pos = 0;
    if (pos >= capacity) pos = capacity - 1;
    const uint8_t* W[3] = {qw, kw, vw};
    const float* A[3] = {qa, ka, va};
    const uint16_t* B[3] = {qb, kb, vb};
    const int64_t R[3] = {2048, 256, 256};
    for (int m = 0; m < 3; ++m) {
        const int64_t pairs = R[m] / 2;
#pragma omp parallel for schedule(static)
        for (int64_t j = 0; j < pairs; ++j) {
            const int64_t r0 = (j / 64) * 128 + (j % 64);
            const int64_t r1 = r0 + 64;
            const float v0 = row2048_dot(W[m], A[m], r0, xn) + bf16_to_f32(B[m][r0]);
            const float v1 = row2048_dot(W[m], A[m], r1, xn) + bf16_to_f32(B[m][r1]);
            float o0 = v0, o1 = v1;
            if (m < 2) {
                const int64_t d = r0 & 127;
                const float c = rope_cos[pos * 64 + d];
                const float s = rope_sin[pos * 64 + d];
                o0 = (v0 * c) - (v1 * s);
                o1 = (v1 * c) + (v0 * s);
            }
            if (m == 0) {
                qo[r0] = f32_to_bf16(o0);
                qo[r1] = f32_to_bf16(o1);
            } else {
                uint16_t* cache = m == 1 ? kcache : vcache;
                const int64_t base = ((r0 >> 7) * capacity + pos) * 128;
                cache[base + (r0 & 127)] = f32_to_bf16(o0);
                cache[base + (r1 & 127)] = f32_to_bf16(o1);
            }
        }
    }
}

KCO_API void kco_swiglu(int act, const uint16_t* x, const uint16_t* gamma, float eps, const uint8_t* gw,
                        const float* ga, const uint8_t* uw, const float* ua, int64_t rows, uint16_t* out) {
    float xn[2048];
    norm_x2048(act, x, gamma, eps, xn);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float g = row2048_dot(gw, ga, r, xn);
        const float u = row2048_dot(uw, ua, r, xn);
        out[r] = act_store(act, silu_fixed(g) * u);
    }
}

/* down projection, K = 11008 (344 chunks over 6 waves). */
KCO_API void kco_down11008(int act, const uint16_t* x, const uint8_t* w, const float* absmax,
                           const uint16_t* residual, int64_t rows, uint16_t* out) {
    enum { NCH = 344, W = 6 };
    float* xf = (float*)malloc(sizeof(float) * NCH * 32);
    for (int i = 0; i < NCH * 32; ++i) xf[i] = act_load(act, x[i]);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const uint8_t* row = w + r * (NCH * 16);
        float s = 0.0f;
        for (int wv = 0; wv < W; ++wv) {
            float part[64];
            for (int l = 0; l < 64; ++l) {
                const int c = wv * 64 + l;
                part[l] = c < NCH ? chunk_dot_raw(row + 16 * c, xf + 32 * c) * absmax[r * (NCH / 2) + (c >> 1)] : 0.0f;
            }
            const float ws = butterfly(part, 64);
            s = wv == 0 ? ws : s + ws;
        }
        if (residual != NULL) s = act_load(act, residual[r]) + act_load(act, act_store(act, s));
        out[r] = act_store(act, s);
    }
    free(xf);
}

/* ------------------------------------------------------------------- GQA */
/* A block's 32 groups of 16 lanes take one token each per round. */
#define GQA_ROUND 32
/* most splits per KV head of an uncapped plan */
#define GQA_SPLIT_CAP 256
/* merges sum splits in groups of GQA_MERGE_GROUP, then the group sums */
#define GQA_MERGE_GROUP 16
/* Split cap of the decode step's plan (its merges are deferred or in-kernel). */
#define GQA_STEP_SPLITS 32

/* tokens per split at kv_len L with at most split_cap splits: the fewest
 * whole rounds that keep the split count within the cap */
KCO_API int64_t kco_gqa_split_tokens(int64_t L, int64_t split_cap) {
    const int64_t rounds = (L + GQA_ROUND - 1) / GQA_ROUND;
    const int64_t per = (rounds + split_cap - 1) / split_cap;
    return GQA_ROUND * (per > 1 ? per : 1);
}

/* The kernels' split plan for a cache of `capacity` rows (split_limit > 0 caps
 * the splits): out = {split_cap, max_splits}. */
KCO_API void kco_gqa_plan(int64_t capacity, int64_t split_limit, int64_t* plan) {
    const int64_t cap = split_limit > 0 && split_limit < GQA_SPLIT_CAP ? split_limit : GQA_SPLIT_CAP;
    const int64_t rounds = (capacity + GQA_ROUND - 1) / GQA_ROUND;
    plan[0] = cap;
    plan[1] = rounds < cap ? rounds : cap;
}

/* 16-lane partial dots of one K row with the 8 query heads of its group,
 * reduced by the lanes' butterfly and scaled into the log2 domain. */
static void gqa_scores(int act, const float qf[8][128], const uint16_t* krow, float qk_scale_log2, float* s8) {
    for (int hl = 0; hl < 8; ++hl) {
        float lanes[16];
        for (int li = 0; li < 16; ++li) {
            float dsum = 0.0f;
            for (int j = 0; j < 8; ++j) dsum = fmaf(qf[hl][8 * li + j], act_load(act, krow[8 * li + j]), dsum);
            lanes[li] = dsum;
        }
        s8[hl] = butterfly(lanes, 16) * qk_scale_log2;
    }
}

/* q [16,128], caches [2, capacity, 128], kv_len L; split s of KV head g owns
 * tokens [s*C, min(s*C + C, L)), C = kco_gqa_split_tokens(L, split_cap),
 * processed in rounds of GQA_ROUND tokens with the online softmax:
 * m' = max(m, round max), rescale r = exp2(m - m'), w_t = exp2(s_t - m'),
 * l = l*r then + w_t in token order, acc = acc*r then fma(w_t, v_t, acc) in
 * token order.  The split partials are merged with w_s = exp2(m_s - M) in
 * groups of GQA_MERGE_GROUP splits (fma in split order), the group sums added
 * in order, and the output is acc * (1 / l) (one correctly rounded reciprocal,
 * then a product, as every merge site of the kernels computes it). */
KCO_API void kco_gqa(int act, const uint16_t* q, const uint16_t* kc, const uint16_t* vc, int64_t capacity,
                     int64_t L, int64_t split_cap, float qk_scale_log2, uint16_t* out) {
    if (L > capacity) L = capacity;
    if (L < 1) {
        /* empty cache: zero output (reference qwen2_gqa_workspace.cuh:118,
         * total > 0 ? weighted / total : 0) */
        memset(out, 0, sizeof(uint16_t) * 16 * 128);
        return;
    }
    const int64_t C = kco_gqa_split_tokens(L, split_cap);
    const int64_t nsplit = (L + C - 1) / C;
    float* part = (float*)malloc(sizeof(float) * 16 * (size_t)nsplit * 130);
#pragma omp parallel for collapse(2) schedule(static)
    for (int g = 0; g < 2; ++g) {
        for (int64_t s = 0; s < nsplit; ++s) {
            float qf[8][128];
            for (int hl = 0; hl < 8; ++hl)
                for (int d = 0; d < 128; ++d) qf[hl][d] = act_load(act, q[(8 * g + hl) * 128 + d]);
            float m[8], l[8], acc[8][128];
            for (int hl = 0; hl < 8; ++hl) {
                m[hl] = -INFINITY;
                l[hl] = 0.0f;
                for (int d = 0; d < 128; ++d) acc[hl][d] = 0.0f;
            }
            const int64_t t0 = s * C;
            const int64_t tend = t0 + C < L ? t0 + C : L;
            for (int64_t base = t0; base < tend; base += GQA_ROUND) {
                const int nv = (int)(tend - base < GQA_ROUND ? tend - base : GQA_ROUND);
                float sc[GQA_ROUND][8];
                for (int t = 0; t < nv; ++t)
                    gqa_scores(act, (const float(*)[128])qf, kc + ((int64_t)g * capacity + base + t) * 128,
                               qk_scale_log2, sc[t]);
                for (int hl = 0; hl < 8; ++hl) {
                    float mr = -INFINITY;
                    for (int t = 0; t < nv; ++t) mr = fmaxf(mr, sc[t][hl]);
                    const float mn = fmaxf(m[hl], mr);
                    const float r = exp2_fixed(m[hl] - mn);
                    float w[GQA_ROUND];
                    for (int t = 0; t < nv; ++t) w[t] = exp2_fixed(sc[t][hl] - mn);
                    l[hl] = l[hl] * r;
                    for (int t = 0; t < nv; ++t) l[hl] = l[hl] + w[t];
                    for (int d = 0; d < 128; ++d) {
                        float a = acc[hl][d] * r;
                        for (int t = 0; t < nv; ++t)
                            a = fmaf(w[t], act_load(act, vc[((int64_t)g * capacity + base + t) * 128 + d]), a);
                        /* the kernel's sum runs over whole quads of tokens, the
                         * slots past the end holding weight 0 and value 0: a
                         * zero product added (turns -0 into +0, else exact) */
                        if (nv & 3) a = fmaf(0.0f, 0.0f, a);
                        acc[hl][d] = a;
                    }
                    m[hl] = mn;
                }
            }
            for (int hl = 0; hl < 8; ++hl) {
                float* dst = part + ((int64_t)(8 * g + hl) * nsplit + s) * 130;
                dst[0] = m[hl];
                dst[1] = l[hl];
                memcpy(dst + 2, acc[hl], sizeof(float) * 128);
            }
        }
    }
    for (int h = 0; h < 16; ++h) {
        const float* src = part + (int64_t)h * nsplit * 130;
        float M = -INFINITY;
        for (int64_t s = 0; s < nsplit; ++s) M = fmaxf(M, src[s * 130]);
        for (int d = 0; d < 128; ++d) {
            float lt = 0.0f, o = 0.0f;
            for (int64_t j = 0; j < nsplit; j += GQA_MERGE_GROUP) {
                float lg = 0.0f, og = 0.0f;
                for (int64_t s = j; s < j + GQA_MERGE_GROUP && s < nsplit; ++s) {
                    const float* p = src + s * 130;
                    const float w = exp2_fixed(p[0] - M);
                    lg = fmaf(p[1], w, lg);
                    og = fmaf(p[2 + d], w, og);
                }
                if (j == 0) {
                    lt = lg;
                    o = og;
                } else {
                    lt = lt + lg;
                    o = o + og;
                }
            }
            out[h * 128 + d] = act_store(act, o * (1.0f / lt));
        }
    }
    free(part);
}

/* --------------------------------------------------------------- lm_head */
KCO_API int32_t kco_lm_head_argmax(const uint16_t* x, const uint16_t* gamma, float eps, const uint16_t* weight,
                                   int64_t vocab, uint16_t* logits) {
    float xs[2048];
    for (int i = 0; i < 2048; ++i) xs[i] = bf16_to_f32(x[i]);
    float r = 1.0f;
    if (gamma != NULL) {
        float part[64];
        for (int l = 0; l < 64; ++l) part[l] = sumsq32(xs + 32 * l);
        r = inv_rms(butterfly(part, 64), 2048.0f, eps);
    }
    float xn[2048]; /* indexed by element */
    for (int e = 0; e < 2048; ++e) xn[e] = gamma != NULL ? (xs[e] * r) * bf16_to_f32(gamma[e]) : xs[e];
    int32_t best_idx = 0x7fffffff;
    float best = -INFINITY;
#pragma omp parallel
    {
        int32_t tb_idx = 0x7fffffff;
        float tb = -INFINITY;
#pragma omp for schedule(static)
        for (int64_t row = 0; row < vocab; ++row) {
            const uint16_t* w = weight + row * 2048;
            float part[64];
            for (int l = 0; l < 64; ++l) {
                float a[4];
                for (int c = 0; c < 4; ++c) {
                    const int e0 = 8 * (l + 64 * c);
                    float acc = 0.0f;
                    for (int j = 0; j < 8; ++j) acc = fmaf(xn[e0 + j], bf16_to_f32(w[e0 + j]), acc);
                    a[c] = acc;
                }
                part[l] = (a[0] + a[1]) + (a[2] + a[3]);
            }
            const uint16_t lb = f32_to_bf16(butterfly(part, 64));
            if (logits != NULL) logits[row] = lb;
            const float v = bf16_to_f32(lb);
            if (v > tb || (v == tb && (int32_t)row < tb_idx)) {
                tb = v;
                tb_idx = (int32_t)row;
            }
        }
#pragma omp critical
        {
            if (tb > best || (tb == best && tb_idx < best_idx)) {
                best = tb;
                best_idx = tb_idx;
            }
        }
    }
    if (best_idx < 0 || best_idx >= vocab) best_idx = 0;
    return best_idx;
}

/* ------------------------------------------------------- Qwen2 decode step */
enum {
    L_INPUT_NORM = 0, L_Q_PACKED, L_Q_ABSMAX, L_Q_BIAS, L_K_PACKED, L_K_ABSMAX, L_K_BIAS, L_V_PACKED, L_V_ABSMAX,
    L_V_BIAS, L_O_PACKED, L_O_ABSMAX, L_POST_NORM, L_GATE_PACKED, L_GATE_ABSMAX, L_UP_PACKED, L_UP_ABSMAX,
    L_DOWN_PACKED, L_DOWN_ABSMAX, L_KEY_CACHE, L_VALUE_CACHE, L_FIELDS
};
enum {
    M_EMBED = 0, M_FINAL_NORM, M_ROPE_COS, M_ROPE_SIN, M_HIDDEN, M_QUERY, M_ATTN, M_MLP, M_LOGITS, M_TOKENS,
    M_CONTROL, M_ATTN_PARTIALS, M_ATTN_COUNTERS, M_LM_BEST, M_LM_COUNTER, M_FIELDS
};
#define P(type, v) ((type)(uintptr_t)(v))

/* One decode step with the same pointer tables as kudacuda_qwen2_model_create
 * (host pointers here).  Workspace/counter fields are ignored. */
KCO_API void kco_qwen2_step(int64_t num_layers, int64_t vocab, int64_t capacity, float eps,
                            const uint64_t* layer_ptrs, const uint64_t* model_ptrs) {
    const uint64_t* G = model_ptrs;
    int32_t* control = P(int32_t*, G[M_CONTROL]);
    int32_t* tokens = P(int32_t*, G[M_TOKENS]);
    uint16_t* hidden = P(uint16_t*, G[M_HIDDEN]);
    uint16_t* query = P(uint16_t*, G[M_QUERY]);
    uint16_t* attn = P(uint16_t*, G[M_ATTN]);
    uint16_t* mlp = P(uint16_t*, G[M_MLP]);
    int64_t pos = control[0];
    if (pos < 0) pos = 0;
    if (pos >= capacity) pos = capacity - 1;
    const int64_t tok_cap = control[2];
    const int64_t tpos = pos < tok_cap ? pos : (tok_cap > 0 ? tok_cap - 1 : 0);
    int64_t tok = tokens[tpos];
    if (tok < 0) tok = 0;
    if (tok >= vocab) tok = vocab - 1;
    memcpy(hidden, P(const uint16_t*, G[M_EMBED]) + tok * 2048, 2048 * sizeof(uint16_t));
    int64_t L = (int64_t)control[0] + 1;
    if (L > capacity) L = capacity;
    const float qk_scale_log2 = (float)(1.0 / sqrt(128.0)) * kLog2e;
    int64_t plan[2];
    kco_gqa_plan(capacity, GQA_STEP_SPLITS, plan);
    /* a stopped decode (control[4]) writes no KV-cache row: the rows the QKV
     * op writes at pos are put back before attention reads the cache */
    const int stopped = control[4] != 0;
    for (int64_t layer = 0; layer < num_layers; ++layer) {
        const uint64_t* Lp = layer_ptrs + layer * L_FIELDS;
        uint16_t saved[2][2][128];
        for (int g = 0; g < 2 && stopped; ++g) {
            memcpy(saved[0][g], P(uint16_t*, Lp[L_KEY_CACHE]) + ((int64_t)g * capacity + pos) * 128, 256);
            memcpy(saved[1][g], P(uint16_t*, Lp[L_VALUE_CACHE]) + ((int64_t)g * capacity + pos) * 128, 256);
        }
        kco_qkv_rope_cache(hidden, P(const uint16_t*, Lp[L_INPUT_NORM]), eps, P(const uint8_t*, Lp[L_Q_PACKED]),
                           P(const float*, Lp[L_Q_ABSMAX]), P(const uint16_t*, Lp[L_Q_BIAS]),
                           P(const uint8_t*, Lp[L_K_PACKED]), P(const float*, Lp[L_K_ABSMAX]),
                           P(const uint16_t*, Lp[L_K_BIAS]), P(const uint8_t*, Lp[L_V_PACKED]),
                           P(const float*, Lp[L_V_ABSMAX]), P(const uint16_t*, Lp[L_V_BIAS]),
                           P(const float*, G[M_ROPE_COS]), P(const float*, G[M_ROPE_SIN]), pos, capacity, query,
                           P(uint16_t*, Lp[L_KEY_CACHE]), P(uint16_t*, Lp[L_VALUE_CACHE]));
        for (int g = 0; g < 2 && stopped; ++g) {
            memcpy(P(uint16_t*, Lp[L_KEY_CACHE]) + ((int64_t)g * capacity + pos) * 128, saved[0][g], 256);
            memcpy(P(uint16_t*, Lp[L_VALUE_CACHE]) + ((int64_t)g * capacity + pos) * 128, saved[1][g], 256);
        }
        kco_gqa(0, query, P(const uint16_t*, Lp[L_KEY_CACHE]), P(const uint16_t*, Lp[L_VALUE_CACHE]), capacity, L,
                plan[0], qk_scale_log2, attn);
        kco_nf4_gemv2048(0, attn, P(const uint8_t*, Lp[L_O_PACKED]), P(const float*, Lp[L_O_ABSMAX]), NULL, hidden,
                         2048, hidden);
        kco_swiglu(0, hidden, P(const uint16_t*, Lp[L_POST_NORM]), eps, P(const uint8_t*, Lp[L_GATE_PACKED]),
                   P(const float*, Lp[L_GATE_ABSMAX]), P(const uint8_t*, Lp[L_UP_PACKED]),
                   P(const float*, Lp[L_UP_ABSMAX]), 11008, mlp);
        kco_down11008(0, mlp, P(const uint8_t*, Lp[L_DOWN_PACKED]), P(const float*, Lp[L_DOWN_ABSMAX]), hidden, 2048,
                      hidden);
    }
    /* bookkeeping: tokens[step + 1] once past the prompt; the stop token
     * (control[3] >= 0) sets the done flag and its position, after which a
     * step neither writes a token nor advances */
    if (stopped) return;
    const int32_t step = control[0];
    const int active = step + 1 >= control[1];
    if (active) {
        const int32_t t = kco_lm_head_argmax(hidden, P(const uint16_t*, G[M_FINAL_NORM]), eps,
                                             P(const uint16_t*, G[M_EMBED]), vocab, P(uint16_t*, G[M_LOGITS]));
        if (step + 1 < control[2]) tokens[step + 1] = t;
        if (control[3] >= 0 && t == control[3]) {
            control[4] = 1;
            control[5] = step + 1;
        }
    }
    control[0] = step + 1;
}
