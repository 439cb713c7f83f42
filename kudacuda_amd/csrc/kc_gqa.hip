// Split-KV grouped-query decode attention for the Qwen2.5-3B shape
// (16 query heads, 2 KV heads, group 8, head_dim 128), in two tactics:
//   * the round path (below): fp32 FMA rounds, every summation order fixed
//     and mirrored by the host oracle bit for bit; all graph-mode calls, the
//     decode step and direct calls under 8192 cached tokens;
//   * the matrix-core tactic (gqa_mfma_partial_kernel, further down): q.K and
//     P.V on MFMA for direct calls from 8192 tokens on, agreeing with the
//     round path to fp32 rounding.
// Both leave split partials in one layout, merged by gqa_merge_kernel.
//
// Round-path partial kernel, grid (max_splits, 2): block (s, g) owns one split of the
// tokens of KV head g and serves all 8 query heads of the group, so every K/V
// byte is read once.  A block is 8 waves = 32 groups of 16 lanes; lane li of a
// group holds dims [8li, 8li+8) of all 8 query heads.  Split s owns tokens
// [s*C, min(s*C+C, L)), C = gqa_split_tokens(L, split_cap): the fewest whole
// 32-token rounds that keep the split count within the cap (chosen from L on
// the device, so a graph replay reads kv_len from memory).
//
// A split is processed in rounds of 32 tokens, one per group.  Per round:
//   * scores: each lane forms 8 dims of the dot of its token's K row with the
//     8 query heads; a reduce-scatter over the 16 lanes (partner distances 8,
//     4, 2, 1 -- the pairs of a full butterfly, so every head's sum is the
//     butterfly's bit for bit) leaves head h's score in lanes 2h and 2h+1,
//     which is why lane li holds its query heads in the order k ^ (li/2 % 8);
//     the V row goes to LDS (zeros for a token past the end);
//   * weights (threads of (head, token)): the round's maximum per head, the
//     new running maximum m', w_t = exp2(s_t - m') and the rescale
//     exp2(m - m') of what the earlier rounds accumulated;
//   * weighted sum: wave w owns dims [16w, 16w+16) of all 8 heads (lane l:
//     head l/8, dims 16w + 2(l%8) and the next, so V is read from LDS by
//     broadcast, once per block): acc = acc * rescale, then
//     acc = fma(w_t, v_t, acc) in token order; wave 0 keeps the 8 sums l the
//     same way.
// The K/V rows of the next two rounds are in flight while a round computes,
// and the LDS is double-buffered, so a round costs two barriers.  A split of
// one round is the plain softmax of its tokens (rescale of zero by zero).
//
// The split partials (max, sum, acc[128] per head) are then, by the number of
// splits at this L:
//   * up to defer_max (the decode step sets it): left for the consumer, the
//     o_proj row kernel, which merges them while its weight rows stream in;
//   * one split: finished in place, out = acc*1 * (1 / (sum*1)), the general merge
//     with weight exp2(0) = 1;
//   * up to ticket_max (<= kInKernelSplits): merged by the last block of the
//     KV head to finish (an agent-scope acquire-release ticket, reset by that block,
//     so the launch is capture-safe);
//   * more: merged by gqa_merge_kernel (grid: query head x 16-dim slice),
//     launched after the partial kernel whenever the grid allows more than
//     ticket_max splits; it returns at once when L needs fewer.
// Every merge computes M = max over splits and w_s = exp2(m_s - M), sums
// fma(l_s, w_s, .) and fma(acc_s, w_s, .) over groups of kGqaMergeGroup
// consecutive splits in order, then adds the group sums in order, and scales
// the sums by one correctly rounded reciprocal of l (acc * (1 / l): one
// division per output instead of one per element where a thread finishes
// several, o_proj's merge prologue 3.79 -> 3.60 us).
// The result depends only on (inputs, kv_len, split_cap).
//
// Math follows the reference's split-KV workspace kernels
// (kernels/common/qwen2_gqa_workspace.cuh:13-120: per-tile max, sum and
// weighted V, merged with exp(m - M)) and the online softmax of
// kernels/common/qwen2_gqa_group_tiled.cuh:122-135; the kv_len < 1 and
// capacity clamps follow kernels/common/qwen2_gqa_workspace.cuh:35-36.
#include "kc_device.h"
#include "kc_kernels.h"

namespace kc {
namespace {

constexpr int kGqaWaves = 8;
constexpr int kGqaThreads = 64 * kGqaWaves;
constexpr int kGroups = 4 * kGqaWaves;      // 16-lane groups per block
constexpr int kRound = kGqaRoundTokens;     // tokens per round, one per group
static_assert(kRound == kGroups, "one token per 16-lane group and round");
constexpr int kHeadsPerGroup = 8;
constexpr int kDim = 128;
constexpr int kPartialStride = kGqaPartialStride;
static_assert(kPartialStride == 2 + kDim, "partial layout: max, sum, acc[128]");
constexpr int kInKernelSplits = 32;
// With kv_len in device memory, only splits below this request their rows
// before kv_len is known: the decode step's grid covers every split the cache
// bucket could need (64 at 2048 tokens) while decode lengths need a few, and
// the rows the idle blocks requested cost the step ~14 us of 1 ms (their
// traffic lands beside the live blocks' and the next kernel's).  16 splits
// cover decode lengths up to 512 tokens; later splits wait for kv_len first.
constexpr int64_t kSpeculativeSplits = 16;
constexpr int kMergeMaxSplits = 256;  // one split's max and sum per merge thread
static_assert(kGqaSplitCap <= kMergeMaxSplits, "every plan's split count (split_limit only lowers it)");
constexpr int kMergeDims = 16;              // dims per merge block
constexpr int kMergeGroups = kMergeMaxSplits / kGqaMergeGroup;
constexpr int kPitch = kRound + 4;          // score / weight rows: the 8 heads on distinct banks
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ int64_t read_kv_len(const GqaArgs& a) {
    int64_t L = a.kv_len_device != nullptr ? static_cast<int64_t>(*a.kv_len_device) + a.kv_len_offset : a.kv_len_host;
    return L < 0 ? 0 : (L > a.capacity ? a.capacity : L);
}

// DPP lane moves inside a row of 16 lanes.
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xb1;          // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4e;          // quad_perm [2,3,0,1]
constexpr int kDppXor3 = 0x1b;          // quad_perm [3,2,1,0]
constexpr int kDppHalfMirror = 0x141;   // lane l <- lane l ^ 7 within each half row
// the value of lane l ^ 4 (a half-row mirror, then a quad reversal)
__device__ __forceinline__ float lane_xor4(float v) { return dpp<kDppXor3>(dpp<kDppHalfMirror>(v)); }

// Maximum over each span of kSpan (32 or 64) lanes; exact, so the order of
// the stages does not matter.  Call with the whole wave active.
template <int kSpan>
__device__ __forceinline__ float span_max(float v) {
    if constexpr (kSpan == 64) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
    }
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
    v = fmaxf(v, row_ror<8>(v));
    v = fmaxf(v, row_ror<4>(v));
    v = fmaxf(v, row_ror<2>(v));
    return fmaxf(v, row_ror<1>(v));
}

// K and V rows of token t for one lane (dims 8li..8li+7), bounded by the
// capacity (rows past kv_len are read, never used).
__device__ __forceinline__ void load_row(const uint16_t* kbase, const uint16_t* vbase, int64_t t, int64_t capacity,
                                         uint4& kr, uint4& vr) {
    const int64_t tc = t < capacity ? t : capacity - 1;
    kr = *reinterpret_cast<const uint4*>(kbase + tc * kDim);
    vr = *reinterpret_cast<const uint4*>(vbase + tc * kDim);
}

// In-kernel merge of the first nsplit (<= N, N = 16 or 32) split partials of
// KV head g (the last block of the head runs it; agent-scope loads: the
// partials come from other blocks of this launch).  Every thread first
// requests the accumulator elements of its two (head, dim) outputs, all
// splits at once (coalesced across a wave), and threads (head t/N, split
// t%N) the splits' maxima and sums; those threads form the weights
// w_s = exp2(m_s - M) into LDS; then each output sums fma(l_s, w_s, .) and
// fma(acc_s, w_s, .) over groups of kGqaMergeGroup splits in order and adds
// the group sums in order.
template <typename T, int N>
__device__ __forceinline__ void ticket_merge(const GqaArgs& a, const float* part, int g, int nsplit,
                                             float (*s_w)[N], float (*s_l)[N]) {
    static_assert(N == 16 || N == 32, "row or half-wave spans");
    const float* head0 = part + static_cast<int64_t>(g * kHeadsPerGroup) * a.max_splits * kPartialStride;
    float vv[2][N];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int idx = threadIdx.x + k * kGqaThreads;
        const float* src = head0 + static_cast<int64_t>(idx / kDim) * a.max_splits * kPartialStride + 2 + idx % kDim;
#pragma unroll
        for (int x = 0; x < N; ++x) {
            vv[k][x] = x < nsplit ? load_agent(src + x * kPartialStride) : 0.0f;
        }
    }
    if (threadIdx.x < kHeadsPerGroup * N) {
        const int hl = threadIdx.x / N;
        const int x = threadIdx.x % N;
        const bool live = x < nsplit;
        const float* row = head0 + (static_cast<int64_t>(hl) * a.max_splits + x) * kPartialStride;
        const float m = live ? load_agent(row) : kNegInf;
        const float l = live ? load_agent(row + 1) : 0.0f;
        float M = m;
        if constexpr (N == 32) {
            M = span_max<32>(M);
        } else {
            M = fmaxf(M, row_ror<8>(M));
            M = fmaxf(M, row_ror<4>(M));
            M = fmaxf(M, row_ror<2>(M));
            M = fmaxf(M, row_ror<1>(M));
        }
        s_w[hl][x] = live ? exp2_fixed(m - M) : 0.0f;
        s_l[hl][x] = l;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int idx = threadIdx.x + k * kGqaThreads;
        const int hl = idx / kDim;
        float lt = 0.0f;
        float o = 0.0f;
#pragma unroll
        for (int j = 0; j < N; j += kGqaMergeGroup) {
            float lg = 0.0f;
            float og = 0.0f;
#pragma unroll
            for (int x = j; x < j + kGqaMergeGroup; ++x) {
                if (x < nsplit) {
                    lg = fmaf(s_l[hl][x], s_w[hl][x], lg);
                    og = fmaf(vv[k][x], s_w[hl][x], og);
                }
            }
            if (j == 0) {
                lt = lg;
                o = og;
            } else if (j < nsplit) {
                lt = lt + lg;
                o = o + og;
            }
        }
        a.out[(g * kHeadsPerGroup + hl) * kDim + idx % kDim] = T::store(o * (1.0f / lt));
    }
}

template <typename T>
__device__ __forceinline__ void gqa_partial_body(const uint16_t* k_rows, const uint16_t* v_rows, const uint16_t* q_vec,
                                                 const int32_t* kv_len_device, int64_t capacity, GqaArgs args) {
    // the leading scalar arguments (what the first loads need) are preloaded
    // into SGPRs at wave launch; they stand for the same fields of `args`
    GqaArgs a = args;
    a.k = k_rows;
    a.v = v_rows;
    a.q = q_vec;
    a.kv_len_device = kv_len_device;
    a.capacity = capacity;
    __shared__ __attribute__((aligned(16))) float s_vf[2][kRound][kDim];           // V rows of a round
    __shared__ __attribute__((aligned(16))) float s_sc[2][kHeadsPerGroup][kPitch];  // scores
    __shared__ __attribute__((aligned(16))) float s_wt[2][kHeadsPerGroup][kPitch];  // weights
    __shared__ float s_cr[2][kHeadsPerGroup];                                       // rescales
    __shared__ float s_M[kHeadsPerGroup];
    __shared__ float s_L[kHeadsPerGroup];
    __shared__ int s_last;

    const int g = blockIdx.y;
    // split s runs on block xcd_contiguous: at decode lengths the few live
    // splits share one XCD's L2 (decode step, attention 4.14 -> 4.07 us)
    const int64_t s = xcd_contiguous(blockIdx.x, gridDim.x);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int gi = wave * 4 + (lane >> 4);
    const int li = lane & 15;
    const int perm = (li >> 1) & 7;  // register k of this lane holds query head k ^ perm
    const uint16_t* kbase = a.k + static_cast<int64_t>(g) * a.capacity * kDim + 8 * li;
    const uint16_t* vbase = a.v + static_cast<int64_t>(g) * a.capacity * kDim + 8 * li;

    // q does not depend on kv_len: request it first, then the rows of this
    // split's first two rounds.  With kv_len in device memory the split size
    // is not known yet; the one-round split of decode lengths is assumed and
    // corrected below when it is wrong.
    uint4 qr[kHeadsPerGroup];
#pragma unroll
    for (int k = 0; k < kHeadsPerGroup; ++k) {
        qr[k] = *reinterpret_cast<const uint4*>(a.q + (g * kHeadsPerGroup + (k ^ perm)) * kDim + 8 * li);
    }
    const bool device_len = a.kv_len_device != nullptr;
    const int64_t c_guess = device_len ? kRound : gqa_split_tokens(read_kv_len(a), a.split_cap);
    // a host kv_len gives the live splits exactly; a device one is guessed
    // (kSpeculativeSplits)
    const bool spec = device_len ? s < kSpeculativeSplits : s * c_guess < read_kv_len(a);
    // Rows are always requested two at a time in this order (round r's K, V,
    // then round r+1's), rows past the split re-reading its last row, so the
    // waves' memory counters see the same sequence every round and each round
    // waits only for its own rows.
    uint4 k0, v0, k1, v1;
    if (spec) {
        // the guessed split's own rows only (a one-round split re-reads its
        // last row instead of the next split's first round)
        const int64_t g0 = s * c_guess;
        const int64_t g_end = g0 + c_guess < a.capacity ? g0 + c_guess : a.capacity;
        load_row(kbase, vbase, g0 + gi, g_end, k0, v0);
        load_row(kbase, vbase, g0 + kRound + gi, g_end, k1, v1);
    }

    const int64_t L = read_kv_len(a);
    const int64_t C = gqa_split_tokens(L, a.split_cap);
    const int64_t nsplit = (L + C - 1) / C;
    if (s >= nsplit) {
        if (nsplit == 0 && s == 0) {
            // empty cache (device kv_len <= 0): zero output, as the reference
            // workspace kernel writes (qwen2_gqa_workspace.cuh:118)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                a.out[(g * kHeadsPerGroup) * kDim + threadIdx.x + k * kGqaThreads] = 0;
            }
        }
        return;
    }
    const int64_t t0 = s * C;
    const int64_t tend = t0 + C < L ? t0 + C : L;
    if (!spec || C != c_guess) {
        load_row(kbase, vbase, t0 + gi, tend, k0, v0);
        load_row(kbase, vbase, t0 + kRound + gi, tend, k1, v1);
    }
    const int rounds = static_cast<int>((tend - t0 + kRound - 1) / kRound);

    float q[kHeadsPerGroup][8];
#pragma unroll
    for (int k = 0; k < kHeadsPerGroup; ++k) {
        unpack8<T>(qr[k], q[k]);
    }

    // weights phase: thread (head wh, token wx) keeps the running maximum of wh
    const int wh = threadIdx.x >> 5;
    const int wx = threadIdx.x & 31;
    float m_run = kNegInf;
    // weighted sum: wave w owns dims [16w, 16w + 16) of all 8 heads; lane l
    // head ph = l/8 at dims da = 16w + 2(l%8) and da + 1, so the 8 lanes of a
    // head read each V pair by broadcast (8-byte loads, two tokens per LDS
    // instruction) and the block reads every V element once; wave 0 also
    // keeps the sums l (lane l: head l/8)
    const int ph = lane >> 3;
    const int da = 16 * wave + 2 * (lane & 7);
    const bool sums = __builtin_amdgcn_readfirstlane(wave) == 0;  // wave-uniform
    float acc0 = 0.0f, acc1 = 0.0f, lsum = 0.0f;

    auto round = [&](int r, int b, uint4& kr, uint4& vr) {
        const int64_t base = t0 + static_cast<int64_t>(kRound) * r;
        const int nv = static_cast<int>(tend - base < kRound ? tend - base : kRound);
        {
            float vf[8];
            unpack8<T>(vr, vf);
            const bool live = gi < nv;
            float4* vrow = reinterpret_cast<float4*>(&s_vf[b][gi][8 * li]);
            vrow[0] = live ? make_float4(vf[0], vf[1], vf[2], vf[3]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            vrow[1] = live ? make_float4(vf[4], vf[5], vf[6], vf[7]) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
        float kf[8];
        unpack8<T>(kr, kf);
        load_row(kbase, vbase, base + 2 * kRound + gi, tend, kr, vr);  // round r + 2
        float d[kHeadsPerGroup];
#pragma unroll
        for (int k = 0; k < kHeadsPerGroup; ++k) {
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                t = fmaf(q[k][j], kf[j], t);
            }
            d[k] = t;
        }
        // reduce-scatter: keep registers 0..3 and take the partner's 4..7
        // (its registers 0..3 are this lane's 4..7 heads), and so on
        const float x0 = d[0] + row_ror<8>(d[4]);
        const float x1 = d[1] + row_ror<8>(d[5]);
        const float x2 = d[2] + row_ror<8>(d[6]);
        const float x3 = d[3] + row_ror<8>(d[7]);
        const float y0 = x0 + lane_xor4(x2);
        const float y1 = x1 + lane_xor4(x3);
        float z = y0 + dpp<kDppXor2>(y1);
        z = z + dpp<kDppXor1>(z);
        if ((li & 1) == 0) {
            s_sc[b][perm][gi] = z * a.qk_scale_log2;  // score of (token gi, head perm)
        }
        __syncthreads();
        if (threadIdx.x < kHeadsPerGroup * kRound) {
            const float sc = s_sc[b][wh][wx];
            const bool valid = wx < nv;
            const float m_new = fmaxf(m_run, span_max<kRound>(valid ? sc : kNegInf));
            s_wt[b][wh][wx] = valid ? exp2_fixed(sc - m_new) : 0.0f;
            if (wx == 0) {
                s_cr[b][wh] = exp2_fixed(m_run - m_new);
            }
            m_run = m_new;
        }
        __syncthreads();
        const float cr = s_cr[b][ph];
        acc0 = acc0 * cr;
        acc1 = acc1 * cr;
        if (sums) {
            lsum = lsum * cr;
        }
        const float* wp = &s_wt[b][ph][0];
        const int nq = (nv + 3) & ~3;  // whole quads: staged zeros past the end add nothing
#pragma unroll 1
        for (int x = 0; x < nq; x += 4) {
            const float4 c = *reinterpret_cast<const float4*>(wp + x);
            const float2 e0 = *reinterpret_cast<const float2*>(&s_vf[b][x + 0][da]);
            const float2 e1 = *reinterpret_cast<const float2*>(&s_vf[b][x + 1][da]);
            const float2 e2 = *reinterpret_cast<const float2*>(&s_vf[b][x + 2][da]);
            const float2 e3 = *reinterpret_cast<const float2*>(&s_vf[b][x + 3][da]);
            acc0 = fmaf(c.x, e0.x, acc0);
            acc1 = fmaf(c.x, e0.y, acc1);
            acc0 = fmaf(c.y, e1.x, acc0);
            acc1 = fmaf(c.y, e1.y, acc1);
            acc0 = fmaf(c.z, e2.x, acc0);
            acc1 = fmaf(c.z, e2.y, acc1);
            acc0 = fmaf(c.w, e3.x, acc0);
            acc1 = fmaf(c.w, e3.y, acc1);
            if (sums) {
                lsum = lsum + c.x;
                lsum = lsum + c.y;
                lsum = lsum + c.z;
                lsum = lsum + c.w;
            }
        }
    };

    // rounds alternate between the two row registers and the two LDS buffers
    int r = 0;
#pragma unroll 1
    for (; r + 1 < rounds; r += 2) {
        round(r, 0, k0, v0);
        round(r + 1, 1, k1, v1);
    }
    if (r < rounds) {
        round(r, 0, k0, v0);
    }
    if (threadIdx.x < kHeadsPerGroup * kRound && wx == 0) {
        s_M[wh] = m_run;
    }
    if (sums && (lane & 7) == 0) {
        s_L[ph] = lsum;
    }
    __syncthreads();

    float* part = a.partials;
    if (nsplit <= a.defer_max) {
        // left for the consumer kernel, which merges them by the same rule;
        // plain stores, visible to the next kernel in the stream
        float* dst = part + ((g * kHeadsPerGroup + ph) * a.max_splits + s) * kPartialStride;
        *reinterpret_cast<float2*>(dst + 2 + da) = make_float2(acc0, acc1);
        if (da == 0) {
            *reinterpret_cast<float2*>(dst) = make_float2(s_M[ph], s_L[ph]);
        }
        return;
    }
    if (nsplit == 1) {
        // single split: the general merge with weight exp2(M - M) = 1
        const float w = exp2_fixed(s_M[ph] - s_M[ph]);
        const float lt = fmaf(s_L[ph], w, 0.0f);
        const float rl = 1.0f / lt;
        const uint32_t lo = T::store(fmaf(acc0, w, 0.0f) * rl);
        const uint32_t hi = T::store(fmaf(acc1, w, 0.0f) * rl);
        *reinterpret_cast<uint32_t*>(a.out + (g * kHeadsPerGroup + ph) * kDim + da) = lo | (hi << 16);
        return;
    }

    {
        // 8-byte pairs (the row's floats 2 + da, 3 + da and 0, 1 are 8-byte aligned)
        float* dst = part + ((g * kHeadsPerGroup + ph) * a.max_splits + s) * kPartialStride;
        store_agent_pair(dst + 2 + da, acc0, acc1);
        if (da == 0) {
            store_agent_pair(dst, s_M[ph], s_L[ph]);
        }
    }
    if (nsplit > a.ticket_max) {
        return;  // gqa_merge_kernel follows
    }

    // ---- ticket: the last block of this KV head merges all splits (the
    // partials travel through agent-scope atomic stores/loads and the
    // acquire-release ticket)
    wait_own_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = take_ticket(a.counters + g);
        s_last = prev == static_cast<uint32_t>(nsplit - 1) ? 1 : 0;
    }
    __syncthreads();
    if (s_last == 0) {
        return;
    }
    if (threadIdx.x == 0) {
        store_agent(a.counters + g, 0u);
    }
    // Up to 16 splits use 16-wide register arrays, more the 32-wide ones (the
    // same operations in the same order).
    // weights and sums in the (now idle) V stage
    static_assert(2 * kHeadsPerGroup * kInKernelSplits <= 2 * kRound * kDim, "merge weights fit the stage");
    float* stage = &s_vf[0][0][0];
    if (nsplit <= kInKernelSplits / 2) {
        constexpr int N = kInKernelSplits / 2;
        ticket_merge<T, N>(a, part, g, static_cast<int>(nsplit), reinterpret_cast<float (*)[N]>(stage),
                           reinterpret_cast<float (*)[N]>(stage + kHeadsPerGroup * N));
    } else {
        constexpr int N = kInKernelSplits;
        ticket_merge<T, N>(a, part, g, static_cast<int>(nsplit), reinterpret_cast<float (*)[N]>(stage),
                           reinterpret_cast<float (*)[N]>(stage + kHeadsPerGroup * N));
    }
}

// Two launch wrappers of the one body.  The bf16 kernel (the decode step and
// the bf16 entry points) carries no occupancy target: it still fits 128
// VGPRs (4 waves per SIMD), and the freer schedule took the step's attention
// from 4.14 to 4.04 us and every standalone length 1..8191 down by ~0.1 us,
// bit-identically.  The fp16 kernel keeps the 4-waves target, without which
// it needs 130 VGPRs (3 waves per SIMD, one 8-wave block per CU).
__global__ __launch_bounds__(kGqaThreads) __attribute__((amdgpu_waves_per_eu(2)))
void gqa_partial_kernel_bf16(const uint16_t* k_rows, const uint16_t* v_rows, const uint16_t* q_vec,
                             const int32_t* kv_len_device, int64_t capacity, GqaArgs args) {
    gqa_partial_body<Bf16>(k_rows, v_rows, q_vec, kv_len_device, capacity, args);
}
__global__ __launch_bounds__(kGqaThreads) __attribute__((amdgpu_waves_per_eu(4)))
void gqa_partial_kernel_f16(const uint16_t* k_rows, const uint16_t* v_rows, const uint16_t* q_vec,
                            const int32_t* kv_len_device, int64_t capacity, GqaArgs args) {
    gqa_partial_body<F16>(k_rows, v_rows, q_vec, kv_len_device, capacity, args);
}

// grid (16 query heads, 8 slices of 16 dims), 256 threads.  Thread t loads
// dim t%16 of the slice for splits t/16, t/16 + 16, ... (16 lanes read one
// 64-byte run of a split row), all in flight before the first LDS store, and
// thread t < nsplit the split's max and sum; the maximum over splits is an
// order-free reduction.  Then thread (dim t%16, group t/16) sums its group of
// kGqaMergeGroup splits in order, and threads 0..15 add the group sums in
// order.
template <typename T>
__global__ __launch_bounds__(256) void gqa_merge_kernel(GqaArgs a) {
    constexpr int kSlice = kMergeDims;
    constexpr int kRowsPerPass = 256 / kSlice;
    constexpr int kPasses = kMergeMaxSplits / kRowsPerPass;
    static_assert(kMergeGroups == kRowsPerPass, "one merge group per thread row");
    __shared__ float s_v[kMergeMaxSplits][kSlice];
    __shared__ float s_w[kMergeMaxSplits];  // weights
    __shared__ float s_l[kMergeMaxSplits];
    __shared__ float s_go[kMergeGroups][kSlice];
    __shared__ float s_gl[kMergeGroups];
    __shared__ float s_red[4];
    const int h = blockIdx.x;
    const int d0 = blockIdx.y * kSlice;
    const int64_t L = read_kv_len(a);
    const int nsplit = static_cast<int>(a.mfma ? gqa_mfma_split_count(L, a.split_cap, a.mfma_quantum)
                                                : gqa_split_count(L, a.split_cap));
    if (a.mfma) {
        // the matrix-core partial kernel merges nothing itself
        if (nsplit == 0) {
            if (threadIdx.x < kSlice) {
                a.out[static_cast<int64_t>(h) * kDim + d0 + threadIdx.x] = 0;  // empty cache
            }
            return;
        }
    } else if (nsplit <= a.ticket_max) {
        return;  // merged by the partial kernel
    }
    const float* src = a.partials + static_cast<int64_t>(h) * a.max_splits * kPartialStride;
    const int d = threadIdx.x % kSlice;
    const int row = threadIdx.x / kSlice;
    // the split's max and sum first, so they travel with the slices
    float mine = kNegInf;
    float lsplit = 0.0f;
    if (static_cast<int>(threadIdx.x) < nsplit) {
        const float2 ml = *reinterpret_cast<const float2*>(src + static_cast<int64_t>(threadIdx.x) * kPartialStride);
        mine = ml.x;
        lsplit = ml.y;
    }
    {
        float v[kPasses];
#pragma unroll
        for (int i = 0; i < kPasses; ++i) {
            const int x = row + kRowsPerPass * i;
            v[i] = x < nsplit ? src[static_cast<int64_t>(x) * kPartialStride + 2 + d0 + d] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kPasses; ++i) {
            const int x = row + kRowsPerPass * i;
            if (x < nsplit) {
                s_v[x][d] = v[i];
            }
        }
    }
    if (static_cast<int>(threadIdx.x) < nsplit) {
        s_l[threadIdx.x] = lsplit;
    }
    const float mloc = span_max<64>(mine);
    if ((threadIdx.x & 63) == 0) {
        s_red[threadIdx.x >> 6] = mloc;
    }
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    if (static_cast<int>(threadIdx.x) < nsplit) {
        s_w[threadIdx.x] = exp2_fixed(mine - M);
    }
    __syncthreads();
    // LDS entries past nsplit (and past ngroups) are read but not used:
    // the loads stay unconditional and in flight together
    const int ngroups = (nsplit + kGqaMergeGroup - 1) / kGqaMergeGroup;
    if (row < ngroups) {
        const int x0 = row * kGqaMergeGroup;
        float vx[kGqaMergeGroup], wx[kGqaMergeGroup], lx[kGqaMergeGroup];
#pragma unroll
        for (int i = 0; i < kGqaMergeGroup; ++i) {
            vx[i] = s_v[x0 + i][d];
            wx[i] = s_w[x0 + i];
            lx[i] = s_l[x0 + i];
        }
        float og = 0.0f;
        float lg = 0.0f;
#pragma unroll
        for (int i = 0; i < kGqaMergeGroup; ++i) {
            const bool live = x0 + i < nsplit;
            og = live ? fmaf(vx[i], wx[i], og) : og;
            lg = live ? fmaf(lx[i], wx[i], lg) : lg;
        }
        s_go[row][d] = og;
        if (d == 0) {
            s_gl[row] = lg;
        }
    }
    __syncthreads();
    if (threadIdx.x < kSlice) {
        float go[kMergeGroups], gl[kMergeGroups];
#pragma unroll
        for (int j = 0; j < kMergeGroups; ++j) {
            go[j] = s_go[j][d];
            gl[j] = s_gl[j];
        }
        float o = go[0];
        float lt = gl[0];
#pragma unroll
        for (int j = 1; j < kMergeGroups; ++j) {
            o = j < ngroups ? o + go[j] : o;
            lt = j < ngroups ? lt + gl[j] : lt;
        }
        a.out[static_cast<int64_t>(h) * kDim + d0 + d] = T::store(o * (1.0f / lt));
    }
}

// ------------------------------------------------------ matrix-core tactic
// Grid (max_splits, 2), kWaves (2 or 4) waves.  Block (s, g) owns split s of
// KV head g (gqa_mfma_split_tokens tokens, a multiple of 32 kWaves); wave w
// takes the split's 32-token chunks w, w + kWaves, ... and keeps its own
// online softmax over them; the wave results are merged in LDS into the split partial (max, sum, acc[128] per
// head: the round path's layout), which gqa_merge_kernel combines.
//
// Operand layouts of v_mfma_f32_16x16x32 (lane l, r = l % 16, c = l / 16):
// A[r][8c + j], B[8c + j][r], D[4c + i][r].  Per chunk:
//   * scores S^T = K q^T over two 16-token tiles and 4 k-steps: A = K rows
//     (lane l: token r of the tile, dims 32k + 8c .. +7, so one load
//     instruction reads 64 contiguous bytes of each of 16 rows), B = q (lane
//     l: query head r of the group, zero for r >= 8).  D leaves lane l the
//     scores of head r for tokens 4c + i (tile 0) and 16 + 4c + i (tile 1);
//   * online softmax: the chunk maximum over the lane's 8 scores and the 4
//     lanes of head r (lane swaps at distance 32 and 16), weights
//     w = exp2(s - m'), rescale exp2(m - m'); each lane keeps its own running
//     sum of w (rescaled alike), the 4 lanes of a head are added at the end;
//   * P.V as D = P V: A = P with k slot 8c + j holding the lane's own tokens
//     (j < 4 tile 0, j >= 4 tile 1), so the scores' output layout is the
//     weights' input layout and nothing moves between lanes.  P enters as two
//     MFMAs, its 16-bit rounding hi and the rounding of the remainder w - hi,
//     which carries ~16 significant bits of each fp32 weight.  B = V^T in
//     the same slot order, staged in the wave's own LDS region (row = dim,
//     80-byte rows: the 16 lanes of one B read fall on distinct banks);
//     acc (lane l: heads 4c + i at dim 16t + r of dim tile t) is rescaled per
//     head first, with factors read from lanes 0..7.
// K/V rows are read once per call and streamed (non-temporal loads).
// Rows past the split's end are loaded clamped to its last row, their scores
// are -inf and their V is zeroed, so every load stays in bounds and nothing
// past the cache end reaches a sum.  The waves of a block exchange data only
// through LDS; a wave's own V^T stores and reads are ordered by the LDS
// executing one wave's instructions in issue order.
typedef __bf16 mfma_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 mfma_f16x8 __attribute__((ext_vector_type(8)));
typedef float mfma_f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct MfmaOps;
template <>
struct MfmaOps<Bf16> {
    typedef mfma_bf16x8 vec;
    static __device__ __forceinline__ mfma_f32x4 mac(vec a, vec b, mfma_f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ void split(const float* w, vec& hi, vec& lo) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const __bf16 h = static_cast<__bf16>(w[j]);
            hi[j] = h;
            lo[j] = static_cast<__bf16>(w[j] - static_cast<float>(h));
        }
    }
};
template <>
struct MfmaOps<F16> {
    typedef mfma_f16x8 vec;
    static __device__ __forceinline__ mfma_f32x4 mac(vec a, vec b, mfma_f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ void split(const float* w, vec& hi, vec& lo) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const _Float16 h = static_cast<_Float16>(w[j]);
            hi[j] = h;
            lo[j] = static_cast<_Float16>(w[j] - static_cast<float>(h));
        }
    }
};

constexpr int kChunk = 32;  // tokens per wave step; a split unit is one chunk per wave
static_assert(kGqaMfmaSplitCap <= kMergeMaxSplits, "the merge kernel takes every split");
constexpr int kVtPitch = 40;  // 16-bit slots per staged V^T row (80 bytes)

struct MfmaChunk {
    uint4 k[2][4];  // K: tile, k-step
    uint4 v[4][2];  // V: token 4va + i, dims 16vb + 8h .. +7
};

__device__ __forceinline__ float lane_swap_max(float v) {
    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
}
__device__ __forceinline__ float lane_swap_sum(float v) {
    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
}

// kPer: chunks per wave of a split (gqa_mfma_split_tokens / quantum) when the
// host knows it (1 or 2: every load is issued up front in straight-line code,
// so each chunk waits only for its own rows); 0: any count, chunks requested
// one pair ahead in a loop.
template <typename T, int kPer, int kWaves>
__global__ __launch_bounds__(64 * kWaves) void gqa_mfma_partial_kernel(GqaArgs a) {
    using Ops = MfmaOps<T>;
    typedef typename Ops::vec vec;
    constexpr int kThreads = 64 * kWaves;
    static_assert(kWaves == 2 || kWaves == 4, "merge layout: 128 or 256 threads");
    __shared__ __attribute__((aligned(16))) uint16_t s_vt[kWaves][kDim * kVtPitch];
    __shared__ float s_m[kWaves][kHeadsPerGroup];
    __shared__ float s_l[kWaves][kHeadsPerGroup];
    static_assert(kWaves * kDim * kHeadsPerGroup * sizeof(float) <= sizeof(s_vt), "wave results fit the V stage");

    const int g = blockIdx.y;
    const int s = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = lane & 15;
    const int c = lane >> 4;

    // q first (every lane loads a row of the group; lanes r >= 8 then clear
    // theirs with a mask, so the loads stay unconditional and in order)
    vec bq[4];
    {
        const uint16_t* qrow = a.q + (g * kHeadsPerGroup + (r & 7)) * kDim + 8 * c;
        const uint32_t keep = r < kHeadsPerGroup ? 0xffffffffu : 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint4 v = *reinterpret_cast<const uint4*>(qrow + 32 * k);
            v.x &= keep;
            v.y &= keep;
            v.z &= keep;
            v.w &= keep;
            bq[k] = __builtin_bit_cast(vec, v);
        }
    }

    const int L = static_cast<int>(read_kv_len(a));
    const int C = static_cast<int>(gqa_mfma_split_tokens(L, a.split_cap, kChunk * kWaves));
    const int nsplit = static_cast<int>(gqa_mfma_split_count(L, a.split_cap, kChunk * kWaves));
    if (s >= nsplit) {
        return;
    }
    const int t0 = s * C;
    const int tend = t0 + C < L ? t0 + C : L;
    const int last = tend - 1;
    const int nchunk = (tend - t0 + kChunk - 1) / kChunk;
    const int64_t head_off = static_cast<int64_t>(g) * a.capacity * kDim;
    const uint16_t* kbase = a.k + head_off + 8 * c;
    const int va = lane >> 3;  // token quad of the lane's V loads
    const int vb = lane & 7;   // 16-dim block of the lane's V loads
    const uint16_t* vbase = a.v + head_off + 16 * vb;

    auto load_chunk = [&](int ci, MfmaChunk& ch) {
        const int tb = t0 + kChunk * ci;
#pragma unroll
        for (int x = 0; x < 2; ++x) {
            const int row = tb + 16 * x + r < last ? tb + 16 * x + r : last;
            const uint16_t* p = kbase + row * kDim;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                ch.k[x][k] = load_stream(reinterpret_cast<const uint4*>(p + 32 * k));
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int row = tb + 4 * va + i < last ? tb + 4 * va + i : last;
            const uint16_t* p = vbase + row * kDim;
            ch.v[i][0] = load_stream(reinterpret_cast<const uint4*>(p));
            ch.v[i][1] = load_stream(reinterpret_cast<const uint4*>(p + 8));
        }
    };

    MfmaChunk ca, cb;
    load_chunk(wave, ca);
    if constexpr (kPer != 1) {
        load_chunk(wave + kWaves, cb);
    }

    uint16_t* vt = s_vt[wave];
    const int sb = va < 4 ? 8 * va : 8 * (va - 4) + 4;  // k slot of the lane's first V token
    float m_run = kNegInf;
    float lsum = 0.0f;
    mfma_f32x4 acc[kDim / 16];
#pragma unroll
    for (int t = 0; t < kDim / 16; ++t) {
        acc[t] = mfma_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }

    auto process = [&](int ci, const MfmaChunk& ch) {
        const int tb = t0 + kChunk * ci;
        const int nv = tend - tb < kChunk ? tend - tb : kChunk;
        // V^T stage: for each dim, the lane's 4 tokens as 4 consecutive slots
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t wv[4][4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool live = 4 * va + i < nv;
                wv[i][0] = live ? ch.v[i][h].x : 0u;
                wv[i][1] = live ? ch.v[i][h].y : 0u;
                wv[i][2] = live ? ch.v[i][h].z : 0u;
                wv[i][3] = live ? ch.v[i][h].w : 0u;
            }
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int d = 16 * vb + 8 * h + 2 * m;
                const uint2 even = make_uint2((wv[0][m] & 0xffffu) | (wv[1][m] << 16), (wv[2][m] & 0xffffu) | (wv[3][m] << 16));
                const uint2 odd = make_uint2((wv[0][m] >> 16) | (wv[1][m] & 0xffff0000u),
                                             (wv[2][m] >> 16) | (wv[3][m] & 0xffff0000u));
                *reinterpret_cast<uint2*>(vt + d * kVtPitch + sb) = even;
                *reinterpret_cast<uint2*>(vt + (d + 1) * kVtPitch + sb) = odd;
            }
        }
        mfma_f32x4 d0 = {0.0f, 0.0f, 0.0f, 0.0f};
        mfma_f32x4 d1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            d0 = Ops::mac(__builtin_bit_cast(vec, ch.k[0][k]), bq[k], d0);
            d1 = Ops::mac(__builtin_bit_cast(vec, ch.k[1][k]), bq[k], d1);
        }
        float sc[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            sc[i] = 4 * c + i < nv ? d0[i] * a.qk_scale_log2 : kNegInf;
            sc[4 + i] = 16 + 4 * c + i < nv ? d1[i] * a.qk_scale_log2 : kNegInf;
        }
        float cm = fmaxf(fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3])), fmaxf(fmaxf(sc[4], sc[5]), fmaxf(sc[6], sc[7])));
        cm = lane_swap_max(cm);
        const float m_new = fmaxf(m_run, cm);
        // a chunk past the split's end (nv <= 0) with nothing before it leaves
        // m at -inf: exponents are taken against 0 then, so all weights and the
        // rescale are exactly 0 instead of NaN
        const float m_ref = m_new == kNegInf ? 0.0f : m_new;
        const float cr = __builtin_amdgcn_exp2f(m_run - m_ref);
        float w[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            w[j] = __builtin_amdgcn_exp2f(sc[j] - m_ref);
        }
        lsum = fmaf(lsum, cr, ((w[0] + w[1]) + (w[2] + w[3])) + ((w[4] + w[5]) + (w[6] + w[7])));
        m_run = m_new;
        vec phi, plo;
        Ops::split(w, phi, plo);
        float crh[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cr), i));
            const float hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(cr), 4 + i));
            crh[i] = c == 0 ? lo : hi;
        }
        __asm__ volatile("" ::: "memory");  // the V^T stores above precede the B reads
#pragma unroll
        for (int t = 0; t < kDim / 16; ++t) {
            const uint4 bv = *reinterpret_cast<const uint4*>(vt + (16 * t + r) * kVtPitch + 8 * c);
            mfma_f32x4 x = acc[t];
            x[0] *= crh[0];
            x[1] *= crh[1];
            x[2] *= crh[2];
            x[3] *= crh[3];
            x = Ops::mac(phi, __builtin_bit_cast(vec, bv), x);
            x = Ops::mac(plo, __builtin_bit_cast(vec, bv), x);
            acc[t] = x;
        }
        __asm__ volatile("" ::: "memory");  // and the next chunk's stores follow them
    };

    // a wave's chunks: wave, wave + 4, ... (< nchunk).  With kPer fixed every
    // chunk is processed unconditionally (one past the end adds nothing), so
    // the compiler keeps its loads ahead of the first wait instead of sinking
    // them into a branch.
    if constexpr (kPer == 1) {
        process(wave, ca);
    } else if constexpr (kPer == 2) {
        process(wave, ca);
        process(wave + kWaves, cb);
    } else {
        // the two register sets alternate; the chunk after next is requested
        // as soon as a set is free (clamped rows, so unconditionally)
#pragma unroll 1
        for (int ci = wave; ci < nchunk; ci += 2 * kWaves) {
            process(ci, ca);
            load_chunk(ci + 2 * kWaves, ca);
            if (ci + kWaves >= nchunk) {
                break;
            }
            process(ci + kWaves, cb);
            load_chunk(ci + 3 * kWaves, cb);
        }
    }
    lsum = lane_swap_sum(lsum);

    __syncthreads();  // every wave is done with its V^T stage
    float* s_acc = reinterpret_cast<float*>(&s_vt[0][0]);  // [wave][dim][head]
    if (c < 2) {
#pragma unroll
        for (int t = 0; t < kDim / 16; ++t) {
            *reinterpret_cast<float4*>(s_acc + ((wave * kDim + 16 * t + r) * kHeadsPerGroup + 4 * c)) =
                make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
        }
    }
    if (lane < kHeadsPerGroup) {
        s_m[wave][lane] = m_run;
        s_l[wave][lane] = lsum;
    }
    __syncthreads();
    // thread: dim d of heads 4hq .. 4hq + 3 (both quads with 128 threads);
    // the waves in order
    const int d = threadIdx.x & (kDim - 1);
#pragma unroll
    for (int hi = 0; hi < 8; hi += kThreads / kDim * 4) {
    const int hq = (threadIdx.x >> 7) + hi / 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int h = 4 * hq + i;
        float M = s_m[0][h];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) {
            M = fmaxf(M, s_m[w][h]);
        }
        float o = 0.0f;
        float lt = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float ww = __builtin_amdgcn_exp2f(s_m[w][h] - M);
            o = fmaf(s_acc[(w * kDim + d) * kHeadsPerGroup + h], ww, o);
            lt = fmaf(s_l[w][h], ww, lt);
        }
        float* dst = a.partials + (static_cast<int64_t>(g * kHeadsPerGroup + h) * a.max_splits + s) * kPartialStride;
        dst[2 + d] = o;
        if (d == 0) {
            *reinterpret_cast<float2*>(dst) = make_float2(M, lt);
        }
    }
    }
}

}  // namespace

GqaPlan gqa_plan(int64_t capacity, int64_t split_limit) {
    GqaPlan p;
    // a caller-sized workspace caps the split count; the uncapped plan keeps up
    // to kGqaSplitCap splits per KV head (512 blocks: two per CU)
    p.split_cap = split_limit > 0 && split_limit < kGqaSplitCap ? split_limit : kGqaSplitCap;
    const int64_t rounds = (capacity + kRound - 1) / kRound;
    p.max_splits = rounds < p.split_cap ? rounds : p.split_cap;
    return p;
}

hipError_t launch_gqa_decode(Act act, const GqaArgs& a, hipStream_t stream) {
    // the grid must cover every split any length up to the capacity produces
    const int64_t rounds = (a.capacity + kRound - 1) / kRound;
    const int64_t need = a.split_cap > 0 && rounds > a.split_cap ? a.split_cap : rounds;
    if (a.capacity <= 0 || a.split_cap <= 0 || a.max_splits < need || a.max_splits > kMergeMaxSplits ||
        a.defer_max < 0 || a.defer_max > kGqaMaxDefer || a.defer_max > a.max_splits || a.ticket_max < 1 ||
        a.ticket_max > kInKernelSplits) {
        return hipErrorInvalidValue;
    }
    const dim3 grid(static_cast<unsigned>(a.max_splits), 2);
    if (act == Act::kBf16) {
        hipLaunchKernelGGL(gqa_partial_kernel_bf16, grid, dim3(kGqaThreads), 0, stream, a.k, a.v, a.q,
                           a.kv_len_device, a.capacity, a);
    } else {
        hipLaunchKernelGGL(gqa_partial_kernel_f16, grid, dim3(kGqaThreads), 0, stream, a.k, a.v, a.q,
                           a.kv_len_device, a.capacity, a);
    }
    hipError_t status = hipGetLastError();
    if (status != hipSuccess || a.max_splits <= a.ticket_max) {
        return status;
    }
    const dim3 mgrid(16, kDim / kMergeDims);
    if (act == Act::kBf16) {
        hipLaunchKernelGGL(gqa_merge_kernel<Bf16>, mgrid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(gqa_merge_kernel<F16>, mgrid, dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

hipError_t launch_gqa_decode_mfma(Act act, GqaArgs a, hipStream_t stream) {
    a.mfma = true;
    // the grid must cover every split of the length a host-length call names,
    // or of any length up to the capacity when the length is in device memory
    if (a.mfma_quantum != 64 && a.mfma_quantum != 128) {
        return hipErrorInvalidValue;
    }
    const int64_t units = (a.capacity + a.mfma_quantum - 1) / a.mfma_quantum;
    const int64_t host_len = a.kv_len_host < 0 ? 0 : (a.kv_len_host > a.capacity ? a.capacity : a.kv_len_host);
    const int64_t need = a.kv_len_device == nullptr ? gqa_mfma_split_count(host_len, a.split_cap, a.mfma_quantum)
                                                     : (units < a.split_cap ? units : a.split_cap);
    if (a.capacity <= 0 || a.capacity > (int64_t{1} << 24) || a.split_cap <= 0 || a.split_cap > kGqaMfmaSplitCap ||
        a.max_splits < need || a.max_splits > kMergeMaxSplits) {
        return hipErrorInvalidValue;
    }
    const dim3 grid(static_cast<unsigned>(a.max_splits), 2);
    // chunks per wave: fixed by the host length, else any
    const int64_t per = a.kv_len_device == nullptr
                            ? gqa_mfma_split_tokens(host_len, a.split_cap, a.mfma_quantum) / a.mfma_quantum
                            : 0;
    const bool two = a.mfma_quantum == 64;
    const dim3 block(two ? 128 : 256);
    if (act == Act::kBf16) {
        auto* kernel = two ? (per == 1 ? gqa_mfma_partial_kernel<Bf16, 1, 2>
                                       : (per == 2 ? gqa_mfma_partial_kernel<Bf16, 2, 2> : gqa_mfma_partial_kernel<Bf16, 0, 2>))
                           : (per == 1 ? gqa_mfma_partial_kernel<Bf16, 1, 4>
                                       : (per == 2 ? gqa_mfma_partial_kernel<Bf16, 2, 4> : gqa_mfma_partial_kernel<Bf16, 0, 4>));
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, a);
    } else {
        auto* kernel = two ? (per == 1 ? gqa_mfma_partial_kernel<F16, 1, 2>
                                       : (per == 2 ? gqa_mfma_partial_kernel<F16, 2, 2> : gqa_mfma_partial_kernel<F16, 0, 2>))
                           : (per == 1 ? gqa_mfma_partial_kernel<F16, 1, 4>
                                       : (per == 2 ? gqa_mfma_partial_kernel<F16, 2, 4> : gqa_mfma_partial_kernel<F16, 0, 4>));
        hipLaunchKernelGGL(kernel, grid, block, 0, stream, a);
    }
    hipError_t status = hipGetLastError();
    if (status != hipSuccess) {
        return status;
    }
    const dim3 mgrid(16, kDim / kMergeDims);
    if (act == Act::kBf16) {
        hipLaunchKernelGGL(gqa_merge_kernel<Bf16>, mgrid, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(gqa_merge_kernel<F16>, mgrid, dim3(256), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace kc
