// Split-KV grouped-query decode attention for the Qwen2.5-3B shape
// (16 query heads, 2 KV heads, group 8, head_dim 128).
//
// Partial kernel, grid (max_splits, 2): block (s, g) owns one split of the
// tokens of KV head g and serves all 8 query heads of the group, so every K/V
// byte is read once.  A block is 8 waves = 32 groups of 16 lanes; lane li of a
// group holds dims [8li, 8li+8) of all 8 query heads.  Two paths, chosen per
// launch from kv_len L (uniform over the grid):
//
// Flat path (L <= flat_max, at most 32 splits): split s owns tokens
// [32s, min(32s+32, L)), one per group.  Each group forms its token's 8 head
// scores (8-dim partial dots and the 16-lane butterfly below), the block takes
// the per-head max M over the split, weights w_t = exp2(s_t - M), sum
// l = w_0 + w_1 + ..., and acc[d] = sum_t w_t v_t[d] in token order, with the
// V rows staged in LDS.  Short caches thus spread over up to 64 CUs instead of
// running a long per-group chain on 2.  Up to 2 * flat_max the same path runs
// with two tokens per group (64-token splits, the same split count).
//
// Round path (longer L): split s owns tokens [s*C, min(s*C+C, L)), C = 128
// up to mid_max and `chunk` (256) beyond, both chosen from L on the device.  Per
// 128-token round, group gi takes tokens base + 4gi + {0..3}: 8 dot products
// of 8 dims per lane and a 16-lane butterfly (DPP) give every lane of the group
// all 32 (token, head) scores (log2 domain: pre-multiplied by scale*log2e).
// The running max is updated redundantly (cheap), but each exponential is
// computed once: lane li evaluates exp2_fixed for (token, head) slots li and
// li+16 and the rescale factor of head li, exchanged through a per-group LDS
// slot (all lanes of a group are in one wave, so no barrier is needed).  The
// next round's K/V rows are loaded before the current round is reduced, and
// split 0 issues its first rows before kv_len arrives.
// The 32 group states are merged through LDS (weights exp2(m_g - M) computed
// once per group and head) into one (max, sum, acc[128]) split partial per
// head.
//
// Either path ends with one (max, sum, acc[128]) partial per split and head.
// Then, by the number of splits at this L:
//   * up to defer_max splits (the decode step sets it): the partials are left
//     for the consumer, the o_proj row kernel, which merges them while its
//     weight rows stream in -- no ticket, no cross-block wait here;
//   * one split finishes in place: out = acc*1 / (sum*1), the general
//     merge formula with weight exp2(0) = 1 (no ticket, no fences);
//   * up to ticket_max (<= kInKernelSplits) splits: the partial is written
//     and the last block of the KV head to finish (a ticket of agent-scope
//     atomics, reset by that block, so the launch is capture-safe) merges the
//     splits;
//   * more splits: the partials are merged by gqa_merge_kernel (grid: query
//     head x 16-dim slice; partials staged through LDS in one pass), which is
//     launched after the partial kernel whenever the grid allows more than
//     ticket_max splits and returns at once when L needs fewer.
// Every merge sums the splits in index order with the same operations, so the
// result depends only on (inputs, kv_len, the split rule).  kv_len may come
// from device memory (graph replay); the rule's bounds come from the cache length
// (gqa_plan), so a direct call and a graph replay at the same L agree.
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
constexpr int kRoundTokens = 4 * kGroups;   // tokens per round
constexpr int kHeadsPerGroup = 8;
constexpr int kDim = 128;
constexpr int kPartialStride = kGqaPartialStride;
static_assert(kPartialStride == 2 + kDim, "partial layout: max, sum, acc[128]");
constexpr int kInKernelSplits = 32;
constexpr int kFlatTokens = kGqaFlatTokens;  // flat path: one token per group, one round per split
static_assert(kFlatTokens == kGroups, "flat path: one token per 16-lane group");
constexpr int kFlatSplits = 32;
constexpr int kMergeMaxSplits = 1024;
constexpr int kMergeDims = 16;              // dims per merge block
constexpr int kSlot = 40;                   // per-group LDS exchange: 32 scores + 8 rescales
constexpr float kNegInf = -__builtin_huge_valf();

__device__ __forceinline__ int64_t read_kv_len(const GqaArgs& a) {
    int64_t L = a.kv_len_device != nullptr ? static_cast<int64_t>(*a.kv_len_device) + a.kv_len_offset : a.kv_len_host;
    return L < 0 ? 0 : (L > a.capacity ? a.capacity : L);
}

__device__ __forceinline__ int64_t split_count(const GqaArgs& a, int64_t L) {
    return gqa_split_count(L, a.flat_max, a.mid_max, a.chunk);
}

// K and V rows of tokens tk .. tk+3 for one lane (dims 8li..8li+7); indices
// past `last` re-read row `last` (read, never used), so the loads are
// unconditional and the wave's memory counter stays exact.
__device__ __forceinline__ void load_rows(const uint16_t* kbase, const uint16_t* vbase, int64_t tk, int64_t last,
                                          uint4* kr, uint4* vr) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t t = tk + k < last ? tk + k : last;
        kr[k] = *reinterpret_cast<const uint4*>(kbase + t * kDim);
        vr[k] = *reinterpret_cast<const uint4*>(vbase + t * kDim);
    }
}

__device__ __forceinline__ int clamp4(int64_t n) { return static_cast<int>(n < 0 ? 0 : (n > 4 ? 4 : n)); }

// In-kernel merge of the first nsplit (<= N) split partials of KV head g
// (the last block of the head runs it): every thread owns two (head, dim)
// outputs, loads every split's max, sum and accumulator element for them
// (agent-scope loads: the partials come from other blocks of this launch),
// and sums in split order with weights exp2(m_s - M).
template <typename T, int N>
__device__ __forceinline__ void ticket_merge(const GqaArgs& a, const float* part, int g, int nsplit) {
#pragma unroll 1
    for (int k = 0; k < 2; ++k) {
        const int idx = threadIdx.x + k * kGqaThreads;
        const int hl = idx / kDim;
        const int d = idx % kDim;
        const float* src = part + (g * kHeadsPerGroup + hl) * a.max_splits * kPartialStride;
        float mv[N], lv[N], vv[N];
#pragma unroll
        for (int x = 0; x < N; ++x) {
            const bool live = x < nsplit;
            mv[x] = live ? load_agent(src + x * kPartialStride) : kNegInf;
            lv[x] = live ? load_agent(src + x * kPartialStride + 1) : 0.0f;
            vv[x] = live ? load_agent(src + x * kPartialStride + 2 + d) : 0.0f;
        }
        float M = kNegInf;
#pragma unroll
        for (int x = 0; x < N; ++x) {
            M = fmaxf(M, mv[x]);
        }
        float lt = 0.0f;
        float o = 0.0f;
#pragma unroll
        for (int x = 0; x < N; ++x) {
            if (x < nsplit) {
                const float w = exp2_fixed(mv[x] - M);
                lt = fmaf(lv[x], w, lt);
                o = fmaf(vv[x], w, o);
            }
        }
        a.out[(g * kHeadsPerGroup + hl) * kDim + d] = T::store(o / lt);
    }
}

template <typename T>
__global__ __launch_bounds__(kGqaThreads) void gqa_partial_kernel(GqaArgs a) {
    __shared__ __attribute__((aligned(16))) float s_x[kGroups][kSlot];
    // group states, head-major so a thread reads one head's 32 groups as
    // 8 contiguous 16-byte loads
    __shared__ __attribute__((aligned(16))) float s_m[kHeadsPerGroup][kGroups];
    __shared__ __attribute__((aligned(16))) float s_l[kHeadsPerGroup][kGroups];
    __shared__ __attribute__((aligned(16))) float s_w[kHeadsPerGroup][kGroups];
    __shared__ float s_M[kHeadsPerGroup];
    __shared__ float s_L[kHeadsPerGroup];
    __shared__ float s_acc[kGroups][kHeadsPerGroup / 2][kDim];  // half the heads at a time
    __shared__ int s_last;

    const int g = blockIdx.y;
    const int64_t s = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int gi = wave * 4 + (lane >> 4);
    const int li = lane & 15;
    const uint16_t* kbase = a.k + static_cast<int64_t>(g) * a.capacity * kDim + 8 * li;
    const uint16_t* vbase = a.v + static_cast<int64_t>(g) * a.capacity * kDim + 8 * li;

    // q does not depend on kv_len: request it first.  Split 0 always exists
    // once kv_len >= 1, so its first rows (bounded by the capacity) are also
    // requested before kv_len is known.
    uint4 qr[kHeadsPerGroup];
#pragma unroll
    for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
        qr[hl] = *reinterpret_cast<const uint4*>(a.q + (g * kHeadsPerGroup + hl) * kDim + 8 * li);
    }
    // flat-path row of this group (token s*32 + gi, bounded by the capacity)
    uint4 kF = make_uint4(0, 0, 0, 0), vF = make_uint4(0, 0, 0, 0);
    if (s * kFlatTokens < a.flat_max) {
        const int64_t t = s * kFlatTokens + gi;
        const int64_t tc = t < a.capacity ? t : a.capacity - 1;
        kF = *reinterpret_cast<const uint4*>(kbase + tc * kDim);
        vF = *reinterpret_cast<const uint4*>(vbase + tc * kDim);
    }
    uint4 kA[4], vA[4], kB[4], vB[4];
    if (s == 0) {
        load_rows(kbase, vbase, 4 * gi, a.capacity - 1, kA, vA);
    }

    const int64_t L = read_kv_len(a);
    const int64_t nsplit = split_count(a, L);
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
    const int64_t C = gqa_split_tokens(L, a.flat_max, a.mid_max, a.chunk);
    const int64_t t0 = s * C;

    float q[kHeadsPerGroup][8];
#pragma unroll
    for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
        unpack8<T>(qr[hl], q[hl]);
    }
    float av_out[2];

    if (L <= a.flat_max) {
        // ---- flat path: group gi scores token s*32 + gi for the 8 heads
        // (same dot and butterfly as a round), then one block-wide softmax
        // per head over the split's tokens and the weighted V sum from LDS.
        float (*s_vf)[kDim] = reinterpret_cast<float (*)[kDim]>(&s_acc[0][0][0]);
        const int64_t f0 = s * kFlatTokens;
        const int nvalid = static_cast<int>(f0 + kFlatTokens < L ? kFlatTokens : L - f0);
        float kf[8], vf[8];
        unpack8<T>(kF, kf);
        unpack8<T>(vF, vf);
        float dots[kHeadsPerGroup];
#pragma unroll
        for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
            float t = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                t = fmaf(q[hl][j], kf[j], t);
            }
            dots[hl] = t;
        }
#pragma unroll
        for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
            dots[hl] += row_ror<8>(dots[hl]);
        }
#pragma unroll
        for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
            dots[hl] += row_ror<4>(dots[hl]);
        }
#pragma unroll
        for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
            dots[hl] += row_ror<2>(dots[hl]);
        }
#pragma unroll
        for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
            dots[hl] += row_ror<1>(dots[hl]);
        }
        float mine = dots[0];
#pragma unroll
        for (int hl = 1; hl < kHeadsPerGroup; ++hl) {
            mine = li == hl ? dots[hl] : mine;
        }
        if (li < kHeadsPerGroup) {
            s_m[li][gi] = mine * a.qk_scale_log2;  // score of (token gi, head li)
        }
        float4* vrow = reinterpret_cast<float4*>(&s_vf[gi][8 * li]);
        vrow[0] = make_float4(vf[0], vf[1], vf[2], vf[3]);
        vrow[1] = make_float4(vf[4], vf[5], vf[6], vf[7]);
        __syncthreads();
        if (threadIdx.x < kGroups * kHeadsPerGroup) {
            const int hl = threadIdx.x / kGroups;
            const int gg = threadIdx.x % kGroups;
            float sv[kGroups];
#pragma unroll
            for (int x = 0; x < kGroups; ++x) {
                sv[x] = s_m[hl][x];
            }
            float M = kNegInf;
#pragma unroll
            for (int x = 0; x < kGroups; ++x) {
                M = x < nvalid ? fmaxf(M, sv[x]) : M;
            }
            s_w[hl][gg] = gg < nvalid ? exp2_fixed(s_m[hl][gg] - M) : 0.0f;
            if (gg == 0) {
                s_M[hl] = M;
            }
        }
        __syncthreads();
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int hl = half * 4 + threadIdx.x / kDim;
            const int dd = threadIdx.x % kDim;
            float acc_f = 0.0f;
            float lsum = 0.0f;
#pragma unroll 8
            for (int x = 0; x < nvalid; ++x) {
                const float w = s_w[hl][x];
                acc_f = fmaf(w, s_vf[x][dd], acc_f);
                lsum = lsum + w;
            }
            av_out[half] = acc_f;
            if (dd == 0) {
                s_L[hl] = lsum;
            }
        }
        __syncthreads();
    } else if (L <= 2 * a.flat_max) {
        // ---- flat path, two tokens per group (64-token splits): group gi
        // scores tokens f0 + gi and f0 + 32 + gi with the dot and butterfly
        // above, then the same block-wide softmax per head over the split's
        // tokens and the weighted V sum in token order.  Its rows are
        // requested here, after kv_len: the early requests are the one-token
        // layout's (requesting both layouts up front costs every short
        // length more than it saves here).
        float (*s_vf)[kDim] = reinterpret_cast<float (*)[kDim]>(&s_acc[0][0][0]);
        float (*s_sc)[2 * kGroups] = reinterpret_cast<float (*)[2 * kGroups]>(&s_x[0][0]);
        float (*s_wt)[2 * kGroups] = s_sc + kHeadsPerGroup;
        static_assert(2 * kHeadsPerGroup * 2 * kGroups <= kGroups * kSlot, "scores and weights fit the slots");
        static_assert(2 * kGroups * kDim <= kGroups * (kHeadsPerGroup / 2) * kDim, "64 V rows fit the stage");
        static_assert(kHeadsPerGroup * 2 * kGroups == kGqaThreads, "one thread per (head, token)");
        const int64_t f0 = s * 2 * kFlatTokens;
        const int nvalid = static_cast<int>(f0 + 2 * kFlatTokens < L ? 2 * kFlatTokens : L - f0);
        uint4 k2[2], v2[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int64_t t = f0 + kFlatTokens * u + gi;
            const int64_t tc = t < a.capacity ? t : a.capacity - 1;
            k2[u] = *reinterpret_cast<const uint4*>(kbase + tc * kDim);
            v2[u] = *reinterpret_cast<const uint4*>(vbase + tc * kDim);
        }
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            float kf[8], vf[8];
            unpack8<T>(k2[u], kf);
            unpack8<T>(v2[u], vf);
            float dots[kHeadsPerGroup];
#pragma unroll
            for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                float t = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    t = fmaf(q[hl][j], kf[j], t);
                }
                dots[hl] = t;
            }
#pragma unroll
            for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                dots[hl] += row_ror<8>(dots[hl]);
            }
#pragma unroll
            for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                dots[hl] += row_ror<4>(dots[hl]);
            }
#pragma unroll
            for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                dots[hl] += row_ror<2>(dots[hl]);
            }
#pragma unroll
            for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                dots[hl] += row_ror<1>(dots[hl]);
            }
            float mine = dots[0];
#pragma unroll
            for (int hl = 1; hl < kHeadsPerGroup; ++hl) {
                mine = li == hl ? dots[hl] : mine;
            }
            const int tok = kFlatTokens * u + gi;
            if (li < kHeadsPerGroup) {
                s_sc[li][tok] = mine * a.qk_scale_log2;  // score of (token tok, head li)
            }
            float4* vrow = reinterpret_cast<float4*>(&s_vf[tok][8 * li]);
            vrow[0] = make_float4(vf[0], vf[1], vf[2], vf[3]);
            vrow[1] = make_float4(vf[4], vf[5], vf[6], vf[7]);
        }
        __syncthreads();
        {
            const int hl = threadIdx.x / (2 * kGroups);
            const int gg = threadIdx.x % (2 * kGroups);
            float M = kNegInf;
#pragma unroll 8
            for (int x = 0; x < 2 * kGroups; ++x) {
                M = x < nvalid ? fmaxf(M, s_sc[hl][x]) : M;
            }
            s_wt[hl][gg] = gg < nvalid ? exp2_fixed(s_sc[hl][gg] - M) : 0.0f;
            if (gg == 0) {
                s_M[hl] = M;
            }
        }
        __syncthreads();
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int hl = half * 4 + threadIdx.x / kDim;
            const int dd = threadIdx.x % kDim;
            float acc_f = 0.0f;
            float lsum = 0.0f;
#pragma unroll 8
            for (int x = 0; x < nvalid; ++x) {
                const float w = s_wt[hl][x];
                acc_f = fmaf(w, s_vf[x][dd], acc_f);
                lsum = lsum + w;
            }
            av_out[half] = acc_f;
            if (dd == 0) {
                s_L[hl] = lsum;
            }
        }
        __syncthreads();
    } else {
        const int64_t tend = (t0 + C < L) ? t0 + C : L;
        // softmax state of head li lives in lane li (< 8) of each group
        float m_own = kNegInf, l_own = 0.0f;
        float acc[kHeadsPerGroup][8];
#pragma unroll
        for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[hl][j] = 0.0f;
            }
        }
        float* slot = s_x[gi];

        // One 128-token round: group gi takes tokens base + 4gi + {0..3}.
        auto round = [&](const uint4* ck, const uint4* cv_in, int64_t base) {
            const int cur_valid = clamp4(tend - (base + 4 * gi));
            // scores, one token at a time: 8 partial dots per lane, the 16-lane
            // butterfly (distances 8, 4, 2, 1) stage by stage over the 8 heads,
            // lane 0 files the scaled sums as two float4
            float4* out4 = reinterpret_cast<float4*>(slot);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                float kf[8];
                unpack8<T>(ck[k], kf);
                float d[kHeadsPerGroup];
#pragma unroll
                for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                    float t = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        t = fmaf(q[hl][j], kf[j], t);
                    }
                    d[hl] = t;
                }
#pragma unroll
                for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                    d[hl] += row_ror<8>(d[hl]);
                }
#pragma unroll
                for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                    d[hl] += row_ror<4>(d[hl]);
                }
#pragma unroll
                for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                    d[hl] += row_ror<2>(d[hl]);
                }
#pragma unroll
                for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                    d[hl] += row_ror<1>(d[hl]);
                }
                if (li == 0) {
                    const float sc = a.qk_scale_log2;
                    out4[2 * k] = make_float4(d[0] * sc, d[1] * sc, d[2] * sc, d[3] * sc);
                    out4[2 * k + 1] = make_float4(d[4] * sc, d[5] * sc, d[6] * sc, d[7] * sc);
                }
            }
            if (cur_valid == 0) {
                return;  // this group has no token in this round
            }
            __builtin_amdgcn_wave_barrier();
            // lane li < 8: online-softmax step of head li; slot k*8+li becomes
            // p = exp2(s - m_new) (0 for a token past the end), slot 32+li the
            // rescale exp2(m_old - m_new)
            if (li < kHeadsPerGroup) {
                float sc[4];
                float mt = kNegInf;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    sc[k] = slot[k * 8 + li];
                    if (k < cur_valid) {
                        mt = fmaxf(mt, sc[k]);
                    }
                }
                const float mnew = fmaxf(m_own, mt);
                const float corr = exp2_fixed(m_own - mnew);
                l_own = l_own * corr;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    float pk = 0.0f;
                    if (k < cur_valid) {
                        pk = exp2_fixed(sc[k] - mnew);
                        l_own = l_own + pk;
                    }
                    slot[k * 8 + li] = pk;
                }
                slot[32 + li] = corr;
                m_own = mnew;
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                const float corr = slot[32 + hl];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    acc[hl][j] = acc[hl][j] * corr;
                }
            }
            // rows past the end contribute 0 * 0: acc is never -0, so
            // fmaf(0, 0, acc) == acc and no branch is needed
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint4 raw = k < cur_valid ? cv_in[k] : make_uint4(0, 0, 0, 0);
                float vf[8];
                unpack8<T>(raw, vf);
#pragma unroll
                for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                    const float pk = slot[k * 8 + hl];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        acc[hl][j] = fmaf(pk, vf[j], acc[hl][j]);
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
        };

        // Ping-pong over two register sets: the next round's rows (clamped, so
        // unconditional) load while the current round computes.
        const int64_t last = tend - 1;
        if (s != 0) {
            load_rows(kbase, vbase, t0 + 4 * gi, last, kA, vA);
        }
        for (int64_t base = t0;;) {
            int64_t nb = base + kRoundTokens;
            load_rows(kbase, vbase, nb + 4 * gi, last, kB, vB);
            round(kA, vA, base);
            if (nb >= tend) {
                break;
            }
            base = nb;
            nb = base + kRoundTokens;
            load_rows(kbase, vbase, nb + 4 * gi, last, kA, vA);
            round(kB, vB, base);
            if (nb >= tend) {
                break;
            }
            base = nb;
        }

        // ---- merge the group states of this block (per head, groups in order;
        // a group that saw no token is skipped)
        if (li < kHeadsPerGroup) {
            s_m[li][gi] = m_own;
            s_l[li][gi] = l_own;
        }
        __syncthreads();
        if (threadIdx.x < kGroups * kHeadsPerGroup) {
            const int hl = threadIdx.x / kGroups;
            const int gg = threadIdx.x % kGroups;
            float mv[kGroups];
#pragma unroll
            for (int x = 0; x < kGroups; ++x) {
                mv[x] = s_m[hl][x];
            }
            float M = kNegInf;
#pragma unroll
            for (int x = 0; x < kGroups; ++x) {
                M = fmaxf(M, mv[x]);
            }
            const float mg = s_m[hl][gg];
            s_w[hl][gg] = mg == kNegInf ? 0.0f : exp2_fixed(mg - M);
            if (gg == 0) {
                s_M[hl] = M;
            }
        }
        __syncthreads();
        if (threadIdx.x < kHeadsPerGroup) {
            const int hl = threadIdx.x;
            float mv[kGroups], lv[kGroups], wv[kGroups];
#pragma unroll
            for (int x = 0; x < kGroups; ++x) {
                mv[x] = s_m[hl][x];
                lv[x] = s_l[hl][x];
                wv[x] = s_w[hl][x];
            }
            float lsum = 0.0f;
#pragma unroll
            for (int x = 0; x < kGroups; ++x) {
                const float t = fmaf(lv[x], wv[x], lsum);
                lsum = mv[x] != kNegInf ? t : lsum;
            }
            s_L[hl] = lsum;
        }

        // merged acc of the block: thread t owns (hl = half*4 + t/128, d = t%128)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            __syncthreads();
#pragma unroll
            for (int hh = 0; hh < kHeadsPerGroup / 2; ++hh) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    s_acc[gi][hh][8 * li + j] = acc[half * 4 + hh][j];
                }
            }
            __syncthreads();
            const int hh = threadIdx.x / kDim;
            const int d = threadIdx.x % kDim;
            const int hl = half * 4 + hh;
            float mv[kGroups], wv[kGroups], xv[kGroups];
#pragma unroll
            for (int x = 0; x < kGroups; ++x) {
                mv[x] = s_m[hl][x];
                wv[x] = s_w[hl][x];
                xv[x] = s_acc[x][hh][d];
            }
            float av = 0.0f;
#pragma unroll
            for (int x = 0; x < kGroups; ++x) {
                const float t = fmaf(xv[x], wv[x], av);
                av = mv[x] != kNegInf ? t : av;
            }
            av_out[half] = av;
        }
    }

    float* part = a.partials;
    if (nsplit <= a.defer_max) {
        // left for the consumer kernel, which merges in split order exactly
        // as below; plain stores, visible to the next kernel in the stream
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int hl = half * 4 + threadIdx.x / kDim;
            const int d = threadIdx.x % kDim;
            float* dst = part + ((g * kHeadsPerGroup + hl) * a.max_splits + s) * kPartialStride;
            dst[2 + d] = av_out[half];
            if (d == 0) {
                dst[0] = s_M[hl];
                dst[1] = s_L[hl];
            }
        }
        return;
    }
    if (nsplit == 1) {
        // single split: the general merge with weight exp2(M - M) = 1
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int hl = half * 4 + threadIdx.x / kDim;
            const int d = threadIdx.x % kDim;
            const float w = exp2_fixed(s_M[hl] - s_M[hl]);
            const float lt = fmaf(s_L[hl], w, 0.0f);
            const float o = fmaf(av_out[half], w, 0.0f);
            a.out[(g * kHeadsPerGroup + hl) * kDim + d] = T::store(o / lt);
        }
        return;
    }

#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int hl = half * 4 + threadIdx.x / kDim;
        const int d = threadIdx.x % kDim;
        float* dst = part + ((g * kHeadsPerGroup + hl) * a.max_splits + s) * kPartialStride;
        store_agent(dst + 2 + d, av_out[half]);
        if (d == 0) {
            store_agent(dst, s_M[hl]);
            store_agent(dst + 1, s_L[hl]);
        }
    }
    if (nsplit > a.ticket_max) {
        return;  // gqa_merge_kernel follows
    }

    // ---- ticket: the last block of this KV head merges all splits (the
    // partials travel through agent-scope atomic stores/loads, no fences)
    wait_own_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(a.counters + g, 1u);
        s_last = prev == static_cast<uint32_t>(nsplit - 1) ? 1 : 0;
    }
    __syncthreads();
    if (s_last == 0) {
        return;
    }
    if (threadIdx.x == 0) {
        store_agent(a.counters + g, 0u);
    }
    // One pass: every thread issues all the loads it needs (the split maxima
    // and sums of its head and its element of every split's accumulator),
    // then forms the weights exp2(m_s - M) itself and sums in split order.
    // Up to 16 splits use 16-wide register arrays, more the 32-wide ones
    // (same operations in the same order; short merges do not pay for the
    // wide form's loads and instructions).
    if (nsplit <= kInKernelSplits / 2) {
        ticket_merge<T, kInKernelSplits / 2>(a, part, g, static_cast<int>(nsplit));
    } else {
        ticket_merge<T, kInKernelSplits>(a, part, g, static_cast<int>(nsplit));
    }
}

// grid (16 query heads, 128 / kMergeDims).  One load pass: thread t brings
// splits t, t+256, ... (max, sum and this block's 16-float slice of the
// accumulator, as float4s) into LDS, all loads in flight together.  The
// maximum over splits is an order-free reduction; the weights exp2(m_s - M)
// and the two sums then run in split order, as in the in-kernel merge.
template <typename T>
__global__ __launch_bounds__(256) void gqa_merge_kernel(GqaArgs a) {
    constexpr int kPerThread = kMergeMaxSplits / 256;
    __shared__ float s_m[kMergeMaxSplits];
    __shared__ float s_l[kMergeMaxSplits];
    __shared__ __attribute__((aligned(16))) float s_v[kMergeMaxSplits][kMergeDims];
    __shared__ float s_red[4];
    __shared__ float s_lt;
    const int h = blockIdx.x;
    const int d0 = blockIdx.y * kMergeDims;
    const int64_t L = read_kv_len(a);
    const int nsplit = static_cast<int>(split_count(a, L));
    if (nsplit <= a.ticket_max) {
        return;  // merged by the partial kernel
    }
    const float* src = a.partials + static_cast<int64_t>(h) * a.max_splits * kPartialStride;
    float mloc = kNegInf;
    float mr[kPerThread], lr[kPerThread];
    float4 vr[kPerThread][kMergeDims / 4];
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const int x = static_cast<int>(threadIdx.x) + 256 * i;
        const int xs = x < nsplit ? x : 0;  // past the end: re-read split 0, unused
        const float* row = src + static_cast<int64_t>(xs) * kPartialStride;
        mr[i] = row[0];
        lr[i] = row[1];
#pragma unroll
        for (int j = 0; j < kMergeDims / 4; ++j) {
            const float* p = row + 2 + d0 + 4 * j;
            vr[i][j] = make_float4(p[0], p[1], p[2], p[3]);
        }
    }
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const int x = static_cast<int>(threadIdx.x) + 256 * i;
        if (x < nsplit) {
            s_m[x] = mr[i];
            s_l[x] = lr[i];
            mloc = fmaxf(mloc, mr[i]);
#pragma unroll
            for (int j = 0; j < kMergeDims / 4; ++j) {
                *reinterpret_cast<float4*>(&s_v[x][4 * j]) = vr[i][j];
            }
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        mloc = fmaxf(mloc, __shfl_xor(mloc, o, 64));
    }
    if ((threadIdx.x & 63) == 0) {
        s_red[threadIdx.x >> 6] = mloc;
    }
    __syncthreads();
    const float M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    // weights in place of the maxima (each thread rewrites its own splits)
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
        const int x = static_cast<int>(threadIdx.x) + 256 * i;
        if (x < nsplit) {
            s_m[x] = exp2_fixed(mr[i] - M);
        }
    }
    __syncthreads();
    const int d = threadIdx.x;
    if (d == kMergeDims) {
        float lt = 0.0f;
        for (int x = 0; x < nsplit; ++x) {
            lt = fmaf(s_l[x], s_m[x], lt);
        }
        s_lt = lt;
    }
    float o = 0.0f;
    if (d < kMergeDims) {
        for (int x = 0; x < nsplit; ++x) {
            o = fmaf(s_v[x][d], s_m[x], o);
        }
    }
    __syncthreads();
    if (d < kMergeDims) {
        a.out[static_cast<int64_t>(h) * kDim + d0 + d] = T::store(o / s_lt);
    }
}

}  // namespace

// Split rule (measured on MI355X): flat path up to 32 x 32 tokens (585-1024
// tokens: 13.4 -> 8.9 us against 128-token round splits) and up to 32 x 64
// tokens with two tokens per group (1100-2048 tokens: 13.3-13.7 -> 12.2-12.7
// us); round path with
// 128-token splits up to 8192 tokens (more blocks at mid lengths: 8192 tokens
// 17.7 -> 15.3 us against 256-token splits), 256-token splits
// beyond (at 32768 tokens 256 splits of 128 cost more in the merge than they
// save: 30.4 vs 22.1 us).
constexpr int64_t kMidMax = 8192;
static_assert(kGqaMidTokens == kRoundTokens, "mid-length splits are one round");

int64_t gqa_chunk_for(int64_t) { return 2 * kRoundTokens; }

GqaPlan gqa_plan(int64_t capacity, int64_t split_limit) {
    GqaPlan p;
    p.chunk = gqa_chunk_for(capacity);
    int64_t flat_splits = kFlatSplits;
    p.mid_max = kMidMax;
    if (split_limit > 0) {
        // a caller-sized workspace: no regime may need more splits than it holds
        flat_splits = split_limit < flat_splits ? split_limit : flat_splits;
        p.mid_max = kGqaMidTokens * split_limit < p.mid_max ? kGqaMidTokens * split_limit : p.mid_max;
        const int64_t need = (capacity + split_limit - 1) / split_limit;
        const int64_t rounded = (need + kRoundTokens - 1) / kRoundTokens * kRoundTokens;
        p.chunk = rounded > p.chunk ? rounded : p.chunk;
    }
    p.flat_max = flat_splits * kFlatTokens;
    p.flat_max = p.flat_max < capacity ? p.flat_max : capacity;
    p.mid_max = p.mid_max < capacity ? p.mid_max : capacity;
    const int64_t flat = (p.flat_max + kFlatTokens - 1) / kFlatTokens;
    const int64_t mid = (p.mid_max + kGqaMidTokens - 1) / kGqaMidTokens;
    const int64_t lng = (capacity + p.chunk - 1) / p.chunk;
    p.max_splits = flat > mid ? flat : mid;
    p.max_splits = lng > p.max_splits ? lng : p.max_splits;
    return p;
}

hipError_t launch_gqa_decode(Act act, const GqaArgs& a, hipStream_t stream) {
    // the grid must cover every split any length up to the capacity produces
    const int64_t flat_splits = (a.flat_max + kFlatTokens - 1) / kFlatTokens;
    const int64_t mid_splits = (a.mid_max + kGqaMidTokens - 1) / kGqaMidTokens;
    const int64_t long_splits = a.chunk > 0 ? (a.capacity + a.chunk - 1) / a.chunk : 0;
    if (a.max_splits <= 0 || a.max_splits > kMergeMaxSplits || a.chunk <= 0 || a.chunk % kRoundTokens != 0 ||
        a.flat_max < 0 || flat_splits > kFlatSplits || a.mid_max < 0 || a.capacity <= 0 ||
        flat_splits > a.max_splits || mid_splits > a.max_splits || long_splits > a.max_splits ||
        a.defer_max < 0 || a.defer_max > kGqaMaxDefer || a.defer_max > a.max_splits || a.ticket_max < 1 ||
        a.ticket_max > kInKernelSplits) {
        return hipErrorInvalidValue;
    }
    const dim3 grid(static_cast<unsigned>(a.max_splits), 2);
    if (act == Act::kBf16) {
        hipLaunchKernelGGL(gqa_partial_kernel<Bf16>, grid, dim3(kGqaThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL(gqa_partial_kernel<F16>, grid, dim3(kGqaThreads), 0, stream, a);
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

}  // namespace kc
