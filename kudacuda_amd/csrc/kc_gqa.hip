// Split-KV grouped-query decode attention for the Qwen2.5-3B shape
// (16 query heads, 2 KV heads, group 8, head_dim 128), one launch per call.
//
// Grid (max_splits, 2): block (s, g) owns tokens [s*C, min(s*C+C, L)) of KV
// head g and serves all 8 query heads of the group, so every K/V byte is read
// once.  A block is 4 waves = 16 groups of 16 lanes; lane li of a group holds
// dims [8li, 8li+8) of all 8 query heads.  Per 64-token round, group gi takes
// tokens base + 4gi + {0..3}: 8 dot products of 8 dims per lane, a 16-lane
// butterfly, then an online-softmax update in the log2 domain (scores are
// pre-multiplied by scale*log2e and exponentiated with exp2_fixed).
// The 16 group states are merged through LDS, each block writes one
// (max, sum, acc[128]) partial per head, and the last block of a KV head to
// finish (device-scope ticket) merges the splits and writes the output.  The
// ticket counter is reset by that block, so the launch is capture-safe and
// needs no memset.  kv_len may come from device memory (graph replay).
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

constexpr int kGqaThreads = 256;
constexpr int kGroups = 16;
constexpr int kHeadsPerGroup = 8;
constexpr int kDim = 128;
constexpr int kPartialStride = 2 + kDim;

template <typename T>
__global__ __launch_bounds__(kGqaThreads) void gqa_split_kernel(GqaArgs a) {
    __shared__ float s_m[kGroups][kHeadsPerGroup];
    __shared__ float s_l[kGroups][kHeadsPerGroup];
    __shared__ float s_acc[kGroups][kHeadsPerGroup / 2][kDim];  // half the heads at a time
    __shared__ int s_last;

    const int g = blockIdx.y;
    const int64_t s = blockIdx.x;
    int64_t L = a.kv_len_device != nullptr ? static_cast<int64_t>(*a.kv_len_device) + a.kv_len_offset : a.kv_len_host;
    L = L < 0 ? 0 : (L > a.capacity ? a.capacity : L);
    const int64_t C = a.chunk;
    const int64_t nsplit = (L + C - 1) / C;
    if (s >= nsplit) {
        return;
    }

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int gi = wave * 4 + (lane >> 4);
    const int li = lane & 15;

    float q[kHeadsPerGroup][8];
#pragma unroll
    for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
        const uint4 v = *reinterpret_cast<const uint4*>(a.q + (g * kHeadsPerGroup + hl) * kDim + 8 * li);
        unpack8<T>(v, q[hl]);
    }
    float m[kHeadsPerGroup], l[kHeadsPerGroup], acc[kHeadsPerGroup][8];
#pragma unroll
    for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
        m[hl] = -__builtin_huge_valf();
        l[hl] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc[hl][j] = 0.0f;
        }
    }

    const uint16_t* kbase = a.k + static_cast<int64_t>(g) * a.capacity * kDim + 8 * li;
    const uint16_t* vbase = a.v + static_cast<int64_t>(g) * a.capacity * kDim + 8 * li;
    const int64_t t0 = s * C;
    const int64_t tend = (t0 + C < L) ? t0 + C : L;
    for (int64_t base = t0; base < tend; base += 64) {
        const int64_t tk = base + 4 * gi;
        int nvalid = static_cast<int>(tend - tk);
        nvalid = nvalid < 0 ? 0 : (nvalid > 4 ? 4 : nvalid);
        uint4 kr[4], vr[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (k < nvalid) {
                kr[k] = *reinterpret_cast<const uint4*>(kbase + (tk + k) * kDim);
                vr[k] = *reinterpret_cast<const uint4*>(vbase + (tk + k) * kDim);
            } else {
                kr[k] = make_uint4(0, 0, 0, 0);
                vr[k] = make_uint4(0, 0, 0, 0);
            }
        }
        float s2[4][kHeadsPerGroup];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float kf[8];
            unpack8<T>(kr[k], kf);
#pragma unroll
            for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
                float d = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    d = fmaf(q[hl][j], kf[j], d);
                }
                s2[k][hl] = group16_sum(d) * a.qk_scale_log2;
            }
        }
        if (nvalid == 0) {
            continue;
        }
        float vf[4][8];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            unpack8<T>(vr[k], vf[k]);
        }
#pragma unroll
        for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
            float mt = -__builtin_huge_valf();
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (k < nvalid) {
                    mt = fmaxf(mt, s2[k][hl]);
                }
            }
            const float mnew = fmaxf(m[hl], mt);
            const float corr = exp2_fixed(m[hl] - mnew);
            l[hl] = l[hl] * corr;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc[hl][j] = acc[hl][j] * corr;
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (k < nvalid) {
                    const float p = exp2_fixed(s2[k][hl] - mnew);
                    l[hl] = l[hl] + p;
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        acc[hl][j] = fmaf(p, vf[k][j], acc[hl][j]);
                    }
                }
            }
            m[hl] = mnew;
        }
    }

    // ---- merge the 16 group states of this block (per head, groups in order)
    if (li == 0) {
#pragma unroll
        for (int hl = 0; hl < kHeadsPerGroup; ++hl) {
            s_m[gi][hl] = m[hl];
            s_l[gi][hl] = l[hl];
        }
    }
    float* part = a.partials;
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
        for (int idx = threadIdx.x; idx < (kHeadsPerGroup / 2) * kDim; idx += kGqaThreads) {
            const int hh = idx / kDim;
            const int d = idx % kDim;
            const int hl = half * 4 + hh;
            float M = -__builtin_huge_valf();
            for (int gg = 0; gg < kGroups; ++gg) {
                M = fmaxf(M, s_m[gg][hl]);
            }
            float lsum = 0.0f, av = 0.0f;
            for (int gg = 0; gg < kGroups; ++gg) {
                const float mg = s_m[gg][hl];
                if (mg == -__builtin_huge_valf()) {
                    continue;
                }
                const float w = exp2_fixed(mg - M);
                lsum = fmaf(s_l[gg][hl], w, lsum);
                av = fmaf(s_acc[gg][hh][d], w, av);
            }
            const int64_t h = g * kHeadsPerGroup + hl;
            float* dst = part + (h * a.max_splits + s) * kPartialStride;
            dst[2 + d] = av;
            if (d == 0) {
                dst[0] = M;
                dst[1] = lsum;
            }
        }
    }

    // ---- ticket: the last block of this KV head merges all splits
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t prev = atomicAdd(a.counters + g, 1u);
        s_last = prev == static_cast<uint32_t>(nsplit - 1) ? 1 : 0;
    }
    __syncthreads();
    if (s_last == 0) {
        return;
    }
    __threadfence();
    if (threadIdx.x == 0) {
        a.counters[g] = 0u;
    }
    for (int idx = threadIdx.x; idx < kHeadsPerGroup * kDim; idx += kGqaThreads) {
        const int hl = idx / kDim;
        const int d = idx % kDim;
        const int64_t h = g * kHeadsPerGroup + hl;
        const float* src = part + h * a.max_splits * kPartialStride;
        float M = -__builtin_huge_valf();
        for (int64_t ss = 0; ss < nsplit; ++ss) {
            M = fmaxf(M, src[ss * kPartialStride]);
        }
        float lt = 0.0f, o = 0.0f;
        for (int64_t ss = 0; ss < nsplit; ++ss) {
            const float* p = src + ss * kPartialStride;
            const float w = exp2_fixed(p[0] - M);
            lt = fmaf(p[1], w, lt);
            o = fmaf(p[2 + d], w, o);
        }
        a.out[h * kDim + d] = T::store(o / lt);
    }
}

}  // namespace

int64_t gqa_chunk_for(int64_t tokens) {
    int64_t chunk = 64;
    while ((tokens + chunk - 1) / chunk > 128) {
        chunk *= 2;
    }
    return chunk;
}

hipError_t launch_gqa_decode(Act act, const GqaArgs& a, hipStream_t stream) {
    if (a.max_splits <= 0) {
        return hipSuccess;
    }
    const dim3 grid(static_cast<unsigned>(a.max_splits), 2);
    if (act == Act::kBf16) {
        hipLaunchKernelGGL(gqa_split_kernel<Bf16>, grid, dim3(kGqaThreads), 0, stream, a);
    } else {
        hipLaunchKernelGGL(gqa_split_kernel<F16>, grid, dim3(kGqaThreads), 0, stream, a);
    }
    return hipGetLastError();
}

}  // namespace kc
