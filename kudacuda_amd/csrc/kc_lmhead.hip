// Dense bf16 lm_head GEMV (tied embedding, vocab x 2048) fused with the final
// RMSNorm, bf16 logit rounding and a device-side greedy argmax.
//
// One wave per vocabulary row: lane l reads 16-byte chunks l, l+64, l+128,
// l+192 of the 4 KiB row (every wave load is a contiguous 1 KiB), keeps one
// accumulator per chunk and combines them as (a0+a1)+(a2+a3) before the wave
// butterfly.  The logit is rounded to bf16 (the model's logits dtype) and the
// argmax runs on the rounded values with the lowest index winning ties, as
// torch.argmax does on the reference's logits
// (tools/benchmark/benchmark_gemma.py:350).  Block winners go to a small
// workspace with plain stores; a one-block second kernel on the same stream
// reads them (the kernel boundary orders the stores before its loads) and
// picks the token.  (A "last block" ticket inside the GEMV kernel cost as much
// as that second launch and needed device-scope fences on every block to be
// correct by the memory model.)
//
// When `control` is given the launch also does the per-token decode
// bookkeeping on device: during the prompt (step + 1 < prompt_len) the GEMV is
// skipped and the next prompt token stays in place; otherwise the winner is
// written to tokens[step + 1]; step then advances.  This removes the host
// argmax/.item() round trip the reference pays per token
// (tools/benchmark/benchmark_gemma.py:328-352).  Stop token (control[3] >= 0):
// the step that emits it keeps it in tokens[], sets the done flag control[4]
// and records its position in control[5]; from then on every step skips the
// GEMV and neither writes a token nor advances -- the reference's EOS stop,
// checked on the device so a host can replay many steps without a per-token
// sync and read where the decode stopped
// (tools/benchmark/benchmark_gemma.py:100-112,147).
#include "kc_device.h"
#include "kc_kernels.h"

namespace kc {
namespace {

constexpr int kLmThreads = 256;
constexpr int kLmMaxBlocks = 768;  // 3072 waves: all resident at 3 waves/SIMD
constexpr int kRing = 4;  // rows in flight per wave

__device__ __forceinline__ bool better(float v, int32_t i, float bv, int32_t bi) {
    return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ float row_dot(const uint4* w, const float* xn) {
    float a[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        float wf[8];
        unpack8<Bf16>(w[c], wf);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc = fmaf(xn[8 * c + j], wf[j], acc);
        }
        a[c] = acc;
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

// The leading scalar arguments (what the first loads need) are preloaded
// into SGPRs at wave launch; they stand for the same fields of `args`.
__global__ __launch_bounds__(kLmThreads) void lm_head_kernel(const uint16_t* weight, const uint16_t* x,
                                                             const uint16_t* gamma, int64_t vocab, LmHeadArgs args) {
    LmHeadArgs a = args;
    a.weight = weight;
    a.x = x;
    a.gamma = gamma;
    a.vocab = vocab;
    __shared__ float s_val[kLmThreads / 64];
    __shared__ int32_t s_idx[kLmThreads / 64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;

    int32_t step = 0;
    bool active = true;
    bool stopped = false;
    if (a.control != nullptr) {
        step = a.control[0];
        stopped = a.control[4] != 0;
        active = !stopped && step + 1 >= a.control[1];
    }

    float best = -__builtin_huge_valf();
    int32_t best_idx = 0x7fffffff;
    if (active) {
        // Loads first, in a fixed order: the first kRing rows of the ring,
        // then the activation chunks (norm layout [32l, 32l+32) and dot
        // layout 8(l + 64c) + j) and gamma.  The rows' HBM requests go out
        // ahead of the activation's L2 reads (decode step 1.1173 -> 1.1160 ms
        // over 10 interleaved runs); every wait is for a known prefix of the
        // issued loads, and the first dot needs its rows anyway.
        const uint4* xv = reinterpret_cast<const uint4*>(a.x);
        const bool has_gamma = a.gamma != nullptr;
        const uint4* gv = reinterpret_cast<const uint4*>(has_gamma ? a.gamma : a.x);
        uint4 xs_raw[4], xd_raw[4], g_raw[4];

        // Ring of kRing rows per wave: row base + i*nwaves sits in slot i and is
        // refilled with the row kRing*nwaves further on as soon as it has been
        // consumed.  The loads are unconditional (rows past the end read the
        // last row again, which stays in cache) so the loop body is straight
        // line code and every dot waits only for its own slot's loads.
        const int64_t nwaves = static_cast<int64_t>(gridDim.x) * (kLmThreads / 64);
        // wave-uniform row numbers (scalar registers, scalar loop control)
        const int64_t first = static_cast<int64_t>(blockIdx.x) * (kLmThreads / 64) +
                              __builtin_amdgcn_readfirstlane(wave);
        const int64_t last_row = a.vocab - 1;
        const uint4* wbase = reinterpret_cast<const uint4*>(a.weight) + lane;
        uint4 w[kRing][4];
#pragma unroll
        for (int i = 0; i < kRing; ++i) {
            __builtin_amdgcn_sched_barrier(0);
            const uint4* src = wbase + (first + i * nwaves < last_row ? first + i * nwaves : last_row) * 256;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                w[i][c] = load_stream(src + 64 * c);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xs_raw[i] = xv[lane * 4 + i];
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            xd_raw[c] = xv[lane + 64 * c];
            g_raw[c] = gv[lane + 64 * c];
        }

        // Final RMSNorm: inverse RMS over elements [32l, 32l+32) per lane,
        // then the lane's dot elements normalised the same way.
        float xs[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            unpack8<Bf16>(xs_raw[i], xs + 8 * i);
        }
        const float r = has_gamma ? inv_rms(wave_sum(sumsq32(xs)), 2048.0f, a.eps) : 1.0f;
        float xn[32];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            unpack8<Bf16>(xd_raw[c], xn + 8 * c);
            float gf[8];
            unpack8<Bf16>(g_raw[c], gf);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                xn[8 * c + j] = has_gamma ? (xn[8 * c + j] * r) * gf[j] : xn[8 * c + j];
            }
        }

        for (int64_t base = first; base < a.vocab; base += kRing * nwaves) {
            float sum[kRing];
#pragma unroll
            for (int i = 0; i < kRing; ++i) {
                sum[i] = row_dot(w[i], xn);
                const int64_t rn = base + (i + kRing) * nwaves;
                const uint4* src = wbase + (rn < last_row ? rn : last_row) * 256;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    w[i][c] = load_stream(src + 64 * c);
                }
                // keep slot i's refill ahead of slot i+1's dot
                __builtin_amdgcn_sched_barrier(0);
            }
            static_assert(kRing % 2 == 0, "rows reduced in pairs");
#pragma unroll
            for (int i = 0; i < kRing; i += 2) {
                const float2 s2 = wave_sum2(sum[i], sum[i + 1]);
                sum[i] = s2.x;
                sum[i + 1] = s2.y;
            }
            // lane i (< kRing) stores slot i's logit: one store per pass
            uint16_t lane_lb = 0;
#pragma unroll
            for (int i = 0; i < kRing; ++i) {
                const int64_t row = base + i * nwaves;
                const uint16_t lb = f32_to_bf16(sum[i]);
                const float v = bf16_to_f32(lb);
                lane_lb = lane == i ? lb : lane_lb;
                if (row < a.vocab && better(v, static_cast<int32_t>(row), best, best_idx)) {
                    best = v;
                    best_idx = static_cast<int32_t>(row);
                }
            }
            const int64_t lane_row = base + lane * nwaves;
            if (a.logits != nullptr && lane < kRing && lane_row < a.vocab) {
                a.logits[lane_row] = lane_lb;
            }
        }
        if (lane == 0) {
            s_val[wave] = best;
            s_idx[wave] = best_idx;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int i = 1; i < kLmThreads / 64; ++i) {
                if (better(s_val[i], s_idx[i], best, best_idx)) {
                    best = s_val[i];
                    best_idx = s_idx[i];
                }
            }
            a.block_best[2 * blockIdx.x] = best;
            a.block_best[2 * blockIdx.x + 1] = __int_as_float(best_idx);
        }
    }
}

// The token from the GEMV launch's `nblocks` block winners, and the decode
// bookkeeping.  One block; the winners' order does not matter (better() is
// the first-max rule on (value, index) pairs).
__global__ __launch_bounds__(kLmThreads) void lm_head_finish_kernel(LmHeadArgs a, int nblocks) {
    __shared__ float s_val[kLmThreads / 64];
    __shared__ int32_t s_idx[kLmThreads / 64];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int32_t step = 0;
    bool active = true;
    bool stopped = false;
    if (a.control != nullptr) {
        step = a.control[0];
        stopped = a.control[4] != 0;
        active = !stopped && step + 1 >= a.control[1];
    }
    float best = -__builtin_huge_valf();
    int32_t best_idx = 0x7fffffff;
    if (active) {
        for (int b = threadIdx.x; b < nblocks; b += kLmThreads) {
            const float2 e = reinterpret_cast<const float2*>(a.block_best)[b];
            const int32_t i = __float_as_int(e.y);
            if (better(e.x, i, best, best_idx)) {
                best = e.x;
                best_idx = i;
            }
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const float ov = __shfl_xor(best, o, 64);
            const int32_t oi = __shfl_xor(best_idx, o, 64);
            if (better(ov, oi, best, best_idx)) {
                best = ov;
                best_idx = oi;
            }
        }
        if (lane == 0) {
            s_val[wave] = best;
            s_idx[wave] = best_idx;
        }
        __syncthreads();
        if (threadIdx.x == 0) {
            for (int i = 1; i < kLmThreads / 64; ++i) {
                if (better(s_val[i], s_idx[i], best, best_idx)) {
                    best = s_val[i];
                    best_idx = s_idx[i];
                }
            }
            if (best_idx < 0 || best_idx >= a.vocab) {
                best_idx = 0;  // every logit was NaN
            }
        }
    }
    if (threadIdx.x == 0) {
        if (active && a.argmax_out != nullptr) {
            a.argmax_out[0] = best_idx;
        }
        if (a.control != nullptr && !stopped) {
            const int32_t next = step + 1;
            if (active && next < a.control[2]) {
                a.tokens[next] = best_idx;
            }
            if (active && a.control[3] >= 0 && best_idx == a.control[3]) {
                a.control[4] = 1;
                a.control[5] = next;
            }
            a.control[0] = next;
        }
    }
}

}  // namespace

hipError_t launch_lm_head_argmax(const LmHeadArgs& a, hipStream_t stream) {
    int64_t blocks = (a.vocab + (kLmThreads / 64) - 1) / (kLmThreads / 64);
    if (blocks > kLmMaxBlocks) {
        blocks = kLmMaxBlocks;
    }
    if (blocks < 1) {
        blocks = 1;
    }
    hipLaunchKernelGGL(lm_head_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kLmThreads), 0, stream, a.weight, a.x,
                       a.gamma, a.vocab, a);
    const hipError_t st = hipGetLastError();
    if (st != hipSuccess) {
        return st;
    }
    hipLaunchKernelGGL(lm_head_finish_kernel, dim3(1), dim3(kLmThreads), 0, stream, a, static_cast<int>(blocks));
    return hipGetLastError();
}

int64_t lm_head_workspace_floats() { return 2 * kLmMaxBlocks; }

}  // namespace kc
