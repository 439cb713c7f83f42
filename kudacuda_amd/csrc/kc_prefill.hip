// Multi-token prefill kernels for gfx950: the NF4 GEMM on MFMA matrix cores.
//
// out[m, n] = epilogue(sum_k x[m, k] * w[n, k]) with w[n, k] the NF4 weight
// dequantised to bf16 (bf16(codebook[code] * absmax), what bitsandbytes'
// dequantize-then-matmul feeds its GEMM; reference
// python/kudacuda_sidecar.py:1719-1738, kernels/common/nf4_device.cuh:10-40)
// and fp32 accumulation in v_mfma_f32_16x16x32_bf16.
//
// Tiling: a block is 4 waves, a wave owns 16 weight rows (kSwiGlu: 16 gate
// rows and the same 16 up rows) and all m <= 64 tokens (4 token tiles of
// 16).  Operand layouts of the 16x16x32 bf16 MFMA (lane l, row l%16, group
// q = l/16): A[l%16][8q + j], B[8q + j][l%16], D[4q + i][l%16].  With
// A = weights (rows n) and B[k][m] = x[m][k], D[n][m] is the output tile.
// k is walked in windows of 128: lane group q owns the 32 contiguous k
// [128w + 32q, 128w + 32q + 32), read as one 16-byte load of codes (and one
// absmax, the 32 codes sit in one 64-block) per weight row and four 16-byte
// loads per token row; MFMA step s of the window takes k = 128w + 32q + 8s + j
// from both operands, so every k of the window is summed exactly once (the
// order of k inside a product sum does not change what is summed).
// Activations (m x k bf16, at most 64 x 11008 x 2 B) are read through the
// caches; the weights stream once.
#include "kc_device.h"
#include "kc_kernels.h"

namespace kc {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kGemmWaves = 4;
constexpr int kGemmThreads = 64 * kGemmWaves;
constexpr int kRowsPerWave = 16;
constexpr int kRowsPerBlock = kRowsPerWave * kGemmWaves;
constexpr int kTokenTiles = kGemmMaxTokens / 16;
constexpr int kWindow = 128;

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// 8 codes of one 32-bit word (byte b: element 2b in the high nibble, 2b+1 in
// the low nibble) times absmax, each rounded to bf16; element j lands in
// 16-bit slot j of the result.
__device__ __forceinline__ uint4 dequant8_bf16(uint32_t word, float am, const float* cb) {
    uint32_t out[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t byte = (word >> (8 * b)) & 0xffu;
        const uint32_t hi = f32_to_bf16(cb[byte >> 4] * am);
        const uint32_t lo = f32_to_bf16(cb[byte & 0xfu] * am);
        out[b] = hi | (lo << 16);
    }
    return make_uint4(out[0], out[1], out[2], out[3]);
}

template <GemmEpi EPI>
__global__ __launch_bounds__(kGemmThreads) void nf4_gemm_kernel(Nf4GemmArgs a) {
    constexpr int NF = EPI == GemmEpi::kSwiGlu ? 2 : 1;  // weight fragments per wave
    __shared__ float cb[16];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r = lane & 15;
    const int q = lane >> 4;
    const int64_t K = a.k;
    const int M = static_cast<int>(a.m);
    const int ntiles = (M + 15) / 16;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + wave * kRowsPerWave;
    const int64_t nrow = n0 + r;  // n % 64 == 0: every row exists

    const uint8_t* wrow[NF];
    const float* arow[NF];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        wrow[f] = a.w[f] + nrow * (K / 2);
        arow[f] = a.absmax[f] + nrow * (K / 64);
    }
    // token rows of the B operand (rows past m re-read row m-1; discarded)
    const uint16_t* xrow[kTokenTiles];
#pragma unroll
    for (int t = 0; t < kTokenTiles; ++t) {
        const int m = 16 * t + r < M ? 16 * t + r : M - 1;
        xrow[t] = a.x + static_cast<int64_t>(m) * K;
    }
    block_codebook_lds(cb);
    __syncthreads();

    floatx4 acc[NF][kTokenTiles];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
#pragma unroll
        for (int t = 0; t < kTokenTiles; ++t) {
            acc[f][t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    }
    for (int64_t kw = 0; kw < K; kw += kWindow) {
        const int64_t kq = kw + 32 * q;
        uint4 wq[NF];
        float am[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            wq[f] = *reinterpret_cast<const uint4*>(wrow[f] + kq / 2);
            am[f] = arow[f][kq / 64];
        }
        uint4 xb[kTokenTiles][4];
#pragma unroll
        for (int t = 0; t < kTokenTiles; ++t) {
            if (t < ntiles) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    xb[t][s] = *reinterpret_cast<const uint4*>(xrow[t] + kq + 8 * s);
                }
            }
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
#pragma unroll
            for (int f = 0; f < NF; ++f) {
                const uint32_t word = s == 0 ? wq[f].x : (s == 1 ? wq[f].y : (s == 2 ? wq[f].z : wq[f].w));
                const bf16x8 A = as_bf16x8(dequant8_bf16(word, am[f], cb));
#pragma unroll
                for (int t = 0; t < kTokenTiles; ++t) {
                    if (t < ntiles) {
                        acc[f][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, as_bf16x8(xb[t][s]), acc[f][t], 0, 0,
                                                                             0);
                    }
                }
            }
        }
    }

    // D[4q + i][r]: rows n0 + 4q + i, token 16t + r; four consecutive rows per
    // lane go out as one 8-byte store
#pragma unroll
    for (int t = 0; t < kTokenTiles; ++t) {
        const int m = 16 * t + r;
        if (t >= ntiles || m >= M) {
            continue;
        }
        const int64_t nb = n0 + 4 * q;
        uint16_t* dst = a.out + static_cast<int64_t>(m) * a.n + nb;
        uint32_t packed[2];
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
            uint16_t h[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int i = 2 * i2 + e;
                float v = acc[0][t][i];
                if constexpr (EPI == GemmEpi::kBias) {
                    if (a.bias != nullptr) {
                        v = v + Bf16::load(a.bias[nb + i]);
                    }
                    h[e] = Bf16::store(v);
                } else if constexpr (EPI == GemmEpi::kResidual) {
                    const float res = Bf16::load(a.residual[static_cast<int64_t>(m) * a.n + nb + i]);
                    h[e] = Bf16::store(res + Bf16::load(Bf16::store(v)));
                } else {
                    const float u = acc[NF - 1][t][i];
                    h[e] = Bf16::store(silu_fixed(v) * u);
                }
            }
            packed[i2] = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
        }
        *reinterpret_cast<uint2*>(dst) = make_uint2(packed[0], packed[1]);
    }
}

}  // namespace

hipError_t launch_nf4_gemm(GemmEpi epi, const Nf4GemmArgs& a, hipStream_t stream) {
    if (a.m < 1 || a.m > kGemmMaxTokens || a.n < kRowsPerBlock || a.n % kRowsPerBlock != 0 || a.k < kWindow ||
        a.k % kWindow != 0 || a.x == nullptr || a.w[0] == nullptr || a.absmax[0] == nullptr || a.out == nullptr ||
        (epi == GemmEpi::kSwiGlu && (a.w[1] == nullptr || a.absmax[1] == nullptr)) ||
        (epi == GemmEpi::kResidual && a.residual == nullptr)) {
        return hipErrorInvalidValue;
    }
    const dim3 grid(static_cast<unsigned>(a.n / kRowsPerBlock));
    switch (epi) {
        case GemmEpi::kBias:
            hipLaunchKernelGGL(nf4_gemm_kernel<GemmEpi::kBias>, grid, dim3(kGemmThreads), 0, stream, a);
            break;
        case GemmEpi::kResidual:
            hipLaunchKernelGGL(nf4_gemm_kernel<GemmEpi::kResidual>, grid, dim3(kGemmThreads), 0, stream, a);
            break;
        case GemmEpi::kSwiGlu:
            hipLaunchKernelGGL(nf4_gemm_kernel<GemmEpi::kSwiGlu>, grid, dim3(kGemmThreads), 0, stream, a);
            break;
    }
    return hipGetLastError();
}

}  // namespace kc

// ---------------------------------------------------------------------------
// Row norm, RoPE + cache write and causal attention of the prefill.
namespace kc {
namespace {

constexpr int kNormRowsPerBlock = 4;  // one wave per row

__global__ __launch_bounds__(256) void prefill_norm_kernel(PrefillNormArgs a) {
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kNormRowsPerBlock + (threadIdx.x >> 6);
    if (row >= a.m) {
        return;
    }
    const uint16_t* x = a.x + row * 2048;
    if (a.embed != nullptr) {
        const int64_t cap = a.control != nullptr ? a.control[2] : a.start + a.m;
        const int64_t at = a.start + row < cap ? a.start + row : (cap > 0 ? cap - 1 : 0);
        int64_t tok = a.tokens[at];
        tok = tok < 0 ? 0 : (tok >= a.vocab ? a.vocab - 1 : tok);
        x = a.embed + tok * 2048;
    }
    uint4 xr[4], gr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xr[i] = reinterpret_cast<const uint4*>(x)[lane * 4 + i];
        gr[i] = reinterpret_cast<const uint4*>(a.gamma)[lane * 4 + i];
    }
    if (a.hidden_out != nullptr) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            reinterpret_cast<uint4*>(a.hidden_out + row * 2048)[lane * 4 + i] = xr[i];
        }
    }
    float xn[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        unpack8<Bf16>(xr[i], xn + 8 * i);
    }
    const float r = inv_rms(wave_sum(sumsq32(xn)), 2048.0f, a.eps);
    uint32_t packed[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float g[8];
        unpack8<Bf16>(gr[i], g);
#pragma unroll
        for (int j = 0; j < 8; j += 2) {
            const uint32_t lo = f32_to_bf16((xn[8 * i + j] * r) * g[j]);
            const uint32_t hi = f32_to_bf16((xn[8 * i + j + 1] * r) * g[j + 1]);
            packed[4 * i + j / 2] = lo | (hi << 16);
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        reinterpret_cast<uint4*>(a.out + row * 2048)[lane * 4 + i] =
            make_uint4(packed[4 * i], packed[4 * i + 1], packed[4 * i + 2], packed[4 * i + 3]);
    }
}

// grid m: thread t rotates the q pairs t, t+256, t+512, t+768 (head p/64,
// dim p%64), k pair t (< 128) and copies k/v element t (< 256) to the caches.
__global__ __launch_bounds__(256) void prefill_rope_cache_kernel(PrefillRopeArgs a) {
    const int64_t row = blockIdx.x;
    const int64_t pos = a.start + row;
    const int t = threadIdx.x;
    const float* cs = a.rope_cos + pos * 64;
    const float* sn = a.rope_sin + pos * 64;
    uint16_t* q = a.q + row * 2048;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int pair = t + 256 * i;
        const int h = pair >> 6;
        const int d = pair & 63;
        const float c = cs[d];
        const float s = sn[d];
        const float v0 = Bf16::load(q[h * 128 + d]);
        const float v1 = Bf16::load(q[h * 128 + d + 64]);
        q[h * 128 + d] = Bf16::store((v0 * c) - (v1 * s));
        q[h * 128 + d + 64] = Bf16::store((v1 * c) + (v0 * s));
    }
    const uint16_t* k = a.k + row * 256;
    const uint16_t* v = a.v + row * 256;
    if (t < 128) {
        const int g = t >> 6;
        const int d = t & 63;
        const float c = cs[d];
        const float s = sn[d];
        const float v0 = Bf16::load(k[g * 128 + d]);
        const float v1 = Bf16::load(k[g * 128 + d + 64]);
        uint16_t* kc = a.kcache + (g * a.capacity + pos) * 128;
        kc[d] = Bf16::store((v0 * c) - (v1 * s));
        kc[d + 64] = Bf16::store((v1 * c) + (v0 * s));
    }
    {
        const int g = t >> 7;
        const int d = t & 127;
        a.vcache[(g * a.capacity + pos) * 128 + d] = v[t];
    }
}

constexpr int kAttnGroups = 32;  // 16-lane groups of a 512-thread block
constexpr int kAttnHeads = 8;
constexpr int kAttnDim = 128;

// grid (m, 2 KV heads), 512 threads.  Query row r (position start + r) of the
// 8 heads of KV head g over cache rows [0, start + r], in rounds of 32 tokens
// (one per 16-lane group): scores by 8-dim partial dots and the 16-lane DPP
// butterfly (log2 domain), then per head m_new = max(m, round max), weights
// exp2(s - m_new), rescale exp2(m - m_new) of the running sum and accumulator,
// weighted V rows from LDS in token order.  out = bf16(acc / sum).
__global__ __launch_bounds__(512) void prefill_attention_kernel(PrefillAttnArgs a) {
    __shared__ __attribute__((aligned(16))) float s_sc[2][kAttnHeads][kAttnGroups];
    __shared__ __attribute__((aligned(16))) float s_w[2][kAttnHeads][kAttnGroups];
    __shared__ float s_corr[2][kAttnHeads];
    __shared__ __attribute__((aligned(16))) float s_v[2][kAttnGroups][kAttnDim];
    const int64_t row = blockIdx.x;
    const int g = blockIdx.y;
    const int lane = threadIdx.x & 63;
    const int gi = threadIdx.x >> 4;
    const int li = lane & 15;
    const int64_t L = a.start + row + 1;
    const int64_t last = L - 1;
    const uint16_t* kbase = a.kcache + static_cast<int64_t>(g) * a.capacity * kAttnDim + 8 * li;
    const uint16_t* vbase = a.vcache + static_cast<int64_t>(g) * a.capacity * kAttnDim + 8 * li;

    float q[kAttnHeads][8];
#pragma unroll
    for (int hl = 0; hl < kAttnHeads; ++hl) {
        const uint4 qr = *reinterpret_cast<const uint4*>(a.q + row * 2048 + (g * kAttnHeads + hl) * kAttnDim + 8 * li);
        unpack8<Bf16>(qr, q[hl]);
    }
    const int sm_h = threadIdx.x / kAttnGroups;  // softmax threads (t < 256)
    const int sm_x = threadIdx.x % kAttnGroups;
    float m_run = -__builtin_huge_valf();
    float acc[2] = {0.0f, 0.0f};
    float l_run[2] = {0.0f, 0.0f};
    const int nround = static_cast<int>((L + kAttnGroups - 1) / kAttnGroups);
    int64_t t = gi < last ? gi : last;
    uint4 kA = *reinterpret_cast<const uint4*>(kbase + t * kAttnDim);
    uint4 vA = *reinterpret_cast<const uint4*>(vbase + t * kAttnDim);
    for (int r = 0; r < nround; ++r) {
        const int buf = r & 1;
        const int64_t base = static_cast<int64_t>(r) * kAttnGroups;
        const int nvalid = static_cast<int>(L - base < kAttnGroups ? L - base : kAttnGroups);
        t = base + kAttnGroups + gi < last ? base + kAttnGroups + gi : last;
        const uint4 kB = *reinterpret_cast<const uint4*>(kbase + t * kAttnDim);
        const uint4 vB = *reinterpret_cast<const uint4*>(vbase + t * kAttnDim);
        float kf[8], vf[8];
        unpack8<Bf16>(kA, kf);
        unpack8<Bf16>(vA, vf);
        float dots[kAttnHeads];
#pragma unroll
        for (int hl = 0; hl < kAttnHeads; ++hl) {
            float acc_d = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc_d = fmaf(q[hl][j], kf[j], acc_d);
            }
            dots[hl] = group16_sum(acc_d);
        }
        float mine = dots[0];
#pragma unroll
        for (int hl = 1; hl < kAttnHeads; ++hl) {
            mine = li == hl ? dots[hl] : mine;
        }
        if (li < kAttnHeads) {
            s_sc[buf][li][gi] = mine * a.qk_scale_log2;
        }
        float4* vrow = reinterpret_cast<float4*>(&s_v[buf][gi][8 * li]);
        vrow[0] = make_float4(vf[0], vf[1], vf[2], vf[3]);
        vrow[1] = make_float4(vf[4], vf[5], vf[6], vf[7]);
        __syncthreads();
        if (threadIdx.x < kAttnGroups * kAttnHeads) {
            float mr = -__builtin_huge_valf();
            for (int x = 0; x < nvalid; ++x) {
                mr = fmaxf(mr, s_sc[buf][sm_h][x]);
            }
            const float m_new = fmaxf(m_run, mr);
            s_w[buf][sm_h][sm_x] = sm_x < nvalid ? exp2_fixed(s_sc[buf][sm_h][sm_x] - m_new) : 0.0f;
            if (sm_x == 0) {
                s_corr[buf][sm_h] = exp2_fixed(m_run - m_new);
            }
            m_run = m_new;
        }
        __syncthreads();
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int hl = half * 4 + threadIdx.x / kAttnDim;
            const int d = threadIdx.x % kAttnDim;
            const float corr = s_corr[buf][hl];
            float av = acc[half] * corr;
            float lv = l_run[half] * corr;
            for (int x = 0; x < nvalid; ++x) {
                const float w = s_w[buf][hl][x];
                av = fmaf(w, s_v[buf][x][d], av);
                lv = lv + w;
            }
            acc[half] = av;
            l_run[half] = lv;
        }
        kA = kB;
        vA = vB;
    }
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const int hl = half * 4 + threadIdx.x / kAttnDim;
        const int d = threadIdx.x % kAttnDim;
        a.out[row * 2048 + (g * kAttnHeads + hl) * kAttnDim + d] = Bf16::store(acc[half] / l_run[half]);
    }
}

__global__ void set_step_kernel(int32_t* control, int32_t step) {
    if (threadIdx.x == 0) {
        control[0] = step;
    }
}

}  // namespace

hipError_t launch_set_step(int32_t* control, int32_t step, hipStream_t stream) {
    hipLaunchKernelGGL(set_step_kernel, dim3(1), dim3(64), 0, stream, control, step);
    return hipGetLastError();
}

hipError_t launch_prefill_norm(const PrefillNormArgs& a, hipStream_t stream) {
    if (a.m < 1 || a.gamma == nullptr || a.out == nullptr || (a.embed == nullptr && a.x == nullptr) ||
        (a.embed != nullptr && (a.tokens == nullptr || a.vocab < 1))) {
        return hipErrorInvalidValue;
    }
    const unsigned blocks = static_cast<unsigned>((a.m + kNormRowsPerBlock - 1) / kNormRowsPerBlock);
    hipLaunchKernelGGL(prefill_norm_kernel, dim3(blocks), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_prefill_rope_cache(const PrefillRopeArgs& a, hipStream_t stream) {
    if (a.m < 1 || a.start < 0 || a.start + a.m > a.capacity || a.q == nullptr || a.k == nullptr ||
        a.v == nullptr || a.kcache == nullptr || a.vcache == nullptr || a.rope_cos == nullptr ||
        a.rope_sin == nullptr) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(prefill_rope_cache_kernel, dim3(static_cast<unsigned>(a.m)), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t stream) {
    if (a.m < 1 || a.start < 0 || a.start + a.m > a.capacity || a.q == nullptr || a.kcache == nullptr ||
        a.vcache == nullptr || a.out == nullptr) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(static_cast<unsigned>(a.m), 2), dim3(512), 0, stream, a);
    return hipGetLastError();
}

}  // namespace kc
