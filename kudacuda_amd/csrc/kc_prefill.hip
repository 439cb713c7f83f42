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
