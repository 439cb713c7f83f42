// Multi-token prefill kernels for gfx950: the NF4 GEMM on MFMA matrix cores.
//
// out[m, n] = epilogue(sum_k x[m, k] * w[n, k]) with w[n, k] the NF4 weight
// dequantised to bf16 (bf16(codebook[code] * absmax), what bitsandbytes'
// dequantize-then-matmul feeds its GEMM; reference
// python/kudacuda_sidecar.py:1719-1738, kernels/common/nf4_device.cuh:10-40)
// and fp32 accumulation in v_mfma_f32_16x16x32_bf16.
//
// Tiling: each wave owns one 16-row weight fragment and all m <= 64 tokens
// (NT token tiles of 16, a template parameter so the window loop is
// straight-line code).  kBias / kResidual / kQkvRope / kResidualNorm: blocks
// of 4 waves own output rows [n0, n0 + 64).  kSwiGlu: blocks of 6 waves,
// waves 0..2 own gate rows [n0, n0 + 48) and waves 3..5 the same up rows; the
// up sums reach the gate waves through LDS for the epilogue.  A block's time
// is set by its CU's LDS and VALU work, so the 11008-row gate/up launch is
// one 6-wave block per CU (230 blocks; 4-wave blocks made 344, and the CUs
// that ran two of them set the launch's length: 64-token prefill
// 2.78 -> 2.72 ms).
//
// Operand layouts of the 16x16x32 bf16 MFMA (lane l, row l%16, group
// q = l/16): A[l%16][8q + j], B[8q + j][l%16], D[4q + i][l%16].  With
// A = weights (rows n) and B[k][m] = x[m][k], D[n][m] is the output tile.
// k is walked in windows of 128: lane group q owns the 32 contiguous k
// [128w + 32q, 128w + 32q + 32) of its weight row, read as one 16-byte load
// of codes (and one absmax: the 32 codes sit in one 64-block); MFMA step s of
// the window takes k = 128w + 32q + 8s + j from both operands, so every k of
// the window is summed exactly once (the order of k inside a product sum does
// not change what is summed).
//
// Activations: the block stages each window's x tile (16 NT rows x 128 k)
// in LDS once, with coalesced 16-byte loads (16 lanes cover one 256-byte row
// slice), rows padded to 272 bytes so that the MFMA operand reads
// (16 bytes per lane, lanes r = 0..7 of a group on distinct banks) do not
// conflict; the tile is double-buffered and the next window's x and weights
// are requested before the current window is computed.
//
// Few row tiles (n = 256 .. 2048) would leave most CUs idle, so K is split
// over a second grid dimension (each block sums a range of windows); the
// fp32 partial tiles are then summed in split order by gemm_reduce_kernel,
// which applies the epilogue.
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
constexpr int kXPitch = kWindow * 2 + 16;  // bytes per staged token row

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8, v); }

// One window's x requests of a thread, kept as one vector value (slots
// 4j..4j+3: its 16-byte piece of token row 16j + tid/16, bytes 16 (tid%16)
// of the row's window slice), and one window's weight requests of a lane
// (slots 0..3: 32 codes of its row, slot 4: their absmax bits).  Plain
// vector values stay in registers through the rotation below.
typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));

template <int NT>
__device__ __forceinline__ u32x16 x_fetch(const uint16_t* const* xrow, int xcol, int64_t kw) {
    u32x16 v = {};
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const uint4 t = *reinterpret_cast<const uint4*>(xrow[j] + kw + xcol);
        v[4 * j] = t.x;
        v[4 * j + 1] = t.y;
        v[4 * j + 2] = t.z;
        v[4 * j + 3] = t.w;
    }
    return v;
}

__device__ __forceinline__ u32x8 w_fetch(const uint8_t* wrow, const float* arow, int64_t kw, int q) {
    const int64_t kq = kw + 32 * q;
    const uint4 t = load_stream(reinterpret_cast<const uint4*>(wrow + kq / 2));  // read once: streamed
    u32x8 v = {};
    v[0] = t.x;
    v[1] = t.y;
    v[2] = t.z;
    v[3] = t.w;
    v[4] = __float_as_uint(arow[kq / 64]);
    return v;
}

template <int NT>
__device__ __forceinline__ void x_stage(uint8_t* buf, const u32x16& o, int tid) {
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        *reinterpret_cast<uint4*>(buf + (16 * j + tid / 16) * kXPitch + 16 * (tid % 16)) =
            make_uint4(o[4 * j], o[4 * j + 1], o[4 * j + 2], o[4 * j + 3]);
    }
}

// 8 codes of one 32-bit word (byte b: element 2b in the high nibble, 2b+1 in
// the low nibble) times absmax, each rounded to bf16 (round to nearest even,
// v_cvt_pk_bf16_f32; the products are finite); element j lands in slot j.
// lookup4 makes the table reads, scale8_bf16 the products.
// Both codes of byte b come from one 8-byte read of the LDS pair table, in
// the block's lane-sliced layout (SlicedLookup: the lane's slot of entry b,
// its address one byte permute; no bank conflicts).  Every prefill GEMM runs
// one block per CU, so its 64 KiB cost no residency: 64-token prefill
// 2.72 -> 2.65 ms against the 32 KiB 16-copy layout (bit-identical).
__device__ __forceinline__ void lookup4(float2* p, uint32_t word, const SlicedLookup& cb) {
    p[0] = *cb.template entry<0>(word);
    p[1] = *cb.template entry<1>(word);
    p[2] = *cb.template entry<2>(word);
    p[3] = *cb.template entry<3>(word);
}

__device__ __forceinline__ bf16x8 scale8_bf16(const float2* p, float am) {
    bf16x8 v;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        v[2 * b] = static_cast<__bf16>(p[b].x * am);
        v[2 * b + 1] = static_cast<__bf16>(p[b].y * am);
    }
    return v;
}

// The 16 table reads of one window's codes.
__device__ __forceinline__ void window_lookups(float2 (&p)[4][4], const u32x8& o, const SlicedLookup& cb) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        lookup4(p[s], o[s], cb);
    }
}

// One window from its table values `p` (read during the previous window):
// the window's 4 NT operand tiles are requested together and the first
// k-step's weights formed while they are in flight; each MFMA is then
// followed by one weight pair of the next k-step, so the products and
// conversions issue while the matrix core works; after the last MFMA `p`
// receives the next window's table reads (codes `on`), whose latency the
// block barrier that ends the window covers.  Reads issued and consumed a
// few at a time left the window a chain of ~25 dependent LDS round trips.
// Against all weights formed before the first MFMA with the next table reads
// ahead of the MFMAs: 64-token prefill 2.53 -> 2.48 ms on one box, ~0.5 % on
// two others (bit-identical).
template <int NT>
__device__ __forceinline__ void gemm_window(const uint8_t* buf, const u32x8& o, float2 (&p)[4][4], const u32x8& on,
                                            floatx4* acc, int r, int q, const SlicedLookup& cb) {
    const float am = __uint_as_float(o[4]);
    uint4 B[4][NT];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            B[s][t] = *reinterpret_cast<const uint4*>(buf + (16 * t + r) * kXPitch + 64 * q + 16 * s);
        }
    }
    bf16x8 A[4];
    A[0] = scale8_bf16(p[0], am);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            if (t < NT) {
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A[s], as_bf16x8(B[s][t]), acc[t], 0, 0, 0);
            }
            if (s < 3) {
                A[s + 1][2 * t] = static_cast<__bf16>(p[s + 1][t].x * am);
                A[s + 1][2 * t + 1] = static_cast<__bf16>(p[s + 1][t].y * am);
            }
            __builtin_amdgcn_sched_barrier(0);  // keeps each MFMA and its pair together
        }
    }
    window_lookups(p, on, cb);
    __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the x staging that follows
}

template <GemmEpi EPI, int NT, int W = kGemmWaves>
__global__ __launch_bounds__(64 * W) void nf4_gemm_kernel(Nf4GemmArgs a) {
    constexpr bool kSw = EPI == GemmEpi::kSwiGlu;
    static_assert(!kSw || W % 2 == 0, "gate and up waves in pairs");
    constexpr int kFrags = kSw ? W / 2 : W;                  // row fragments of the block per weight
    constexpr int kBlockRows = kFrags * kRowsPerWave;        // output rows of the block
    __shared__ __attribute__((aligned(16))) float s_cb[kNf4SlicedFloats];
    __shared__ __attribute__((aligned(16))) uint8_t s_x[2][16 * NT * kXPitch];
    const SlicedLookup cb = sliced_lookup(s_cb);
    static_assert(64 * W >= kNf4PairEntries, "one pair-table entry per thread");
    const float2 pair_entry = pair_entry_fetch();  // first request: its wait below waits for nothing else
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int tx = tid & 255;  // x staging: threads 256.. repeat the first 256 (same data, same place)
    const int r = lane & 15;
    const int q = lane >> 4;
    const int64_t K = a.k;
    const int M = static_cast<int>(a.m);  // 16 * (NT - 1) < M <= 16 * NT
    const int S = static_cast<int>(gridDim.y);
    const int64_t windows = K / kWindow;
    const int64_t per_split = (windows + S - 1) / S;
    const int64_t k_begin = static_cast<int64_t>(blockIdx.y) * per_split * kWindow;
    const int64_t k_end = k_begin + per_split * kWindow < K ? k_begin + per_split * kWindow : K;
    // this wave's fragment: f = 0 (gate or plain) / 1 (up), first output
    // column n0w; kQkvRope: the block's 64 rows lie in the q, k or v weight
    // (segment boundaries are multiples of 64), row0 is the row in it.  A
    // fragment past the last row (the last block of a 48-row gate/up split)
    // computes the last fragment again and stores nothing.
    const int f = kSw ? wave / kFrags : 0;
    const int frag = kSw ? wave % kFrags : wave;
    const int64_t n0w = static_cast<int64_t>(blockIdx.x) * kBlockRows + frag * kRowsPerWave;
    const bool live = n0w < a.n;
    int seg = f;
    int64_t row0 = live ? n0w : a.n - kRowsPerWave;
    if constexpr (EPI == GemmEpi::kQkvRope) {
        seg = n0w < a.q_rows ? 0 : (n0w < a.q_rows + a.kv_rows ? 1 : 2);
        row0 = n0w - (seg == 0 ? 0 : (seg == 1 ? a.q_rows : a.q_rows + a.kv_rows));
    }
    const uint8_t* wrow = a.w[seg] + (row0 + r) * (K / 2);  // every row exists (multiples of 64)
    const float* arow = a.absmax[seg] + (row0 + r) * (K / 64);
    // x rows this thread stages (rows past m re-read row m - 1; never used)
    const uint16_t* xrow[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int m = 16 * j + tx / 16 < M ? 16 * j + tx / 16 : M - 1;
        xrow[j] = a.x + static_cast<int64_t>(m) * K;
    }
    const int xcol = 8 * (tx % 16);

    floatx4 acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        acc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // x and weights are requested two windows ahead into three register
    // slots that rotate through the unrolled loop; x of window w + 1 is
    // staged into the other LDS buffer while window w is computed, and only
    // waits for requests older than the ones just issued.  Requests past the
    // split's last window are clamped to a window of the split, never used.
    constexpr int kBuf = 16 * NT * kXPitch;
    uint8_t* const sx = &s_x[0][0];
    const int64_t k1 = k_begin + kWindow < k_end ? k_begin + kWindow : k_begin;
    u32x16 x0 = x_fetch<NT>(xrow, xcol, k_begin);
    u32x8 w0 = w_fetch(wrow, arow, k_begin, q);
    u32x16 x1 = x_fetch<NT>(xrow, xcol, k1);
    u32x8 w1 = w_fetch(wrow, arow, k1, q);
    u32x16 x2;
    u32x8 w2;
    x_stage<NT>(sx, x0, tx);
    sliced_entry_store(s_cb, pair_entry);
    __syncthreads();
    float2 p[4][4];  // table values of the window about to be computed
    window_lookups(p, w0, cb);
    int buf = 0;
    int64_t kw = k_begin;
#define KC_GEMM_STEP(XF, WF, WC, WN, XS)                                           \
    {                                                                              \
        const int64_t kf = kw + 2 * kWindow < k_end ? kw + 2 * kWindow : kw;       \
        XF = x_fetch<NT>(xrow, xcol, kf);                                          \
        WF = w_fetch(wrow, arow, kf, q);                                           \
        __builtin_amdgcn_sched_barrier(0); /* requests ahead of the compute */     \
        gemm_window<NT>(sx + buf * kBuf, WC, p, WN, acc, r, q, cb);                \
        x_stage<NT>(sx + (buf ^ 1) * kBuf, XS, tx);                                \
        __syncthreads();                                                           \
        buf ^= 1;                                                                  \
        kw += kWindow;                                                             \
        if (kw >= k_end) {                                                         \
            break;                                                                 \
        }                                                                          \
    }
    while (true) {
        KC_GEMM_STEP(x2, w2, w0, w1, x1)
        KC_GEMM_STEP(x0, w0, w1, w2, x2)
        KC_GEMM_STEP(x1, w1, w2, w0, x0)
    }
#undef KC_GEMM_STEP

    // D[4q + i][r]: rows n0w + 4q + i, token 16t + r; four consecutive rows
    // per lane go out as one store
    if (S > 1) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int m = 16 * t + r;
            if (m < M && live) {
                float* dst = a.partials + ((static_cast<int64_t>(f) * S + blockIdx.y) * M + m) * a.n + n0w + 4 * q;
                *reinterpret_cast<float4*>(dst) = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
            }
        }
        return;
    }
    if constexpr (EPI == GemmEpi::kQkvRope || EPI == GemmEpi::kResidualNorm) {
        return;  // always split: the epilogue is in the split reduce
    }
    floatx4 up[NT];
    if constexpr (kSw) {
        // the up waves hand their sums to the gate waves of the same rows
        // (the staging buffers are free: the loop ended on a barrier)
        floatx4* s_up = reinterpret_cast<floatx4*>(&s_x[0][0]);
        if (f == 1) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                s_up[(frag * NT + t) * 64 + lane] = acc[t];
            }
        }
        __syncthreads();
        if (f == 1) {
            return;
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            up[t] = s_up[(frag * NT + t) * 64 + lane];
        }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int m = 16 * t + r;
        if (m >= M || !live) {
            continue;
        }
        const int64_t nb = n0w + 4 * q;
        uint16_t* dst = a.out + static_cast<int64_t>(m) * a.n + nb;
        uint32_t packed[2];
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
            uint16_t h[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int i = 2 * i2 + e;
                float v = acc[t][i];
                if constexpr (EPI == GemmEpi::kBias) {
                    if (a.bias != nullptr) {
                        v = v + Bf16::load(a.bias[nb + i]);
                    }
                    h[e] = Bf16::store(v);
                } else if constexpr (EPI == GemmEpi::kResidual) {
                    const float res = Bf16::load(a.residual[static_cast<int64_t>(m) * a.n + nb + i]);
                    h[e] = Bf16::store(res + Bf16::load(Bf16::store(v)));
                } else {
                    h[e] = Bf16::store(silu_fixed(v) * up[t][i]);
                }
            }
            packed[i2] = static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16);
        }
        *reinterpret_cast<uint2*>(dst) = make_uint2(packed[0], packed[1]);
    }
}

// Sum of the S split partials of V consecutive floats at `src` (splits
// `plane` floats apart) in split order.  The loads of up to 8 splits are
// issued together (split index clamped; the clamped repeats are not added),
// so S splits cost ceil((S - 1) / 8) memory round trips instead of S - 1.
template <int V>
__device__ __forceinline__ void split_sum(const float* src, int64_t plane, int S, float* out) {
    typedef float vec __attribute__((ext_vector_type(V)));
    vec acc = *reinterpret_cast<const vec*>(src);
    for (int s0 = 1; s0 < S; s0 += 8) {
        vec p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int s = s0 + j < S ? s0 + j : S - 1;
            p[j] = *reinterpret_cast<const vec*>(src + s * plane);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (s0 + j < S) {
#pragma unroll
                for (int i = 0; i < V; ++i) {
                    acc[i] = acc[i] + p[j][i];
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < V; ++i) {
        out[i] = acc[i];
    }
}

// One thread per 4 consecutive outputs of one token: the split partials are
// summed in split order (fp32), then the GEMM's epilogue.
template <GemmEpi EPI>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(Nf4GemmArgs a, int S) {
    constexpr int NF = EPI == GemmEpi::kSwiGlu ? 2 : 1;
    const int64_t quads = a.m * a.n / 4;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= quads) {
        return;
    }
    const int64_t m = idx / (a.n / 4);
    const int64_t nb = (idx % (a.n / 4)) * 4;
    float v[NF][4];
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        const float* src = a.partials + (static_cast<int64_t>(f) * S * a.m + m) * a.n + nb;
        split_sum<4>(src, a.m * a.n, S, v[f]);
    }
    uint16_t h[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (EPI == GemmEpi::kBias) {
            h[i] = Bf16::store(a.bias != nullptr ? v[0][i] + Bf16::load(a.bias[nb + i]) : v[0][i]);
        } else if constexpr (EPI == GemmEpi::kResidual) {
            const float res = Bf16::load(a.residual[m * a.n + nb + i]);
            h[i] = Bf16::store(res + Bf16::load(Bf16::store(v[0][i])));
        } else {
            h[i] = Bf16::store(silu_fixed(v[0][i]) * v[NF - 1][i]);
        }
    }
    *reinterpret_cast<uint2*>(a.out + m * a.n + nb) =
        make_uint2(static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16),
                   static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16));
}

// kQkvRope epilogue.  Per token, thread u handles (d, d + 1) and their RoPE
// partners (d + 64, d + 65) of one q head (u < q_rows / 4) or k head (next
// kv_rows / 4), or 4 consecutive v values (last kv_rows / 4): split partials
// summed in split order, bias added in fp32 and the sum rounded to bf16 (the
// plain kBias epilogue), then the rotation in fp32 from the bf16 values,
// rounded again.  Rotated q goes to out [m, q_rows], rotated k and v to the
// caches at position start + row.
__global__ __launch_bounds__(256) void qkv_rope_reduce_kernel(Nf4GemmArgs a, int S) {
    const int64_t per_row = (a.q_rows + 2 * a.kv_rows) / 4;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= a.m * per_row) {
        return;
    }
    const int64_t m = idx / per_row;
    const int64_t u = idx % per_row;
    const int64_t pos = a.start + m;
    const int64_t q_units = a.q_rows / 4;
    const int64_t k_units = a.kv_rows / 4;
    const float* src = a.partials + m * a.n;
    const int64_t plane = a.m * a.n;
    if (u >= q_units + k_units) {
        const int64_t c = a.q_rows + a.kv_rows + 4 * (u - q_units - k_units);  // v column
        const int64_t cv = c - a.q_rows - a.kv_rows;
        // the bias is read unconditionally (a stand-in address when there is
        // none) so that its request goes out with the partials'
        const uint16_t* b = a.seg_bias[2];
        const uint2 braw = *reinterpret_cast<const uint2*>(b != nullptr ? b + cv : a.x);
        float vs[4];
        split_sum<4>(src + c, plane, S, vs);
        const uint16_t bb[4] = {static_cast<uint16_t>(braw.x), static_cast<uint16_t>(braw.x >> 16),
                                static_cast<uint16_t>(braw.y), static_cast<uint16_t>(braw.y >> 16)};
        uint16_t h[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h[i] = Bf16::store(b != nullptr ? vs[i] + Bf16::load(bb[i]) : vs[i]);
        }
        uint16_t* dst = a.vcache + ((cv / 128) * a.capacity + pos) * 128 + cv % 128;
        *reinterpret_cast<uint2*>(dst) = make_uint2(static_cast<uint32_t>(h[0]) | (static_cast<uint32_t>(h[1]) << 16),
                                                    static_cast<uint32_t>(h[2]) | (static_cast<uint32_t>(h[3]) << 16));
        return;
    }
    const bool is_q = u < q_units;
    const int64_t uu = is_q ? u : u - q_units;
    const int64_t head = uu / 32;
    const int d = static_cast<int>(uu % 32) * 2;
    const int64_t c0 = (is_q ? 0 : a.q_rows) + head * 128 + d;  // partial column of (d, d + 1)
    const uint16_t* b = is_q ? a.seg_bias[0] : a.seg_bias[1];
    const int64_t cb0 = head * 128 + d;  // column within the segment
    // bias (a stand-in address when there is none) and rotary factors are
    // requested with the partials, not after them
    const uint32_t blo = *reinterpret_cast<const uint32_t*>(b != nullptr ? b + cb0 : a.x);
    const uint32_t bhi = *reinterpret_cast<const uint32_t*>(b != nullptr ? b + cb0 + 64 : a.x);
    const float2 cs = *reinterpret_cast<const float2*>(a.rope_cos + pos * 64 + d);
    const float2 sn = *reinterpret_cast<const float2*>(a.rope_sin + pos * 64 + d);
    float lov[2], hiv[2];
    split_sum<2>(src + c0, plane, S, lov);
    split_sum<2>(src + c0 + 64, plane, S, hiv);
    const float2 lo = make_float2(lov[0], lov[1]);
    const float2 hi = make_float2(hiv[0], hiv[1]);
    const bool hb = b != nullptr;
    const float l0 = Bf16::load(Bf16::store(hb ? lo.x + Bf16::load(static_cast<uint16_t>(blo)) : lo.x));
    const float l1 = Bf16::load(Bf16::store(hb ? lo.y + Bf16::load(static_cast<uint16_t>(blo >> 16)) : lo.y));
    const float h0 = Bf16::load(Bf16::store(hb ? hi.x + Bf16::load(static_cast<uint16_t>(bhi)) : hi.x));
    const float h1 = Bf16::load(Bf16::store(hb ? hi.y + Bf16::load(static_cast<uint16_t>(bhi >> 16)) : hi.y));
    const float c_0 = cs.x;
    const float c_1 = cs.y;
    const float s_0 = sn.x;
    const float s_1 = sn.y;
    const uint32_t rl = static_cast<uint32_t>(Bf16::store((l0 * c_0) - (h0 * s_0))) |
                        (static_cast<uint32_t>(Bf16::store((l1 * c_1) - (h1 * s_1))) << 16);
    const uint32_t rh = static_cast<uint32_t>(Bf16::store((h0 * c_0) + (l0 * s_0))) |
                        (static_cast<uint32_t>(Bf16::store((h1 * c_1) + (l1 * s_1))) << 16);
    uint16_t* dst = is_q ? a.out + m * a.q_rows + head * 128 + d : a.kcache + (head * a.capacity + pos) * 128 + d;
    *reinterpret_cast<uint32_t*>(dst) = rl;
    *reinterpret_cast<uint32_t*>(dst + 64) = rh;
}

// kResidualNorm epilogue: one block per token row of 2048, thread t owns
// columns 8t..8t+7.  Split partials summed in split order, the residual
// epilogue bf16(res + bf16(sum)) written back to out, then (with norm_gamma)
// the row's RMSNorm: fp32 sum of squares of the new bf16 row (8 fmaf per
// thread, wave butterfly, the 4 wave sums (w0 + w1) + (w2 + w3)), the decode
// kernels' inv_rms and bf16((h * inv) * gamma) into norm_out.
__global__ __launch_bounds__(256) void residual_norm_reduce_kernel(Nf4GemmArgs a, int S) {
    __shared__ float s_ss[4];
    const int64_t m = blockIdx.x;
    const int t = threadIdx.x;
    const int64_t c = 8 * t;
    const float* src = a.partials + m * a.n + c;
    const int64_t plane = a.m * a.n;
    // residual and gamma (the residual again when there is no norm) are
    // requested with the partials, so no load waits behind the barrier below
    const uint4 rv = *reinterpret_cast<const uint4*>(a.residual + m * a.n + c);
    const uint4 gv = *reinterpret_cast<const uint4*>(a.norm_gamma != nullptr ? a.norm_gamma + c : a.residual + m * a.n + c);
    float v[8];
    split_sum<8>(src, plane, S, v);
    float res[8];
    unpack8<Bf16>(rv, res);
    float h[8];
    uint32_t packed[4];
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const uint16_t lo = Bf16::store(res[i] + Bf16::load(Bf16::store(v[i])));
        const uint16_t hi = Bf16::store(res[i + 1] + Bf16::load(Bf16::store(v[i + 1])));
        h[i] = Bf16::load(lo);
        h[i + 1] = Bf16::load(hi);
        packed[i / 2] = static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
    }
    *reinterpret_cast<uint4*>(a.out + m * a.n + c) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    if (a.norm_gamma == nullptr) {
        return;
    }
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        ss = fmaf(h[i], h[i], ss);
    }
    ss = wave_sum(ss);
    if ((t & 63) == 0) {
        s_ss[t >> 6] = ss;
    }
    __syncthreads();
    const float r = inv_rms((s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]), 2048.0f, a.eps);
    float g[8];
    unpack8<Bf16>(gv, g);
#pragma unroll
    for (int i = 0; i < 8; i += 2) {
        const uint32_t lo = Bf16::store((h[i] * r) * g[i]);
        const uint32_t hi = Bf16::store((h[i + 1] * r) * g[i + 1]);
        packed[i / 2] = lo | (hi << 16);
    }
    *reinterpret_cast<uint4*>(a.norm_out + m * a.n + c) = make_uint4(packed[0], packed[1], packed[2], packed[3]);
}

template <GemmEpi EPI>
hipError_t launch_gemm_epi(const Nf4GemmArgs& a, hipStream_t stream) {
    constexpr int NF = EPI == GemmEpi::kSwiGlu ? 2 : 1;
    int64_t S = 1;
    if (a.partials != nullptr) {
        // (kQkvRope: at least 2, its epilogue is the split reduce)
        // ~1024 waves: one 16-row fragment per wave, K windows split over blocks
        const int64_t row_waves = NF * a.n / kRowsPerWave;
        const int64_t windows = a.k / kWindow;
        S = (1024 + row_waves - 1) / row_waves;
        S = S < windows ? S : windows;
        S = S < 64 ? S : 64;
        while (S > 1 && NF * S * a.m * a.n > a.partial_floats) {
            --S;
        }
        if ((EPI == GemmEpi::kQkvRope || EPI == GemmEpi::kResidualNorm) && S < 2) {
            S = 2;
        }
        if (S > 1) {
            const int64_t per_split = (windows + S - 1) / S;
            S = (windows + per_split - 1) / per_split;  // no empty split
        }
    }
    if constexpr (EPI == GemmEpi::kSwiGlu) {
        // 6-wave blocks of 48 gate + 48 up rows: 11008 rows make 230 blocks,
        // one per CU (4-wave blocks made 344, so a third of the CUs ran two)
        constexpr int kSwWaves = 6;
        constexpr int64_t kSwRows = kSwWaves / 2 * kRowsPerWave;
        const dim3 grid(static_cast<unsigned>((a.n + kSwRows - 1) / kSwRows), static_cast<unsigned>(S));
        const dim3 block(64 * kSwWaves);
        switch ((a.m + 15) / 16) {
            case 1:
                hipLaunchKernelGGL((nf4_gemm_kernel<EPI, 1, kSwWaves>), grid, block, 0, stream, a);
                break;
            case 2:
                hipLaunchKernelGGL((nf4_gemm_kernel<EPI, 2, kSwWaves>), grid, block, 0, stream, a);
                break;
            case 3:
                hipLaunchKernelGGL((nf4_gemm_kernel<EPI, 3, kSwWaves>), grid, block, 0, stream, a);
                break;
            default:
                hipLaunchKernelGGL((nf4_gemm_kernel<EPI, kTokenTiles, kSwWaves>), grid, block, 0, stream, a);
                break;
        }
    } else {
        const dim3 grid(static_cast<unsigned>(a.n / kRowsPerBlock), static_cast<unsigned>(S));
        switch ((a.m + 15) / 16) {
            case 1:
                hipLaunchKernelGGL((nf4_gemm_kernel<EPI, 1>), grid, dim3(kGemmThreads), 0, stream, a);
                break;
            case 2:
                hipLaunchKernelGGL((nf4_gemm_kernel<EPI, 2>), grid, dim3(kGemmThreads), 0, stream, a);
                break;
            case 3:
                hipLaunchKernelGGL((nf4_gemm_kernel<EPI, 3>), grid, dim3(kGemmThreads), 0, stream, a);
                break;
            default:
                hipLaunchKernelGGL((nf4_gemm_kernel<EPI, kTokenTiles>), grid, dim3(kGemmThreads), 0, stream, a);
                break;
        }
    }
    hipError_t status = hipGetLastError();
    if (status != hipSuccess || S == 1) {
        return status;
    }
    const int64_t quads = a.m * a.n / 4;
    if constexpr (EPI == GemmEpi::kQkvRope) {
        hipLaunchKernelGGL(qkv_rope_reduce_kernel, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                           stream, a, static_cast<int>(S));
    } else if constexpr (EPI == GemmEpi::kResidualNorm) {
        hipLaunchKernelGGL(residual_norm_reduce_kernel, dim3(static_cast<unsigned>(a.m)), dim3(256), 0, stream, a,
                           static_cast<int>(S));
    } else {
        hipLaunchKernelGGL(gemm_reduce_kernel<EPI>, dim3(static_cast<unsigned>((quads + 255) / 256)), dim3(256), 0,
                           stream, a, static_cast<int>(S));
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_nf4_gemm(GemmEpi epi, const Nf4GemmArgs& a, hipStream_t stream) {
    if (a.m < 1 || a.m > kGemmMaxTokens || a.n < kRowsPerBlock || a.n % kRowsPerBlock != 0 || a.k < kWindow ||
        a.k % kWindow != 0 || a.x == nullptr || a.w[0] == nullptr || a.absmax[0] == nullptr || a.out == nullptr ||
        (epi == GemmEpi::kSwiGlu && (a.w[1] == nullptr || a.absmax[1] == nullptr)) ||
        ((epi == GemmEpi::kResidual || epi == GemmEpi::kResidualNorm) && a.residual == nullptr)) {
        return hipErrorInvalidValue;
    }
    if (epi == GemmEpi::kResidualNorm &&
        (a.partials == nullptr || a.n != 2048 || 2 * a.m * a.n > a.partial_floats ||
         (a.norm_gamma != nullptr && a.norm_out == nullptr))) {
        return hipErrorInvalidValue;
    }
    // the split-only epilogues need two windows at least (two splits)
    if ((epi == GemmEpi::kQkvRope || epi == GemmEpi::kResidualNorm) && a.k < 2 * kWindow) {
        return hipErrorInvalidValue;
    }
    if (epi == GemmEpi::kQkvRope &&
        (a.partials == nullptr || a.q_rows < 128 || a.q_rows % 128 != 0 || a.kv_rows < 128 || a.kv_rows % 128 != 0 ||
         a.n != a.q_rows + 2 * a.kv_rows || a.w[1] == nullptr || a.w[2] == nullptr || a.absmax[1] == nullptr ||
         a.absmax[2] == nullptr || a.rope_cos == nullptr || a.rope_sin == nullptr || a.kcache == nullptr ||
         a.vcache == nullptr || a.start < 0 || a.start + a.m > a.capacity ||
         2 * a.m * a.n > a.partial_floats)) {
        return hipErrorInvalidValue;
    }
    switch (epi) {
        case GemmEpi::kBias:
            return launch_gemm_epi<GemmEpi::kBias>(a, stream);
        case GemmEpi::kResidual:
            return launch_gemm_epi<GemmEpi::kResidual>(a, stream);
        case GemmEpi::kSwiGlu:
            return launch_gemm_epi<GemmEpi::kSwiGlu>(a, stream);
        case GemmEpi::kQkvRope:
            return launch_gemm_epi<GemmEpi::kQkvRope>(a, stream);
        case GemmEpi::kResidualNorm:
            return launch_gemm_epi<GemmEpi::kResidualNorm>(a, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace kc

// ---------------------------------------------------------------------------
// Row norm and causal attention of the prefill.
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
constexpr int kAttnGroups = 32;  // 16-lane groups of a 512-thread block
constexpr int kAttnHeads = 8;    // query heads per KV head
constexpr int kAttnBlockHeads = 4;
constexpr int kAttnDim = 128;

// grid (m, 2 KV heads, 2 head halves), 512 threads.  Query row r (position
// start + r) of query heads 4z .. 4z + 3 of KV head g (8 per KV head; each
// head's arithmetic is independent of the others', so halving the heads per
// block doubles the blocks -- 256 for 64 tokens -- and leaves every result as
// it was) over cache rows [0, start + r], in rounds of 32 tokens
// (one per 16-lane group): scores by 8-dim partial dots and the 16-lane DPP
// butterfly (log2 domain), then per head m_new = max(m, round max), weights
// exp2(s - m_new), rescale exp2(m - m_new) of the running sum and accumulator,
// weighted V rows from LDS in token order.  out = bf16(acc / sum).
__global__ __launch_bounds__(512) void prefill_attention_kernel(PrefillAttnArgs a) {
    constexpr int H = kAttnBlockHeads;
    static_assert(H * kAttnDim == 512, "one thread per (head, dim) in the weighted sum");
    __shared__ __attribute__((aligned(16))) float s_sc[2][H][kAttnGroups];
    __shared__ __attribute__((aligned(16))) float s_w[2][H][kAttnGroups];
    __shared__ float s_corr[2][H];
    __shared__ __attribute__((aligned(16))) float s_v[2][kAttnGroups][kAttnDim];
    const int64_t row = blockIdx.x;
    const int g = blockIdx.y;
    const int h0 = g * kAttnHeads + static_cast<int>(blockIdx.z) * H;  // first query head of the block
    const int lane = threadIdx.x & 63;
    const int gi = threadIdx.x >> 4;
    const int li = lane & 15;
    const int64_t L = a.start + row + 1;
    const int64_t last = L - 1;
    const uint16_t* kbase = a.kcache + static_cast<int64_t>(g) * a.capacity * kAttnDim + 8 * li;
    const uint16_t* vbase = a.vcache + static_cast<int64_t>(g) * a.capacity * kAttnDim + 8 * li;

    float q[H][8];
#pragma unroll
    for (int hl = 0; hl < H; ++hl) {
        const uint4 qr = *reinterpret_cast<const uint4*>(a.q + row * 2048 + (h0 + hl) * kAttnDim + 8 * li);
        unpack8<Bf16>(qr, q[hl]);
    }
    const int sm_h = threadIdx.x / kAttnGroups;  // softmax threads (t < 128)
    const int sm_x = threadIdx.x % kAttnGroups;
    float m_run = -__builtin_huge_valf();
    float acc = 0.0f;
    float l_run = 0.0f;
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
        float dots[H];
#pragma unroll
        for (int hl = 0; hl < H; ++hl) {
            float acc_d = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                acc_d = fmaf(q[hl][j], kf[j], acc_d);
            }
            dots[hl] = group16_sum(acc_d);
        }
        float mine = dots[0];
#pragma unroll
        for (int hl = 1; hl < H; ++hl) {
            mine = li == hl ? dots[hl] : mine;
        }
        if (li < H) {
            s_sc[buf][li][gi] = mine * a.qk_scale_log2;
        }
        float4* vrow = reinterpret_cast<float4*>(&s_v[buf][gi][8 * li]);
        vrow[0] = make_float4(vf[0], vf[1], vf[2], vf[3]);
        vrow[1] = make_float4(vf[4], vf[5], vf[6], vf[7]);
        __syncthreads();
        if (threadIdx.x < kAttnGroups * H) {
            // the round's maximum per head: a 32-lane butterfly over the
            // head's softmax threads (a maximum is exact in any order)
            const float sc = s_sc[buf][sm_h][sm_x];
            float mr = sm_x < nvalid ? sc : -__builtin_huge_valf();
#pragma unroll
            for (int o = 16; o >= 1; o >>= 1) {
                mr = fmaxf(mr, __shfl_xor(mr, o, kAttnGroups));
            }
            const float m_new = fmaxf(m_run, mr);
            s_w[buf][sm_h][sm_x] = sm_x < nvalid ? exp2_fixed(sc - m_new) : 0.0f;
            if (sm_x == 0) {
                s_corr[buf][sm_h] = exp2_fixed(m_run - m_new);
            }
            m_run = m_new;
        }
        __syncthreads();
        {
            const int hl = threadIdx.x / kAttnDim;
            const int d = threadIdx.x % kAttnDim;
            const float corr = s_corr[buf][hl];
            float av = acc * corr;
            float lv = l_run * corr;
            for (int x = 0; x < nvalid; ++x) {
                const float w = s_w[buf][hl][x];
                av = fmaf(w, s_v[buf][x][d], av);
                lv = lv + w;
            }
            acc = av;
            l_run = lv;
        }
        kA = kB;
        vA = vB;
    }
    {
        const int hl = threadIdx.x / kAttnDim;
        const int d = threadIdx.x % kAttnDim;
        a.out[row * 2048 + (h0 + hl) * kAttnDim + d] = Bf16::store(acc / l_run);
    }
}

// A prefill starts a generation: step = its last prompt position, stop state
// cleared (control[4] done flag, control[5] stop position).
__global__ void set_step_kernel(int32_t* control, int32_t step) {
    if (threadIdx.x == 0) {
        control[0] = step;
        control[4] = 0;
        control[5] = 0;
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

hipError_t launch_prefill_attention(const PrefillAttnArgs& a, hipStream_t stream) {
    if (a.m < 1 || a.start < 0 || a.start + a.m > a.capacity || a.q == nullptr || a.kcache == nullptr ||
        a.vcache == nullptr || a.out == nullptr) {
        return hipErrorInvalidValue;
    }
    hipLaunchKernelGGL(prefill_attention_kernel, dim3(static_cast<unsigned>(a.m), 2, kAttnHeads / kAttnBlockHeads),
                       dim3(512), 0, stream, a);
    return hipGetLastError();
}

}  // namespace kc
