// NF4 kernels for gfx950: blockwise quantise / dequantise, the K = 2048 row
// family (GEMV, fused RMSNorm+QKV(+bias), fused QKV+RoPE+KV-cache write,
// fused gate/up SwiGLU) and the K = 11008 down projection.
//
// Design (wave64, bandwidth-bound, no MFMA because M = 1):
//  * one wave owns a whole 2048-wide row: lane l streams the 16 packed bytes
//    of chunk l with one 128-bit load, so a wave load is one contiguous
//    1 KiB row (fully coalesced) and the lane's 32 activations stay in
//    registers for every row the wave visits;
//  * codes are looked up in a block-shared LDS table of code pairs (one
//    8-byte entry per byte value), one byte-select shift per byte; gate/up,
//    with one large block per CU, reads a lane-sliced copy (32 interleaved
//    copies, one byte permute per byte) whose lookups never share a bank;
//  * the RMSNorm is computed inside the consumer kernel: waves 0..3 of a
//    block each normalise a quarter into LDS and every wave of the block
//    (4, 7 in QKV+RoPE, 11 in gate/up) reads it, so no separate norm launch is needed;
//  * loads are issued in dependency order (activations, epilogue operands,
//    rows), and a gate/up wave requests task i + 1's rows only once task
//    i's have arrived, then computes task i (a wave stalled on a full memory
//    queue stops in order, its arithmetic with it);
//  * reductions are wave64 butterflies on lane-swap and DPP instructions,
//    two rows per chain.
// Semantics follow the reference's tiled NF4 kernels
// (kernels/common/nf4_tiled_gemv.cuh:61-168: norm in fp32, dot in fp32,
// bias added in fp32 before the single output rounding) and its SwiGLU
// (kernels/common/nf4_swiglu_bf16.cuh:61-164: silu(g) * u in fp32).
#include <utility>

#include "kc_device.h"
#include "kc_kernels.h"

namespace kc {
namespace {

constexpr int kRowsThreads = 256;
// gate/up blocks: 11 waves, of which waves 0..3 compute the shared norm and
// the rest only read it; 4 tasks per wave (kSwiGluWaves waves in all), so
// ~251 blocks give about one block and 43 tasks per CU.  Measured in step
// shape against 12-wave blocks of 2 tasks (8.76 -> 8.05 us) and 12-wave
// blocks of 4 tasks (8.2 us).
constexpr int kSwiGluThreads = 704;
constexpr int64_t kSwiGluWaves = 2816;
// QKV+RoPE blocks: 7 waves (waves 0..3 compute the shared norm, 4..6 read
// it), ~183 blocks.  Decode step, 10 interleaved runs of 128 steps on each of
// two boxes: 1.1191 ms against 1.1215 for 4-wave blocks (5, 6, 8, 9 waves:
// 1.1225, 1.1222, 1.1322, 1.1266).
constexpr int kQkvRopeThreads = 448;
constexpr int kNormPitch = 36;  // floats per lane row of the shared norm (32 + 4: conflict-free)
// Launch cap of the other row kernels (GEMV, QKV): up to 6144 waves (24 per
// CU on 256 CUs), one task per wave at the model's shapes; measured faster
// than fewer waves with more tasks each there.
constexpr int64_t kMaxRowWaves = 6144;

// Decision points between adjacent codebook values: fp32 of the fp64
// midpoint.  A scaled value s maps to the number of midpoints it exceeds, so
// an exact tie goes to the lower code.
__device__ constexpr float kNf4Mid[15] = {
    -0x1.b239b0p-1f, -0x1.38a4e0p-1f, -0x1.d70900p-2f, -0x1.5bd4ecp-2f, -0x1.e079d8p-3f,
    -0x1.1a7178p-3f, -0x1.74f0e2p-5f, 0x1.45f5fep-5f,  0x1.ec90c4p-4f,  0x1.a0cfc0p-3f,
    0x1.2b05a8p-2f,  0x1.8ea7f2p-2f,  0x1.00da08p-1f,  0x1.491b5ep-1f,  0x1.b913b4p-1f,
};

struct RowPair {
    int m0 = 0, m1 = 0;      // matrix index of each row
    int64_t r0 = 0, r1 = 0;  // row within its matrix
    bool has1 = false;
};

template <RowMode MODE>
__device__ __forceinline__ RowPair map_task(const Nf4RowsArgs& a, int64_t task) {
    RowPair p;
    if constexpr (MODE == RowMode::kGemv) {
        p.r0 = 2 * task;
        p.r1 = 2 * task + 1;
        p.has1 = p.r1 < a.rows[0];
    } else if constexpr (MODE == RowMode::kSwiGlu) {
        p.m0 = 0;
        p.m1 = 1;
        p.r0 = task;
        p.r1 = task;
        p.has1 = true;
    } else {
        // Q, K, V rows paired as (d, d + 64) inside each 128-row head so the
        // rotary rotation of a pair happens in registers.
        int64_t j = task;
        int m = 0;
        while (m < 2 && j >= a.rows[m] / 2) {
            j -= a.rows[m] / 2;
            ++m;
        }
        const int64_t head = j / 64;
        const int64_t d = j % 64;
        p.m0 = m;
        p.m1 = m;
        p.r0 = head * 128 + d;
        p.r1 = head * 128 + d + 64;
        p.has1 = true;
    }
    return p;
}

// Entry m of a three-pointer field by selects: the kernel's argument struct
// is a local copy (its leading pointers come preloaded), and a runtime index
// into one of its arrays would put the whole copy in scratch memory.
template <typename P>
__device__ __forceinline__ P pick3(const P (&arr)[3], int m) {
    return m == 0 ? arr[0] : (m == 1 ? arr[1] : arr[2]);
}

__device__ __forceinline__ void fetch_row(const Nf4RowsArgs& a, int m, int64_t r, int lane, uint4& pk, float& am) {
    pk = load_stream(reinterpret_cast<const uint4*>(pick3(a.w, m) + r * 1024) + lane);
    am = load_stream(pick3(a.absmax, m) + r * 32 + (lane >> 1));
}

// wx[x] = lane x's value of every lane's 16-lane row, for x in X
template <int... X>
__device__ __forceinline__ void row_bcast_all(float v, float* wx, std::integer_sequence<int, X...>) {
    ((wx[X] = row_bcast<X>(v)), ...);
}

// Small per-task operands of the epilogue (bias, residual, rotary
// cos/sin), loaded with the weights so the epilogue itself never waits on
// memory.  Every lane loads the same addresses (one request per wave); lane 0
// (and lane 1 for a GEMV pair) uses them.
struct Epi {
    uint16_t b0 = 0, b1 = 0;  // bias (GEMV: lane's bias) raw 16-bit
    uint16_t res = 0;         // GEMV residual of the lane's row
    float c = 1.0f, s = 0.0f; // rotary cos/sin
};

template <typename T, RowMode MODE>
__device__ __forceinline__ Epi fetch_epilogue(const Nf4RowsArgs& a, const RowPair& p, int lane, int64_t pos) {
    Epi e;
    if constexpr (MODE == RowMode::kGemv) {
        const int64_t r = (lane == 1 && p.has1) ? p.r1 : p.r0;
        // null operands read x[0] instead (always valid) and are ignored
        const uint16_t* bias = a.bias[0] != nullptr ? a.bias[0] + r : a.x;
        const uint16_t* res = a.residual != nullptr ? a.residual + r : a.x;
        e.b0 = *bias;
        e.res = *res;
    } else if constexpr (MODE == RowMode::kQkv || MODE == RowMode::kQkvRope) {
        const uint16_t* bias = pick3(a.bias, p.m0);
        e.b0 = bias[p.r0];
        e.b1 = bias[p.r1];
        if constexpr (MODE == RowMode::kQkvRope) {
            const int64_t d = p.r0 & 127;
            e.c = a.rope_cos[pos * 64 + d];
            e.s = a.rope_sin[pos * 64 + d];
        }
    }
    return e;
}

// Epilogue of one task (row pair) once both dots are reduced; every lane
// holds d0/d1, lane 0 (and lane 1 for a GEMV pair) stores.
template <typename T, RowMode MODE>
__device__ __forceinline__ void row_epilogue(const Nf4RowsArgs& a, const RowPair& cur, const Epi& e, float d0,
                                             float d1, int lane, int64_t pos, bool write_cache) {
    if constexpr (MODE == RowMode::kGemv) {
        if (lane < 2 && (lane == 0 || cur.has1)) {
            const int64_t r = lane == 0 ? cur.r0 : cur.r1;
            float v = lane == 0 ? d0 : d1;
            if (a.bias[0] != nullptr) {
                v = v + T::load(e.b0);
            }
            if (a.residual != nullptr) {
                v = T::load(e.res) + T::load(T::store(v));
            }
            a.out[0][r] = T::store(v);
        }
    } else if constexpr (MODE == RowMode::kSwiGlu) {
        // the row kernel stores SwiGLU outputs itself, one lane per task
    } else {
        if (lane == 0) {
            const int m = cur.m0;
            const float v0 = d0 + T::load(e.b0);
            const float v1 = d1 + T::load(e.b1);
            if constexpr (MODE == RowMode::kQkv) {
                pick3(a.out, m)[cur.r0] = T::store(v0);
                pick3(a.out, m)[cur.r1] = T::store(v1);
            } else {
                float o0 = v0, o1 = v1;
                if (m < 2) {
                    o0 = (v0 * e.c) - (v1 * e.s);
                    o1 = (v1 * e.c) + (v0 * e.s);
                }
                if (m == 0) {
                    a.out[0][cur.r0] = T::store(o0);
                    a.out[0][cur.r1] = T::store(o1);
                } else if (write_cache) {
                    uint16_t* cache = m == 1 ? a.kcache : a.vcache;
                    const int64_t g = cur.r0 >> 7;
                    const int64_t base = (g * a.capacity + pos) * 128;
                    cache[base + (cur.r0 & 127)] = T::store(o0);
                    cache[base + (cur.r1 & 127)] = T::store(o1);
                }
            }
        }
    }
}

// Fields of Nf4RowsArgs passed again as the row kernel's leading pointer
// arguments, per mode: the weight rows and absmax, and what the mode loads
// first besides (GEMV: the attention partials and length, x, residual;
// SwiGLU: x and the norm weight).
template <RowMode MODE>
struct RowsHot {
    static constexpr bool kQkvRows = MODE == RowMode::kQkv || MODE == RowMode::kQkvRope;
    static void get(const Nf4RowsArgs& a, const void* (&h)[6]) {
        if constexpr (MODE == RowMode::kGemv) {
            h[0] = a.w[0], h[1] = a.absmax[0], h[2] = a.attn.partials, h[3] = a.attn.kv_len_device, h[4] = a.x,
            h[5] = a.residual;
        } else if constexpr (kQkvRows) {
            h[0] = a.w[0], h[1] = a.w[1], h[2] = a.w[2], h[3] = a.absmax[0], h[4] = a.absmax[1], h[5] = a.absmax[2];
        } else {
            h[0] = a.w[0], h[1] = a.w[1], h[2] = a.absmax[0], h[3] = a.absmax[1], h[4] = a.x, h[5] = a.gamma;
        }
    }
    __device__ __forceinline__ static void apply(Nf4RowsArgs& a, const void* h0, const void* h1, const void* h2,
                                                 const void* h3, const void* h4, const void* h5) {
        if constexpr (MODE == RowMode::kGemv) {
            a.w[0] = static_cast<const uint8_t*>(h0);
            a.absmax[0] = static_cast<const float*>(h1);
            a.attn.partials = static_cast<const float*>(h2);
            a.attn.kv_len_device = static_cast<const int32_t*>(h3);
            a.x = static_cast<const uint16_t*>(h4);
            a.residual = static_cast<const uint16_t*>(h5);
        } else if constexpr (kQkvRows) {
            a.w[0] = static_cast<const uint8_t*>(h0);
            a.w[1] = static_cast<const uint8_t*>(h1);
            a.w[2] = static_cast<const uint8_t*>(h2);
            a.absmax[0] = static_cast<const float*>(h3);
            a.absmax[1] = static_cast<const float*>(h4);
            a.absmax[2] = static_cast<const float*>(h5);
        } else {
            a.w[0] = static_cast<const uint8_t*>(h0);
            a.w[1] = static_cast<const uint8_t*>(h1);
            a.absmax[0] = static_cast<const float*>(h2);
            a.absmax[1] = static_cast<const float*>(h3);
            a.x = static_cast<const uint16_t*>(h4);
            a.gamma = static_cast<const uint16_t*>(h5);
        }
    }
};

// Each wave owns up to TPW tasks (task = gwave + i * nwaves).  Loads are
// issued in one fixed order before any arithmetic: activation and norm
// weight, epilogue operands, then every row of every task (tasks past the end
// re-read the last task's rows and are discarded).  Vector memory returns in
// issue order, so the norm waits only for the small vectors while the rows
// stream in, and each task's dot waits only for its own rows.
//
// ATTN > 0 (kGemv only): x is the output of split-KV attention.  When the
// partials were left unmerged (split count <= attn.defer_max = ATTN), thread t
// merges head t/16, dims 8(t%16)..+7: M = max of the split maxima, weights
// exp2(m_s - M), sum and acc accumulated in split order, x = T(acc * (1 / sum)) --
// the attention kernel's own merge -- into LDS before the block barrier.
// The kv_len word, the partials and x (used when the attention merged
// itself) are requested before the weight rows.
//
// The six leading pointer arguments are preloaded into SGPRs at wave launch
// (the fields the first, longest loads need; RowsHot maps them per mode) and
// stand for the same fields of `args`.
template <typename T, RowMode MODE, int TPW, int ATTN = 0, int NTH = kRowsThreads>
__global__ __launch_bounds__(NTH) void nf4_rows2048_kernel(const void* h0, const void* h1, const void* h2,
                                                           const void* h3, const void* h4, const void* h5,
                                                           Nf4RowsArgs args, int64_t ntasks) {
    Nf4RowsArgs a = args;
    RowsHot<MODE>::apply(a, h0, h1, h2, h3, h4, h5);
    static_assert(ATTN >= 0 && ATTN <= kGqaMaxDefer, "deferred split slots");
    static_assert(!ATTN || MODE == RowMode::kGemv, "attention merge feeds the GEMV only");
    static_assert(!ATTN || kRowsThreads * 8 == 2048, "one thread per 8 merged outputs");
    // kQkv / kQkvRope / kSwiGlu: the block shares the RMSNorm (waves 0..3 each
    // normalise a quarter of the vector into LDS, every wave reads it)
    constexpr bool kCoop = MODE != RowMode::kGemv;
    static_assert(!kCoop || (NTH >= 256 && NTH % 64 == 0), "waves 0..3 compute the shared norm");
    static_assert(!ATTN || NTH == kRowsThreads, "merge layout");
    // gate/up (one large block per CU) reads the lane-sliced table, the other
    // modes (many small blocks per CU) the single one
    constexpr bool kSliced = MODE == RowMode::kSwiGlu;
    __shared__ __attribute__((aligned(16))) float cb[kSliced ? kNf4SlicedFloats : 2 * kNf4PairEntries];
    __shared__ __attribute__((aligned(16))) uint16_t s_xa[ATTN ? 2048 : 8];
    __shared__ float s_ss[4];
    __shared__ __attribute__((aligned(16))) float s_xn[kCoop ? 64 * kNormPitch : 4];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t waves_per_block = NTH / 64;
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * waves_per_block;
    const int64_t first = static_cast<int64_t>(xcd_contiguous(blockIdx.x, gridDim.x)) * waves_per_block + wave;
    static_assert(NTH >= kNf4PairEntries, "one pair-table entry per thread");
    const float2 pair_entry = pair_entry_fetch();

    int64_t pos = 0;
    bool write_cache = true;
    if constexpr (MODE == RowMode::kQkvRope) {
        pos = a.control[0];
        pos = pos < 0 ? 0 : (pos >= a.capacity ? a.capacity - 1 : pos);
        write_cache = a.done == nullptr || *a.done == 0;  // a stopped decode writes no cache row
    }
    const uint16_t* x = a.x;
    if (a.embed != nullptr) {
        // tokens[] holds control[2] entries; never read past it
        const int64_t tok_cap = a.control[2];
        const int64_t tpos = pos < tok_cap ? pos : (tok_cap > 0 ? tok_cap - 1 : 0);
        int64_t tok = a.tokens[tpos];
        tok = tok < 0 ? 0 : (tok >= a.vocab ? a.vocab - 1 : tok);
        x = a.embed + tok * 2048;
    }
    const bool has_gamma = !ATTN && a.gamma != nullptr;
    int64_t attn_len = 0;
    // one slot per split the attention may defer (ATTN = attn.defer_max)
    float2 pml[ATTN ? ATTN : 1];
    float2 pv[ATTN ? ATTN : 1][4];
    if constexpr (ATTN > 0) {
        // every slot is requested (loads unconditional); slots past the
        // split count at this length are read, never used
        attn_len = static_cast<int64_t>(*a.attn.kv_len_device) + a.attn.kv_len_offset;
        const float* src = a.attn.partials + static_cast<int64_t>(threadIdx.x >> 4) * a.attn.max_splits *
                                                 kGqaPartialStride;
        const int d0 = 8 * (threadIdx.x & 15);
#pragma unroll
        for (int x = 0; x < ATTN; ++x) {
            const float* row = src + x * kGqaPartialStride;
            pml[x] = *reinterpret_cast<const float2*>(row);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                pv[x][j] = *reinterpret_cast<const float2*>(row + 2 + d0 + 2 * j);
            }
        }
    }
    // kCoop: lane l of wave w holds elements 512w + 8l .. +7 (xq, gq);
    // otherwise the lane's own 32 elements [32l, 32l + 32) (xr, gr)
    uint4 xr[4], gr[4], xq, gq;
    const bool norm_wave = wave < 4;
    if constexpr (kCoop) {
        if (norm_wave) {
            xq = reinterpret_cast<const uint4*>(x)[64 * wave + lane];
            gq = reinterpret_cast<const uint4*>(has_gamma ? a.gamma : x)[64 * wave + lane];
        }
    } else {
        const uint4* xv = reinterpret_cast<const uint4*>(x) + lane * 4;
        const uint4* gv = reinterpret_cast<const uint4*>(has_gamma ? a.gamma : x) + lane * 4;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xr[i] = xv[i];
        }
        if constexpr (!ATTN) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                gr[i] = gv[i];
            }
        }
    }

    RowPair tasks[TPW];
    Epi epi[TPW];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        const int64_t t = first + i * nwaves;
        tasks[i] = map_task<MODE>(a, t < ntasks ? t : ntasks - 1);
        epi[i] = fetch_epilogue<T, MODE>(a, tasks[i], lane, pos);
    }
    // Rows of the first kEarly tasks are requested up front.  Gate/up keeps
    // one task in flight behind the current one: once task i's rows have
    // arrived the wave requests task i + 1 and only then computes task i.  A
    // wave whose load cannot be issued yet (the CU's memory queue is full
    // while the launch's weights stream in) stalls in order, so requesting
    // every task at once leaves the waves idle until the stream drains (and
    // two tasks of lookahead measured slower than one: 8.67 vs 8.05 us).
    uint4 pk[TPW][2];
    float am[TPW][2];
    constexpr int kEarly = MODE == RowMode::kSwiGlu ? 1 : TPW;
    auto fetch_task = [&](int i) {
        fetch_row(a, tasks[i].m0, tasks[i].r0, lane, pk[i][0], am[i][0]);
        fetch_row(a, tasks[i].m1, tasks[i].has1 ? tasks[i].r1 : tasks[i].r0, lane, pk[i][1], am[i][1]);
    };
#pragma unroll
    for (int i = 0; i < kEarly; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        fetch_task(i);
    }
    __builtin_amdgcn_sched_barrier(0);

    bool merged = false;
    if constexpr (ATTN > 0) {
        const int64_t L = attn_len < 0 ? 0 : (attn_len > a.attn.capacity ? a.attn.capacity : attn_len);
        const int64_t nsplit = gqa_split_count(L, a.attn.split_cap);
        merged = nsplit >= 1 && nsplit <= a.attn.defer_max;
        if (merged) {
            float M = -__builtin_huge_valf();
#pragma unroll
            for (int x = 0; x < ATTN; ++x) {
                M = x < nsplit ? fmaxf(M, pml[x].x) : M;
            }
            // the 16 threads of a head form one DPP row: lane x of the row
            // evaluates exp2(m_x - M) once and row broadcasts hand it out
            const int ri = threadIdx.x & 15;
            float mi = pml[0].x;
#pragma unroll
            for (int x = 1; x < ATTN; ++x) {
                mi = ri == x ? pml[x].x : mi;
            }
            const float wi = exp2_fixed(mi - M);
            float wx[ATTN];
            static_assert(ATTN <= 16, "one broadcast per deferred split, within a 16-lane row");
            row_bcast_all(wi, wx, std::make_integer_sequence<int, ATTN>{});
            float lt = 0.0f;
            float o[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int x = 0; x < ATTN; ++x) {
                if (x < nsplit) {
                    const float w = wx[x];
                    lt = fmaf(pml[x].y, w, lt);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        o[2 * j] = fmaf(pv[x][j].x, w, o[2 * j]);
                        o[2 * j + 1] = fmaf(pv[x][j].y, w, o[2 * j + 1]);
                    }
                }
            }
            uint32_t packed[4];
            const float rl = 1.0f / lt;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                packed[j] = static_cast<uint32_t>(T::store(o[2 * j] * rl)) |
                            (static_cast<uint32_t>(T::store(o[2 * j + 1] * rl)) << 16);
            }
            const uint4 xm = make_uint4(packed[0], packed[1], packed[2], packed[3]);
            reinterpret_cast<uint4*>(s_xa)[threadIdx.x] = xm;
            if (blockIdx.x == 0 && a.attn.out != nullptr) {
                reinterpret_cast<uint4*>(a.attn.out)[threadIdx.x] = xm;
            }
        }
    }
    float xq8[8];
    if (kCoop && norm_wave) {
        // this wave's quarter of the sum of squares (8 fmaf per lane, wave
        // butterfly); the four quarters meet in LDS behind the codebook barrier
        unpack8<T>(xq, xq8);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc = fmaf(xq8[j], xq8[j], acc);
        }
        acc = wave_sum(acc);
        if (lane == 0) {
            s_ss[wave] = acc;
        }
    }
    if constexpr (kSliced) {
        sliced_entry_store(cb, pair_entry);
    } else {
        pair_entry_store(cb, pair_entry);
    }
    __syncthreads();
    if constexpr (ATTN) {
        if (merged) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xr[i] = reinterpret_cast<const uint4*>(s_xa)[lane * 4 + i];
            }
        }
    }

    // RMSNorm of the lane's 32 elements against the whole vector
    float xn[32];
    if constexpr (kCoop) {
        // r from the four quarter sums ((w0 + w1) + (w2 + w3)); this lane
        // normalises its 8 elements into the padded LDS row of their owner
        // lane (elements [32L, 32L + 32) at s_xn[L * kNormPitch]), then every
        // lane reads its own 32
        if (norm_wave) {
            const float r = inv_rms((s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]), 2048.0f, a.eps);
            float g8[8];
            unpack8<T>(gq, g8);
            float y[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                y[j] = has_gamma ? (xq8[j] * r) * g8[j] : xq8[j];
            }
            float* dst = s_xn + (16 * wave + (lane >> 2)) * kNormPitch + 8 * (lane & 3);
            reinterpret_cast<float4*>(dst)[0] = make_float4(y[0], y[1], y[2], y[3]);
            reinterpret_cast<float4*>(dst)[1] = make_float4(y[4], y[5], y[6], y[7]);
        }
        __syncthreads();
        const float4* src = reinterpret_cast<const float4*>(s_xn + lane * kNormPitch);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float4 v = src[i];
            xn[4 * i] = v.x;
            xn[4 * i + 1] = v.y;
            xn[4 * i + 2] = v.z;
            xn[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            unpack8<T>(xr[i], xn + 8 * i);
        }
        if (has_gamma) {
            const float r = inv_rms(wave_sum(sumsq32(xn)), 2048.0f, a.eps);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float g[8];
                unpack8<T>(gr[i], g);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    xn[8 * i + j] = (xn[8 * i + j] * r) * g[j];
                }
            }
        }
    }

    // kSwiGlu: lane i keeps task i's gate and up sums, and the epilogue runs
    // once for the wave (lanes 0 .. TPW-1)
    float gate = 0.0f, up = 0.0f;
    int64_t out_row = tasks[0].r0;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
        if (MODE == RowMode::kSwiGlu && i + 1 < TPW) {
            // the empty asm consumes task i's rows, so the wave waits for them here
            asm volatile("" ::"v"(pk[i][0].x), "v"(pk[i][1].x), "v"(am[i][0]), "v"(am[i][1]));
            __builtin_amdgcn_sched_barrier(0);
            fetch_task(i + 1);
            __builtin_amdgcn_sched_barrier(0);
        } else if (MODE != RowMode::kSwiGlu && i >= kEarly) {
            __builtin_amdgcn_sched_barrier(0);
            fetch_task(i);
            __builtin_amdgcn_sched_barrier(0);
        }
        float d0, d1 = 0.0f;
        auto dot = [&](const uint4& w) {
            if constexpr (kSliced) {
                return nf4_chunk_dot(w, xn, sliced_lookup(cb));
            } else {
                return nf4_chunk_dot_raw(w, xn, cb);
            }
        };
        if (tasks[i].has1) {
            const float2 d = wave_sum2(dot(pk[i][0]) * am[i][0], dot(pk[i][1]) * am[i][1]);
            d0 = d.x;
            d1 = d.y;
        } else {
            d0 = wave_sum(dot(pk[i][0]) * am[i][0]);
        }
        if constexpr (MODE == RowMode::kSwiGlu) {
            gate = lane == i ? d0 : gate;
            up = lane == i ? d1 : up;
            out_row = lane == i ? tasks[i].r0 : out_row;
        } else if (first + i * nwaves < ntasks) {
            row_epilogue<T, MODE>(a, tasks[i], epi[i], d0, d1, lane, pos, write_cache);
        }
    }
    if constexpr (MODE == RowMode::kSwiGlu) {
        if (lane < TPW && first + lane * nwaves < ntasks) {
            a.out[0][out_row] = T::store(silu_fixed(gate) * up);
        }
    }

    if (blockIdx.x == 0 && a.hidden_out != nullptr) {
        if constexpr (kCoop) {
            if (norm_wave) {
                reinterpret_cast<uint4*>(a.hidden_out)[64 * wave + lane] = xq;
            }
        } else if (wave == 0) {
            uint4* dst = reinterpret_cast<uint4*>(a.hidden_out) + lane * 4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dst[i] = xr[i];
            }
        }
    }
    if (blockIdx.x == 0 && wave == 0) {
        if (a.norm_out != nullptr) {
            float4* dst = reinterpret_cast<float4*>(a.norm_out) + lane * 8;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                dst[i] = make_float4(xn[4 * i], xn[4 * i + 1], xn[4 * i + 2], xn[4 * i + 3]);
            }
        }
    }
}

// K = 11008 (NCHUNK = 344 chunks): a block of W = 6 waves covers R rows
// (chunk c -> wave c/64, lane c%64); each lane keeps its chunk's 32 inputs in
// registers.  Loads in issue order: activation chunk, residuals of the
// block's rows, then the R rows (lanes past the last chunk re-read it and
// contribute 0).  Row total = sum of the W wave sums in wave order.
template <typename T, int NCHUNK, int R>
//
// The arguments are scalars so that all of them are preloaded into SGPRs at
// wave launch.
__global__ __launch_bounds__(64 * ((NCHUNK + 63) / 64)) void nf4_down_kernel(const uint16_t* x, const uint8_t* w,
                                                                            const float* absmax,
                                                                            const uint16_t* residual, uint16_t* out,
                                                                            int64_t rows) {
    Nf4DownArgs a;
    a.x = x;
    a.w = w;
    a.absmax = absmax;
    a.residual = residual;
    a.out = out;
    a.rows = rows;
    constexpr int W = (NCHUNK + 63) / 64;
    // the pair table and one spare entry that threads past the table overwrite
    __shared__ __attribute__((aligned(16))) float cb[2 * kNf4PairEntries + 2];
    __shared__ float red[R][W];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int c = wave * 64 + lane;
    const bool valid = c < NCHUNK;
    const int cc = valid ? c : NCHUNK - 1;
    const int64_t row_chunks = NCHUNK;
    const int64_t row_blocks = NCHUNK / 2;
    const int64_t rbase = static_cast<int64_t>(xcd_contiguous(blockIdx.x, gridDim.x)) * R;  // XCD-contiguous rows
    const int64_t last_row = a.rows - 1;
    static_assert(64 * W >= kNf4PairEntries, "one pair-table entry per thread");
    const float2 pair_entry = pair_entry_fetch();

    uint4 xr[4];
    const uint4* src = reinterpret_cast<const uint4*>(a.x) + static_cast<int64_t>(cc) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xr[i] = src[i];
    }
    // thread t < R finishes row rbase + t.  The residual load is unconditional
    // (from x when there is none): a load under a branch makes the compiler
    // wait for every load issued before it, so the rows would be requested
    // only after the activation chunk had arrived.
    const int64_t my_row = rbase + (threadIdx.x % R) < last_row ? rbase + (threadIdx.x % R) : last_row;
    const bool has_res = a.residual != nullptr;
    const uint16_t res = *(has_res ? a.residual + my_row : a.x);

    uint4 pk[R];
    float am[R];
    const uint4* wv = reinterpret_cast<const uint4*>(a.w) + cc;
#pragma unroll
    for (int i = 0; i < R; ++i) {
        __builtin_amdgcn_sched_barrier(0);
        const int64_t r = rbase + i < last_row ? rbase + i : last_row;
        pk[i] = load_stream(wv + r * row_chunks);
        am[i] = load_stream(a.absmax + r * row_blocks + (cc >> 1));
    }
    __builtin_amdgcn_sched_barrier(0);

    // Every thread stores (those past the table into the spare entry): a
    // store under a branch lets the compiler sink the entry's load behind the
    // rows and wait for all of them before the barrier.
    reinterpret_cast<float2*>(cb)[threadIdx.x < kNf4PairEntries ? threadIdx.x : kNf4PairEntries] = pair_entry;
    __builtin_amdgcn_sched_barrier(0);  // nothing that waits for a row before the barrier
    __syncthreads();
    float xv[32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        unpack8<T>(xr[i], xv + 8 * i);
    }

    static_assert(R % 2 == 0, "rows reduced in pairs");
#pragma unroll
    for (int i = 0; i < R; i += 2) {
        const float p0 = nf4_chunk_dot_raw(pk[i], xv, cb) * am[i];
        const float p1 = nf4_chunk_dot_raw(pk[i + 1], xv, cb) * am[i + 1];
        const float2 p = wave_sum2(valid ? p0 : 0.0f, valid ? p1 : 0.0f);
        if (lane == 0) {
            red[i][wave] = p.x;
            red[i + 1][wave] = p.y;
        }
    }
    __syncthreads();
    if (threadIdx.x < R && rbase + threadIdx.x < a.rows) {
        const int64_t r = rbase + threadIdx.x;
        float s = red[threadIdx.x][0];
#pragma unroll
        for (int w = 1; w < W; ++w) {
            s = s + red[threadIdx.x][w];
        }
        if (has_res) {
            s = T::load(res) + T::load(T::store(s));
        }
        a.out[r] = T::store(s);
    }
}

struct SrcF32 {
    static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
};
struct SrcBf16 {
    static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
};

// One wave per 64-element block: absmax by a max-butterfly (order free),
// scale by the reciprocal, pick the code by counting decision points.
template <typename S, typename P>
__global__ __launch_bounds__(256) void nf4_quantize_kernel(const P* src, int64_t nblocks, uint8_t* packed,
                                                           float* absmax) {
    const int lane = threadIdx.x & 63;
    const int64_t blk = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (blk >= nblocks) {
        return;
    }
    const float v = S::load(src, blk * 64 + lane);
    float m = fabsf(v);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        m = fmaxf(m, __shfl_xor(m, o, 64));
    }
    int code = 7;
    if (m > 0.0f) {
        const float s = v * (1.0f / m);
        code = 0;
#pragma unroll
        for (int i = 0; i < 15; ++i) {
            code += s > kNf4Mid[i] ? 1 : 0;
        }
    }
    const int partner = __shfl_xor(code, 1, 64);
    if ((lane & 1) == 0) {
        packed[blk * 32 + (lane >> 1)] = static_cast<uint8_t>((code << 4) | partner);
    }
    if (lane == 0) {
        absmax[blk] = m;
    }
}

__global__ __launch_bounds__(256) void nf4_dequantize_kernel(const uint8_t* packed, const float* absmax, int64_t n,
                                                             int64_t blocksize, int out_kind, void* out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) {
        return;
    }
    const uint32_t byte = packed[i >> 1];
    const uint32_t code = (i & 1) == 0 ? (byte >> 4) : (byte & 0xfu);
    const float v = kNf4Codebook[code] * absmax[i / blocksize];
    if (out_kind == 0) {
        static_cast<float*>(out)[i] = v;
    } else if (out_kind == 1) {
        static_cast<uint16_t*>(out)[i] = f32_to_bf16(v);
    } else {
        static_cast<uint16_t*>(out)[i] = f32_to_f16(v);
    }
}

// The o_proj GEMV with the attention merge prologue for k deferral slots:
// instantiations K = 1 .. kGqaMaxDefer, tried in turn.
template <typename T, RowMode MODE, int TPW, int K>
hipError_t launch_attn_rows(int k, dim3 grid, const void* const* h, const Nf4RowsArgs& a, int64_t ntasks,
                            hipStream_t stream) {
    if constexpr (K > kGqaMaxDefer) {
        return hipErrorInvalidValue;
    } else {
        if (k != K) {
            return launch_attn_rows<T, MODE, TPW, K + 1>(k, grid, h, a, ntasks, stream);
        }
        hipLaunchKernelGGL((nf4_rows2048_kernel<T, MODE, TPW, K>), grid, dim3(kRowsThreads), 0, stream, h[0], h[1],
                           h[2], h[3], h[4], h[5], a, ntasks);
        return hipGetLastError();
    }
}

template <typename T, RowMode MODE, int TPW>
hipError_t launch_rows_tpw(const Nf4RowsArgs& a, int64_t ntasks, int64_t blocks, hipStream_t stream) {
    const void* h[6];
    RowsHot<MODE>::get(a, h);
    const dim3 grid(static_cast<unsigned>(blocks));
    if constexpr (MODE == RowMode::kGemv && TPW == 1) {
        if (a.attn.partials != nullptr) {
            // one instantiation per deferral slot count (1..kGqaMaxDefer, checked by the caller)
            return launch_attn_rows<T, MODE, TPW, 1>(static_cast<int>(a.attn.defer_max), grid, h, a, ntasks, stream);
        }
    }
    if constexpr (MODE == RowMode::kSwiGlu) {
        hipLaunchKernelGGL((nf4_rows2048_kernel<T, MODE, TPW, false, kSwiGluThreads>), grid, dim3(kSwiGluThreads), 0,
                           stream, h[0], h[1], h[2], h[3], h[4], h[5], a, ntasks);
        return hipGetLastError();
    }
    if constexpr (MODE == RowMode::kQkvRope) {
        hipLaunchKernelGGL((nf4_rows2048_kernel<T, MODE, TPW, false, kQkvRopeThreads>), grid, dim3(kQkvRopeThreads),
                           0, stream, h[0], h[1], h[2], h[3], h[4], h[5], a, ntasks);
        return hipGetLastError();
    }
    hipLaunchKernelGGL((nf4_rows2048_kernel<T, MODE, TPW>), grid, dim3(kRowsThreads), 0, stream, h[0], h[1], h[2],
                       h[3], h[4], h[5], a, ntasks);
    return hipGetLastError();
}

template <typename T, RowMode MODE>
hipError_t launch_rows_t(const Nf4RowsArgs& a, hipStream_t stream) {
    int64_t ntasks = 0;
    if (MODE == RowMode::kGemv) {
        ntasks = (a.rows[0] + 1) / 2;
    } else if (MODE == RowMode::kSwiGlu) {
        ntasks = a.rows[0];
    } else {
        ntasks = (a.rows[0] + a.rows[1] + a.rows[2]) / 2;
    }
    if (ntasks <= 0) {
        return hipSuccess;
    }
    if (a.attn.partials != nullptr) {
        // the merge runs in the one-task-per-wave GEMV only
        const AttnSplits& at = a.attn;
        if (MODE != RowMode::kGemv || ntasks > kMaxRowWaves || a.gamma != nullptr || a.embed != nullptr ||
            at.kv_len_device == nullptr || at.capacity <= 0 || at.split_cap <= 0 || at.max_splits <= 0 ||
            at.defer_max < 1 || at.defer_max > kGqaMaxDefer || at.defer_max > at.max_splits) {
            return hipErrorInvalidValue;
        }
    }
    // every wave's tasks in flight at once
    const int64_t waves_per_block =
        (MODE == RowMode::kSwiGlu ? kSwiGluThreads : (MODE == RowMode::kQkvRope ? kQkvRopeThreads : kRowsThreads)) / 64;
    const int64_t max_waves = MODE == RowMode::kSwiGlu ? kSwiGluWaves : kMaxRowWaves;
    int64_t tpw = (ntasks + max_waves - 1) / max_waves;
    tpw = tpw <= 1 ? 1 : (tpw <= 2 ? 2 : (tpw <= 4 ? 4 : 8));
    const int64_t waves = (ntasks + tpw - 1) / tpw;
    const int64_t blocks = (waves + waves_per_block - 1) / waves_per_block;
    switch (tpw) {
        case 1:
            return launch_rows_tpw<T, MODE, 1>(a, ntasks, blocks, stream);
        case 2:
            return launch_rows_tpw<T, MODE, 2>(a, ntasks, blocks, stream);
        case 4:
            return launch_rows_tpw<T, MODE, 4>(a, ntasks, blocks, stream);
        default:
            return launch_rows_tpw<T, MODE, 8>(a, ntasks, blocks, stream);
    }
}

template <typename T>
hipError_t launch_rows_mode(RowMode mode, const Nf4RowsArgs& a, hipStream_t stream) {
    switch (mode) {
        case RowMode::kGemv:
            return launch_rows_t<T, RowMode::kGemv>(a, stream);
        case RowMode::kQkv:
            return launch_rows_t<T, RowMode::kQkv>(a, stream);
        case RowMode::kQkvRope:
            return launch_rows_t<T, RowMode::kQkvRope>(a, stream);
        case RowMode::kSwiGlu:
            return launch_rows_t<T, RowMode::kSwiGlu>(a, stream);
    }
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_nf4_rows2048(RowMode mode, Act act, const Nf4RowsArgs& a, hipStream_t stream) {
    return act == Act::kBf16 ? launch_rows_mode<Bf16>(mode, a, stream) : launch_rows_mode<F16>(mode, a, stream);
}

hipError_t launch_nf4_down11008(Act act, const Nf4DownArgs& a, hipStream_t stream) {
    constexpr int kChunks = 11008 / 32;
    constexpr int kRows = 4;  // 512 blocks of 6 waves: measured faster than 2 or 8 rows per block
    constexpr int kThreads = 64 * ((kChunks + 63) / 64);
    if (a.rows <= 0) {
        return hipSuccess;
    }
    if (a.x == nullptr || a.w == nullptr || a.absmax == nullptr || a.out == nullptr) {
        return hipErrorInvalidValue;  // the kernel also reads x in place of an absent residual
    }
    const int64_t blocks = (a.rows + kRows - 1) / kRows;
    if (act == Act::kBf16) {
        hipLaunchKernelGGL((nf4_down_kernel<Bf16, kChunks, kRows>), dim3(static_cast<unsigned>(blocks)),
                           dim3(kThreads), 0, stream, a.x, a.w, a.absmax, a.residual, a.out, a.rows);
    } else {
        hipLaunchKernelGGL((nf4_down_kernel<F16, kChunks, kRows>), dim3(static_cast<unsigned>(blocks)),
                           dim3(kThreads), 0, stream, a.x, a.w, a.absmax, a.residual, a.out, a.rows);
    }
    return hipGetLastError();
}

hipError_t launch_nf4_quantize_f32(const float* src, int64_t n, uint8_t* packed, float* absmax, hipStream_t stream) {
    const int64_t nblocks = n / 64;
    if (nblocks <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL((nf4_quantize_kernel<SrcF32, float>), dim3(static_cast<unsigned>((nblocks + 3) / 4)),
                       dim3(256), 0, stream, src, nblocks, packed, absmax);
    return hipGetLastError();
}

hipError_t launch_nf4_quantize_bf16(const uint16_t* src, int64_t n, uint8_t* packed, float* absmax,
                                    hipStream_t stream) {
    const int64_t nblocks = n / 64;
    if (nblocks <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL((nf4_quantize_kernel<SrcBf16, uint16_t>), dim3(static_cast<unsigned>((nblocks + 3) / 4)),
                       dim3(256), 0, stream, src, nblocks, packed, absmax);
    return hipGetLastError();
}

hipError_t launch_nf4_dequantize(const uint8_t* packed, const float* absmax, int64_t n, int64_t blocksize,
                                 int out_kind, void* out, hipStream_t stream) {
    if (n <= 0) {
        return hipSuccess;
    }
    hipLaunchKernelGGL(nf4_dequantize_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream,
                       packed, absmax, n, blocksize, out_kind, out);
    return hipGetLastError();
}

}  // namespace kc
