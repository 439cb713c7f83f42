// Device-side numerics shared by every gfx950 kernel in libkudacuda.
//
// Every reduction below has ONE fixed order (lane -> chunk mapping, per-lane
// accumulator split, butterfly stages).  The decode path's results are a pure
// function of its inputs, so greedy tokens are reproducible run to run and can
// be matched bit for bit by a host restatement that follows the same order.
//
// Conventions (wave64):
//  * NF4 "chunk": 16 packed bytes = 32 consecutive logical elements; chunk c of
//    a row holds elements [32c, 32c+32) and uses absmax block c/2 (blocksize
//    64).  Byte i of a chunk carries element 2i in its high nibble and 2i+1 in
//    its low nibble (bitsandbytes packing, reference
//    kernels/common/nf4_device.cuh:36-39).
//  * chunk dot: four accumulators, one per 32-bit word (8 elements each),
//    sequential fmaf inside a word, combined as (a0+a1)+(a2+a3), then multiplied
//    by the block's absmax.
//  * wave_sum: butterfly v += shfl_xor(v, o) for o = 32,16,8,4,2,1; the result
//    is identical in every lane because IEEE addition is commutative.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kc {

// bitsandbytes NF4 codebook (the 16 fp32 values of the format; reference
// kernels/common/nf4_device.cuh:10-27).  Kept as exact hex literals.
__device__ constexpr float kNf4Codebook[16] = {
    -0x1.000000p+0f, -0x1.647362p-1f, -0x1.0cd660p-1f, -0x1.946540p-2f,
    -0x1.23449ap-2f, -0x1.7a6a7ep-3f, -0x1.74f0e2p-4f, 0x0.0p+0f,
    0x1.45f5fep-4f,  0x1.4995c6p-3f,  0x1.f809bap-3f,  0x1.5a0674p-2f,
    0x1.c34970p-2f,  0x1.200f56p-1f,  0x1.722766p-1f,  0x1.000000p+0f,
};

constexpr float kLog2e = 0x1.715476p+0f;  // fp32(log2(e))

// ---------------------------------------------------------------- conversions
__device__ __forceinline__ float bf16_to_f32(uint16_t v) {
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even fp32 -> bf16; NaN becomes a quiet NaN with its sign.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return static_cast<uint16_t>((u >> 16) | 0x0040u);
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t v) {
    return static_cast<float>(__builtin_bit_cast(_Float16, v));
}

// fp32 -> fp16, round to nearest even.  The value passes through an empty asm
// first: otherwise the compiler folds a preceding fp32 multiply into a
// mixed-precision FMA that rounds the exact product to fp16 once, which
// differs from rounding the fp32 product when that product is an fp16 tie.
__device__ __forceinline__ uint16_t f32_to_f16(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// Activation element types travel as 16-bit storage; the tag picks the
// conversion.  Bf16 is the decode path's type, F16 serves the reference's
// fp16 entry points.
struct Bf16 {
    static __device__ __forceinline__ float load(uint16_t v) { return bf16_to_f32(v); }
    static __device__ __forceinline__ uint16_t store(float f) { return f32_to_bf16(f); }
};
struct F16 {
    static __device__ __forceinline__ float load(uint16_t v) { return f16_to_f32(v); }
    static __device__ __forceinline__ uint16_t store(float f) { return f32_to_f16(f); }
};

// Weight streams are loaded non-temporally (global_load ... nt): each weight
// byte is read once per token, and a streamed line would otherwise displace
// what every kernel of the step re-reads from the caches -- its code, kernel
// arguments, tables and activations.  Measured on the decode step: the hint
// on lm_head alone saves its own ~9 us, on the row kernels and down alone
// nothing, and on all three 1.047 -> 1.010 ms per token (any one stream left
// cached evicts those lines again every layer).
__device__ __forceinline__ uint4 load_stream(const uint4* p) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ float load_stream(const float* p) { return __builtin_nontemporal_load(p); }

// Unpack 8 consecutive 16-bit elements held in a uint4.
template <typename T>
__device__ __forceinline__ void unpack8(const uint4 v, float* out) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        out[2 * i] = T::load(static_cast<uint16_t>(w[i] & 0xffffu));
        out[2 * i + 1] = T::load(static_cast<uint16_t>(w[i] >> 16));
    }
}

// ---------------------------------------------------------------------- exp2
// 2^y by exact reduction y = n + f (n = rint(y), |f| <= 1/2, f exact) and the
// degree-7 Taylor polynomial of e^(f ln 2) in Horner form, scaled by ldexp.
// Results below 2^-125 flush to +0 (so no subnormal is ever produced) and
// y >= 128 gives +inf.  Max error about 2 ulp over the whole range.
__device__ __forceinline__ float exp2_fixed(float y) {
    if (!(y >= -125.0f)) {
        return (y != y) ? y : 0.0f;
    }
    if (y >= 128.0f) {
        return __builtin_huge_valf();
    }
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
    return ldexpf(p, static_cast<int>(n));
}

// silu(g) = g / (1 + e^-g), with e^-g = exp2_fixed(g * -log2e).
__device__ __forceinline__ float silu_fixed(float g) {
    const float e = exp2_fixed(g * -kLog2e);
    return g / (1.0f + e);
}

// ---------------------------------------------------------------- reductions
// DPP row rotation (row_ror:N, rotate within each row of 16 lanes).
template <int N>
__device__ __forceinline__ float row_ror(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 | N, 0xf, 0xf, false));
}

// DPP row broadcast (row_newbcast:N): every lane of a 16-lane row receives
// lane N of its row.
template <int N>
__device__ __forceinline__ float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 | N, 0xf, 0xf, false));
}

// Butterfly over the 16 lanes of a row: v += partner for partner distance
// 8, 4, 2, 1.  Implemented with row rotations: after the distance-8 stage the
// row holds a period-8 pattern, after distance 4 a period-4 one, ..., so a
// rotation by d pairs every lane with the same value as lane ^ d, and the sums
// equal the xor butterfly's bit for bit (IEEE addition is commutative).
__device__ __forceinline__ float group16_sum(float v) {
    v += row_ror<8>(v);
    v += row_ror<4>(v);
    v += row_ror<2>(v);
    v += row_ror<1>(v);
    return v;
}

// Butterfly over the wave: partner distance 32, 16 (cross-row stages), then
// the in-row stages 8..1.  Every lane ends with the same value.  The cross-row
// stages use the lane-swap instructions on two copies of v: afterwards every
// lane holds the pair {v[l], v[l ^ d]} (one value in each result), and their
// sum is the stage's v[l] + v[l ^ d] (IEEE addition is commutative).  Call
// with the whole wave active.
__device__ __forceinline__ float wave_sum(float v) {
    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
    return group16_sum(v);
}

// Two butterflies at the price of one: the first lane swap takes a's upper
// half and b's lower half, so after its sum lanes 0..31 hold a's distance-32
// stage and lanes 32..63 b's; the remaining stages pair lanes inside each half
// only.  A last swap hands out {sum(a), sum(b)} to every lane.  Each row's
// additions are the pairs and order of wave_sum, so the sums are identical to
// wave_sum(a) and wave_sum(b).  Call with the whole wave active.
__device__ __forceinline__ float2 wave_sum2(float a, float b) {
    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(a), __float_as_uint(b), false, false);
    float v = __uint_as_float(p32[0]) + __uint_as_float(p32[1]);
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(p16[0]) + __uint_as_float(p16[1]);
    v = group16_sum(v);
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// -------------------------------------------------- cross-block exchange
// Blocks of one launch that hand results to a "last block" (ticket pattern)
// exchange only a few words.  The hand-over, and what each step compiles to
// on gfx950 (checked in this build's assembly):
//   1. each thread writes its words with agent-scope atomic stores
//      (global_store_* ... sc1: written through the XCD's L2, which is not
//      coherent with the other XCDs' L2 caches);
//   2. every wave waits for its own stores (s_waitcnt vmcnt(0)), then the
//      block barrier;
//   3. one thread takes the ticket with an agent-scope acquire-release
//      fetch-add (buffer_wbl2 sc1, global_atomic_add, buffer_inv sc1): the
//      release orders the block's stores before the increment under the HIP
//      memory model, the acquire orders the other blocks' stores before this
//      block's reads;
//   4. the last block reads the words with agent-scope atomic loads
//      (global_load_* ... sc1).
// Steps 1, 2 and 4 alone carry the data on this hardware; step 3's fences
// make the hand-over correct by the memory model instead of by those cache
// bits, for ~0.2 us per launch of a few publishing blocks.  Each release's L2
// write-back costs ~0.3 us and those of one XCD serialise, so a launch with
// hundreds of publishing blocks (lm_head) takes no ticket: its blocks write
// with plain stores and a second kernel reads them after the kernel boundary.
__device__ __forceinline__ void store_agent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// two adjacent floats (8-byte aligned) as one 8-byte agent-scope store
__device__ __forceinline__ void store_agent_pair(float* p, float lo, float hi) {
    const uint64_t v = static_cast<uint64_t>(__float_as_uint(lo)) | (static_cast<uint64_t>(__float_as_uint(hi)) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The ticket of step 3: returns the counter's value before the increment.
__device__ __forceinline__ uint32_t take_ticket(uint32_t* counter) {
    return __hip_atomic_fetch_add(counter, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until this wave's vector memory operations (the exchange stores) have
// completed; call before the barrier that precedes the ticket increment.
__device__ __forceinline__ void wait_own_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ------------------------------------------------------------ block placement
// Workgroups go to the 8 XCDs round-robin by block index.  A kernel that
// streams a weight matrix in block order runs block b as block
// xcd_contiguous(b, n) instead, so that each XCD covers one contiguous eighth
// of the blocks (and of the matrix) rather than every eighth block across all
// of it: a bijection of [0, n), XCD x = b % 8 taking the range that starts at
// x * (n / 8) + min(x, n % 8).  Decode step on one box, 3 interleaved runs:
// 1.0088 -> 0.9988 ms with down and the row kernels placed this way.
__device__ __forceinline__ uint32_t xcd_contiguous(uint32_t b, uint32_t n) {
    const uint32_t x = b & 7u;
    const uint32_t q = n >> 3;
    const uint32_t r = n & 7u;
    return x * q + (x < r ? x : r) + (b >> 3);
}

// ------------------------------------------------------------------ NF4 dots
// (byte B of x) << S in one instruction (a byte-select shift), written as
// asm: the compiler folds a byte-select operand back into a shift and an AND.
template <int B, int S>
__device__ __forceinline__ uint32_t byte_shl(uint32_t x) {
    uint32_t r;
    if constexpr (B == 0) {
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_0"
            : "=v"(r) : "v"(static_cast<uint32_t>(S)), "v"(x));
    } else if constexpr (B == 1) {
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_1"
            : "=v"(r) : "v"(static_cast<uint32_t>(S)), "v"(x));
    } else if constexpr (B == 2) {
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_2"
            : "=v"(r) : "v"(static_cast<uint32_t>(S)), "v"(x));
    } else {
        asm("v_lshlrev_b32_sdwa %0, %1, %2 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:BYTE_3"
            : "=v"(r) : "v"(static_cast<uint32_t>(S)), "v"(x));
    }
    return r;
}

template <int B>
__device__ __forceinline__ uint32_t byte_shl3(uint32_t x) {
    return byte_shl<B, 3>(x);
}

// Where a lane finds byte value e's entry of the pair table in LDS: the
// block's single copy (offset e * 8, one byte-select shift) ...
struct PairLookup {
    const char* base;
    template <int B>
    __device__ __forceinline__ const float2* entry(uint32_t w) const {
        return reinterpret_cast<const float2*>(base + byte_shl3<B>(w));
    }
};
// ... or the lane-sliced copy (see sliced_entry_store): offset e * 256 + 8 s for
// the lane's slot s = lane % 32, formed by one byte permute from the code
// word and the lane's 8 s (bytes, low to high: 8 s, byte B of w, 0, 0).
struct SlicedLookup {
    const char* base;
    uint32_t slot8;
    template <int B>
    __device__ __forceinline__ const float2* entry(uint32_t w) const {
        return reinterpret_cast<const float2*>(base + __builtin_amdgcn_perm(w, slot8, 0x0c0c0400u | (B << 8)));
    }
};

// Codebook values of the 32 codes of one chunk, gathered from the LDS pair
// table before any arithmetic so the lookups overlap.  Entry e of the table
// holds (code[e >> 4], code[e & 15]), the values of both nibbles of byte e
// (even element in the high nibble), so each byte costs one offset
// instruction and one 8-byte LDS read.
template <typename Lookup>
__device__ __forceinline__ void nf4_gather32(const uint4 pk, const Lookup& lut, float* cw) {
    const uint32_t w[4] = {pk.x, pk.y, pk.z, pk.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float2 p0 = *lut.template entry<0>(w[i]);
        const float2 p1 = *lut.template entry<1>(w[i]);
        const float2 p2 = *lut.template entry<2>(w[i]);
        const float2 p3 = *lut.template entry<3>(w[i]);
        cw[8 * i + 0] = p0.x;
        cw[8 * i + 1] = p0.y;
        cw[8 * i + 2] = p1.x;
        cw[8 * i + 3] = p1.y;
        cw[8 * i + 4] = p2.x;
        cw[8 * i + 5] = p2.y;
        cw[8 * i + 6] = p3.x;
        cw[8 * i + 7] = p3.y;
    }
}

// Dot of one 32-element chunk with x[0..31] (already in fp32), before the
// absmax multiply, with the pair table in LDS at `lut`.
template <typename Lookup>
__device__ __forceinline__ float nf4_chunk_dot(const uint4 pk, const float* x, const Lookup& lut) {
    float cw[32];
    nf4_gather32(pk, lut, cw);
    float a[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc = fmaf(x[8 * i + j], cw[8 * i + j], acc);
        }
        a[i] = acc;
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}
// ... with the block's single copy of the table at `pairs`.
__device__ __forceinline__ float nf4_chunk_dot_raw(const uint4 pk, const float* x, const float* pairs) {
    return nf4_chunk_dot(pk, x, PairLookup{reinterpret_cast<const char*>(pairs)});
}

// Sum of squares of 32 consecutive elements, same accumulator split as a
// chunk dot.
__device__ __forceinline__ float sumsq32(const float* x) {
    float a[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            acc = fmaf(x[8 * i + j], x[8 * i + j], acc);
        }
        a[i] = acc;
    }
    return (a[0] + a[1]) + (a[2] + a[3]);
}

// 1 / sqrt(sumsq / n + eps), every step correctly rounded.
__device__ __forceinline__ float inv_rms(float sumsq, float n, float eps) {
    return 1.0f / sqrtf(sumsq / n + eps);
}

// Load the 32 activation elements of chunk `lane` (elements [32*lane, +32))
// from a 16-bit vector, RMS-normalise them against the whole 2048-element
// vector and return them in fp32: x_n = (x * inv_rms) * gamma.  When gamma is
// null the raw values are returned.
template <typename T>
__device__ __forceinline__ void load_norm_x2048(const uint16_t* __restrict__ x,
                                                const uint16_t* __restrict__ gamma,
                                                float eps, int lane, float* xn) {
    const uint4* xv = reinterpret_cast<const uint4*>(x) + lane * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        unpack8<T>(xv[i], xn + 8 * i);
    }
    if (gamma == nullptr) {
        return;
    }
    const float ss = wave_sum(sumsq32(xn));
    const float r = inv_rms(ss, 2048.0f, eps);
    float g[32];
    const uint4* gv = reinterpret_cast<const uint4*>(gamma) + lane * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        unpack8<T>(gv[i], g + 8 * i);
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) {
        xn[j] = (xn[j] * r) * g[j];
    }
}

// Entries of the byte pair table: one per byte value, 8 bytes each.
constexpr int kNf4PairEntries = 256;

// The byte pair table (see nf4_gather32), entry e = (code[e >> 4],
// code[e & 15]), built at compile time into the code object.
struct Nf4PairTable {
    float v[2 * kNf4PairEntries];
};
constexpr Nf4PairTable nf4_make_pair_table() {
    Nf4PairTable t{};
    for (int e = 0; e < kNf4PairEntries; ++e) {
        t.v[2 * e] = kNf4Codebook[e >> 4];
        t.v[2 * e + 1] = kNf4Codebook[e & 15];
    }
    return t;
}
__device__ constexpr Nf4PairTable kNf4PairTable = nf4_make_pair_table();

// Block-shared LDS copy of the pair table, in two steps so the global load
// can be issued before the kernel's weight loads (a wait for it then does not
// wait for them): pair_entry_fetch() returns this thread's entry (threads past
// the table re-read entry t & 255), pair_entry_store() writes it (threads
// below 256 only; blocks have at least 256 threads).  The caller publishes the
// table with a block barrier.
__device__ __forceinline__ float2 pair_entry_fetch() {
    return reinterpret_cast<const float2*>(kNf4PairTable.v)[threadIdx.x & (kNf4PairEntries - 1)];
}
__device__ __forceinline__ void pair_entry_store(float* pairs, float2 e) {
    if (threadIdx.x < kNf4PairEntries) {
        reinterpret_cast<float2*>(pairs)[threadIdx.x] = e;
    }
}

// Lane-sliced copy of the pair table for kernels with few, large blocks: 32
// copies interleaved so that slot s of entry e sits at byte e * 256 + 8 s.
// Lane l reads slot l % 32, so its lookups always fall in bank pair l % 32,
// and the 32 lanes an LDS pass serves for 8-byte reads (64 banks of 4 bytes)
// never share a bank; random entries of the single table collide (about two
// thirds of its LDS cycles were bank-conflict stalls).  Fewer slots (16 or
// 8, half or a quarter of the fill) put two or four lanes of a pass on one
// bank pair and measured slower.  64 KiB; the entry stride (kNf4SlotStride
// slots, 256 bytes) is what one byte permute can form, kNf4Slots of its
// slots are filled and read.
constexpr int kNf4SlotStride = 32;
constexpr int kNf4Slots = 32;
static_assert(kNf4Slots <= kNf4SlotStride && (kNf4Slots & (kNf4Slots - 1)) == 0, "slots tile the stride");
constexpr int kNf4SlicedFloats = 2 * kNf4PairEntries * kNf4SlotStride;
// Thread t < 256 writes its entry (pair_entry_fetch) into every slot, slot
// (j + t) % kNf4Slots at step j, so the 32 lanes of a pass write 32 bank
// pairs.  The caller publishes the table with a block barrier.
__device__ __forceinline__ void sliced_entry_store(float* sliced, float2 e) {
    if (threadIdx.x < kNf4PairEntries) {
        float2* row = reinterpret_cast<float2*>(sliced) + threadIdx.x * kNf4SlotStride;
#pragma unroll 8
        for (int j = 0; j < kNf4Slots; ++j) {
            row[(j + threadIdx.x) & (kNf4Slots - 1)] = e;
        }
    }
}
__device__ __forceinline__ SlicedLookup sliced_lookup(const float* sliced) {
    return SlicedLookup{reinterpret_cast<const char*>(sliced), (threadIdx.x & (kNf4Slots - 1)) * 8u};
}

}  // namespace kc
