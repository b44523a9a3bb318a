// Decode-side MoE on gfx950 (the reference's Window MoE, T <= 8 rows): the first-appearance
// expert plan, the precise Q8_1 activation quantizer, the grouped gate/up and down
// mat-vecs over Q8_1 activations, the F32 SwiGLU and the decode combine
// (moe.metal:101-275, quantize_q8_1.metal, 04-metal-kernels.md sections 5.8 and 5.10).
//
// With at most 8 rows, every token routes to distinct experts, so a group (one expert) has at
// most 8 entries. The mat-vecs read each active expert's weights once: one workgroup per
// (group, 32 weight rows); within a wave, LPR lanes share a weight row, each taking whole
// 32-value Q8_1 blocks of K, and every lane keeps one accumulator per entry of the group.
// Integer block dots run on v_dot4_i32_i8 (codes times Q8_1 codes, exact), then the block's
// float scales; a butterfly over the row's lanes finishes the row.
#include <stdint.h>

#include "sm_device.h"
#include "sm_launch.h"
#include "sm_topk.h"

namespace sm {
namespace {

constexpr uint32_t kQ81Bytes = 36;  // half2 ds (d, sum), int8 qs[32] (types.h:128-131)

__device__ __forceinline__ uint32_t f32_bits(float x) { return __builtin_bit_cast(uint32_t, x); }
__device__ __forceinline__ float bits_f32(uint32_t b) { return __builtin_bit_cast(float, b); }

// C's round(): half away from zero (the reference's round_half_away, common/math.h:42-44).
__device__ __forceinline__ int round_away(float x) { return int(__builtin_roundf(x)); }

// ---- the precise Q8_1 quantizer's exceptional paths (quantize_q8_1.metal) ----------------
// d = amax / 127 for an amax whose exponent field is at most 7, correctly rounded, in units
// of the smallest subnormal (integer arithmetic, so no hardware denormal handling is needed).
__device__ uint32_t q81_subnormal_scale_bits(uint32_t amax_bits) {
    const uint32_t e = (amax_bits >> 23) & 0xffu;
    const uint32_t sig = e == 0u ? amax_bits & 0x007fffffu : (amax_bits & 0x007fffffu) | 0x00800000u;
    const uint32_t shift = e == 0u ? 0u : e - 1u;
    const uint32_t units = sig << shift;
    uint32_t q = units / 127u;
    const uint32_t rem = units % 127u, twice = 2u * rem;
    if (twice > 127u || (twice == 127u && (q & 1u) != 0u)) ++q;
    return q;
}

// round(multiplier * value / denominator) from the exact significands, clamped to 127 (the
// path for d rounding to zero).
__device__ int q81_round_ratio(uint32_t value_bits, uint32_t den_bits, uint32_t mult) {
    const uint32_t mag = value_bits & 0x7fffffffu;
    const uint32_t ve = (mag >> 23) & 0xffu, de = (den_bits >> 23) & 0xffu;
    const uint32_t vs = ve == 0u ? mag & 0x007fffffu : (mag & 0x007fffffu) | 0x00800000u;
    const uint32_t ds = de == 0u ? den_bits & 0x007fffffu : (den_bits & 0x007fffffu) | 0x00800000u;
    const int vp = ve == 0u ? -149 : int(ve) - 150, dp = de == 0u ? -149 : int(de) - 150;
    const int shift = dp - vp;
    if (ds == 0u) return 0;
    uint64_t num = uint64_t(vs) * mult, den = ds;
    if (shift >= 0) {
        if (shift >= 32) return 0;
        den <<= uint32_t(shift);
    } else {
        if (-shift >= 32) return (value_bits & 0x80000000u) ? -127 : 127;
        num <<= uint32_t(-shift);
    }
    const uint64_t quo = num / den, rem = num % den;
    uint64_t r = quo + (rem * 2u >= den ? 1u : 0u);
    if (r > 127u) r = 127u;
    return (value_bits & 0x80000000u) ? -int(r) : int(r);
}

// round(x / d) for a subnormal, non-zero d: both significands rescaled before the division.
__device__ int q81_round_subnormal_division(uint32_t value_bits, uint32_t d_bits) {
    const uint32_t mag = value_bits & 0x7fffffffu;
    const uint32_t ve = (mag >> 23) & 0xffu;
    const uint32_t vs = ve == 0u ? mag & 0x007fffffu : (mag & 0x007fffffu) | 0x00800000u;
    const uint32_t ds = d_bits & 0x007fffffu;
    if (ds == 0u) return 0;
    const uint32_t vshift = ve == 0u ? 0u : ve - 1u;
    const float sv = float(vs) * float(1u << vshift);
    const float sd = float(ds);
    int m = round_away(__fdiv_rn(sv, sd));
    if (m > 127) m = 127;
    return (value_bits & 0x80000000u) ? -m : m;
}

// round(x / d) for a subnormal x and a normal d: zero unless d's exponent field is 1.
__device__ int q81_round_subnormal_input(uint32_t value_bits, uint32_t d_bits) {
    const uint32_t mag = value_bits & 0x7fffffffu;
    const uint32_t de = (d_bits >> 23) & 0xffu;
    if (mag == 0u || de > 1u) return 0;
    const uint32_t vs = mag & 0x007fffffu;
    const uint32_t ds = (d_bits & 0x007fffffu) | 0x00800000u;
    const int m = round_away(__fdiv_rn(float(vs), float(ds)));
    return (value_bits & 0x80000000u) ? -m : m;
}

// Quantizes value i of a row (its F32 bits vb) into the row's Q8_1 blocks y; all 32 lanes of
// the value's block call it together (lanes 32 apart hold the same position of two blocks).
// amax is reduced over the absolute bit patterns and the sum over the unrounded values, both
// with xor 16, 8, 4, 2, 1 butterflies.
__device__ __forceinline__ void q8_1_value(uint32_t vb, uint8_t* y, uint32_t i) {
    const float xi = bits_f32(vb);
    uint32_t amax = vb & 0x7fffffffu;
    float sum = xi;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) {
        const uint32_t om = uint32_t(__shfl_xor(int(amax), o));
        amax = om > amax ? om : amax;
        sum = sum + __shfl_xor(sum, o);
    }
    const uint32_t ae = (amax >> 23) & 0xffu;
    const uint32_t d_bits = ae <= 7u ? q81_subnormal_scale_bits(amax) : f32_bits(__fdiv_rn(bits_f32(amax), 127.0f));
    const float d = bits_f32(d_bits);
    const uint32_t de = (d_bits >> 23) & 0xffu, ve = (vb >> 23) & 0xffu;
    int q;
    if (amax == 0u) q = 0;
    else if (d_bits == 0u) q = q81_round_ratio(vb, amax, 127u);
    else if (de == 0u) q = q81_round_subnormal_division(vb, d_bits);
    else if (ve == 0u) q = q81_round_subnormal_input(vb, d_bits);
    else q = round_away(__fdiv_rn(xi, d));
    uint8_t* blk = y + uint64_t(i / 32u) * kQ81Bytes;
    blk[4 + (i & 31u)] = uint8_t(int8_t(q));
    if ((i & 31u) == 0u) {
        const uint32_t ds = uint32_t(f16_bits(_Float16(d))) | (uint32_t(f16_bits(_Float16(sum))) << 16);
        *reinterpret_cast<uint32_t*>(blk) = ds;
    }
}

// One thread per value (n is a multiple of 32, so each 32-lane half of a wave exits or stays
// as a whole).
template <bool F32IN>
__global__ __launch_bounds__(256) void q8_1_kernel(const void* x, uint8_t* y, uint32_t n, uint32_t rows) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x, r = blockIdx.y;
    if (r >= rows || i >= n) return;
    const uint32_t vb = F32IN ? reinterpret_cast<const uint32_t*>(x)[uint64_t(r) * n + i]
                              : f32_bits(float(reinterpret_cast<const _Float16*>(x)[uint64_t(r) * n + i]));
    q8_1_value(vb, y + uint64_t(r) * (n / 32u) * kQ81Bytes, i);
}

// The decode SwiGLU fused with the Q8_1 quantization of its output: hidden = silu(g) * u in F32
// (moe.metal:213-221), stored, and quantized for the down mat-vec. One thread per value of a
// rows x n array (n a multiple of 32).
__global__ __launch_bounds__(256) void swiglu_q8_1_kernel(const float* gate, const float* up, float* hidden, uint8_t* y,
                                                          uint32_t n, uint32_t rows) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x, r = blockIdx.y;
    if (r >= rows || i >= n) return;
    const uint64_t at = uint64_t(r) * n + i;
    const float h = silu(gate[at]) * up[at];
    hidden[at] = h;
    q8_1_value(f32_bits(h), y + uint64_t(r) * (n / 32u) * kQ81Bytes, i);
}

// ---- the plan ----------------------------------------------------------------------------
// MoePlan (moe.metal:101-111): 1620 bytes.
struct DecodePlan {
    uint32_t n_groups, n_entries, n_miss, skip;
    int32_t grp_e[80], grp_res[80], grp_start[81], ent_tok[80], ent_dst[80];
};
static_assert(sizeof(DecodePlan) == 1620, "MoePlan layout");

// First-appearance grouping of n = rows * top_k <= 80 entries, one workgroup of 128 or 256
// threads (threads past 127 hold no entry)
// (moe.metal:124-210): entry i's group is the rank of its expert's first appearance among
// first appearances; its slot is the group's start plus the number of earlier entries with
// the same expert. The groups' starts are a prefix sum of their sizes in first-appearance
// order. An id outside [0, E) sets status bit 1 and leaves an empty plan (n_groups = 0).
// ids_lds (may be null): the route ids, already in LDS.
__device__ __forceinline__ void moe_plan_body(const DecodePlanArgs& a, const int32_t* ids_lds = nullptr) {
    __shared__ int32_t e_s[128];
    __shared__ uint32_t mask_s[2][2];
    __shared__ uint32_t size_w[2];
    __shared__ int32_t gstart_s[81], gidx_s[128];
    __shared__ uint32_t bad_s;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t n = a.rows * a.top_k;
    DecodePlan* P = reinterpret_cast<DecodePlan*>(a.plan);
    if (tid == 0) {
        bad_s = 0;
        if (a.status != nullptr) *a.status = 0u;  // the stage's status word starts clear
    }
    const int32_t e = tid < n ? (ids_lds != nullptr ? ids_lds[tid] : a.ids[tid]) : -1;
    if (tid < 128u) e_s[tid] = e;  // a 256-thread workgroup (the fused front launch) runs it too
    __syncthreads();
    if (tid < n && (e < 0 || uint32_t(e) >= a.n_experts)) atomicOr(&bad_s, 1u);
    __syncthreads();
    const bool bad = bad_s != 0u;
    uint32_t first = tid, rank = 0, size = 0;
    if (tid < n) {
        for (uint32_t j = 0; j < tid; ++j)
            if (e_s[j] == e) {
                if (first == tid) first = j;
                ++rank;
            }
        if (first == tid)
            for (uint32_t j = tid; j < n; ++j) size += e_s[j] == e ? 1u : 0u;
    }
    const bool is_first = !bad && tid < n && first == tid;
    // Group index of a first appearance: first appearances before it (ballot prefix).
    const uint64_t m = __ballot(is_first);
    if (lane == 0 && wave < 2u) {
        mask_s[wave][0] = uint32_t(m);
        mask_s[wave][1] = uint32_t(m >> 32);
    }
    // Group start: sizes of earlier first appearances (inclusive scan within the wave).
    uint32_t incl = is_first ? size : 0u;
#pragma unroll
    for (uint32_t off = 1; off < 64u; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off);
        if (lane >= off) incl += y;
    }
    if (lane == 63u && wave < 2u) size_w[wave] = incl;
    __syncthreads();
    const uint64_t m0 = uint64_t(mask_s[0][0]) | (uint64_t(mask_s[0][1]) << 32);
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64u - lane));
    const uint32_t gi = uint32_t(__builtin_popcountll(m & lt)) + (wave == 1u ? uint32_t(__builtin_popcountll(m0)) : 0u);
    const uint32_t start = incl - (is_first ? size : 0u) + (wave == 1u ? size_w[0] : 0u);
    const uint32_t m1c = uint32_t(__builtin_popcountll(uint64_t(mask_s[1][0]) | (uint64_t(mask_s[1][1]) << 32)));
    const uint32_t n_groups = bad ? 0u : uint32_t(__builtin_popcountll(m0)) + m1c;
    // Clear the arrays, then fill (a barrier keeps the clears first).
    if (tid < 80u) {
        P->grp_e[tid] = 0;
        P->grp_res[tid] = 0;
        P->ent_tok[tid] = 0;
        P->ent_dst[tid] = 0;
    }
    if (tid < 81u) P->grp_start[tid] = 0;
    __syncthreads();
    uint32_t res_miss = 0;
    if (is_first) {
        gidx_s[tid] = int32_t(gi);
        gstart_s[gi] = int32_t(start);
        const bool resident = a.resident == nullptr || a.resident[e] >= 0;
        P->grp_e[gi] = e;
        P->grp_start[gi] = int32_t(start);
        P->grp_res[gi] = resident ? 1 : 0;
        res_miss = resident ? 0u : 1u;
    }
    const uint32_t miss_total = __syncthreads_count(res_miss != 0u);
    if (tid == 0) {
        P->n_groups = n_groups;
        P->n_entries = bad ? 0u : n;
        P->n_miss = miss_total;
        P->skip = miss_total == 0u ? 1u : 0u;
        P->grp_start[n_groups] = bad ? 0 : int32_t(n);
        if (bad && a.status != nullptr) atomicOr(a.status, 2u);
    }
    if (!bad && tid < n) {
        const uint32_t slot = uint32_t(gstart_s[gidx_s[first]]) + rank;
        P->ent_dst[slot] = int32_t(tid);
        P->ent_tok[slot] = int32_t(tid / a.top_k);
        // Tiered mode: one use per entry (exact in F32 below 2^24).
        if (a.usage != nullptr) atomicAdd(&a.usage[e], 1.0f);
    }
}

__global__ __launch_bounds__(128) void moe_plan_kernel(DecodePlanArgs a) { moe_plan_body(a); }

// ---- block dots over Q8_1 ----------------------------------------------------------------
__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(int(a), int(b), c, false);
}

// A Q8_1 block of an activation row: its 8 code words and the float d.
struct Act {
    uint32_t q[8];
    float d;
};
__device__ __forceinline__ Act load_act(const uint8_t* blk) {  // 36-byte blocks: 4-byte aligned
    Act a;
#pragma unroll
    for (int i = 0; i < 8; ++i) a.q[i] = ld_global<uint32_t>(blk + 4 + 4 * i);
    a.d = f16_lo(ld_global<uint32_t>(blk));
    return a;
}

// Weight side of a row, per format, in units that a lane takes whole: a Q4_K or Q2_K
// super-block (256 values) or a pair of Q8_0 blocks (64 values). raw() issues the unit's
// loads (kRaw dwords, every byte of the unit, nothing else); dot() takes sub-block s (32
// values) of the loaded unit against one activation block.
typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

struct UnitQ80 {  // 2 x 34 B: d0, q0[32], d1, q1[32]; 4-byte aligned (rows hold whole pairs)
    static constexpr uint32_t kVals = 64, kSub = 2, kRaw = 17;
    __device__ __forceinline__ static void raw(const uint8_t* row, uint32_t u, uint32_t* r) {
        const uint8_t* p = row + 68u * u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const u32x4a v = ld_global<u32x4a>(p + 16 * i);
#pragma unroll
            for (int j = 0; j < 4; ++j) r[4 * i + j] = v[j];
        }
        r[16] = ld_global<uint32_t>(p + 64);
    }
    __device__ __forceinline__ static float dot(const uint32_t* r, uint32_t sb, const Act& x, float acc) {
        // block 0: d in bytes 0-1, codes in bytes 2..33; block 1: d in bytes 34-35, codes 36..67
        int s = 0;
        float d;
        if (sb == 0u) {
#pragma unroll
            for (int i = 0; i < 8; ++i) s = sdot4(__builtin_amdgcn_alignbyte(r[i + 1], r[i], 2), x.q[i], s);
            d = f16_lo(r[0]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) s = sdot4(r[9 + i], x.q[i], s);
            d = f16_hi(r[8]);
        }
        return __builtin_fmaf(d * x.d, float(s), acc);  // moe/native table: fma(d0 * d1, float(sumi), acc)
    }
};

struct UnitQ4K {  // 144 B: d, dmin, scales[12], qs[128]; 16-byte aligned
    static constexpr uint32_t kVals = 256, kSub = 8, kRaw = 36;
    __device__ __forceinline__ static void raw(const uint8_t* row, uint32_t u, uint32_t* r) {
        const uint8_t* p = row + 144u * u;
#pragma unroll
        for (int i = 0; i < 9; ++i) {
            const u32x4 v = ld_global<u32x4>(p + 16 * i);
#pragma unroll
            for (int j = 0; j < 4; ++j) r[4 * i + j] = v[j];
        }
    }
    __device__ __forceinline__ static float dot(const uint32_t* r, uint32_t j, const Act& x, float acc) {
        // Sub-block j: the low (j even) or high nibbles of qs bytes 32 (j/2) .. +32, i.e. words
        // 4 + 8 (j/2) .. +8; get_scale_min_k4 (dequant.hpp:157-190) over header bytes 4..15.
        const uint32_t sh = 4u * (j & 1u), q0 = 4u + 8u * (j >> 1);
        auto byte = [&](uint32_t k) { return (r[1 + k / 4] >> (8u * (k & 3u))) & 0xffu; };
        int sc, mn;
        if (j < 4) {
            sc = int(byte(j) & 63u);
            mn = int(byte(j + 4) & 63u);
        } else {
            sc = int((byte(j + 4) & 0xFu) | ((byte(j - 4) >> 6) << 4));
            mn = int((byte(j + 4) >> 4) | ((byte(j) >> 6) << 4));
        }
        int s = 0, t = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s = sdot4((r[q0 + i] >> sh) & 0x0F0F0F0Fu, x.q[i], s);
            t = sdot4(0x01010101u, x.q[i], t);
        }
        const float sd = x.d * float(s * sc), sm = x.d * float(t * mn);
        return acc + __builtin_fmaf(-f16_hi(r[0]), sm, f16_lo(r[0]) * sd);  // q4_K: fma(-dm.y, sm, dm.x * sd), then acc + v
    }
};

struct UnitQ2K {  // 84 B: scales[16] @0, q[64] @16, d @80, dmin @82; 4-byte aligned
    static constexpr uint32_t kVals = 256, kSub = 8, kRaw = 21;
    __device__ __forceinline__ static void raw(const uint8_t* row, uint32_t u, uint32_t* r) {
        const uint8_t* p = row + 84u * u;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const u32x4a v = ld_global<u32x4a>(p + 16 * i);
#pragma unroll
            for (int j = 0; j < 4; ++j) r[4 * i + j] = v[j];
        }
        r[20] = ld_global<uint32_t>(p + 80);
    }
    __device__ __forceinline__ static float dot(const uint32_t* r, uint32_t bb, const Act& x, float acc) {
        // Values 128n + 32j + w (w < 32) use bits 2j of q[32n + w]; scale byte 8n + 2j + (w >= 16).
        const uint32_t nn = bb >> 2, j = bb & 3u;
        const uint32_t scw = r[2 * nn + (j >> 1)];
        const uint32_t s0 = (scw >> (16u * (j & 1u))) & 0xffu, s1 = (scw >> (16u * (j & 1u) + 8u)) & 0xffu;
        int a0 = 0, a1 = 0, t0 = 0, t1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            a0 = sdot4((r[4 + 8 * nn + i] >> (2u * j)) & 0x03030303u, x.q[i], a0);
            t0 = sdot4(0x01010101u, x.q[i], t0);
            a1 = sdot4((r[4 + 8 * nn + 4 + i] >> (2u * j)) & 0x03030303u, x.q[4 + i], a1);
            t1 = sdot4(0x01010101u, x.q[4 + i], t1);
        }
        const float sd = x.d * float(a0 * int(s0 & 0xFu) + a1 * int(s1 & 0xFu));
        const float sm = x.d * float(t0 * int(s0 >> 4) + t1 * int(s1 >> 4));
        return acc + __builtin_fmaf(-f16_hi(r[20]), sm, f16_lo(r[20]) * sd);
    }
};

// ---- grouped mat-vecs --------------------------------------------------------------------
// Group g = blockIdx.y (blocks past n_groups exit). LPR lanes share a weight row (its unit
// count where that is 6 or 10, which leaves 4 of a wave's 64 lanes idle, else the smallest
// power of two covering its units), each lane taking one whole unit, so a row's bytes are all
// in flight at once and every byte loaded is used. A workgroup takes `iters`
// consecutive slices of 4 * 64/LPR rows of the stage (gate/up: gate rows 0..I-1 then up rows
// I..2I-1; down: output rows 0..d-1), one row per LPR-lane segment of a wave. The group's
// activation blocks are staged in LDS once. Each lane keeps one accumulator per entry of the
// group, a butterfly over the row's lanes finishes the row, and finished rows go to LDS; the
// workgroup stores them after its last slice, consecutive lanes on consecutive columns (a
// global store inside the loop would hold its registers until it completes).

// A group holds at most one entry per token (a token's top-k experts are distinct), so at most
// max_group = T entries: the LDS staging is sized for that, and a larger group is a bad plan.

__host__ __device__ constexpr uint32_t matvec_rows_per_block(uint32_t lpr) { return 4u * (64u / lpr); }

template <class Unit, int MODE, uint32_t LPR>
__global__ __launch_bounds__(256, 4) void moe_matvec_kernel(DecodeMatvec m) {  // >= 4 waves per SIMD
    constexpr uint32_t RPW = 64u / LPR, RPI = 4u * RPW;  // rows per wave, rows per slice
    constexpr bool kPow2 = (LPR & (LPR - 1u)) == 0u;
    // LDS: codes [entry][block] (8 words), then d [entry][block], then results [slice row][entry]
    extern __shared__ uint32_t act_s[];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t g = blockIdx.y;
    const DecodePlan* P = reinterpret_cast<const DecodePlan*>(m.plan);
    if (g >= 80u) return;
    // A plan whose header is unusable: workgroup (0, 0) reports it and zeroes every output row
    // this stage could have written.
    // Every plan field this workgroup needs, read in one round trip (g < 80: all inside the plan).
    const uint32_t p_entries = P->n_entries, p_groups = P->n_groups;
    const int32_t p_s = P->grp_start[g], p_t = P->grp_start[g + 1], p_e = P->grp_e[g];
    const bool plan_ok = p_entries == m.n_entries && p_groups <= m.n_entries;  // a group holds >= 1 entry
    if (!plan_ok) {
        if (g != 0u || blockIdx.x != 0u) return;
        if (tid == 0) atomicOr(m.status, 2u);
        const uint64_t total = uint64_t(m.n_entries) * m.out_width;
        float* outs[2] = {m.out0, MODE == kGateUp ? m.out1 : nullptr};
        for (int o = 0; o < 2; ++o)
            if (outs[o] != nullptr)
                for (uint64_t i = tid; i < total; i += 256u) outs[o][i] = 0.0f;
        return;
    }
    if (g >= p_groups) return;
    if (p_groups == 0u || p_s < 0 || p_t <= p_s || uint32_t(p_t) > m.n_entries || uint32_t(p_t - p_s) > m.max_group ||
        p_e < 0 || uint32_t(p_e) >= m.n_experts) {
        if (tid == 0 && blockIdx.x == 0u) atomicOr(m.status, 2u);
        return;  // the group's rows cannot be named: the whole stage's status reports it
    }
    const uint32_t a0 = uint32_t(p_s), a1 = uint32_t(p_t), ex = uint32_t(p_e);
    const uint32_t n_e = a1 - a0;
    // Entries: activation row (gate/up: the token; down: the grouped entry) and output row
    // (gate/up: the grouped entry; down: the route index from ent_dst).
    uint32_t arow[8], orow[8];
    bool entries_ok = true;
#pragma unroll
    for (uint32_t c = 0; c < 8u; ++c) {
        const uint32_t a = a0 + (c < n_e ? c : n_e - 1u);
        if (MODE == kGateUp) {
            const int32_t t = P->ent_tok[a];
            entries_ok = entries_ok && t >= 0 && uint32_t(t) < m.act_rows;
            arow[c] = uint32_t(t);
            orow[c] = a;
        } else {
            const int32_t dd = P->ent_dst[a];
            entries_ok = entries_ok && dd >= 0 && uint32_t(dd) < m.n_entries;
            arow[c] = a;
            orow[c] = uint32_t(dd);
        }
    }
    const uint64_t* addr = m.addresses + 3u * ex;
    const uint8_t* w0 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[0] : addr[2]);
    const uint8_t* w1 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[1] : addr[2]);
    const uint32_t fault = entries_ok ? weight_fault(w0, w1) : 2u;
    const uint32_t n_rows = MODE == kGateUp ? 2u * m.out_width : m.out_width;
    const uint32_t rows_wg = m.iters * RPI, r_first = rows_wg * blockIdx.x;
    if (fault != 0u) {
        // The group's output rows of this workgroup are zeroed; the status reports the fault.
        for (uint32_t i = r_first + tid; i < min(n_rows, r_first + rows_wg); i += 256u) {
            const bool up = MODE == kGateUp && i >= m.out_width;
            float* out = up ? m.out1 : m.out0;
            const uint32_t col = up ? i - m.out_width : i;
            for (uint32_t c = 0; c < n_e; ++c)  // a damaged entry's row cannot be named: skipped
                if (orow[c] < m.n_entries) out[uint64_t(orow[c]) * m.out_width + col] = 0.0f;
        }
        if (tid == 0 && blockIdx.x == 0u) atomicOr(m.status, fault);
        return;
    }
    const uint32_t nblk = m.k / 32u, nunit = m.k / Unit::kVals;
    const uint32_t seg = lane % LPR, rin = lane / LPR;
    const bool lane_ok = rin < RPW;  // lanes past the wave's last whole row segment (LPR 6 or 10) idle
    const bool unit_ok = lane_ok && seg < nunit;
    const uint32_t u = unit_ok ? seg : nunit - 1u;
    auto row_ptr = [&](uint32_t it) {  // this lane's row of slice it (clamped into the stage)
        const uint32_t row = r_first + it * RPI + wave * RPW + (lane_ok ? rin : 0u);
        const uint32_t rowc = row < n_rows ? row : n_rows - 1u;
        const bool up = MODE == kGateUp && rowc >= m.out_width;
        return (up ? w1 : w0) + uint64_t(up ? rowc - m.out_width : rowc) * m.row_bytes;
    };
    uint32_t* codes_s = act_s;                                               // [entry][block][8]
    float* d_s = reinterpret_cast<float*>(act_s + m.max_group * nblk * 8u);  // [entry][block]
    float* res_s = d_s + m.max_group * nblk;                                 // [slice row][entry]
    // Stage the group's activation blocks (n_e rows of nblk Q8_1 blocks) into LDS. The first
    // kStageRegs words per thread are loaded into registers before the first slice's weight
    // units are requested and stored after, so the two round trips overlap (the loads return in
    // order, so storing the staged words waits only for them); the barrier then waits for the
    // LDS stores alone and leaves the weight loads in flight.
    constexpr uint32_t kStageRegs = 4;
    const uint32_t n_words = n_e * nblk * 9u;  // >= 9
    const uint32_t d_base = m.max_group * nblk * 8u;
    auto stage_src = [&](uint32_t i) {
        const uint32_t c = i / (nblk * 9u), rem = i - c * nblk * 9u, b = rem / 9u, w = rem - b * 9u;
        return m.act + (uint64_t(arow[c]) * nblk + b) * kQ81Bytes + 4u * w;
    };
    // LDS word of staged word i: its block's d (as F32) or one of its 8 code words.
    auto stage_dst = [&](uint32_t i, uint32_t& v) {
        const uint32_t c = i / (nblk * 9u), rem = i - c * nblk * 9u, b = rem / 9u, w = rem - b * 9u;
        v = w == 0u ? f32_bits(f16_lo(v)) : v;
        return w == 0u ? d_base + c * nblk + b : (c * nblk + b) * 8u + (w - 1u);
    };
    // Branch-free, so the stores wait for the staged words only: loads clamped into the range,
    // and a thread past it stores to the first result word, which the first slice overwrites.
    uint32_t sv[kStageRegs];
#pragma unroll
    for (uint32_t j = 0; j < kStageRegs; ++j) {
        const uint32_t i = tid + 256u * j;
        sv[j] = ld_global<uint32_t>(stage_src(i < n_words ? i : n_words - 1u));
    }
    uint32_t r[Unit::kRaw];
    Unit::raw(row_ptr(0u), u, r);
#pragma unroll
    for (uint32_t j = 0; j < kStageRegs; ++j) {
        const uint32_t i = tid + 256u * j;
        uint32_t v = sv[j];
        const uint32_t at = stage_dst(i < n_words ? i : n_words - 1u, v);
        act_s[i < n_words ? at : d_base + m.max_group * nblk] = v;
    }
    if (n_words > 256u * kStageRegs)  // more than eight entries' worth at d = 2560: the rest in the plain way
        for (uint32_t i = tid + 256u * kStageRegs; i < n_words; i += 256u) {
            uint32_t v = ld_global<uint32_t>(stage_src(i));
            const uint32_t at = stage_dst(i, v);  // converts v first
            act_s[at] = v;
        }
    __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    for (uint32_t it = 0; it < m.iters; ++it) {
        const uint32_t lr = it * RPI + wave * RPW + (lane_ok ? rin : 0u);
        if (it > 0u) Unit::raw(row_ptr(it), u, r);
        // One entry at a time (n_e is uniform over the workgroup): the unit's sub-blocks against
        // the entry's activation blocks, then the butterfly over the row's LPR lanes.
        for (uint32_t c = 0; c < n_e; ++c) {
            // Opaque to the optimiser, so the codes are decoded per entry instead of all eight
            // sub-blocks being decoded once and held (64 more registers).
#pragma unroll
            for (uint32_t i = 0; i < Unit::kRaw; ++i) __asm__ volatile("" : "+v"(r[i]));
            float acc = 0.0f;
            if (unit_ok) {
#pragma unroll
                for (uint32_t sb = 0; sb < Unit::kSub; ++sb) {
                    const uint32_t b = u * Unit::kSub + sb;
                    const uint32_t* cs = codes_s + (c * nblk + b) * 8u;
                    const u32x4 qa = *reinterpret_cast<const u32x4*>(cs), qb = *reinterpret_cast<const u32x4*>(cs + 4);
                    Act a;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        a.q[i] = qa[i];
                        a.q[4 + i] = qb[i];
                    }
                    a.d = d_s[c * nblk + b];
                    acc = Unit::dot(r, sb, a, acc);
                    // The next pair's LDS reads stay below this pair's dots (register budget).
                    if (sb & 1u) __builtin_amdgcn_sched_barrier(0);
                }
            }
            if constexpr (kPow2) {
#pragma unroll
                for (uint32_t o = LPR / 2u; o > 0u; o >>= 1) acc = acc + __shfl_xor(acc, int(o));
            } else {
                // A tree within the row's segment: at stride o, segment lane s (s % 2o == 0) adds
                // lane s + o when that lies inside the segment; the sum ends in segment lane 0.
#pragma unroll
                for (uint32_t o = 1u; o < LPR; o <<= 1) {
                    const float v = __shfl(acc, int(lane + o < 64u ? lane + o : 63u));
                    if (seg % (2u * o) == 0u && seg + o < LPR) acc = acc + v;
                }
            }
            if (lane_ok && seg == 0u) res_s[lr * m.max_group + c] = acc;
        }
    }
    __syncthreads();  // every slice's rows are in LDS
    for (uint32_t i = tid; i < rows_wg * n_e; i += 256u) {
        const uint32_t c = i / rows_wg, lr = i - c * rows_wg, row = r_first + lr;
        if (row >= n_rows) continue;
        const bool up = MODE == kGateUp && row >= m.out_width;
        float* out = up ? m.out1 : m.out0;
        const uint32_t col = up ? row - m.out_width : row;
        out[uint64_t(orow[c]) * m.out_width + col] = res_s[lr * m.max_group + c];
    }
}

// ---- dense mat-vecs: the shared expert (F16 / BF16 weights) and the router (F32 weights) --
// 4 * 64/LPR output rows per workgroup, one per LPR-lane segment of a wave; the row's lanes
// take 16-byte weight chunks lane % LPR + LPR * i (8 F16/BF16 values or 4 F32 values), up to
// kPerLane at once before using any, and keep one accumulator per activation row (two in
// gate/up: the gate and up rows of the same output column); a butterfly finishes each row.
// gate/up applies the F32 SwiGLU silu(g) * u before its one store (the reference's shx
// SwiGLU, moe.metal:243-251); the router adds the bias after the dot.
enum { kWF16 = 0, kWBF16 = 1, kWF32 = 2 };
constexpr uint32_t kPerLane = 4;

// The shared expert's sigmoid-gate logits gl[t] = x_t . gv (one workgroup: wave w takes
// tokens w and w + 4; each lane 8 consecutive values per 16-byte load into two partial sums,
// then a fixed xor butterfly).
template <int WT>
__device__ __forceinline__ void gate_logit_block(const DenseDecode& m) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    const _Float16* x = reinterpret_cast<const _Float16*>(m.x);
    for (uint32_t t = wave; t < m.rows; t += 4u) {
        float s0 = 0.0f, s1 = 0.0f;
        for (uint32_t k = 8u * lane; k < m.k; k += 512u) {
            const half8 xv = ld_global<half8>(x + uint64_t(t) * m.k + k);
            const u32x4 wv = ld_global<u32x4>(m.gv + 2u * k);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t pair = wv[i];
                const float w0 = WT == kWBF16 ? bits_f32(pair << 16) : f16_lo(pair);
                const float w1 = WT == kWBF16 ? bits_f32(pair & 0xffff0000u) : f16_hi(pair);
                s0 = __builtin_fmaf(float(xv[2 * i]), w0, s0);
                s1 = __builtin_fmaf(float(xv[2 * i + 1]), w1, s1);
            }
        }
        float sum = s0 + s1;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sum = sum + __shfl_xor(sum, off);
        if (lane == 0) m.gl[t] = sum;
    }
}

// Workgroup bx of nb of one dense mat-vec (a launch of its own, or one part of a fused launch),
// x_lds its dynamic LDS.
template <int WT, bool GATE_UP, bool XF32, uint32_t LPR>
__device__ __forceinline__ void dense_decode_body(const DenseDecode& m, uint32_t bx, uint32_t nb, uint8_t* x_lds) {
    if (GATE_UP && m.gv != nullptr && bx == nb - 1u) {
        gate_logit_block<WT>(m);  // the job's last workgroup
        return;
    }
    if (!GATE_UP && bx >= m.row_blocks) {
        // The router launch's extra workgroups: one 8-byte word each per thread of the
        // validated address tables (pinned ring slots) into their device snapshots, read once
        // across PCIe beside the router's own work.
        const uint32_t w = (bx - m.row_blocks) * 256u + threadIdx.x;
        if (w < m.snap_words) m.snap_dst[w] = m.snap_src[w];
        else if (w - m.snap_words < m.snap_words2) m.snap_dst2[w - m.snap_words] = m.snap_src2[w - m.snap_words];
        return;
    }
    constexpr uint32_t RPW = 64u / LPR;
    constexpr uint32_t NW = GATE_UP ? 2u : 1u;
    constexpr uint32_t VPC = WT == kWF32 ? 4u : 8u;  // values per 16-byte chunk
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    // The T activation rows ([rows][k], F16 or F32) are staged in LDS once per workgroup: every
    // weight chunk meets all T rows, and LDS reads cost far less issue than a global load per
    // (chunk, row). The copy is LDS-DMA, 1 KB per wave instruction (the allocation is rounded up
    // to whole kilobytes; lanes past the rows' end re-read their last 16 bytes into that tail),
    // issued before the first weight loads so that both are one round trip.
    {
        const uint32_t xbytes = m.rows * m.k * (XF32 ? 4u : 2u);  // k % 64 == 0: whole 16-byte pieces
        const uint8_t* xg = reinterpret_cast<const uint8_t*>(m.x);
        for (uint32_t q = wave; q < (xbytes + 1023u) / 1024u; q += 4u) {
            const uint32_t off = 1024u * q + 16u * lane;
            __builtin_amdgcn_global_load_lds(
                reinterpret_cast<const __attribute__((address_space(1))) void*>(
                    reinterpret_cast<uintptr_t>(xg + (off < xbytes ? off : xbytes - 16u))),
                reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(x_lds + 1024u * q)),
                16, 0, 0);
        }
    }
    const uint32_t nch = m.k / VPC;
    const uint32_t per_lane = (nch + LPR - 1u) / LPR;
    const uint32_t row = matvec_rows_per_block(LPR) * bx + wave * RPW + lane / LPR;
    const bool row_ok = row < m.n_out;  // uniform within each LPR-lane segment
    const uint32_t wbytes = WT == kWF32 ? 4u : 2u;
    float acc[NW][8];
#pragma unroll
    for (uint32_t w = 0; w < NW; ++w)
#pragma unroll
        for (uint32_t t = 0; t < 8u; ++t) acc[w][t] = 0.0f;
    const uint8_t* wr[2] = {m.w0 + uint64_t(row_ok ? row : 0u) * m.k * wbytes,
                            GATE_UP ? m.w1 + uint64_t(row_ok ? row : 0u) * m.k * wbytes : nullptr};
    // Chunks in flight per lane (at most): ten for the router's F32 rows, eight for F16/BF16
    // rows, so the rows of the reference model's widths (2560 values: ten F32 or five F16 chunks
    // per lane of a 64-lane row) are one round trip.
    constexpr uint32_t NB = WT == kWF32 ? 10u : 8u;
    u32x4 raw[NW][NB];
    auto load_batch = [&](uint32_t base) {
#pragma unroll
        for (uint32_t i = 0; i < NB; ++i) {
            const uint32_t c = lane % LPR + LPR * (base + i);
            if (c < nch)
#pragma unroll
                for (uint32_t w = 0; w < NW; ++w) raw[w][i] = ld_global<u32x4>(wr[w] + 16u * c);
        }
    };
    if (row_ok) load_batch(0u);
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the staged rows (and the first weights)
    __syncthreads();
    if (row_ok) {
        for (uint32_t base = 0; base < per_lane; base += NB) {
            if (base > 0u) load_batch(base);
#pragma unroll
            for (uint32_t i = 0; i < NB; ++i) {
                const uint32_t c = lane % LPR + LPR * (base + i);
                if (c >= nch) continue;
                float wv[NW][VPC];
#pragma unroll
                for (uint32_t w = 0; w < NW; ++w)
#pragma unroll
                    for (uint32_t j = 0; j < 4u; ++j) {
                        const uint32_t q = raw[w][i][j];
                        if (WT == kWF32) {
                            wv[w][j] = bits_f32(q);
                        } else if (WT == kWBF16) {
                            wv[w][2 * j] = bits_f32(q << 16);
                            wv[w][2 * j + 1] = bits_f32(q & 0xffff0000u);
                        } else {
                            wv[w][2 * j] = f16_lo(q);
                            wv[w][2 * j + 1] = f16_hi(q);
                        }
                    }
#pragma unroll
                for (uint32_t t = 0; t < 8u; ++t) {
                    if (t >= m.rows) break;
                    float xv[VPC];
                    if (XF32) {
                        const float* xp = reinterpret_cast<const float*>(x_lds) + t * m.k + VPC * c;
                        const float4v a = *reinterpret_cast<const float4v*>(xp);
#pragma unroll
                        for (uint32_t j = 0; j < 4u; ++j) xv[j] = a[j];
                        if (VPC == 8u) {
                            const float4v b = *reinterpret_cast<const float4v*>(xp + 4);
#pragma unroll
                            for (uint32_t j = 0; j < 4u; ++j) xv[(4u + j) % VPC] = b[j];
                        }
                    } else {
                        const uint8_t* xp = x_lds + (t * m.k + VPC * c) * 2u;
                        if (VPC == 8u) {
                            const u32x4 q = *reinterpret_cast<const u32x4*>(xp);
#pragma unroll
                            for (uint32_t j = 0; j < 4u; ++j) {
                                xv[(2u * j) % VPC] = f16_lo(q[j]);
                                xv[(2u * j + 1u) % VPC] = f16_hi(q[j]);
                            }
                        } else {
                            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                            const u32x2 q = *reinterpret_cast<const u32x2*>(xp);
                            xv[0] = f16_lo(q[0]);
                            xv[1] = f16_hi(q[0]);
                            xv[2 % VPC] = f16_lo(q[1]);
                            xv[3 % VPC] = f16_hi(q[1]);
                        }
                    }
#pragma unroll
                    for (uint32_t w = 0; w < NW; ++w)
#pragma unroll
                        for (uint32_t j = 0; j < VPC; ++j) acc[w][t] = __builtin_fmaf(wv[w][j], xv[j], acc[w][t]);
                }
            }
        }
    }
#pragma unroll
    for (uint32_t w = 0; w < NW; ++w)
#pragma unroll
        for (uint32_t t = 0; t < 8u; ++t)
            if (t < m.rows)
#pragma unroll
                for (uint32_t o = LPR / 2u; o > 0u; o >>= 1) acc[w][t] = acc[w][t] + __shfl_xor(acc[w][t], int(o));
    if (row_ok && lane % LPR == 0u) {
        const float b = (!GATE_UP && m.bias != nullptr) ? m.bias[row] : 0.0f;
#pragma unroll
        for (uint32_t t = 0; t < 8u; ++t)
            if (t < m.rows)
                m.out[uint64_t(t) * m.n_out + row] = GATE_UP ? silu(acc[0][t]) * acc[NW - 1][t] : acc[0][t] + b;
    }
}

template <int WT, bool GATE_UP, bool XF32, uint32_t LPR>
__global__ __launch_bounds__(256) void dense_decode_kernel(DenseDecode m) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t x_lds[];
    dense_decode_body<WT, GATE_UP, XF32, LPR>(m, blockIdx.x, gridDim.x, x_lds);
}

// The decode layer's router (F32 rows, with its snapshot copies) and its shared expert's gate/up
// (F16/BF16 rows, with the gate logit) in one launch: both read only the layer's F16 input
// rows, staged alike, and neither reads what the other writes. Workgroups [0, r_blocks) are the
// router's, the rest the shared gate/up's.
template <int WT, uint32_t LPR>
__global__ __launch_bounds__(256) void router_shared_decode_kernel(DenseDecode r, DenseDecode g, uint32_t r_blocks) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t x_lds[];
    if (blockIdx.x < r_blocks) dense_decode_body<kWF32, false, false, LPR>(r, blockIdx.x, r_blocks, x_lds);
    else dense_decode_body<WT, true, false, LPR>(g, blockIdx.x - r_blocks, gridDim.x - r_blocks, x_lds);
}

// A decode layer's front launch after the router: the plan (workgroup 0; with a.logits, the
// top-k first, its ids handed to the plan through LDS), the Q8_1 quantization of the F16 input
// rows (the next q_blocks workgroups, 256 values each) and the shared expert's down mat-vec
// (the remaining workgroups, F32 hidden rows; WT < 0: none). None of the three reads what
// another writes.
template <int WT, uint32_t LPR>
__global__ __launch_bounds__(256) void decode_front_kernel(DecodePlanArgs a, const _Float16* x, uint8_t* y, uint32_t n,
                                                           uint32_t q_blocks, DenseDecode sd) {
    extern __shared__ __attribute__((aligned(1024))) uint8_t x_lds[];
    if (blockIdx.x == 0) {
        if (a.logits == nullptr) {
            moe_plan_body(a);
            return;
        }
        // The route first: up to 4 tokens one per wave, up to 8 two per wave (slots for E <= 512).
        __shared__ int32_t ids_s[80];
        const uint32_t wave = threadIdx.x >> 6;
        if (a.rows <= 4u)
            topk_token<8, true>(a.logits, a.route_ids, a.route_weights, a.rows, a.n_experts, a.top_k, 0, nullptr, wave,
                                ids_s);
        else
            topk_token<16, false>(a.logits, a.route_ids, a.route_weights, a.rows, a.n_experts, a.top_k, 0, nullptr,
                                  threadIdx.x >> 5, ids_s);
        __syncthreads();
        moe_plan_body(a, ids_s);
        return;
    }
    if (blockIdx.x <= q_blocks) {
        const uint32_t per_row = (n + 255u) / 256u, b = blockIdx.x - 1u;
        const uint32_t r = b / per_row, i = (b - r * per_row) * 256u + threadIdx.x;
        if (i >= n) return;  // n % 32 == 0: whole 32-lane blocks leave together
        q8_1_value(f32_bits(float(x[uint64_t(r) * n + i])), y + uint64_t(r) * (n / 32u) * kQ81Bytes, i);
        return;
    }
    if constexpr (WT >= 0) {
        const uint32_t first = 1u + q_blocks;
        dense_decode_body<WT, false, true, LPR>(sd, blockIdx.x - first, gridDim.x - first, x_lds);
    }
}

// Lanes per weight row: the smallest power of two from 8 to 64 that leaves each lane at most
// kPerLane 16-byte chunks of a row of k values (VPC values per chunk).
__host__ __device__ constexpr uint32_t dense_lpr(uint32_t k, uint32_t vpc) {
    uint32_t lpr = 8;
    while (lpr < 64u && (k / vpc + lpr - 1u) / lpr > kPerLane) lpr <<= 1;
    return lpr;
}

// Workgroups of one dense job: its row blocks, then the gate-logit workgroup (gate/up with a
// gate vector) or the snapshot-copy workgroups (router). Sets m.row_blocks.
inline uint32_t dense_blocks(DenseDecode& m, bool gate_up, uint32_t lpr) {
    m.row_blocks = (m.n_out + matvec_rows_per_block(lpr) - 1u) / matvec_rows_per_block(lpr);
    const uint32_t extra = gate_up ? (m.gv != nullptr ? 1u : 0u) : (m.snap_words + m.snap_words2 + 255u) / 256u;
    return m.row_blocks + extra;
}

template <int WT, bool GATE_UP, bool XF32>
hipError_t launch_dense_decode_t(const DenseDecode& m, hipStream_t s) {
    const uint32_t lpr = dense_lpr(m.k, WT == kWF32 ? 4u : 8u);
    DenseDecode mm = m;
    const dim3 grid(dense_blocks(mm, GATE_UP, lpr));
    // The staged activation rows: rows x k values, at most 8 x SM_DECODE_MAX_WIDTH F32 (128 KB),
    // rounded up to whole kilobytes (the copy's unit).
    const size_t lds = (size_t(m.rows) * m.k * (XF32 ? 4u : 2u) + 1023u) & ~size_t(1023);
    if (lds > 131072u) return hipErrorInvalidValue;
    auto go = [&](auto kern) {
        // Above 64 KB of dynamic LDS the launch needs the kernel's limit raised first (the
        // widest rows only: T = 8 at K >= 2048 with F32 rows, or K = 4096 with F16 rows).
        if (lds > 65536u) {
            const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
            if (attr != hipSuccess) return attr;
        }
        kern<<<grid, 256, lds, s>>>(mm);
        return hipGetLastError();
    };
    switch (lpr) {
        case 64: return go(dense_decode_kernel<WT, GATE_UP, XF32, 64>);
        case 32: return go(dense_decode_kernel<WT, GATE_UP, XF32, 32>);
        case 16: return go(dense_decode_kernel<WT, GATE_UP, XF32, 16>);
        default: return go(dense_decode_kernel<WT, GATE_UP, XF32, 8>);
    }
}

// ---- post ops ----------------------------------------------------------------------------
// eh = silu(g) * u in F32 (moe.metal:213-221).
__global__ __launch_bounds__(256) void swiglu_f32_kernel(const float* gate, const float* up, float* out, uint64_t n) {
    const uint64_t i = uint64_t(blockIdx.x) * 256u + threadIdx.x;
    if (i < n) out[i] = silu(gate[i]) * up[i];
}

// The decode combine (moe.metal:253-274): the first rank is a product, the others fma in
// rank order, and the gated shared output is added last. The ranks' values are loaded eight at
// a time (a rank past top_k reloads the last one and is not used) before their fmas, so a
// thread keeps eight loads in flight instead of paying one round trip per rank.
constexpr uint32_t kCombineBatch = 8;
__global__ __launch_bounds__(256) void combine_decode_kernel(const float* parts, const float* w, const float* shared,
                                                             const float* gl, float* out, uint32_t top_k, uint32_t d) {
    const uint32_t t = blockIdx.y, c = blockIdx.x * 256u + threadIdx.x;
    if (c >= d) return;
    const float* p = parts + uint64_t(t) * top_k * d + c;
    const float* wt = w + uint64_t(t) * top_k;
    // The shared row's value and gate logit go out with the first batch.
    const float sh = shared != nullptr ? shared[uint64_t(t) * d + c] : 0.0f;
    const float g = shared != nullptr ? gl[t] : 0.0f;
    float s = 0.0f;
    for (uint32_t k0 = 0; k0 < top_k; k0 += kCombineBatch) {
        float pv[kCombineBatch];
#pragma unroll
        for (uint32_t j = 0; j < kCombineBatch; ++j) {
            const uint32_t k = k0 + j < top_k ? k0 + j : top_k - 1u;
            pv[j] = p[uint64_t(k) * d];
        }
#pragma unroll
        for (uint32_t j = 0; j < kCombineBatch; ++j) {
            const uint32_t k = k0 + j;
            if (k < top_k) s = k == 0u ? pv[j] * wt[0] : __builtin_fmaf(pv[j], wt[k], s);
        }
    }
    out[uint64_t(t) * d + c] = shared != nullptr ? s + sh * sigmoid(g) : s;
}

// Copies a validated address table (pinned host ring slot) into its device snapshot and clears
// the stage's status word (a standalone expert stage, whose plan came from elsewhere).
__global__ __launch_bounds__(256) void snapshot_copy_kernel(const uint64_t* src, uint64_t* dst, uint32_t words,
                                                            uint32_t* status) {
    for (uint32_t w = threadIdx.x; w < words; w += 256u) dst[w] = src[w];
    if (threadIdx.x == 0 && status != nullptr) *status = 0u;
}

template <class Unit, int MODE>
hipError_t launch_matvec_t(const DecodeMatvec& mm, hipStream_t s) {
    DecodeMatvec m = mm;
    const uint32_t n_rows = MODE == kGateUp ? 2u * m.out_width : m.out_width;
    const uint32_t nblk = m.k / 32u, nunit = m.k / Unit::kVals;
    if (nunit == 0u || nunit > 64u || m.k % Unit::kVals != 0u) return hipErrorInvalidValue;  // host-checked
    if (m.max_group == 0u || m.max_group > 8u || m.n_entries == 0u || m.n_entries > 80u) return hipErrorInvalidValue;
    uint32_t lpr = 1;
    while (lpr < nunit) lpr <<= 1;
    if (lpr < 8u) lpr = 8u;
    if (nunit == 10u || nunit == 6u) lpr = nunit;  // 60 of 64 lanes busy instead of 40 or 48
    // Slices per workgroup: up to 4 once the groups (at most one per routed entry) give the
    // chip about four workgroups per CU without them; one when there are few groups (T = 1).
    const uint32_t rpi = matvec_rows_per_block(lpr);
    const uint32_t slices = (n_rows + rpi - 1u) / rpi;
    const uint32_t per_iter = m.n_entries * slices;  // workgroups at one slice each (upper bound)
    m.iters = per_iter >= 4096u ? 4u : per_iter >= 2048u ? 2u : 1u;
    // One grid row per possible group: a valid plan has at most one group per entry (<= 80).
    const dim3 grid((slices + m.iters - 1u) / m.iters, m.n_entries);
    const size_t lds = size_t(m.max_group) * nblk * 9u * 4u + size_t(m.iters) * rpi * m.max_group * 4u;
    switch (lpr) {
        case 64: moe_matvec_kernel<Unit, MODE, 64><<<grid, 256, lds, s>>>(m); break;
        case 32: moe_matvec_kernel<Unit, MODE, 32><<<grid, 256, lds, s>>>(m); break;
        case 16: moe_matvec_kernel<Unit, MODE, 16><<<grid, 256, lds, s>>>(m); break;
        case 10: moe_matvec_kernel<Unit, MODE, 10><<<grid, 256, lds, s>>>(m); break;
        case 6: moe_matvec_kernel<Unit, MODE, 6><<<grid, 256, lds, s>>>(m); break;
        default: moe_matvec_kernel<Unit, MODE, 8><<<grid, 256, lds, s>>>(m); break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_plan(const DecodePlanArgs& a, hipStream_t s) {
    moe_plan_kernel<<<1, 128, 0, s>>>(a);
    return hipGetLastError();
}

namespace {
template <int WT>
hipError_t launch_front_t(const DecodePlanArgs& a, const _Float16* x, uint8_t* y, uint32_t n, uint32_t rows,
                          const DenseDecode* sd, hipStream_t s) {
    const uint32_t q_blocks = rows * ((n + 255u) / 256u);
    DenseDecode m = sd != nullptr ? *sd : DenseDecode{};
    uint32_t lpr = 8, extra = 0;
    size_t lds = 0;
    if (WT >= 0) {
        lpr = dense_lpr(m.k, 8u);
        extra = dense_blocks(m, false, lpr);
        lds = (size_t(m.rows) * m.k * 4u + 1023u) & ~size_t(1023);  // F32 hidden rows
        if (lds > 131072u) return hipErrorInvalidValue;
    }
    const dim3 grid(1u + q_blocks + extra);
    auto go = [&](auto kern) {
        if (lds > 65536u) {
            const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
            if (attr != hipSuccess) return attr;
        }
        kern<<<grid, 256, lds, s>>>(a, x, y, n, q_blocks, m);
        return hipGetLastError();
    };
    if constexpr (WT < 0) {
        return go(decode_front_kernel<-1, 8>);
    } else {
        switch (lpr) {
            case 64: return go(decode_front_kernel<WT, 64>);
            case 32: return go(decode_front_kernel<WT, 32>);
            case 16: return go(decode_front_kernel<WT, 16>);
            default: return go(decode_front_kernel<WT, 8>);
        }
    }
}
}  // namespace

hipError_t launch_decode_front(const DecodePlanArgs& a, const _Float16* x, uint8_t* y, uint32_t n, uint32_t rows,
                               Fmt shared_fmt, const DenseDecode* shared_down, hipStream_t s) {
    if (rows == 0u || rows > 8u || n == 0u || n % 32u != 0u || a.rows != rows) return hipErrorInvalidValue;
    if (a.logits != nullptr && (a.n_experts == 0u || a.n_experts > 512u || a.top_k == 0u || a.top_k > a.n_experts ||
                                rows * a.top_k > 80u || a.route_ids == nullptr || a.route_weights == nullptr))
        return hipErrorInvalidValue;
    if (shared_down == nullptr) return launch_front_t<-1>(a, x, y, n, rows, nullptr, s);
    if (shared_down->rows != rows || shared_down->k == 0u || shared_down->k % 64u != 0u) return hipErrorInvalidValue;
    switch (shared_fmt) {
        case Fmt::F16: return launch_front_t<kWF16>(a, x, y, n, rows, shared_down, s);
        case Fmt::BF16: return launch_front_t<kWBF16>(a, x, y, n, rows, shared_down, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_swiglu_q8_1(const float* gate, const float* up, float* hidden, uint8_t* y, uint32_t n, uint32_t rows,
                              hipStream_t s) {
    if (n == 0u || n % 32u != 0u) return hipErrorInvalidValue;
    swiglu_q8_1_kernel<<<dim3((n + 255u) / 256u, rows), 256, 0, s>>>(gate, up, hidden, y, n, rows);
    return hipGetLastError();
}

hipError_t launch_snapshot_copy(const uint64_t* src, uint64_t* dst, uint32_t words, uint32_t* status, hipStream_t s) {
    snapshot_copy_kernel<<<1, 256, 0, s>>>(src, dst, words, status);
    return hipGetLastError();
}

hipError_t launch_quantize_q8_1(const void* x, bool f32_input, uint8_t* y, uint32_t n, uint32_t rows, hipStream_t s) {
    const dim3 grid((n + 255u) / 256u, rows);
    if (f32_input) q8_1_kernel<true><<<grid, 256, 0, s>>>(x, y, n, rows);
    else q8_1_kernel<false><<<grid, 256, 0, s>>>(x, y, n, rows);
    return hipGetLastError();
}

hipError_t launch_decode_matvec(Fmt fmt, bool gate_up, const DecodeMatvec& m, hipStream_t s) {
    switch (fmt) {
        case Fmt::Q8_0: return gate_up ? launch_matvec_t<UnitQ80, kGateUp>(m, s) : launch_matvec_t<UnitQ80, kDown>(m, s);
        case Fmt::Q4_K: return gate_up ? launch_matvec_t<UnitQ4K, kGateUp>(m, s) : launch_matvec_t<UnitQ4K, kDown>(m, s);
        case Fmt::Q2_K: return gate_up ? launch_matvec_t<UnitQ2K, kGateUp>(m, s) : launch_matvec_t<UnitQ2K, kDown>(m, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dense_decode(Fmt fmt, bool gate_up, const DenseDecode& m, hipStream_t s) {
    if (m.rows == 0u || m.rows > 8u || m.k == 0u || m.k % 64u != 0u) return hipErrorInvalidValue;
    switch (fmt) {  // gate/up reads the F16 mixed activation; down the F32 hidden
        case Fmt::F16:
            return gate_up ? launch_dense_decode_t<kWF16, true, false>(m, s) : launch_dense_decode_t<kWF16, false, true>(m, s);
        case Fmt::BF16:
            return gate_up ? launch_dense_decode_t<kWBF16, true, false>(m, s) : launch_dense_decode_t<kWBF16, false, true>(m, s);
        default: return hipErrorInvalidValue;
    }
}

namespace {
DenseDecode router_job(const _Float16* x, const float* w, const float* bias, float* logits, uint32_t rows, uint32_t d,
                       uint32_t E, const SnapshotCopy& snap) {
    DenseDecode m{};
    m.snap_src = snap.src;
    m.snap_dst = snap.dst;
    m.snap_words = snap.words;
    m.snap_src2 = snap.src2;
    m.snap_dst2 = snap.dst2;
    m.snap_words2 = snap.words2;
    m.w0 = reinterpret_cast<const uint8_t*>(w);
    m.x = x;
    m.bias = bias;
    m.out = logits;
    m.rows = rows;
    m.k = d;
    m.n_out = E;
    return m;
}

template <int WT>
hipError_t launch_router_shared_t(DenseDecode r, DenseDecode g, uint32_t lpr, hipStream_t s) {
    const uint32_t rb = dense_blocks(r, false, lpr), gb = dense_blocks(g, true, lpr);
    const size_t lds = (size_t(r.rows) * r.k * 2u + 1023u) & ~size_t(1023);  // F16 rows, as one job stages them
    if (lds > 131072u) return hipErrorInvalidValue;
    auto go = [&](auto kern) {
        if (lds > 65536u) {
            const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                        hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
            if (attr != hipSuccess) return attr;
        }
        kern<<<rb + gb, 256, lds, s>>>(r, g, rb);
        return hipGetLastError();
    };
    switch (lpr) {
        case 64: return go(router_shared_decode_kernel<WT, 64>);
        case 32: return go(router_shared_decode_kernel<WT, 32>);
        case 16: return go(router_shared_decode_kernel<WT, 16>);
        default: return go(router_shared_decode_kernel<WT, 8>);
    }
}
}  // namespace

hipError_t launch_router_decode(const _Float16* x, const float* w, const float* bias, float* logits, uint32_t rows,
                                uint32_t d, uint32_t E, const SnapshotCopy& snap, hipStream_t s) {
    if (rows == 0u || rows > 8u || d == 0u || d % 64u != 0u) return hipErrorInvalidValue;
    return launch_dense_decode_t<kWF32, false, false>(router_job(x, w, bias, logits, rows, d, E, snap), s);
}

hipError_t launch_router_shared_decode(const _Float16* x, const float* w, const float* bias, float* logits,
                                       uint32_t rows, uint32_t d, uint32_t E, const SnapshotCopy& snap, Fmt shared_fmt,
                                       const DenseDecode& shared_gate_up, hipStream_t s) {
    if (rows == 0u || rows > 8u || d == 0u || d % 64u != 0u) return hipErrorInvalidValue;
    if (shared_gate_up.rows != rows || shared_gate_up.k != d || shared_gate_up.x != x) return hipErrorInvalidValue;
    if (shared_fmt != Fmt::F16 && shared_fmt != Fmt::BF16) return hipErrorInvalidValue;
    const DenseDecode r = router_job(x, w, bias, logits, rows, d, E, snap);
    const uint32_t lpr = dense_lpr(d, 4u);
    if (lpr != dense_lpr(d, 8u)) {  // the two jobs split their rows differently: two launches
        const hipError_t e = launch_dense_decode_t<kWF32, false, false>(r, s);
        return e != hipSuccess ? e : launch_dense_decode(shared_fmt, true, shared_gate_up, s);
    }
    return shared_fmt == Fmt::F16 ? launch_router_shared_t<kWF16>(r, shared_gate_up, lpr, s)
                                  : launch_router_shared_t<kWBF16>(r, shared_gate_up, lpr, s);
}

hipError_t launch_swiglu_f32(const float* gate, const float* up, float* out, uint64_t n, hipStream_t s) {
    swiglu_f32_kernel<<<uint32_t((n + 255u) / 256u), 256, 0, s>>>(gate, up, out, n);
    return hipGetLastError();
}

hipError_t launch_combine_decode(const float* parts, const float* w, const float* shared, const float* gl, float* out,
                                 uint32_t rows, uint32_t top_k, uint32_t d, hipStream_t s) {
    combine_decode_kernel<<<dim3((d + 255u) / 256u, rows), 256, 0, s>>>(parts, w, shared, gl, out, top_k, d);
    return hipGetLastError();
}

}  // namespace sm
