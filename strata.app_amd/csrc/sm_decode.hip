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

// One thread per value, 32 lanes per block (n is a multiple of 32, so each 32-lane half of a
// wave exits or stays as a whole). amax is reduced over the absolute bit patterns and the
// sum over the unrounded values, both with xor 16, 8, 4, 2, 1 butterflies.
template <bool F32IN>
__global__ __launch_bounds__(256) void q8_1_kernel(const void* x, uint8_t* y, uint32_t n, uint32_t rows) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x, r = blockIdx.y;
    if (r >= rows || i >= n) return;
    uint32_t vb;
    if (F32IN) {
        vb = reinterpret_cast<const uint32_t*>(x)[uint64_t(r) * n + i];
    } else {
        vb = f32_bits(float(reinterpret_cast<const _Float16*>(x)[uint64_t(r) * n + i]));
    }
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
    uint8_t* blk = y + (uint64_t(r) * (n / 32u) + i / 32u) * kQ81Bytes;
    blk[4 + (i & 31u)] = uint8_t(int8_t(q));
    if ((i & 31u) == 0u) {
        const uint32_t ds = uint32_t(f16_bits(_Float16(d))) | (uint32_t(f16_bits(_Float16(sum))) << 16);
        *reinterpret_cast<uint32_t*>(blk) = ds;
    }
}

// ---- the plan ----------------------------------------------------------------------------
// MoePlan (moe.metal:101-111): 1620 bytes.
struct DecodePlan {
    uint32_t n_groups, n_entries, n_miss, skip;
    int32_t grp_e[80], grp_res[80], grp_start[81], ent_tok[80], ent_dst[80];
};
static_assert(sizeof(DecodePlan) == 1620, "MoePlan layout");

// First-appearance grouping of n = rows * top_k <= 80 entries, one 128-thread workgroup
// (moe.metal:124-210): entry i's group is the rank of its expert's first appearance among
// first appearances; its slot is the group's start plus the number of earlier entries with
// the same expert. The groups' starts are a prefix sum of their sizes in first-appearance
// order. An id outside [0, E) sets status bit 1 and leaves an empty plan (n_groups = 0).
// The workgroup also copies the layer's validated address tables into their device snapshots.
__global__ __launch_bounds__(128) void moe_plan_kernel(DecodePlanArgs a) {
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
    const int32_t e = tid < n ? a.ids[tid] : -1;
    e_s[tid] = e;
    __syncthreads();
    if (tid < n && (e < 0 || uint32_t(e) >= a.n_experts)) atomicOr(&bad_s, 1u);
    // Snapshot copies (validated on the host into pinned ring slots).
    for (uint32_t w = tid; w < a.snap_words; w += 128u) a.snap_dst[w] = a.snap_src[w];
    for (uint32_t w = tid; w < a.snap_words2; w += 128u) a.snap_dst2[w] = a.snap_src2[w];
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
    if (lane == 0) {
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
    if (lane == 63u) size_w[wave] = incl;
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

// Weight side of one 32-value block b of a row, per format: load() reads it once for every
// entry; dot() returns the block's float contribution for one activation block.
struct DotQ80 {  // 34 B / 32 values: d, int8 q[32] (blocks 2-byte aligned)
    uint32_t w[8];
    float d;
    __device__ __forceinline__ void load(const uint8_t* row, uint32_t b) {
        const uint8_t* p = row + 34u * b;
        const uintptr_t a = reinterpret_cast<uintptr_t>(p);
        const uint8_t* base = reinterpret_cast<const uint8_t*>(a & ~uintptr_t(3));
        // Nine dwords cover the block either way; the last may hold two bytes past the block
        // (never past the page holding its last byte).
        uint32_t v[9];
#pragma unroll
        for (int i = 0; i < 9; ++i) v[i] = ld_global<uint32_t>(base + 4 * i);
        // 4-aligned block: d at byte 0, codes at 2; otherwise d at byte 2, codes at 4.
        const bool odd = (a & 3u) != 0u;
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = odd ? v[i + 1] : __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);
        d = odd ? f16_hi(v[0]) : f16_lo(v[0]);
    }
    __device__ __forceinline__ float dot(const Act& x, float acc) const {
        int s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) s = sdot4(w[i], x.q[i], s);
        return __builtin_fmaf(d * x.d, float(s), acc);  // moe/native table: fma(d0 * d1, float(sumi), acc)
    }
};

struct DotQ4K {  // 144 B / 256 values: sub-block j (32 values) of the super-block per call
    uint32_t w[8];
    float d, dmin;
    int sc, mn;
    __device__ __forceinline__ void load(const uint8_t* row, uint32_t b) {
        const uint8_t* sb = row + 144u * (b >> 3);
        const uint32_t j = b & 7u, g = j >> 1, sh = 4u * (j & 1u);
        const u32x4 hdr = ld_global<u32x4>(sb);
        const u32x4 q0 = ld_global<u32x4>(sb + 16 + 32 * g), q1 = ld_global<u32x4>(sb + 32 + 32 * g);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = (q0[i] >> sh) & 0x0F0F0F0Fu;
            w[4 + i] = (q1[i] >> sh) & 0x0F0F0F0Fu;
        }
        d = f16_lo(hdr[0]);
        dmin = f16_hi(hdr[0]);
        // get_scale_min_k4 (dequant.hpp:157-190): scales bytes 0-11 are header bytes 4-15.
        auto byte = [&](uint32_t k) { return (hdr[1 + k / 4] >> (8u * (k & 3u))) & 0xffu; };
        if (j < 4) {
            sc = int(byte(j) & 63u);
            mn = int(byte(j + 4) & 63u);
        } else {
            sc = int((byte(j + 4) & 0xFu) | ((byte(j - 4) >> 6) << 4));
            mn = int((byte(j + 4) >> 4) | ((byte(j) >> 6) << 4));
        }
    }
    __device__ __forceinline__ float dot(const Act& x, float acc) const {
        int s = 0, t = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            s = sdot4(w[i], x.q[i], s);
            t = sdot4(0x01010101u, x.q[i], t);
        }
        const float sd = x.d * float(s * sc), sm = x.d * float(t * mn);
        return acc + __builtin_fmaf(-dmin, sm, d * sd);  // q4_K: fma(-dm.y, sm, dm.x * sd), then acc + v
    }
};

struct DotQ2K {  // 84 B / 256: scales[16] @0, q[64] @16, d @80, dmin @82
    uint32_t w[8];
    float d, dmin;
    int sc0, mn0, sc1, mn1;
    __device__ __forceinline__ void load(const uint8_t* row, uint32_t b) {
        const uint8_t* sb = row + 84u * (b >> 3);
        const uint32_t bb = b & 7u, nn = bb >> 2, j = bb & 3u;
        // Values 128n + 32j + w (w < 32) use bits 2j of q[32n + w]; scale byte 8n + 2j + (w >= 16).
#pragma unroll
        for (int i = 0; i < 8; ++i) w[i] = (ld_global<uint32_t>(sb + 16 + 32 * nn + 4 * i) >> (2u * j)) & 0x03030303u;
        const uint32_t scw = ld_global<uint32_t>(sb + 8 * nn + 2 * (j & 2u));  // 4-aligned: bytes 8n + 4(j/2) ..
        const uint32_t s0 = (scw >> (16u * (j & 1u))) & 0xffu, s1 = (scw >> (16u * (j & 1u) + 8u)) & 0xffu;
        sc0 = int(s0 & 0xFu);
        mn0 = int(s0 >> 4);
        sc1 = int(s1 & 0xFu);
        mn1 = int(s1 >> 4);
        const uint32_t dd = ld_global<uint32_t>(sb + 80);
        d = f16_lo(dd);
        dmin = f16_hi(dd);
    }
    __device__ __forceinline__ float dot(const Act& x, float acc) const {
        int s0 = 0, s1 = 0, t0 = 0, t1 = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            s0 = sdot4(w[i], x.q[i], s0);
            t0 = sdot4(0x01010101u, x.q[i], t0);
            s1 = sdot4(w[4 + i], x.q[4 + i], s1);
            t1 = sdot4(0x01010101u, x.q[4 + i], t1);
        }
        const float sd = x.d * float(s0 * sc0 + s1 * sc1), sm = x.d * float(t0 * mn0 + t1 * mn1);
        return acc + __builtin_fmaf(-dmin, sm, d * sd);
    }
};

// ---- grouped mat-vecs --------------------------------------------------------------------
// Group g = blockIdx.y (blocks past n_groups exit); weight rows [32 * blockIdx.x, +32) of the
// stage (gate/up: gate rows 0..I-1 then up rows I..2I-1; down: output rows 0..d-1), 8 per
// wave. LPR lanes share a row (8..64, a power of two), each taking blocks lane % LPR + LPR * i
// below K/32; the other lanes of the wave take the next rows. The launch picks the largest LPR
// dividing K/32 so that every lane takes the same number of blocks; where no such LPR >= 8
// exists (K = 640: 20 blocks) LPR is 8 and the last step leaves some lanes idle.
constexpr uint32_t kRowsPerGroupBlock = 32;

__device__ __forceinline__ bool plan_header_ok(const DecodePlan* P, uint32_t n_entries, uint32_t n_experts, uint32_t g,
                                               uint32_t& a0, uint32_t& a1, uint32_t& ex) {
    if (P->n_entries != n_entries || P->n_groups == 0u || P->n_groups > 80u || g >= P->n_groups) return false;
    const int32_t s = P->grp_start[g], t = P->grp_start[g + 1], e = P->grp_e[g];
    if (s < 0 || t <= s || uint32_t(t) > n_entries || uint32_t(t - s) > 8u || e < 0 || uint32_t(e) >= n_experts) return false;
    a0 = uint32_t(s);
    a1 = uint32_t(t);
    ex = uint32_t(e);
    return true;
}

template <class Dot, int MODE, uint32_t LPR>
__global__ __launch_bounds__(256) void moe_matvec_kernel(DecodeMatvec m) {
    constexpr uint32_t RPW = 64u / LPR;  // rows per wave pass
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t g = blockIdx.y;
    const DecodePlan* P = reinterpret_cast<const DecodePlan*>(m.plan);
    if (g >= 80u) return;
    // A plan whose header is unusable: workgroup (0, 0) reports it and zeroes every output row
    // this stage could have written.
    const bool plan_ok = P->n_entries == m.n_entries && P->n_groups <= 80u;
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
    if (g >= P->n_groups) return;
    uint32_t a0, a1, ex;
    if (!plan_header_ok(P, m.n_entries, m.n_experts, g, a0, a1, ex)) {
        if (tid == 0 && blockIdx.x == 0u) atomicOr(m.status, 2u);
        return;  // the group's rows cannot be named: the whole stage's status reports it
    }
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
    const uint32_t nblk = m.k / 32u;
    const uint32_t per_lane = (nblk + LPR - 1u) / LPR;
    for (uint32_t it = 0; it < kRowsPerGroupBlock / (4u * RPW); ++it) {
        const uint32_t row = kRowsPerGroupBlock * blockIdx.x + (it * 4u + wave) * RPW + lane / LPR;
        const bool row_ok = row < n_rows;  // uniform within each LPR-lane segment
        float acc[8];
#pragma unroll
        for (uint32_t c = 0; c < 8u; ++c) acc[c] = 0.0f;
        if (row_ok && fault == 0u) {
            const bool up = MODE == kGateUp && row >= m.out_width;
            const uint8_t* wr = (up ? w1 : w0) + uint64_t(up ? row - m.out_width : row) * m.row_bytes;
            for (uint32_t i = 0; i < per_lane; ++i) {
                const uint32_t b = lane % LPR + LPR * i;  // the block of K this lane takes
                if (b >= nblk) break;                     // ragged last step (K/32 not a multiple of LPR)
                Dot wd;
                wd.load(wr, b);
#pragma unroll
                for (uint32_t c = 0; c < 8u; ++c)
                    if (c < n_e) acc[c] = wd.dot(load_act(m.act + (uint64_t(arow[c]) * nblk + b) * kQ81Bytes), acc[c]);
            }
        }
        // Butterfly over the row's LPR lanes (xor LPR/2 .. 1).
#pragma unroll
        for (uint32_t c = 0; c < 8u; ++c)
#pragma unroll
            for (uint32_t o = LPR / 2u; o > 0u; o >>= 1) acc[c] = acc[c] + __shfl_xor(acc[c], int(o));
        if (row_ok && lane % LPR == 0u) {
            const bool up = MODE == kGateUp && row >= m.out_width;
            float* out = up ? m.out1 : m.out0;
            const uint32_t col = up ? row - m.out_width : row;
#pragma unroll
            for (uint32_t c = 0; c < 8u; ++c)
                if (c < n_e) out[uint64_t(orow[c]) * m.out_width + col] = fault == 0u ? acc[c] : 0.0f;
        }
    }
    if (fault != 0u && tid == 0 && blockIdx.x == 0u) atomicOr(m.status, fault);
}

// ---- the shared expert: dense mat-vecs over F16 / BF16 weights ---------------------------
// Rows [32 * blockIdx.x, +32) of the output, 8 per wave; LPR lanes share a weight row, each
// taking 8-value chunks lane % LPR + LPR * i (one 16-byte load of the weight row). Every lane
// keeps one accumulator per activation row (two in gate/up: the gate and up rows of the same
// output column), and a butterfly over the row's lanes finishes them. gate/up applies the
// F32 SwiGLU silu(g) * u before its one store (the reference's shx_swiglu, moe.metal:237-245).
template <bool BF, bool GATE_UP, uint32_t LPR>
__global__ __launch_bounds__(256) void dense_decode_kernel(DenseDecode m) {
    constexpr uint32_t RPW = 64u / LPR;
    constexpr uint32_t NW = GATE_UP ? 2u : 1u;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t nch = m.k / 8u;
    const uint32_t per_lane = (nch + LPR - 1u) / LPR;
    for (uint32_t it = 0; it < kRowsPerGroupBlock / (4u * RPW); ++it) {
        const uint32_t row = kRowsPerGroupBlock * blockIdx.x + (it * 4u + wave) * RPW + lane / LPR;
        const bool row_ok = row < m.n_out;  // uniform within each LPR-lane segment
        float acc[NW][8];
#pragma unroll
        for (uint32_t w = 0; w < NW; ++w)
#pragma unroll
            for (uint32_t t = 0; t < 8u; ++t) acc[w][t] = 0.0f;
        if (row_ok) {
            const uint8_t* wr[2] = {m.w0 + uint64_t(row) * m.k * 2u, GATE_UP ? m.w1 + uint64_t(row) * m.k * 2u : nullptr};
            for (uint32_t i = 0; i < per_lane; ++i) {
                const uint32_t c = lane % LPR + LPR * i;
                if (c >= nch) break;
                float wv[NW][8];
#pragma unroll
                for (uint32_t w = 0; w < NW; ++w) {
                    const u32x4 q = ld_global<u32x4>(wr[w] + 16u * c);
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        if (BF) {
                            wv[w][2 * j] = bits_f32(q[j] << 16);
                            wv[w][2 * j + 1] = bits_f32(q[j] & 0xffff0000u);
                        } else {
                            wv[w][2 * j] = f16_lo(q[j]);
                            wv[w][2 * j + 1] = f16_hi(q[j]);
                        }
                    }
                }
#pragma unroll
                for (uint32_t t = 0; t < 8u; ++t) {
                    if (t >= m.rows) break;
                    float xv[8];
                    if (GATE_UP) {
                        const u32x4 q = ld_global<u32x4>(reinterpret_cast<const uint8_t*>(m.x) + (uint64_t(t) * m.k + 8u * c) * 2u);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            xv[2 * j] = f16_lo(q[j]);
                            xv[2 * j + 1] = f16_hi(q[j]);
                        }
                    } else {
                        const float* xp = reinterpret_cast<const float*>(m.x) + uint64_t(t) * m.k + 8u * c;
                        const float4v a = ld_global<float4v>(xp), b = ld_global<float4v>(xp + 4);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            xv[j] = a[j];
                            xv[4 + j] = b[j];
                        }
                    }
#pragma unroll
                    for (uint32_t w = 0; w < NW; ++w)
#pragma unroll
                        for (int j = 0; j < 8; ++j) acc[w][t] = __builtin_fmaf(wv[w][j], xv[j], acc[w][t]);
                }
            }
        }
#pragma unroll
        for (uint32_t w = 0; w < NW; ++w)
#pragma unroll
            for (uint32_t t = 0; t < 8u; ++t)
#pragma unroll
                for (uint32_t o = LPR / 2u; o > 0u; o >>= 1) acc[w][t] = acc[w][t] + __shfl_xor(acc[w][t], int(o));
        if (row_ok && lane % LPR == 0u) {
#pragma unroll
            for (uint32_t t = 0; t < 8u; ++t)
                if (t < m.rows)
                    m.out[uint64_t(t) * m.n_out + row] = GATE_UP ? silu(acc[0][t]) * acc[NW - 1][t] : acc[0][t];
        }
    }
}

template <bool BF, bool GATE_UP>
hipError_t launch_dense_decode_t(const DenseDecode& m, hipStream_t s) {
    const uint32_t nch = m.k / 8u;
    uint32_t lpr = 64;
    while (lpr > 8u && nch % lpr != 0u) lpr >>= 1;
    const dim3 grid((m.n_out + kRowsPerGroupBlock - 1) / kRowsPerGroupBlock);
    switch (lpr) {
        case 64: dense_decode_kernel<BF, GATE_UP, 64><<<grid, 256, 0, s>>>(m); break;
        case 32: dense_decode_kernel<BF, GATE_UP, 32><<<grid, 256, 0, s>>>(m); break;
        case 16: dense_decode_kernel<BF, GATE_UP, 16><<<grid, 256, 0, s>>>(m); break;
        default: dense_decode_kernel<BF, GATE_UP, 8><<<grid, 256, 0, s>>>(m); break;
    }
    return hipGetLastError();
}

// ---- post ops ----------------------------------------------------------------------------
// eh = silu(g) * u in F32 (moe.metal:213-221).
__global__ __launch_bounds__(256) void swiglu_f32_kernel(const float* gate, const float* up, float* out, uint64_t n) {
    const uint64_t i = uint64_t(blockIdx.x) * 256u + threadIdx.x;
    if (i < n) out[i] = silu(gate[i]) * up[i];
}

// The decode combine (moe.metal:253-274): the first rank is a product, the others fma in
// rank order, and the gated shared output is added last.
__global__ __launch_bounds__(256) void combine_decode_kernel(const float* parts, const float* w, const float* shared,
                                                             const float* gl, float* out, uint32_t top_k, uint32_t d) {
    const uint32_t t = blockIdx.y, c = blockIdx.x * 256u + threadIdx.x;
    if (c >= d) return;
    const float* p = parts + uint64_t(t) * top_k * d + c;
    const float* wt = w + uint64_t(t) * top_k;
    float s = p[0] * wt[0];
    for (uint32_t k = 1; k < top_k; ++k) s = __builtin_fmaf(p[uint64_t(k) * d], wt[k], s);
    float o = s;
    if (shared != nullptr) {
        const float gs = sigmoid(gl[t]);
        o = s + shared[uint64_t(t) * d + c] * gs;
    }
    out[uint64_t(t) * d + c] = o;
}

// Copies a validated address table (pinned host ring slot) into its device snapshot and clears
// the stage's status word (a standalone expert stage, whose plan came from elsewhere).
__global__ __launch_bounds__(256) void snapshot_copy_kernel(const uint64_t* src, uint64_t* dst, uint32_t words,
                                                            uint32_t* status) {
    for (uint32_t w = threadIdx.x; w < words; w += 256u) dst[w] = src[w];
    if (threadIdx.x == 0 && status != nullptr) *status = 0u;
}

template <class Dot, int MODE>
hipError_t launch_matvec_t(const DecodeMatvec& m, hipStream_t s) {
    const uint32_t n_rows = MODE == kGateUp ? 2u * m.out_width : m.out_width;
    const dim3 grid((n_rows + kRowsPerGroupBlock - 1) / kRowsPerGroupBlock, 80);
    const uint32_t nblk = m.k / 32u;
    if (nblk == 0u) return hipErrorInvalidValue;
    uint32_t lpr = 64;
    while (lpr > 8u && nblk % lpr != 0u) lpr >>= 1;
    switch (lpr) {
        case 64: moe_matvec_kernel<Dot, MODE, 64><<<grid, 256, 0, s>>>(m); break;
        case 32: moe_matvec_kernel<Dot, MODE, 32><<<grid, 256, 0, s>>>(m); break;
        case 16: moe_matvec_kernel<Dot, MODE, 16><<<grid, 256, 0, s>>>(m); break;
        default: moe_matvec_kernel<Dot, MODE, 8><<<grid, 256, 0, s>>>(m); break;
    }
    return hipGetLastError();
}

}  // namespace

hipError_t launch_decode_plan(const DecodePlanArgs& a, hipStream_t s) {
    moe_plan_kernel<<<1, 128, 0, s>>>(a);
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
        case Fmt::Q8_0: return gate_up ? launch_matvec_t<DotQ80, kGateUp>(m, s) : launch_matvec_t<DotQ80, kDown>(m, s);
        case Fmt::Q4_K: return gate_up ? launch_matvec_t<DotQ4K, kGateUp>(m, s) : launch_matvec_t<DotQ4K, kDown>(m, s);
        case Fmt::Q2_K: return gate_up ? launch_matvec_t<DotQ2K, kGateUp>(m, s) : launch_matvec_t<DotQ2K, kDown>(m, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dense_decode(Fmt fmt, bool gate_up, const DenseDecode& m, hipStream_t s) {
    if (m.rows == 0u || m.rows > 8u || m.k == 0u || m.k % 64u != 0u) return hipErrorInvalidValue;
    switch (fmt) {
        case Fmt::F16: return gate_up ? launch_dense_decode_t<false, true>(m, s) : launch_dense_decode_t<false, false>(m, s);
        case Fmt::BF16: return gate_up ? launch_dense_decode_t<true, true>(m, s) : launch_dense_decode_t<true, false>(m, s);
        default: return hipErrorInvalidValue;
    }
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
