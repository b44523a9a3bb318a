// Router GEMM, softmax top-k, stable expert grouping, F16 row gather, and the plan /
// destination validators for gfx950.
#include "sm_device.h"
#include "sm_launch.h"
#include "sm_topk.h"

namespace sm {
namespace {

constexpr uint32_t kTopkWaveRows = 1024;  // top-k: one token per wave up to this many tokens

// ---------------------------------------------------------------------------------------
// Router GEMM: logits[t,e] = sum_k x[t,k] * W[e,k], F16 activations, F32 weights.
// Each F32 weight is split into an F16 head and an F16 tail scaled by 2^11
// (w = hi + lo * 2^-11 to about 2^-22 relative); two MFMA accumulators carry the head and
// tail products and are merged as fma(lo, 2^-11, hi). Tile: ROWS tokens (32, 64 or 128) x
// 64 experts per 512-thread workgroup. Wave w owns experts 16 (w & 3) .. +15 and, of each
// 64-column stage, the 32-column k-step w >> 2, so the two waves of a SIMD multiply the same
// experts over different columns and their partial sums are added once at the end (through
// LDS). Each expert's weights are read and split once per workgroup, so larger token tiles
// divide that work; the launcher takes the largest tile that still gives every CU a
// workgroup.
// The reduction is streamed in stages of 64 columns through an LDS ring of NST slots: each
// stage holds the ROWS x 64 activation slab and the 64 x 64 F32 weight slab, both copied by
// LDS-DMA (16 bytes per lane, XOR-swizzled chunk positions) by waves 0-3, and the copies run
// NST - 1 stages ahead, so a wave waits only for the oldest stage while the later ones stay
// in flight. The ring stays within 96 KB so that a workgroup of the shared expert's GEMM,
// which runs beside the router on the second stream, still fits on the same CU. Within a
// wave the k-steps keep the order of a plain loop over its columns.
// ---------------------------------------------------------------------------------------
constexpr int kRouterCols = 64;
constexpr int kRouterThreads = 512;

template <int ROWS>
struct RouterStage {
    static constexpr int KS = 64;                      // reduction columns per stage
    static constexpr int NST = ROWS == 128 ? 3 : 4;    // ring slots (NST - 1 stages in flight)
    static constexpr int CPR = KS / 8;                 // 16-byte activation chunks per row
    static constexpr int RPI = 64 / CPR;               // activation rows per copy instruction
    static constexpr int NA = ROWS / (4 * RPI);        // activation copies per copying wave and stage
    static constexpr int WCPR = KS / 4;                // 16-byte weight chunks per expert row
    static constexpr int WPI = 64 / WCPR;              // expert rows per copy instruction
    static constexpr int NW = 16 / WPI;                // weight copies per copying wave (its 16 experts)
    static constexpr int A_BYTES = ROWS * KS * 2;
    static constexpr int BYTES = A_BYTES + kRouterCols * KS * 4;
    static_assert(NA * 4 * RPI == ROWS && NW * WPI == 16, "copy map covers the stage");
    static_assert(NST * BYTES <= 96 * 1024, "LDS ring leaves room for a co-resident workgroup");
    // The second k-half's partial sums (ROWS / 16 blocks x 4 values x head and tail, for
    // 256 lanes) pass through the ring after the last stage.
    static_assert(ROWS / 16 * 8 * 256 * 4 <= NST * BYTES, "partial sums fit the ring");
};

// s_waitcnt immediate that waits for at most n vector-memory operations (gfx9 encoding:
// vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt left at their no-wait maxima).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

template <int ROWS>
__global__ __launch_bounds__(kRouterThreads) void router_gemm_kernel(const _Float16* __restrict__ x,
                                                                    const float* __restrict__ w,
                                                                    const float* __restrict__ bias,
                                                                    float* __restrict__ logits,
                                                                    uint32_t rows, uint32_t d, uint32_t E,
                                                                    RouterPrep prep) {
    using S = RouterStage<ROWS>;
    constexpr int RB = ROWS / 16;  // 16-row MFMA blocks
    typedef float f2v __attribute__((ext_vector_type(2)));
    typedef _Float16 h2v __attribute__((ext_vector_type(2)));
    __shared__ __attribute__((aligned(1024))) uint8_t ring[S::NST * S::BYTES];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = (tid >> 6) & 3, kh = tid >> 8;  // expert quarter, k-half of each stage
    const bool copier = kh == 0;
    const int n = lane & 15, g = lane >> 4;
    const uint32_t t0 = blockIdx.x * ROWS;
    const uint32_t e0 = blockIdx.y * kRouterCols;
    const uint32_t e = e0 + 16 * wave + n;
    const bool e_ok = e < E;
    if (prep.hist != nullptr) {  // the grouping histogram's counts, before top-k adds to them
        const uint32_t nb = gridDim.x * gridDim.y, b = blockIdx.y * gridDim.x + blockIdx.x;
        for (uint32_t i = b * kRouterThreads + uint32_t(tid); i < prep.hist_words; i += nb * kRouterThreads)
            prep.hist[i] = 0u;
        if (b == 0 && tid == 0) *prep.arrive = 0u;
    }
    // Copy maps (element offsets at k = 0, in 64 bits: rows x d may exceed 2^32).
    // Activation copy q = NA*wave + j fills LDS chunk positions [64q, 64q + 64): row
    // R = RPI*q + lane / CPR, position p = lane % CPR holding chunk p ^ (R % CPR).
    uint64_t aofs[S::NA];
#pragma unroll
    for (int j = 0; j < S::NA; ++j) {
        const uint32_t R = uint32_t(S::RPI * (S::NA * wave + j)) + uint32_t(lane) / S::CPR;
        const uint32_t C = (uint32_t(lane) % S::CPR) ^ (R % S::CPR);
        const uint32_t t = t0 + R < rows ? t0 + R : rows - 1u;
        aofs[j] = uint64_t(t) * d + 8u * C;
    }
    // Weight copy q = NW*wave + j: expert row Rw = WPI*q + lane / WCPR of the tile (wave w
    // copies the 16 experts of its quarter), position p = lane % WCPR holding chunk
    // p ^ (Rw & 15). Row 0 stands in for experts past E; those outputs are never stored.
    uint64_t wofs[S::NW];
#pragma unroll
    for (int j = 0; j < S::NW; ++j) {
        const uint32_t Rw = uint32_t(S::WPI * (S::NW * wave + j)) + uint32_t(lane) / S::WCPR;
        const uint32_t C = (uint32_t(lane) % S::WCPR) ^ (Rw & 15u);
        wofs[j] = uint64_t(e0 + Rw < E ? e0 + Rw : 0u) * d + 4u * C;
    }
    auto issue = [&](uint32_t st, uint32_t slot) {
        uint8_t* base = ring + slot * S::BYTES;
        const uint32_t k0 = st * S::KS;
#pragma unroll
        for (int j = 0; j < S::NA; ++j)
            __builtin_amdgcn_global_load_lds(
                reinterpret_cast<const __attribute__((address_space(1))) void*>(reinterpret_cast<uintptr_t>(x + aofs[j] + k0)),
                reinterpret_cast<__attribute__((address_space(3))) void*>(
                    reinterpret_cast<uintptr_t>(base + (S::NA * wave + j) * 1024)),
                16, 0, 0);
#pragma unroll
        for (int j = 0; j < S::NW; ++j)
            __builtin_amdgcn_global_load_lds(
                reinterpret_cast<const __attribute__((address_space(1))) void*>(reinterpret_cast<uintptr_t>(w + wofs[j] + k0)),
                reinterpret_cast<__attribute__((address_space(3))) void*>(
                    reinterpret_cast<uintptr_t>(base + S::A_BYTES + (S::NW * wave + j) * 1024)),
                16, 0, 0);
    };
    float4v acc_hi[RB], acc_lo[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) { acc_hi[rb] = float4v{0, 0, 0, 0}; acc_lo[rb] = float4v{0, 0, 0, 0}; }
    const uint32_t n_st = d / S::KS;
    if (copier) {
#pragma unroll
        for (int i = 0; i < S::NST - 1; ++i)
            if (uint32_t(i) < n_st) issue(i, i);
    }
    const uint32_t wrow = 16u * wave + n;  // this lane's expert row in the weight slab
    const uint32_t c0 = 8u * kh + 2u * g;   // lane group g holds columns 8g .. 8g + 7 of the k-step
    for (uint32_t st = 0; st < n_st; ++st) {
        // Stage st's copies (of every copying wave, hence the barrier); stage st + 1 may stay
        // in flight. A bare s_barrier: __syncthreads() would add a workgroup release that
        // waits for every copy in flight. A copying wave's stage-st copies are complete after
        // the wait, and the slot refilled below was last read in the previous iteration, whose
        // LDS reads every wave consumed before reaching this barrier.
        if (copier) {
            const uint32_t later = n_st - 1u - st;  // stages issued after st (at most NST - 2)
            if (S::NST == 4 && later >= 2u) __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * (S::NA + S::NW)));
            else if (later >= 1u) __builtin_amdgcn_s_waitcnt(vmcnt_imm(S::NA + S::NW));
            else __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
        __builtin_amdgcn_s_barrier();
        if (copier && st + S::NST - 1 < n_st) issue(st + S::NST - 1, (st + S::NST - 1) % S::NST);
        const uint8_t* base = ring + (st % S::NST) * S::BYTES;
        const uint8_t* wb = base + S::A_BYTES + wrow * (S::KS * 4);
        // Every operand read of the k-step first, then the split, so one wait covers them.
        const float4v w0 = *reinterpret_cast<const float4v*>(wb + 16u * (c0 ^ uint32_t(n)));
        const float4v w1 = *reinterpret_cast<const float4v*>(wb + 16u * ((c0 + 1u) ^ uint32_t(n)));
        half8 a[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const uint32_t r = 16u * rb + n;
            const uint32_t pos = (4u * kh + g) ^ (r % S::CPR);
            a[rb] = *reinterpret_cast<const half8*>(base + r * (S::KS * 2) + 16u * pos);
        }
        __builtin_amdgcn_sched_barrier(0);
        half8 bh, bl;
#pragma unroll
        for (int i = 0; i < 8; i += 2) {
            const f2v wv = i < 4 ? f2v{w0[i], w0[i + 1]} : f2v{w1[i - 4], w1[i - 3]};
            const h2v hp = __builtin_convertvector(wv, h2v);                                     // head, RNE
            const h2v lp = __builtin_convertvector((wv - __builtin_convertvector(hp, f2v)) * 2048.0f, h2v);  // tail
            bh[i] = hp.x;
            bh[i + 1] = hp.y;
            bl[i] = lp.x;
            bl[i + 1] = lp.y;
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            acc_hi[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[rb], bh, acc_hi[rb], 0, 0, 0);
            acc_lo[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[rb], bl, acc_lo[rb], 0, 0, 0);
        }
    }
    // The second k-half hands its partial sums to the first through the ring (every wave's
    // last reads of it are done at the barrier).
    __syncthreads();
    float* part = reinterpret_cast<float*>(ring);
    const uint32_t pl = 64u * wave + lane;
    if (!copier) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                part[(8 * rb + 2 * i) * 256 + pl] = acc_hi[rb][i];
                part[(8 * rb + 2 * i + 1) * 256 + pl] = acc_lo[rb][i];
            }
    }
    __syncthreads();
    if (!copier || !e_ok) return;
    const float b = bias != nullptr ? bias[e] : 0.0f;
    float v[RB][4];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float hi = acc_hi[rb][i] + part[(8 * rb + 2 * i) * 256 + pl];
            const float lo = acc_lo[rb][i] + part[(8 * rb + 2 * i + 1) * 256 + pl];
            v[rb][i] = __builtin_fmaf(lo, 4.8828125e-4f, hi) + b;
        }
    // A full token tile stores without per-row branches, so the bias load is waited for once
    // (a wait per branch would also wait for each earlier store).
    if (t0 + ROWS <= rows) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) logits[uint64_t(t0 + 16 * rb + 4 * g + i) * E + e] = v[rb][i];
    } else {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t t = t0 + 16 * rb + 4 * g + i;
                if (t < rows) logits[uint64_t(t) * E + e] = v[rb][i];
            }
    }
}

template <int NV, bool WAVE>
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits,
                                                         int32_t* __restrict__ ids,
                                                         float* __restrict__ weights,
                                                         uint32_t rows, uint32_t E, uint32_t K,
                                                         int divide, uint32_t* __restrict__ hist) {
    const uint32_t t = WAVE ? blockIdx.x * 4u + (threadIdx.x >> 6) : blockIdx.x * 8u + (threadIdx.x >> 5);
    topk_token<NV, WAVE>(logits, ids, weights, rows, E, K, divide, hist, t, nullptr);
}

// ---------------------------------------------------------------------------------------
// Grouping. Results equal a stable counting sort of the valid entries by expert id:
//   count   one 256-entry tile per workgroup, LDS histogram, raw counts to hist[tile][e]
//   scan    per expert column, exclusive prefix over tiles (32 tile slices per column in
//           parallel); then the last workgroup to finish: block scans over experts give
//           each expert's first slot, group index and first tile; writes the PfPlan slot
//           and the 64-entry tile list, and the expert's first slot to the extra row
//           hist[n_tiles][e]
//   scatter one 256-entry tile per workgroup: hist row += first slot (the reference's
//           "cursor at tile start"); stable in-tile rank from per-wave ballot matching of
//           the 9-bit ids plus the counts of earlier waves; src[slot] = i/k, dst[slot] = i
// ---------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void group_count_kernel(const int32_t* __restrict__ ids, uint32_t N,
                                                          uint32_t E, uint32_t* __restrict__ hist,
                                                          uint32_t* __restrict__ arrive) {
    __shared__ uint32_t cnt[512];
    const uint32_t tile = blockIdx.x, tid = threadIdx.x;
    if (tile == 0 && tid == 0) *arrive = 0u;
    for (uint32_t e = tid; e < E; e += 256) cnt[e] = 0;
    __syncthreads();
    const uint64_t entry = uint64_t(tile) * kCountTile + tid;
    if (entry < N) {
        const int32_t id = ids[entry];
        if (id >= 0 && uint32_t(id) < E) atomicAdd(&cnt[id], 1u);
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += 256) hist[uint64_t(tile) * E + e] = cnt[e];
}

// Exclusive scan over the NT threads of a workgroup; returns the prefix and the total.
template <uint32_t NT>
__device__ __forceinline__ uint32_t block_scan(uint32_t v, uint32_t* wave_tot, uint32_t& total) {
    constexpr uint32_t kWaves = NT / 64;
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t inc = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(inc, off);
        if (lane >= uint32_t(off)) inc += o;
    }
    if (lane == 63u) wave_tot[wave] = inc;
    __syncthreads();
    uint32_t before = 0, all = 0;
#pragma unroll
    for (uint32_t w = 0; w < kWaves; ++w) {
        if (w < wave) before += wave_tot[w];
        all += wave_tot[w];
    }
    __syncthreads();
    total = all;
    return before + inc - v;
}

// Column scan, then the plan. Workgroup c scans expert columns [32c, 32c + 32): thread
// (slice, e) takes a contiguous run of tiles, the slice partials give each run's exclusive
// start, each run is rewritten in place with its column prefix, and the column total goes to
// the extra row hist[n_tiles][e] (a device-coherent store). Each workgroup then counts itself
// in at `arrive` (zeroed by the count kernel, which runs just before) with an acquire-release
// add, and the last to arrive reads the totals with device-coherent loads and builds the plan: block
// scans over the experts give each expert's first slot, group index and first tile; the slot
// is filled, the group fields written, tile i finds its group by binary search over the
// groups' first tiles (no serial per-expert loop), and hist[n_tiles][e] becomes the expert's
// first slot. `prep` (a full layer) zeroes the two stage status words and the destination
// bitset that the gather's checks use.
constexpr uint32_t kScanThreads = 1024;
__global__ __launch_bounds__(kScanThreads) void group_scan_plan_kernel(uint32_t* __restrict__ hist, uint32_t E,
                                                                       uint32_t N, uint32_t n_tiles,
                                                                       Plan* __restrict__ plan,
                                                                       uint32_t* __restrict__ tiles,
                                                                       uint32_t* __restrict__ arrive, GroupPrep prep,
                                                                       const int32_t* __restrict__ resident) {
    __shared__ uint32_t part[32][33];
    __shared__ uint32_t wave_tot[kScanThreads / 64];
    __shared__ uint32_t s_tstart[512], s_first[512], s_last;
    const uint32_t tid = threadIdx.x;
    if (blockIdx.x == 0 && tid == 0) {
        if (prep.status != nullptr) *prep.status = 0u;
        if (prep.status2 != nullptr) *prep.status2 = 0u;
    }
    for (uint32_t i = blockIdx.x * kScanThreads + tid; i < prep.clear_words; i += gridDim.x * kScanThreads)
        prep.clear[i] = 0u;
    {
        const uint32_t el = tid & 31u, slice = tid >> 5;
        const uint32_t e = blockIdx.x * 32u + el;
        const uint32_t per = (n_tiles + 31u) / 32u;
        const uint32_t t_begin = slice * per < n_tiles ? slice * per : n_tiles;
        const uint32_t t_end = t_begin + per < n_tiles ? t_begin + per : n_tiles;
        // Up to kScanHeld counts per thread are loaded at once and kept for the rewrite (one
        // round trip, where a load after each store would cost one per tile).
        constexpr uint32_t kScanHeld = 16;
        const bool held = per <= kScanHeld;
        uint32_t hv[kScanHeld];
        uint32_t local = 0;
        if (e < E) {
            if (held) {
#pragma unroll
                for (uint32_t j = 0; j < kScanHeld; ++j)
                    hv[j] = t_begin + j < t_end ? hist[uint64_t(t_begin + j) * E + e] : 0u;
#pragma unroll
                for (uint32_t j = 0; j < kScanHeld; ++j) local += hv[j];
            } else {
                for (uint32_t t = t_begin; t < t_end; ++t) local += hist[uint64_t(t) * E + e];
            }
        }
        part[slice][el] = local;
        __syncthreads();
        if (e < E) {
            uint32_t run = 0;
            for (uint32_t sl = 0; sl < slice; ++sl) run += part[sl][el];
            // The total is the only value another workgroup reads in this launch: an
            // agent-scope atomic store, published by the acquire-release add on `arrive`.
            if (slice == 31u)
                __hip_atomic_store(&hist[uint64_t(n_tiles) * E + e], run + local, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
            if (held) {
#pragma unroll
                for (uint32_t j = 0; j < kScanHeld; ++j)
                    if (t_begin + j < t_end) {
                        hist[uint64_t(t_begin + j) * E + e] = run;
                        run += hv[j];
                    }
            } else {
                for (uint32_t t = t_begin; t < t_end; ++t) {
                    const uint64_t h = uint64_t(t) * E + e;
                    const uint32_t c = hist[h];
                    hist[h] = run;
                    run += c;
                }
            }
        }
    }
    // Count in once this workgroup's totals are stored: the workgroup barrier orders every
    // thread's total before thread 0's acquire-release add on `arrive` (agent scope), and the
    // last workgroup to arrive acquires every earlier workgroup's totals through that same
    // word before its barrier hands them to its other threads. The rewritten rows are read
    // only by the scatter launch.
    __syncthreads();
    if (tid == 0)
        s_last = __hip_atomic_fetch_add(arrive, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1u
                     ? 1u : 0u;
    __syncthreads();
    if (!s_last) return;

    const uint32_t count =
        tid < E ? __hip_atomic_load(&hist[uint64_t(n_tiles) * E + tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                : 0u;
    uint32_t total_count, total_groups, total_tiles;
    const uint32_t first = block_scan<kScanThreads>(count, wave_tot, total_count);
    const uint32_t grp = block_scan<kScanThreads>(count ? 1u : 0u, wave_tot, total_groups);
    const uint32_t ntile_e = (count + kExpertTile - 1) / kExpertTile;
    const uint32_t tstart = block_scan<kScanThreads>(ntile_e, wave_tot, total_tiles);
    // Residency of the layer's experts (tiered mode): a used expert whose table entry is < 0
    // is a miss the host resolves before the expert stages run.
    const bool res = resident == nullptr || tid >= E || resident[tid] >= 0;
    uint32_t total_miss;
    (void)block_scan<kScanThreads>(count != 0u && !res ? 1u : 0u, wave_tot, total_miss);
    // Whole 6400-byte slot: every word defined (unused group slots -1 / 0, tail zero).
    uint32_t* words = reinterpret_cast<uint32_t*>(plan);
    for (uint32_t i = tid; i < kPlanSlotBytes / 4; i += kScanThreads) {
        uint32_t val = 0;
        if (i >= 8 && i < 8 + 1024) val = 0xffffffffu;  // grp_e[], grp_res[] = -1
        words[i] = val;
    }
    if (count) {
        s_tstart[grp] = tstart;
        s_first[grp] = first;
    }
    __syncthreads();
    if (count) {
        plan->grp_e[grp] = int32_t(tid);
        plan->grp_res[grp] = res ? 1 : 0;
        plan->grp_start[grp] = int32_t(first);
    }
    if (tid < E) hist[uint64_t(n_tiles) * E + tid] = first;
    if (tid == 0) {
        plan->n_groups = total_groups;
        plan->n_entries = N;
        plan->n_miss = total_miss;
        plan->skip = total_miss == 0u ? 1u : 0u;
        plan->n_tiles = total_tiles;
        plan->bad = N - total_count;
        plan->grp_start[total_groups] = int32_t(total_count);
    }
    // Every group has at least one tile, so the groups' first tiles ascend strictly.
    for (uint32_t i = tid; i < total_tiles; i += kScanThreads) {
        uint32_t lo = 0, hi = total_groups;
        while (hi - lo > 1u) {
            const uint32_t mid = (lo + hi) >> 1;
            if (s_tstart[mid] <= i) lo = mid;
            else hi = mid;
        }
        tiles[2 * i] = lo;
        tiles[2 * i + 1] = s_first[lo] + kExpertTile * (i - s_tstart[lo]);
    }
}

__global__ __launch_bounds__(256) void group_scatter_kernel(const int32_t* __restrict__ ids, uint32_t N,
                                                            uint32_t K, uint32_t E, uint32_t n_tiles,
                                                            uint32_t* __restrict__ hist,
                                                            int32_t* __restrict__ src,
                                                            int32_t* __restrict__ dst) {
    __shared__ uint32_t wcnt[4][512];
    __shared__ uint32_t base[512];
    const uint32_t tile = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    for (uint32_t i = tid; i < 4 * 512; i += 256) (&wcnt[0][0])[i] = 0;
    for (uint32_t e = tid; e < E; e += 256) {
        const uint64_t h = uint64_t(tile) * E + e;
        const uint32_t fin = hist[h] + hist[uint64_t(n_tiles) * E + e];
        hist[h] = fin;
        base[e] = fin;
    }
    const uint64_t entry = uint64_t(tile) * kCountTile + tid;
    const int32_t id = entry < N ? ids[entry] : -1;
    const bool valid = id >= 0 && uint32_t(id) < E;
    const uint32_t key = valid ? uint32_t(id) : 1023u;
    uint64_t match = ~0ull;
#pragma unroll
    for (int b = 0; b < 10; ++b) {
        const bool bit = (key >> b) & 1u;
        const uint64_t bal = __ballot(bit);
        match &= bit ? bal : ~bal;
    }
    const uint64_t lt = (1ull << lane) - 1ull;
    const uint32_t rank = __popcll(match & lt);
    const uint64_t gt = lane == 63u ? 0ull : (~0ull << (lane + 1u));
    __syncthreads();
    if (valid && (match & gt) == 0ull) wcnt[wave][id] = rank + 1u;
    __syncthreads();
    if (!valid) return;
    uint32_t slot = base[id] + rank;
    for (uint32_t w = 0; w < wave; ++w) slot += wcnt[w][id];
    src[slot] = int32_t(entry / K);
    dst[slot] = int32_t(entry);
}

// ---------------------------------------------------------------------------------------
// Expert-stage validation (prefill_moe.metal:603-733): status is cleared, then bit 1 set
// when the plan header, the tile chain, or the destination permutation is inconsistent.
// ---------------------------------------------------------------------------------------
// The header and per-group checks run one group per thread; the tile-count sum is a block
// reduction, so the whole plan is checked in a few dependent memory round trips.
// The whole check runs in one workgroup of NT threads; `reset_status` clears the status
// words first (a full layer's gather leaves that to the grouping, see GroupPrep).
template <uint32_t NT>
__device__ __forceinline__ void check_plan(const PlanCheck& c, bool reset_status) {
    __shared__ uint32_t s_header_ok, s_groups_ok, s_wave_tiles[NT / 64];
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    if (tid < c.n_counters) c.counters[tid] = 0u;
    // Address snapshots: every load of a thread is issued before its stores, so the reads
    // of pinned host memory cost one round trip (tables are at most 3 x 512 words).
    constexpr int kPer = 1536 / NT;
    uint64_t v1[kPer], v2[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const uint32_t i = tid + NT * j;
        v1[j] = c.snap_src != nullptr && i < c.snap_words ? c.snap_src[i] : 0u;
        v2[j] = c.snap_src2 != nullptr && i < c.snap_words2 ? c.snap_src2[i] : 0u;
    }
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
        const uint32_t i = tid + NT * j;
        if (c.snap_src != nullptr && i < c.snap_words) c.snap_dst[i] = v1[j];
        if (c.snap_src2 != nullptr && i < c.snap_words2) c.snap_dst2[i] = v2[j];
    }
    const Plan* p = c.plan;
    const uint32_t N = c.n_entries, E = c.n_experts;
    const uint32_t ng = p->n_groups, nt = p->n_tiles;
    auto fail = [&]() {
        atomicOr(c.status, 2u);
        if (c.status2 != nullptr) atomicOr(c.status2, 2u);
    };
    if (tid == 0) {
        if (reset_status) {
            *c.status = 0u;
            if (c.status2 != nullptr) *c.status2 = 0u;
        }
        s_groups_ok = 1u;
        s_header_ok = (p->bad == 0u && ng != 0u && ng <= E && ng <= 512u && p->n_entries == N &&
                       nt <= c.tile_capacity && nt <= p->n_entries && p->grp_start[0] == 0 &&
                       p->grp_start[ng] == int32_t(N))
                          ? 1u : 0u;
    }
    __syncthreads();
    if (!s_header_ok) {
        if (tid == 0) fail();
        return;
    }
    // Group g: non-empty, inside [0, N), expert in range and strictly ascending.
    uint32_t my_tiles = 0;
    for (uint32_t g = tid; g < ng; g += NT) {
        const int32_t first = p->grp_start[g], end = p->grp_start[g + 1], ex = p->grp_e[g];
        bool ok = end > first && uint32_t(end) <= N && ex >= 0 && uint32_t(ex) < E;
        if (g != 0u) ok = ok && ex > p->grp_e[g - 1];
        if (!ok) s_groups_ok = 0u;
        else my_tiles += (uint32_t(end - first) + kExpertTile - 1) / kExpertTile;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) my_tiles += __shfl_xor(my_tiles, off);
    if (lane == 0) s_wave_tiles[wave] = my_tiles;
    __syncthreads();
    uint32_t expected = 0;
    for (uint32_t w = 0; w < NT / 64; ++w) expected += s_wave_tiles[w];
    if (!s_groups_ok || expected != nt) {
        if (tid == 0) fail();
        return;
    }
    const uint32_t* tiles = c.tiles;
    for (uint32_t i = tid; i < nt; i += NT) {
        const uint32_t tg = tiles[2 * i], ty = tiles[2 * i + 1];
        bool ok = tg < ng;
        if (ok) {
            const uint32_t first = uint32_t(p->grp_start[tg]), end = uint32_t(p->grp_start[tg + 1]);
            ok = ty >= first && ty < end && (ty - first) % kExpertTile == 0u;
            if (i == 0u) {
                ok = ok && tg == 0u && ty == 0u;
            } else {
                const uint32_t pg = tiles[2 * (i - 1)], py = tiles[2 * (i - 1) + 1];
                if (pg >= ng) ok = false;
                else if (pg == tg) ok = ok && ty == py + kExpertTile;
                else if (pg + 1u == tg) ok = ok && py + kExpertTile >= uint32_t(p->grp_start[pg + 1]) && ty == first;
                else ok = false;
            }
            if (i + 1u == nt) ok = ok && tg + 1u == ng && ty + kExpertTile >= end;
        }
        if (!ok) fail();
    }
}

__global__ __launch_bounds__(512) void plan_validate_kernel(PlanCheck c) {
    for (uint32_t i = blockIdx.x * 512u + threadIdx.x; i < c.clear_words; i += gridDim.x * 512u) c.clear[i] = 0u;
    if (blockIdx.x != 0) return;
    check_plan<512>(c, c.keep_status == 0u);
}

// Xs[a,:] = X[token(a),:] for every valid entry a < the plan's valid-entry count, walked in
// route order. Workgroup (tile, part) takes the kCountTile route entries of histogram tile
// `tile` and column part `part` of the rows (kGatherPart 16-byte chunks, 256 bytes). It
// recomputes each entry's grouped slot exactly as the scatter wrote it (the tile's final
// cursors in hist plus the entry's stable rank among the tile's equal ids), then loads each
// token's row part once and stores it to the slots of that token's entries in the tile: X is
// read once (a token whose entries straddle two tiles, twice), and each thread keeps its
// token's loads ahead of a run of up to top-k stores. The stores are non-temporal: the grouped
// rows are a write-once stream. The plan header is checked first as in the reference's gather
// (prefill_moe.metal:282-297); an inconsistent plan writes nothing.
// CHECK (a full layer, both expert stages on the grouping's plan): workgroup 0 runs the
// stages' plan check (prefill_moe.metal:603-733) and the copy workgroups are 1..; copy
// workgroup (tile, part) also marks its share of the tile's entries of `dst` in the bitset,
// which is the reference's destination check (prefill_moe_down_dispatch.mm:470-520) spread
// over the gather: an entry outside [0, N) or one already marked sets bit 1 of the down status.
constexpr uint32_t kGatherPart = 16, kGatherBatch = 2;
template <bool CHECK>
__global__ __launch_bounds__(256) void gather_kernel(const u32x4* __restrict__ x, uint32_t vpr,
                                                     const int32_t* __restrict__ ids,
                                                     const uint32_t* __restrict__ hist, uint32_t K, uint32_t E,
                                                     uint32_t parts, const Plan* __restrict__ plan, uint32_t N,
                                                     u32x4* __restrict__ xs, PlanCheck c,
                                                     const int32_t* __restrict__ dst, uint32_t* __restrict__ bits) {
    __shared__ uint32_t wcnt[4][512];
    __shared__ uint32_t s_base[512];
    __shared__ uint32_t s_slot[kCountTile];
    uint32_t b = blockIdx.x;
    if constexpr (CHECK) {
        if (b == 0) {
            check_plan<256>(c, false);
            return;
        }
        b -= 1u;
    }
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const uint32_t tile = b / parts, part = b - tile * parts;
    const uint32_t i0 = tile * kCountTile, i1 = i0 + kCountTile < N ? i0 + kCountTile : N;
    // Thread (row lane j, chunk) copies tokens t0 + j, t0 + j + rpar, ... of the tile; the first
    // kGatherBatch of them are loaded before anything else (they depend on the tile alone).
    const uint32_t rpar = 256u / kGatherPart, j = tid / kGatherPart;
    const uint32_t col = part * kGatherPart + (tid - j * kGatherPart);
    const uint32_t t0 = i0 / K, t1 = (i1 - 1u) / K;
    u32x4 v[kGatherBatch];
    auto load_batch = [&](uint32_t tb) {
#pragma unroll
        for (uint32_t q = 0; q < kGatherBatch; ++q) {
            const uint32_t t = tb + j + q * rpar;
            if (t <= t1) v[q] = x[uint64_t(t) * vpr + col];
        }
    };
    load_batch(t0);
    const uint64_t entry = uint64_t(i0) + tid;
    const int32_t id = entry < N ? ids[entry] : -1;  // issued before the plan reads
    for (uint32_t e = tid; e < E; e += 256u) s_base[e] = hist[uint64_t(tile) * E + e];
    // CHECK: this workgroup's share of the tile's destinations, loaded with the other first
    // loads and marked after the copies (a returning atomic would hold the copies behind its
    // round trip).
    bool marks = false;
    uint32_t dv = 0;
    if constexpr (CHECK) {
        const uint32_t per = (kCountTile + parts - 1u) / parts;
        const uint32_t i = i0 + part * per + tid;
        marks = tid < per && i < i1;
        if (marks) dv = uint32_t(dst[i]);
    }
    auto mark = [&]() {
        if (!marks) return;
        if (dv >= N) {
            atomicOr(c.status2, 2u);
        } else {
            const uint32_t mask = 1u << (dv % 32u);
            if (atomicOr(&bits[dv / 32u], mask) & mask) atomicOr(c.status2, 2u);
        }
    };
    for (uint32_t k = tid; k < 4u * 512u; k += 256u) (&wcnt[0][0])[k] = 0u;
    const uint32_t ng = plan->n_groups;
    if (ng > 512u || plan->n_entries != N || plan->bad > plan->n_entries) {
        mark();
        return;
    }
    const int32_t sorted_signed = plan->grp_start[ng];
    if (sorted_signed < 0 || uint32_t(sorted_signed) != N - plan->bad) {
        mark();
        return;
    }
    // The entry's slot, as group_scatter_kernel computed it.
    const bool valid = id >= 0 && uint32_t(id) < E;
    const uint32_t key = valid ? uint32_t(id) : 1023u;
    uint64_t match = ~0ull;
#pragma unroll
    for (int bit = 0; bit < 10; ++bit) {
        const bool on = (key >> bit) & 1u;
        const uint64_t bal = __ballot(on);
        match &= on ? bal : ~bal;
    }
    const uint32_t rank = __popcll(match & ((1ull << lane) - 1ull));
    const uint64_t gt = lane == 63u ? 0ull : (~0ull << (lane + 1u));
    __syncthreads();
    if (valid && (match & gt) == 0ull) wcnt[wave][id] = rank + 1u;
    __syncthreads();
    uint32_t slot = ~0u;
    if (valid) {
        slot = s_base[id] + rank;
        for (uint32_t w = 0; w < wave; ++w) slot += wcnt[w][id];
        if (slot >= uint32_t(sorted_signed)) slot = ~0u;  // only behind an inconsistent histogram
    }
    s_slot[tid] = slot;
    __syncthreads();
    for (uint32_t tb = t0;; tb += kGatherBatch * rpar) {
        if (tb != t0) load_batch(tb);
#pragma unroll
        for (uint32_t q = 0; q < kGatherBatch; ++q) {
            const uint32_t t = tb + j + q * rpar;
            if (t > t1) break;
            const uint32_t r0 = t * K < i0 ? i0 - t * K : 0u;
            const uint32_t r1 = t * K + K > i1 ? i1 - t * K : K;
            for (uint32_t r = r0; r < r1; ++r) {
                const uint32_t sl = s_slot[t * K + r - i0];
                if (sl != ~0u) __builtin_nontemporal_store(v[q], &xs[uint64_t(sl) * vpr + col]);
            }
        }
        if (tb + kGatherBatch * rpar > t1) break;
    }
    mark();
}

__global__ __launch_bounds__(256) void bitset_clear_kernel(uint32_t* __restrict__ bits, uint32_t words) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i < words) bits[i] = 0u;
}

__global__ __launch_bounds__(256) void destination_validate_kernel(const int32_t* __restrict__ dst,
                                                                   uint32_t* __restrict__ bits,
                                                                   uint32_t* __restrict__ status,
                                                                   uint32_t N) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= N) return;
    const uint32_t d = uint32_t(dst[i]);
    if (d >= N) { atomicOr(status, 2u); return; }
    const uint32_t mask = 1u << (d % 32u);
    if (atomicOr(&bits[d / 32u], mask) & mask) atomicOr(status, 2u);
}

}  // namespace

hipError_t launch_router_gemm(const _Float16* x, const float* w, const float* bias, float* logits,
                              uint32_t rows, uint32_t d, uint32_t E, hipStream_t s, const RouterPrep* prep) {
    const RouterPrep rp = prep != nullptr ? *prep : RouterPrep{};
    // The largest token tile that still launches at least one workgroup per CU (256), so
    // each expert's weights are split as few times as the layer allows.
    const uint32_t ecols = (E + kRouterCols - 1) / kRouterCols;
    auto blocks = [&](uint32_t r) { return ((rows + r - 1) / r) * ecols; };
    if (blocks(128) >= 256u) {
        router_gemm_kernel<128><<<dim3((rows + 127) / 128, ecols), kRouterThreads, 0, s>>>(x, w, bias, logits, rows, d, E, rp);
    } else if (blocks(64) >= 256u) {
        router_gemm_kernel<64><<<dim3((rows + 63) / 64, ecols), kRouterThreads, 0, s>>>(x, w, bias, logits, rows, d, E, rp);
    } else {
        router_gemm_kernel<32><<<dim3((rows + 31) / 32, ecols), kRouterThreads, 0, s>>>(x, w, bias, logits, rows, d, E, rp);
    }
    return hipGetLastError();
}

hipError_t launch_route_topk(const float* logits, int32_t* ids, float* weights, uint32_t rows,
                             uint32_t E, uint32_t K, int divide, hipStream_t s, uint32_t* hist) {
    if (E == 0u || E > 512u || K == 0u || K > 32u || K > E) return hipErrorInvalidValue;
    // Up to 1024 tokens (one wave per SIMD at most) a token takes a whole wave; more tokens
    // share waves two by two.
    if (rows <= kTopkWaveRows) {
        const uint32_t blocks = (rows + 3u) / 4u, nv = (E + 63u) / 64u;
        if (nv <= 1) route_topk_kernel<1, true><<<blocks, 256, 0, s>>>(logits, ids, weights, rows, E, K, divide, hist);
        else if (nv <= 2) route_topk_kernel<2, true><<<blocks, 256, 0, s>>>(logits, ids, weights, rows, E, K, divide, hist);
        else if (nv <= 4) route_topk_kernel<4, true><<<blocks, 256, 0, s>>>(logits, ids, weights, rows, E, K, divide, hist);
        else route_topk_kernel<8, true><<<blocks, 256, 0, s>>>(logits, ids, weights, rows, E, K, divide, hist);
    } else {
        const uint32_t blocks = (rows + 7u) / 8u, nv = (E + 31u) / 32u;
        if (nv <= 1) route_topk_kernel<1, false><<<blocks, 256, 0, s>>>(logits, ids, weights, rows, E, K, divide, hist);
        else if (nv <= 2) route_topk_kernel<2, false><<<blocks, 256, 0, s>>>(logits, ids, weights, rows, E, K, divide, hist);
        else if (nv <= 4) route_topk_kernel<4, false><<<blocks, 256, 0, s>>>(logits, ids, weights, rows, E, K, divide, hist);
        else if (nv <= 8) route_topk_kernel<8, false><<<blocks, 256, 0, s>>>(logits, ids, weights, rows, E, K, divide, hist);
        else route_topk_kernel<16, false><<<blocks, 256, 0, s>>>(logits, ids, weights, rows, E, K, divide, hist);
    }
    return hipGetLastError();
}

hipError_t launch_grouping(const int32_t* ids, uint32_t rows, uint32_t K, uint32_t E, uint32_t* hist,
                           Plan* plan, uint32_t* tiles, int32_t* src, int32_t* dst, const GroupPrep* prep,
                           const int32_t* resident,
                           hipStream_t s, bool counted) {
    const uint32_t N = rows * K;
    const uint32_t n_tiles = (N + kCountTile - 1) / kCountTile;
    uint32_t* arrive = reinterpret_cast<uint32_t*>(reinterpret_cast<uint8_t*>(plan) + kArriveBytes);
    if (!counted) group_count_kernel<<<n_tiles, 256, 0, s>>>(ids, N, E, hist, arrive);
    group_scan_plan_kernel<<<(E + 31) / 32, kScanThreads, 0, s>>>(hist, E, N, n_tiles, plan, tiles, arrive,
                                                                  prep != nullptr ? *prep : GroupPrep{}, resident);
    group_scatter_kernel<<<n_tiles, 256, 0, s>>>(ids, N, K, E, n_tiles, hist, src, dst);
    return hipGetLastError();
}

hipError_t launch_gather(const _Float16* x, uint32_t d, const int32_t* ids, const uint32_t* hist, uint32_t K,
                         uint32_t E, const Plan* plan, uint32_t N, _Float16* xs, hipStream_t s) {
    const uint32_t vpr = d / 8, parts = vpr / kGatherPart;  // d % 256 == 0
    const uint32_t blocks = parts * ((N + kCountTile - 1) / kCountTile);  // (tile, part) pairs
    gather_kernel<false><<<blocks, 256, 0, s>>>(reinterpret_cast<const u32x4*>(x), vpr, ids, hist, K, E, parts,
                                                plan, N, reinterpret_cast<u32x4*>(xs), PlanCheck{}, nullptr, nullptr);
    return hipGetLastError();
}

hipError_t launch_gather_checked(const _Float16* x, uint32_t d, const int32_t* ids, const uint32_t* hist, uint32_t K,
                                 uint32_t E, const Plan* plan, uint32_t N, _Float16* xs, const PlanCheck& c,
                                 const int32_t* dst, uint32_t* bits, hipStream_t s) {
    if (c.snap_words > 1536u || c.snap_words2 > 1536u || c.status2 == nullptr) return hipErrorInvalidValue;
    const uint32_t vpr = d / 8, parts = vpr / kGatherPart;
    const uint32_t blocks = 1u + parts * ((N + kCountTile - 1) / kCountTile);  // check + copy workgroups
    gather_kernel<true><<<blocks, 256, 0, s>>>(reinterpret_cast<const u32x4*>(x), vpr, ids, hist, K, E, parts, plan,
                                               N, reinterpret_cast<u32x4*>(xs), c, dst, bits);
    return hipGetLastError();
}

hipError_t launch_plan_validate(const PlanCheck& c, hipStream_t s) {
    if (c.snap_words > 1536u || c.snap_words2 > 1536u) return hipErrorInvalidValue;  // E <= 512
    const uint32_t blocks = 1u + c.clear_words / (512u * 16u);
    plan_validate_kernel<<<blocks, 512, 0, s>>>(c);
    return hipGetLastError();
}

hipError_t launch_destination_validate(const int32_t* dst, uint32_t* bits, uint32_t* status, uint32_t N,
                                       bool bitset_clear, hipStream_t s) {
    const uint32_t words = (N + 31) / 32;
    if (bitset_clear) bitset_clear_kernel<<<(words + 255) / 256, 256, 0, s>>>(bits, words);
    destination_validate_kernel<<<(N + 255) / 256, 256, 0, s>>>(dst, bits, status, N);
    return hipGetLastError();
}

}  // namespace sm
