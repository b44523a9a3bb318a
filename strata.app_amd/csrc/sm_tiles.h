// The 64-row tile machinery of the routed expert products on gfx950 (groups below the wide
// kernel's threshold): enumeration of the small groups' tiles, LDS-DMA copies of activation
// slabs and packed weight images, per-lane decode into the MFMA B layout, and the fused
// epilogues. Included by the translation units that launch tile items: the standalone
// staged kernel (sm_gemm.hip) and the routed stage kernel, which runs a stage's wide units
// and then its tiles in one launch (sm_wide.hip).
#pragma once

#include <type_traits>

#include "sm_device.h"
#include "sm_launch.h"

namespace sm {
namespace {

constexpr int kSlab = 256;  // values per K slab (one Q4_K / Q2_K super-block, eight Q8_0 blocks)

// ---------------------------------------------------------------------------------------
// Routed products, staged: 512-thread workgroups (8 waves) over a 64-row tile and `npi`
// consecutive column tiles. Each wave owns NF 16-column weight fragments (NF = 2 or 4) and
// all 64 rows, so one column tile covers 128*NF weight rows (gate/up: 64*NF gate rows and
// the 64*NF up rows of the same hidden columns; down: 128*NF output columns). Per (column
// tile, slab) step the 64 x 256 activation slab and the weight-row slabs are copied
// global -> LDS by LDS-DMA (global_load_lds), one step ahead and interleaved with the
// multiplies; lanes then read their raw fragments from LDS, decode them into the MFMA B
// layout and multiply against A fragments from the XOR-swizzled activation slab. The steps
// of a workgroup form one flat pipeline, so short reductions (down: K = I) do not drain it
// between column tiles.
// ---------------------------------------------------------------------------------------
constexpr int kV2Threads = 512;

// Position (in 16-byte chunks) of chunk c of row r inside a swizzled 64 x 256 slab. LDS has
// 64 banks of 4 bytes, so a 16-byte chunk at position p sits in bank group p % 16, and a
// ds_read_b128 of 64 lanes is served in passes of 16 lanes that never pair two lanes with the
// same lane % 16 (a plain linear read is conflict-free) but do pair lanes of different
// 16-lane quarters. An A-fragment read (lane n + 16 gq: row 16 rb + n, chunk 8 gq + s) must
// therefore put every lane in a bank group that depends on n alone: here n ^ s. Positions
// are grouped as [rb][gq][n & 7][16], so each 16-chunk group holds chunks 8 gq .. 8 gq + 7 of
// rows n and n + 8 (two whole 128-byte lines of the activation rows).
__device__ __forceinline__ uint32_t a_pos(uint32_t r, uint32_t c) {
    const uint32_t n = r & 15u;
    return 16u * (32u * (r >> 4) + 8u * (c >> 3) + (n & 7u)) + (n ^ (c & 7u));
}

template <int MODE>
__device__ void zero_cols(const RoutedGemm& g, uint32_t r0, uint32_t r1, uint32_t c0, uint32_t c1, bool by_dst) {
    const uint32_t width = c1 - c0;
    for (uint32_t i = threadIdx.x; i < 64u * width; i += blockDim.x) {
        const uint32_t r = r0 + i / width, c = c0 + i % width;
        if (r >= r1 || r >= g.n_entries) continue;
        if (MODE == kGateUp) {
            g.out_h[uint64_t(r) * g.n_out + c] = _Float16(0.0f);
        } else if (!by_dst) {
            g.out_f[uint64_t(r) * g.n_out + c] = 0.0f;
        } else {
            const uint32_t d = uint32_t(g.dst[r]);
            if (d < g.n_entries) g.out_f[uint64_t(d) * g.n_out + c] = 0.0f;
            else atomicOr(g.status, 2u);
        }
    }
}

// The work item of one staged workgroup: tile rows [a0, a1) of one expert group and column
// tiles [nt_begin, nt_end), with the expert's two weight matrices.
struct TileWork {
    uint32_t a0, a1, nt_begin, nt_end;
    const uint8_t* w0;
    const uint8_t* w1;
};

// Tile enumeration of the persistent staged kernels (512 threads), once per workgroup:
// reads the status word and counts, per plan group below wide_min entries, its
// ceil(size / 64) tiles; s_pref[gi] = tiles of the groups before gi. The plan has been
// checked against the tile list by the plan validator, so these are exactly the list's
// tiles of those groups, in order. A group that fails the range checks contributes no
// tiles and reports status bit 1 (it cannot occur behind a passed plan check). Returns the
// status word read at start.
// The plan's group starts and experts kept in LDS by the enumeration pass (s_grp: starts
// [0, 513), experts [513, 1025)), so the item lookups cost no plan round trip.
constexpr uint32_t kGrpWords = 1025;
__device__ __forceinline__ void stash_groups(int32_t* s_grp, uint32_t tid, int32_t f, int32_t e, int32_t ex) {
    s_grp[tid] = f;
    if (tid == 511u) s_grp[512] = e;
    s_grp[513u + tid] = ex;
}
// Start, end and expert of group gi (gi < 512): from the stash when there is one.
__device__ __forceinline__ void group_fields(const Plan* p, const int32_t* s_grp, uint32_t gi, uint32_t& f, uint32_t& e,
                                             uint32_t& ex) {
    if (s_grp != nullptr) {
        f = uint32_t(s_grp[gi]);
        e = uint32_t(s_grp[gi + 1u]);
        ex = uint32_t(s_grp[513u + gi]);
    } else {
        f = uint32_t(p->grp_start[gi]);
        e = uint32_t(p->grp_start[gi + 1u]);
        ex = uint32_t(p->grp_e[gi]);
    }
}

// Small-tile enumeration (512 threads, once per workgroup): groups below wide_min entries,
// ceil(size / 64) tiles each; s_pref[gi] = tiles of the groups before gi, s_pref[512] = all.
// Every group field is loaded without waiting for n_groups (thread gi < 512 reads inside the
// plan's arrays whatever n_groups holds), so the scan costs one round trip. An unusable group
// sets status bit 1. Returns the status word read at start.
__device__ __forceinline__ uint32_t scan_small_tiles(const RoutedGemm& g, uint32_t* s_pref, uint32_t* s_wsum, uint32_t* s_flag,
                                                     int32_t* s_grp = nullptr) {
    const Plan* p = g.plan;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    if (tid == 0) *s_flag = __hip_atomic_load(g.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t ng_raw = p->n_groups;
    const int32_t f = p->grp_start[tid], e = p->grp_start[tid + 1], ex = p->grp_e[tid];
    if (s_grp != nullptr) stash_groups(s_grp, tid, f, e, ex);
    const uint32_t ng = ng_raw < 512u ? ng_raw : 512u;
    uint32_t n = 0;
    if (tid < ng) {
        if (f >= 0 && e > f && uint32_t(e) <= g.n_entries && ex >= 0 && uint32_t(ex) < g.n_experts) {
            if (uint32_t(e - f) < g.wide_min) n = (uint32_t(e - f) + 63u) / 64u;
        } else {
            atomicOr(g.status, 2u);
        }
    }
#pragma unroll
    for (uint32_t off = 1; off < 64u; off <<= 1) {
        const uint32_t y = __shfl_up(n, off);
        if (lane >= off) n += y;
    }
    if (lane == 63u) s_wsum[wave] = n;
    __syncthreads();
    uint32_t base = 0;
    for (uint32_t w = 0; w < wave; ++w) base += s_wsum[w];
    s_pref[tid + 1] = base + n;
    if (tid == 0) s_pref[0] = 0;
    __syncthreads();
    return *s_flag;
}

// Item `item` (tile k = item / n_chunks of the enumeration, column chunk item % n_chunks):
// its rows, column tiles and weights, and the weight fault code (0: usable). No side
// effects. Uniform per workgroup.
template <int MODE>
__device__ __forceinline__ uint32_t staged_item_work(const RoutedGemm& g, const uint32_t* s_pref, uint32_t item,
                                                     uint32_t n_ntiles, uint32_t npi, uint32_t n_chunks, TileWork& t,
                                                     const int32_t* s_grp) {
    const Plan* p = g.plan;
    const uint32_t k = item / n_chunks, chunk = item - k * n_chunks;
    uint32_t lo = 0, hi = 512;
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (s_pref[mid] <= k) lo = mid;
        else hi = mid;
    }
    uint32_t f, e, ex;
    group_fields(p, s_grp, lo, f, e, ex);
    t.nt_begin = chunk * npi;
    t.nt_end = t.nt_begin + npi < n_ntiles ? t.nt_begin + npi : n_ntiles;
    t.a0 = f + 64u * (k - s_pref[lo]);
    t.a1 = t.a0 + 64u < e ? t.a0 + 64u : e;
    const uint64_t* addr = g.addresses + 3u * ex;
    t.w0 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[0] : addr[2]);
    t.w1 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[1] : addr[2]);
    return weight_fault(t.w0, t.w1);
}

// staged_item_work, and false when the item is done already: an expert without usable
// weights has zeroed its rows and set status bit 0 (missing) or 2 (unleased tiered slot).
template <int MODE>
__device__ bool staged_item(const RoutedGemm& g, const uint32_t* s_pref, uint32_t item, uint32_t n_ntiles,
                            uint32_t npi, uint32_t n_chunks, uint32_t out_per_nt, TileWork& t, const int32_t* s_grp) {
    if (const uint32_t fault = staged_item_work<MODE>(g, s_pref, item, n_ntiles, npi, n_chunks, t, s_grp)) {
        if (threadIdx.x == 0) atomicOr(g.status, fault);
        zero_cols<MODE>(g, t.a0, t.a1, t.nt_begin * out_per_nt, t.nt_end * out_per_nt, MODE == kDown);
        return false;
    }
    return true;
}

// Activation copy map of one 64 x 256 slab: wave instruction q = 4*wave + j (j = 0..3)
// fills chunk positions [64q, 64q + 64), the inverse of a_pos: position 16 Q + rho holds
// row 16 (Q >> 5) + ((Q & 7) | (rho & 8)), chunk 8 ((Q >> 3) & 3) + ((rho & 7) ^ (Q & 7)).
// Each instruction reads eight whole 128-byte lines (8 rows x 8 chunks). Rows past the
// tile's end repeat its last row.
__device__ __forceinline__ void slab_sources(const RoutedGemm& g, const TileWork& t, int wave, int lane,
                                             const _Float16* (&asrc)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t Q = 4u * (4u * wave + j) + (uint32_t(lane) >> 4), rho = uint32_t(lane) & 15u;
        const uint32_t R = 16u * (Q >> 5) + ((Q & 7u) | (rho & 8u));
        const uint32_t C = 8u * ((Q >> 3) & 3u) + ((rho & 7u) ^ (Q & 7u));
        uint32_t row = t.a0 + R;
        if (row > t.a1 - 1u) row = t.a1 - 1u;
        asrc[j] = g.a + uint64_t(row) * g.k + 8u * C;
    }
}

// Issues LDS-DMA copy j (0..3, 16 B per lane) of this wave's share of the slab at k0.
__device__ __forceinline__ void issue_slab_part(const _Float16* const (&asrc)[4], uint32_t k0, _Float16* slab,
                                                int wave, int j) {
    __builtin_amdgcn_global_load_lds(
        reinterpret_cast<const __attribute__((address_space(1))) void*>(reinterpret_cast<uintptr_t>(asrc[j] + k0)),
        reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(slab + (4 * wave + j) * 512)),
        16, 0, 0);
}
__device__ __forceinline__ void issue_slab(const _Float16* const (&asrc)[4], uint32_t k0, _Float16* slab, int wave) {
#pragma unroll
    for (int j = 0; j < 4; ++j) issue_slab_part(asrc, k0, slab, wave, j);
}

// Geometry of a staged step with NF fragments per wave.
template <int MODE, int NF>
struct Staged {
    static constexpr uint32_t kImageRows = 128u * NF;                          // weight rows per step
    static constexpr uint32_t kHalf = 64u * NF;                                // gate/up: gate rows, then up rows
    static constexpr uint32_t kOut = MODE == kGateUp ? 64u * NF : 128u * NF;   // output columns per column tile
    // Column of lane n's fragment f within the column tile (gate/up: the hidden column, the
    // same for gate fragment f and up fragment f + NF/2). Down interleaves the fragments, so
    // lane n holds NF adjacent output columns and 16 lanes store whole 128-byte row pieces.
    __device__ static __forceinline__ uint32_t col(int wave, int n, int f) {
        if (MODE == kGateUp) return uint32_t(wave) * (8u * NF) + 16u * uint32_t(f % (NF / 2)) + uint32_t(n);
        return uint32_t(wave) * (16u * NF) + NF * uint32_t(n) + uint32_t(f);
    }
    // Row of the packed weight image holding that fragment.
    __device__ static __forceinline__ uint32_t image_row(int wave, int n, int f) {
        if (MODE == kGateUp) return (f < NF / 2 ? 0u : kHalf) + col(wave, n, f);
        return col(wave, n, f);
    }
};

// One 256-value slab of the wave's block. Only the first RB 16-row blocks of the tile hold
// entries (the rest of a 64-row tile past its group's end would multiply padding), so the
// others are skipped. The A fragments and decoded B fragments of k-step s + 1 are read and
// decoded while the MFMAs of k-step s run (two register sets), so no MFMA waits on the LDS
// read or the decode just before it. after_s(s) runs after k-step s: the staged kernel
// issues part s of the next step's copies there, so a wave never blocks on a long burst of
// memory instructions while it could be multiplying.
template <class Frag, int NF, int RB, class After>
__device__ __forceinline__ void slab_mma(const _Float16* buf, int n, int gq, const Frag (&c)[NF],
                                         float4v (&acc)[NF][4], After after_s) {
    half8 a[2][RB], b[2][NF];
    auto fetch = [&](int s, int z) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) a[z][rb] = *reinterpret_cast<const half8*>(buf + 8u * a_pos(16u * rb + n, 8u * gq + s));
#pragma unroll
        for (int f = 0; f < NF; ++f) b[z][f] = c[f].step(s);
    };
    fetch(0, 0);
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const int z = s & 1;
        if (s + 1 < 8) fetch(s + 1, z ^ 1);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int f = 0; f < NF; ++f) acc[f][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[z][rb], b[z][f], acc[f][rb], 0, 0, 0);
        after_s(s);
    }
}

// Writes a finished column tile and clears the accumulators. gate/up: eh[a][col] =
// half_sat(silu(gate) * up); down: parts[dst[a]][col], with a destination outside [0, N)
// reported (status bit 1) and the entry's own row zeroed instead.
template <int MODE, int NF, int RB>
__device__ __forceinline__ void staged_epilogue(const RoutedGemm& g, const uint32_t* s_dst, uint32_t a0, uint32_t a1,
                                                uint32_t col0, int wave, int n, int gq, float4v (&acc)[NF][4]) {
    using S = Staged<MODE, NF>;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = a0 + 16u * rb + 4u * gq + i;
            if (a >= a1) continue;
            if (MODE == kGateUp) {
#pragma unroll
                for (int f = 0; f < NF / 2; ++f)
                    g.out_h[uint64_t(a) * g.n_out + col0 + S::col(wave, n, f)] =
                        half_sat(silu_fast(acc[f][rb][i]) * acc[f + NF / 2][rb][i]);
            } else {
                const uint32_t d = s_dst[16 * rb + 4 * gq + i];
                const bool good = d < g.n_entries;
                if (!good) atomicOr(g.status, 2u);
                const uint64_t row = good ? d : a;
                typedef float vecf __attribute__((ext_vector_type(NF)));
                vecf v;
#pragma unroll
                for (int f = 0; f < NF; ++f) v[f] = good ? acc[f][rb][i] : 0.0f;
                // Write-once rows: non-temporal, so they do not evict the weight lines that the
                // next step of this or another item still reads.
                __builtin_nontemporal_store(v, reinterpret_cast<vecf*>(g.out_f + row * g.n_out + col0 + S::col(wave, n, 0)));
            }
        }
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[f][rb] = float4v{0, 0, 0, 0};
}

// Gate/up with a free weight image (two images, NF = 2): the column tile's F16 rows go
// through LDS (the image this step has finished reading, [64 rows][128 columns + 8 pad]), so
// each wave stores 8 whole 256-byte row pieces with 16-byte stores (2 instructions) instead of
// 16 scattered 2-byte stores. Rows past the tile's end are not stored.
template <int RB>
__device__ __forceinline__ void staged_epilogue_lds(const RoutedGemm& g, uint32_t a0, uint32_t a1, uint32_t col0,
                                                    int wave, int lane, float4v (&acc)[2][4], uint8_t* stage) {
    constexpr uint32_t kRowB = 272u;  // 128 halves + 16 bytes of pad: the 4 rows of a write hit distinct banks
    const int n = lane & 15, gq = lane >> 4;
    // LDS-only barriers: the next step's copies, in flight, need not land here.
    __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // fragments read from the image
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t row = 16u * rb + 4u * gq + i;
            *reinterpret_cast<_Float16*>(stage + row * kRowB + 2u * (16u * wave + n)) =
                half_sat(silu_fast(acc[0][rb][i]) * acc[1][rb][i]);
        }
#pragma unroll
    for (int f = 0; f < 2; ++f)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[f][rb] = float4v{0, 0, 0, 0};
    __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // the tile's rows are in LDS
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const uint32_t row = 8u * wave + 4u * j + uint32_t(gq), a = a0 + row;
        if (row < 16u * RB && a < a1)
            *reinterpret_cast<u32x4*>(g.out_h + uint64_t(a) * g.n_out + col0 + 8u * n) =
                *reinterpret_cast<const u32x4*>(stage + row * kRowB + 16u * n);
    }
}

// Bytes moved per lane by one LDS-DMA copy of weight-row slabs: 16 where the slab size
// allows, else 4 (Q2_K's 84-byte slabs). Lane l of a copy writes at LDS base + l * size.
template <int SB> struct ChunkBytes { static constexpr int value = SB % 16 == 0 ? 16 : 4; };

// The weight-row slabs of one (column tile, slab) step are copied into an LDS image packed
// as [128*NF rows][SB bytes] by LDS-DMA: wave instruction q moves the 64 consecutive chunks
// [64q, 64q + 64) of that image, so each instruction reads a few whole row slabs
// (contiguous bytes) instead of 64 scattered fragments. gate/up: image rows [0, 64*NF) are
// gate rows nt*64*NF + r, the rest the up rows of the same hidden columns; down: rows
// nt*128*NF + r. Every instruction is full (128*NF rows x SB/CS chunks is a multiple of 64)
// and lies wholly in the gate or the up half. Wave w issues instructions q = w + 8j;
// `off` keeps each lane's byte offset within its matrix for column tile 0, slab 0.
template <class Frag, int MODE, int NF>
struct WeightCopy {
    static constexpr int SB = SlabBytes<Frag>::value;
    static constexpr int CS = ChunkBytes<SB>::value;
    static constexpr uint32_t kPerRow = SB / CS;
    static constexpr uint32_t kInstr = Staged<MODE, NF>::kImageRows * kPerRow / 64u;
    static constexpr uint32_t kPerWave = (kInstr + 7u) / 8u;
    static_assert((Staged<MODE, NF>::kImageRows * kPerRow) % 128u == 0u, "copies must be whole wave instructions");
    uint32_t off[kPerWave];
    __device__ __forceinline__ void init(const RoutedGemm& g, int wave, int lane) {
#pragma unroll
        for (uint32_t j = 0; j < kPerWave; ++j) {
            const uint32_t c = 64u * (uint32_t(wave) + 8u * j) + uint32_t(lane);
            uint32_t r = c / kPerRow;
            const uint32_t piece = c - r * kPerRow;
            if (MODE == kGateUp && r >= Staged<MODE, NF>::kHalf) r -= Staged<MODE, NF>::kHalf;
            off[j] = r * g.row_bytes + piece * CS;  // < 512 rows x row_bytes: 32 bits suffice
        }
    }
    // Issues item j (instruction q = wave + 8j) of the copy for (nt, sb) into `wbuf`.
    __device__ __forceinline__ void issue(const RoutedGemm& g, const TileWork& t, uint32_t nt, uint32_t sb,
                                          uint8_t* wbuf, int wave, uint32_t j) const {
        const uint32_t q = uint32_t(wave) + 8u * j;
        if (q >= kInstr) return;
        const bool up = MODE == kGateUp && q >= kInstr / 2u;
        const uint8_t* base = up ? t.w1 : t.w0;
        const uint32_t rows_per_tile = MODE == kGateUp ? Staged<MODE, NF>::kHalf : Staged<MODE, NF>::kImageRows;
        const uint64_t tile_off = uint64_t(nt) * rows_per_tile * g.row_bytes + uint64_t(sb) * SB;
        const uint8_t* src = base + tile_off + off[j];
        auto* gsrc = reinterpret_cast<const __attribute__((address_space(1))) void*>(reinterpret_cast<uintptr_t>(src));
        auto* ldst = reinterpret_cast<__attribute__((address_space(3))) void*>(reinterpret_cast<uintptr_t>(wbuf + q * 64u * CS));
        if constexpr (CS == 16) __builtin_amdgcn_global_load_lds(gsrc, ldst, 16, 0, 0);
        else __builtin_amdgcn_global_load_lds(gsrc, ldst, 4, 0, 0);
    }
};

// Weight images per workgroup: two (one filled while the other is read) when they fit
// beside the activation double buffer within 140 KB of LDS, else one, read into registers
// behind a second barrier before it is refilled.
template <class Frag, int NF>
struct StagedBuffers {
    static constexpr uint32_t kImage = 128u * NF * SlabBytes<Frag>::value;
    static constexpr int kWBuf = 65536u + 2u * kImage <= 143360u ? 2 : 1;
    static_assert(65536u + kImage <= 143360u, "weight image too large for LDS");
};

// LDS of the staged tile kernels: the activation slabs (or the resident tile), the weight
// image(s), the tile's destination rows (down) and the next dynamically drawn item.
template <class Frag, int NF>
struct TileSmem {
    _Float16 sa[2][64 * kSlab] __attribute__((aligned(1024)));
    uint8_t sw[StagedBuffers<Frag, NF>::kWBuf][StagedBuffers<Frag, NF>::kImage] __attribute__((aligned(1024)));
    uint32_t s_dst[64];  // down: destination row of each tile row
    uint32_t s_next;
};

// Weights straight to registers instead of through an LDS image: where only one image would
// fit beside the resident activation tile (Q8_0 down, K <= 512), each lane loads its own
// fragments for the next step while it multiplies the current one, so the weight stream
// never waits for a barrier. (For the other formats and shapes the LDS image measured faster.)
template <class Frag, int MODE, bool RESIDENT>
struct DirectWeights {
    static constexpr bool value = MODE == kDown && RESIDENT && StagedBuffers<Frag, 2>::kWBuf == 1;
};

// Launch shape of the staged tile kernels for one stage: column tiles of 128*NF weight rows,
// `npi` of them per item (about 8 (column tile, slab) steps per item; with the activation tile
// resident (K <= 512) every column tile of a row tile goes to one item, so the tile is read
// once).
struct TilePlan {
    uint32_t n_ntiles, npi, n_chunks;
    bool resident;
};
template <int MODE, int NF>
inline TilePlan tile_plan(uint32_t k, uint32_t n_out) {
    TilePlan p;
    p.n_ntiles = n_out / Staged<MODE, NF>::kOut;
    const uint32_t n_slabs = k / kSlab;
    p.npi = n_slabs <= 2 ? p.n_ntiles : (n_slabs >= 8 ? 1u : 8u / n_slabs);
    if (p.npi > p.n_ntiles) p.npi = p.n_ntiles;
    p.n_chunks = (p.n_ntiles + p.npi - 1) / p.npi;
    p.resident = n_slabs <= 2;
    return p;
}

// Invalid plan or permutation: every tile slot writes zeros (the wide units' rows included,
// since slots cover every row the tile list can name).
template <int MODE, int NF>
__device__ void zero_tile_slots(const RoutedGemm& g, uint32_t n_ntiles, uint32_t npi, uint32_t n_chunks) {
    using S = Staged<MODE, NF>;
    for (uint32_t slot = blockIdx.x; slot < g.tile_capacity * n_chunks; slot += gridDim.x) {
        const uint32_t ti = slot / n_chunks, ch = slot % n_chunks;
        const uint32_t nb = ch * npi, ne = nb + npi < n_ntiles ? nb + npi : n_ntiles;
        zero_cols<MODE>(g, ti * 64u, ti * 64u + 64u, nb * S::kOut, ne * S::kOut, false);
    }
}

// The items of the tiles s_pref enumerates (scan_small_tiles). XCD x (workgroups b with
// b % 8 == x) takes the contiguous item range [x * per, (x + 1) * per), so the column chunks
// of a tile share that XCD's L2. Static: workgroup b takes items x * per + b / 8 + j * P.
// Dynamic (a kernel whose workgroups reach their tiles at different times): they draw the
// range's items from counter x of g.counters (zeroed by the stage's plan check); thread 0
// fetches the next item when it starts the current one and publishes it in s_next at the
// end, so the atomic's round trip overlaps the item's first copies.
// RESIDENT (K <= 512): both activation slabs are copied once and stay in LDS for all of
// the workgroup's column tiles, instead of being re-read from L2 for each of them.
template <class Frag, int MODE, int NF, bool RESIDENT, bool DYNAMIC>
__device__ __forceinline__ void tile_items(const RoutedGemm& g, TileSmem<Frag, NF>& sm, const uint32_t* s_pref,
                                           uint32_t n_ntiles, uint32_t npi, uint32_t n_chunks, const int32_t* s_grp) {
    constexpr bool dynamic = DYNAMIC;
    using S = Staged<MODE, NF>;
    using WC = WeightCopy<Frag, MODE, NF>;
    constexpr int SB = SlabBytes<Frag>::value;
    constexpr int WBUF = StagedBuffers<Frag, NF>::kWBuf;
    auto& sa = sm.sa;
    auto& sw = sm.sw;
    uint32_t* s_dst = sm.s_dst;
    const uint32_t items = s_pref[512] * n_chunks;
    const uint32_t per = (items + 7u) >> 3, x = blockIdx.x & 7u, P = gridDim.x >> 3;
    const uint32_t i_end = (x + 1u) * per < items ? (x + 1u) * per : items;
    uint32_t* counter = g.counters + x;
    uint32_t item_static = x * per + (blockIdx.x >> 3);
    if (dynamic && threadIdx.x == 0) sm.s_next = x * per + atomicAdd(counter, 1u);
    // Static order with streamed slabs and two weight images: the next item's work is looked
    // up at the start of the current one and its first copies are issued in the current
    // item's last step, into the buffers that step does not read, so an item starts without
    // the plan, address and copy round trips. Buffers then alternate across items: step s of
    // an item uses parity (par0 + s) & 1.
    constexpr bool XPF = !DYNAMIC && !RESIDENT && WBUF == 2;
    bool pf_have = false;  // the current item's work and first copies came from the previous one
    TileWork t_pf{};
    uint32_t par0 = 0;
    for (;; item_static += P) {
    __syncthreads();  // the previous item's reads of LDS are done; s_next is visible
    const uint32_t item = dynamic ? sm.s_next : item_static;
    if (item >= i_end) break;
    uint32_t next = 0;
    if (dynamic && threadIdx.x == 0) next = atomicAdd(counter, 1u);
    TileWork t;
    const bool pf = XPF && pf_have;
    if (pf) {
        t = t_pf;
    } else if (!staged_item<MODE>(g, s_pref, item, n_ntiles, npi, n_chunks, S::kOut, t, s_grp)) {
        __syncthreads();  // every thread has read s_next
        if (dynamic && threadIdx.x == 0) sm.s_next = x * per + next;
        continue;
    }
    TileWork t_nx{};
    bool nx_ok = false;  // an item whose weights fault is left to its own turn
    if (XPF && item + P < i_end)
        nx_ok = staged_item_work<MODE>(g, s_pref, item + P, n_ntiles, npi, n_chunks, t_nx, s_grp) == 0u;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, n = lane & 15, gq = lane >> 4;
    // Read once here rather than in each epilogue, where a dependent global load would also
    // wait for the copies of the next step (visible after the first loop barrier).
    if (MODE == kDown && tid < 64) s_dst[tid] = t.a0 + uint32_t(tid) < t.a1 ? uint32_t(g.dst[t.a0 + tid]) : ~0u;
    const uint32_t n_slabs = g.k / kSlab;
    const uint32_t n_steps = (t.nt_end - t.nt_begin) * n_slabs;
    const _Float16* asrc[4];
    slab_sources(g, t, wave, lane, asrc);
    WC wc;
    wc.init(g, wave, lane);
    // Part p (0..7) of the copies of `step`: activation copy p (p < 4, streamed slabs only)
    // and weight items j with j % 8 == p.
    // Part p (0..7) of the copies of step (nt, sb) into buffer `buf` (computed once per step by
    // the caller: the division by n_slabs stays out of the k-step loop).
    auto issue_part_of = [&](const TileWork& tw, const _Float16* const (&as)[4], uint32_t nt, uint32_t sb,
                             uint32_t buf, int p) {
        if (!RESIDENT && p < 4) issue_slab_part(as, sb * kSlab, sa[buf], wave, p);
        uint8_t* wb = sw[WBUF == 2 ? buf : 0u];
#pragma unroll
        for (uint32_t j = uint32_t(p); j < WC::kPerWave; j += 8u) wc.issue(g, tw, nt, sb, wb, wave, j);
    };
    auto issue_part = [&](uint32_t nt, uint32_t sb, uint32_t buf, int p) { issue_part_of(t, asrc, nt, sb, buf, p); };
    if (RESIDENT)
        for (uint32_t sb = 0; sb < n_slabs; ++sb) issue_slab(asrc, sb * kSlab, sa[sb], wave);
    constexpr bool DIRECT = DirectWeights<Frag, MODE, RESIDENT>::value;
    if constexpr (DIRECT) {
        // Steps are (column tile, half f): the wave's 16 weight rows of fragment f, rows
        // 128 f + 16 wave + n of the column tile, with every slab of them loaded at once, so a
        // step's eight waves read 128 consecutive rows whole. The 128-byte lines that two slabs
        // of a row share, and the end of one row with the start of the next (rows are 4.25
        // lines), are then fetched by one step, where loads a step apart fetched some of them
        // twice (lines evicted in between). The column tile's F32 results go out through LDS
        // (the weight image is unused here), so `parts` rows are written as whole 1 KB pieces.
        auto load_step = [&](auto& c, uint32_t tile, int f) {
            const uint32_t r = (t.nt_begin + tile) * S::kImageRows + 128u * uint32_t(f) + 16u * uint32_t(wave) + uint32_t(n);
#pragma unroll
            for (int sb = 0; sb < int(sizeof(c) / sizeof(c[0])); ++sb)
                c[sb][0].template load<FromGlobal>(t.w0 + uint64_t(r) * g.row_bytes + uint64_t(sb) * SB, gq);
        };
        // The finished column tile: accumulators -> LDS [row][256 + 4 pad] (the pad puts the
        // four lane groups' rows in distinct banks), then each wave stores 8 rows, 64 lanes x 16
        // bytes per row. Rows past the tile's end are not stored; a destination outside [0, N)
        // is reported (status bit 1) and the entry's own row is zeroed instead.
        constexpr uint32_t kStageRow = 260u;
        static_assert(64u * kStageRow * 4u <= StagedBuffers<Frag, NF>::kImage, "output tile must fit the image buffer");
        float* stage = reinterpret_cast<float*>(sw[0]);
        auto epilogue = [&](auto rb_const, float4v (&acc)[2][1][4], uint32_t tile) {
            constexpr int RB = decltype(rb_const)::value;
            __syncthreads();  // the previous tile's rows have been read out
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int rb = 0; rb < RB; ++rb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t row = 16u * rb + 4u * gq + i, col = 128u * f + 16u * wave + n;
                        stage[row * kStageRow + col] = acc[f][0][rb][i];
                        acc[f][0][rb][i] = 0.0f;
                    }
            __syncthreads();
            const uint32_t col0 = (t.nt_begin + tile) * S::kOut;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t row = 8u * wave + j, a = t.a0 + row;
                if (row >= 16u * RB || a >= t.a1) continue;  // wave-uniform
                const uint32_t d = s_dst[row];
                const bool good = d < g.n_entries;
                if (!good && lane == 0) atomicOr(g.status, 2u);
                float4v v = *reinterpret_cast<const float4v*>(stage + row * kStageRow + 4u * lane);
                if (!good) v = float4v{0, 0, 0, 0};
                // Write-once rows: non-temporal, so they do not evict the weight lines that the
                // next step of this or another item still reads.
                __builtin_nontemporal_store(v, reinterpret_cast<float4v*>(g.out_f + uint64_t(good ? d : a) * g.n_out + col0 + 4u * lane));
            }
        };
        auto run_direct = [&](auto rb_const, auto ns_const) {
            constexpr int RB = decltype(rb_const)::value;
            constexpr int NS = decltype(ns_const)::value;  // slabs (K = 256 NS)
            float4v acc[2][1][4];
#pragma unroll
            for (int f = 0; f < 2; ++f)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) acc[f][0][rb] = float4v{0, 0, 0, 0};
            const uint32_t n_tiles = t.nt_end - t.nt_begin;
            Frag fa[NS][1], fb[NS][1];
            load_step(fa, 0, 0);
            auto do_step = [&](Frag (&cur)[NS][1], float4v (&acc_f)[1][4]) {
#pragma unroll
                for (int sb = 0; sb < NS; ++sb) {
                    cur[sb][0].prepare();
                    slab_mma<Frag, 1, RB>(sa[sb], n, gq, cur[sb], acc_f, [](int) {});
                }
            };
            for (uint32_t tile = 0; tile < n_tiles; ++tile) {
                __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // fa: (tile, f = 0)
                if (tile == 0) __syncthreads();                         // the resident slabs
                load_step(fb, tile, 1);
                // The loads stay ahead of this step's work (left alone, the scheduler sinks them
                // below the multiplies, and the next step then waits for their whole latency).
                __builtin_amdgcn_sched_barrier(0);
                do_step(fa, acc[0]);
                __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // fb: (tile, f = 1)
                load_step(fa, tile + 1 < n_tiles ? tile + 1 : tile, 0);
                __builtin_amdgcn_sched_barrier(0);
                do_step(fb, acc[1]);
                epilogue(rb_const, acc, tile);
            }
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the repeated last loads
        };
        auto run_ns = [&](auto rb_const) {
            if (n_slabs == 2u) run_direct(rb_const, std::integral_constant<int, 2>());
            else run_direct(rb_const, std::integral_constant<int, 1>());
        };
        switch ((t.a1 - t.a0 + 15u) / 16u) {  // workgroup-uniform
            case 1: run_ns(std::integral_constant<int, 1>()); break;
            case 2: run_ns(std::integral_constant<int, 2>()); break;
            case 3: run_ns(std::integral_constant<int, 3>()); break;
            default: run_ns(std::integral_constant<int, 4>()); break;
        }
        if (dynamic && threadIdx.x == 0) sm.s_next = x * per + next;
        continue;
    }
    if (!pf) {
#pragma unroll
        for (int p = 0; p < 8; ++p) issue_part(t.nt_begin, 0u, par0, p);
    }
    // The step loop, specialised on the number of 16-row blocks holding entries.
    auto run = [&](auto rb_const) {
        constexpr int RB = decltype(rb_const)::value;
        float4v acc[NF][4];
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) acc[f][rb] = float4v{0, 0, 0, 0};
        uint32_t cur_nt = 0, cur_sb = 0;
        for (uint32_t step = 0; step < n_steps; ++step) {
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this step's copies ...
            __syncthreads();                                       // ... from every wave
            const bool more = step + 1 < n_steps;
            const uint32_t par = (par0 + step) & 1u;
            const uint8_t* wb = sw[WBUF == 2 ? par : 0u];
            Frag c[NF];
#pragma unroll
            for (int f = 0; f < NF; ++f) c[f].template load<FromLds>(wb + S::image_row(wave, n, f) * SB, gq);
            // A barrier waits for every outstanding load of the wave, so with one weight image
            // the next step's copies start only after the second barrier.
            if (WBUF == 1) __syncthreads();  // every wave holds its fragments: the image may be refilled
            // Column tile and slab of this step and the next (workgroup-uniform counters).
            const uint32_t nt = t.nt_begin + cur_nt, sb = cur_sb;
            const uint32_t nx_sb = sb + 1u == n_slabs ? 0u : sb + 1u;
            const uint32_t nx_nt = sb + 1u == n_slabs ? nt + 1u : nt;
            // Every copy of the next step is issued here, a whole step ahead of its wait (the
            // buffers it fills were last read in the previous step, or, with one weight image,
            // before the second barrier).
            if (more) {
#pragma unroll
                for (int p = 0; p < 8; ++p) issue_part(nx_nt, nx_sb, par ^ 1u, p);
            } else if (XPF && nx_ok) {
                const _Float16* asrc_nx[4];
                slab_sources(g, t_nx, wave, lane, asrc_nx);
#pragma unroll
                for (int p = 0; p < 8; ++p) issue_part_of(t_nx, asrc_nx, t_nx.nt_begin, 0u, par ^ 1u, p);
            }
#pragma unroll
            for (int f = 0; f < NF; ++f) c[f].prepare();
            slab_mma<Frag, NF, RB>(sa[RESIDENT ? sb : par], n, gq, c, acc, [](int) {});
            if (sb == n_slabs - 1u) {  // column tile complete
                if constexpr (MODE == kGateUp && NF == 2 && WBUF == 2)
                    staged_epilogue_lds<RB>(g, t.a0, t.a1, nt * S::kOut, wave, lane, acc, sw[par]);
                else
                    staged_epilogue<MODE, NF, RB>(g, s_dst, t.a0, t.a1, nt * S::kOut, wave, n, gq, acc);
            }
            cur_sb = nx_sb;
            cur_nt = nx_nt - t.nt_begin;
        }
    };
    switch ((t.a1 - t.a0 + 15u) / 16u) {  // workgroup-uniform
        case 1: run(std::integral_constant<int, 1>()); break;
        case 2: run(std::integral_constant<int, 2>()); break;
        case 3: run(std::integral_constant<int, 3>()); break;
        default: run(std::integral_constant<int, 4>()); break;
    }
    if (XPF) {
        pf_have = nx_ok;
        t_pf = t_nx;
        par0 = (par0 + n_steps) & 1u;
    }
    // Every thread read s_next before the item's first step barrier.
    if (dynamic && threadIdx.x == 0) sm.s_next = x * per + next;
    }
}

template <class Frag, int MODE, int NF, bool RESIDENT>
__global__ __launch_bounds__(kV2Threads) void routed_gemm_staged_kernel(RoutedGemm g, uint32_t n_ntiles, uint32_t npi,
                                                                        uint32_t n_chunks) {
    __shared__ TileSmem<Frag, NF> sm;
    __shared__ uint32_t s_pref[513], s_wsum[8], s_flag;
    __shared__ int32_t s_grp[kGrpWords];
    const uint32_t flag = scan_small_tiles(g, s_pref, s_wsum, &s_flag, s_grp);
    if (flag & 2u) {
        zero_tile_slots<MODE, NF>(g, n_ntiles, npi, n_chunks);
        return;
    }
    tile_items<Frag, MODE, NF, RESIDENT, false>(g, sm, s_pref, n_ntiles, npi, n_chunks, s_grp);
}


}  // namespace
}  // namespace sm
