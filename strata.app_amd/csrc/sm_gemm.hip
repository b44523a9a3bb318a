// Grouped expert products and the dense shared-expert products for gfx950.
//
// Workgroup tile: 64 rows x 128 weight columns, 256 threads (4 wave64s). Wave w owns two
// 16-column groups (c0, c1) and all 64 rows as four 16x16 MFMA accumulators per group.
//   gate/up: c0 = gate rows j, c1 = up rows j for j in [64*nt + 16w, +16), so the SwiGLU
//            epilogue pairs gate and up values that sit in the same lane and register;
//   down:    c0, c1 = output columns [128*nt + 32w, +16) and [128*nt + 32w + 16, +16).
// The K dimension runs in 256-value slabs. Each lane decodes its own weight values
// straight into the MFMA B-operand layout (no LDS round trip for weights); the 64 x 256
// activation slab is staged in LDS and shared by the four waves.
// Routed workgroups walk the grouping's 64-entry tile list; the flat workgroup id is
// remapped so that consecutive work items (the column tiles of one row tile) land on
// the same XCD and share its L2.
#include <type_traits>

#include "sm_device.h"
#include "sm_launch.h"

namespace sm {
namespace {

constexpr int kRows = 64;
constexpr int kSlab = 256;
constexpr int kLdsRow = kSlab + 8;  // halves

enum Mode { kGateUp = 0, kDown = 1 };

// Hardware dispatches workgroup b to XCD b % 8. Give each XCD a contiguous run of the
// `real` work items (so the column tiles of one row tile share an XCD's L2), spread over
// all eight XCDs; returns `real` (no work) for blocks past the last item.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t b, uint32_t real) {
    const uint32_t per = (real + 7u) >> 3;
    const uint32_t slot = b >> 3;
    if (slot >= per) return real;
    const uint32_t w = (b & 7u) * per + slot;
    return w < real ? w : real;
}

// One 64-row x 128-column tile over all K. Software-pipelined: while slab sb is decoded
// and multiplied, the raw weight fragments and the activation chunk of slab sb+1 are
// already in flight into registers; one LDS buffer holds the current activation slab.
// FULL: K is a multiple of 256, so every load is unconditional and the loop has no
// divergent branches; otherwise (Q8_0 widths that end mid-slab) lane groups past K load
// from a clamped in-bounds address and contribute zero weights and activations.
template <class Frag, bool FULL>
__device__ __forceinline__ void tile_mma(const _Float16* __restrict__ a_rows, uint32_t a0,
                                         uint32_t a_last, uint32_t K, uint32_t n_rb, const uint8_t* w0row,
                                         const uint8_t* w1row, _Float16* sa, float4v (&acc0)[4],
                                         float4v (&acc1)[4]) {
    const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, g = lane >> 4;
    constexpr int kSB = SlabBytes<Frag>::value;
    const uint32_t n_slabs = (K + kSlab - 1) / kSlab;
    // Activation staging: thread covers rows r0 + 8i (i = 0..7), 16-byte column cc.
    const int cc = tid & 31, r0 = tid >> 5;
    const _Float16* arow[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        uint32_t row = a0 + r0 + 8 * i;
        if (row > a_last) row = a_last;
        arow[i] = a_rows + uint64_t(row) * K + 8 * cc;
    }
    const half8 zero{0, 0, 0, 0, 0, 0, 0, 0};
    half8 areg[8];
    Frag f0, f1;
    auto load_slab = [&](uint32_t sb) {
        uint32_t ka = sb * kSlab, kb = sb;
        if (!FULL) {
            if (ka + 8u * cc >= K) ka = 0;             // clamped; zeroed below
            if (sb * kSlab + 64u * g >= K) kb = 0;     // clamped; zeroed at decode time
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) areg[i] = *reinterpret_cast<const half8*>(arow[i] + ka);
        if (!FULL && sb * kSlab + 8u * cc >= K) {
#pragma unroll
            for (int i = 0; i < 8; ++i) areg[i] = zero;
        }
        f0.load(w0row + uint64_t(kb) * kSB, g);
        f1.load(w1row + uint64_t(kb) * kSB, g);
    };
    load_slab(0);
    for (uint32_t sb = 0; sb < n_slabs; ++sb) {
        __syncthreads();  // every wave is done reading the previous slab
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<half8*>(sa + (r0 + 8 * i) * kLdsRow + 8 * cc) = areg[i];
        Frag c0 = f0, c1 = f1;
        const bool kok = FULL || sb * kSlab + 64u * g < K;
        if (sb + 1 < n_slabs) load_slab(sb + 1);
        __syncthreads();
        c0.prepare();
        c1.prepare();
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            half8 b0 = c0.step(s), b1 = c1.step(s);
            if (!FULL && !kok) { b0 = zero; b1 = zero; }
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const half8 a = *reinterpret_cast<const half8*>(sa + (16 * rb + n) * kLdsRow + 64 * g + 8 * s);
                acc0[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b0, acc0[rb], 0, 0, 0);
                acc1[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b1, acc1[rb], 0, 0, 0);
            }
        }
    }
}

// Dequantize rows x K weights of one format to K-major F16 [K][rows] through the same
// per-lane fragments the products use (one wave per 16 rows x one 256-value slab).
template <class Frag>
__global__ __launch_bounds__(64) void decode_rows_kernel(const uint8_t* __restrict__ w, uint32_t rows,
                                                         uint32_t K, uint64_t row_bytes,
                                                         uint16_t* __restrict__ out) {
    const int lane = threadIdx.x, n = lane & 15, g = lane >> 4;
    const uint32_t row = blockIdx.x * 16u + n, sb = blockIdx.y;
    constexpr int kSB = SlabBytes<Frag>::value;
    if (row >= rows || sb * kSlab + 64u * g >= K) return;
    Frag f;
    f.load(w + uint64_t(row) * row_bytes + uint64_t(sb) * kSB, g);
    f.prepare();
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const half8 h = f.step(s);
#pragma unroll
        for (int i = 0; i < 8; ++i) out[uint64_t(sb * kSlab + 64u * g + 8u * s + i) * rows + row] = f16_bits(h[i]);
    }
}

// Zero the block's output tile for rows [r0, r1) (route order for gate/up, entry order for
// the down tile, as the reference's zero paths do: prefill_moe.metal:556-601).
template <int MODE>
__device__ void zero_tile(const RoutedGemm& g, uint32_t r0, uint32_t r1, uint32_t nt) {
    if (MODE == kGateUp) {
        for (uint32_t i = threadIdx.x; i < 64u * 64u; i += 256u) {
            const uint32_t r = r0 + i / 64u, c = nt * 64u + i % 64u;
            if (r < r1 && r < g.n_entries) g.out_h[uint64_t(r) * g.n_out + c] = _Float16(0.0f);
        }
    } else {
        for (uint32_t i = threadIdx.x; i < 64u * 128u; i += 256u) {
            const uint32_t r = r0 + i / 128u, c = nt * 128u + i % 128u;
            if (r < r1 && r < g.n_entries) g.out_f[uint64_t(r) * g.n_out + c] = 0.0f;
        }
    }
}

template <class Frag, int MODE, bool FULL>
__global__ __launch_bounds__(256) void routed_gemm_kernel(RoutedGemm g, uint32_t n_ntiles, uint32_t total) {
    __shared__ __attribute__((aligned(16))) _Float16 sa[kRows * kLdsRow];
    __shared__ uint32_t s_flag, s_tiles;
    const Plan* p = g.plan;
    const uint32_t N = g.n_entries;
    if (threadIdx.x == 0) {
        s_flag = __hip_atomic_load(g.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_tiles = p->n_tiles;
    }
    __syncthreads();
    if (s_flag & 2u) {  // invalid plan or permutation: every tile slot writes zeros
        if (blockIdx.x >= total) return;
        const uint32_t tile_index = blockIdx.x / n_ntiles, nt = blockIdx.x % n_ntiles;
        zero_tile<MODE>(g, tile_index * 64u, tile_index * 64u + 64u, nt);
        return;
    }
    // A valid plan has n_tiles <= capacity; only those tiles carry work.
    const uint32_t real = (s_tiles < g.tile_capacity ? s_tiles : g.tile_capacity) * n_ntiles;
    const uint32_t w = xcd_remap(blockIdx.x, real);
    if (w >= real) return;
    const uint32_t tile_index = w / n_ntiles, nt = w % n_ntiles;
    const uint32_t tg = g.tiles[2 * tile_index], a0 = g.tiles[2 * tile_index + 1];
    bool ok = tg < p->n_groups;
    uint32_t gfirst = 0, gend = 0;
    int32_t ex = -1;
    if (ok) {
        const int32_t f = p->grp_start[tg], e = p->grp_start[tg + 1];
        ex = p->grp_e[tg];
        ok = f >= 0 && e > f && uint32_t(e) <= p->n_entries && ex >= 0 && uint32_t(ex) < g.n_experts;
        if (ok) {
            gfirst = uint32_t(f);
            gend = uint32_t(e);
            ok = a0 >= gfirst && a0 < gend && (a0 - gfirst) % 64u == 0u;
        }
    }
    if (!ok) {
        if (threadIdx.x == 0) atomicOr(g.status, 2u);
        zero_tile<MODE>(g, tile_index * 64u, tile_index * 64u + 64u, nt);
        return;
    }
    if (gend - gfirst >= g.wide_min) return;  // the wide kernel's group
    const uint32_t a1 = a0 + 64u < gend ? a0 + 64u : gend;
    const uint64_t* addr = g.addresses + 3u * uint32_t(ex);
    const uint8_t* w0 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[0] : addr[2]);
    const uint8_t* w1 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[1] : addr[2]);
    if (w0 == nullptr || w1 == nullptr) {
        if (threadIdx.x == 0) atomicOr(g.status, 1u);
        if (MODE == kGateUp) {
            zero_tile<MODE>(g, a0, a1, nt);
        } else {  // down rows live in route order
            for (uint32_t i = threadIdx.x; i < 64u * 128u; i += 256u) {
                const uint32_t a = a0 + i / 128u, c = nt * 128u + i % 128u;
                if (a >= a1) continue;
                const uint32_t d = uint32_t(g.dst[a]);
                if (d < N) g.out_f[uint64_t(d) * g.n_out + c] = 0.0f;
                else atomicOr(g.status, 2u);
            }
        }
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15, gq = lane >> 4;
    uint32_t col0, col1;
    if (MODE == kGateUp) { col0 = nt * 64u + 16u * wave + n; col1 = col0; }
    else { col0 = nt * 128u + 32u * wave + n; col1 = col0 + 16u; }
    float4v acc0[4], acc1[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) { acc0[rb] = float4v{0, 0, 0, 0}; acc1[rb] = float4v{0, 0, 0, 0}; }
    tile_mma<Frag, FULL>(g.a, a0, a1 - 1u, g.k, (a1 - a0 + 15u) / 16u, w0 + uint64_t(col0) * g.row_bytes,
                   w1 + uint64_t(col1) * g.row_bytes, sa, acc0, acc1);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = a0 + 16u * rb + 4u * gq + i;
            if (a >= a1) continue;
            if (MODE == kGateUp) {
                g.out_h[uint64_t(a) * g.n_out + col0] = half_sat(silu_fast(acc0[rb][i]) * acc1[rb][i]);
            } else {
                const uint32_t d = uint32_t(g.dst[a]);
                if (d < N) {
                    g.out_f[uint64_t(d) * g.n_out + col0] = acc0[rb][i];
                    g.out_f[uint64_t(d) * g.n_out + col1] = acc1[rb][i];
                } else {
                    atomicOr(g.status, 2u);
                    g.out_f[uint64_t(a) * g.n_out + col0] = 0.0f;
                    g.out_f[uint64_t(a) * g.n_out + col1] = 0.0f;
                }
            }
        }
}

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

// Position (in 16-byte chunks) of chunk c of row r inside a swizzled 64 x 256 slab: the
// 16 rows one MFMA A-fragment read touches map to 16 distinct 4-bank groups.
__device__ __forceinline__ uint32_t a_pos(uint32_t r, uint32_t c) { return r * 32u + (c ^ (r & 15u)); }

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
__device__ uint32_t scan_small_tiles(const RoutedGemm& g, uint32_t* s_pref, uint32_t* s_wsum, uint32_t* s_flag) {
    const Plan* p = g.plan;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    if (tid == 0) *s_flag = __hip_atomic_load(g.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t ng = p->n_groups < 512u ? p->n_groups : 512u;
    uint32_t n = 0;
    if (tid < ng) {
        const int32_t f = p->grp_start[tid], e = p->grp_start[tid + 1], ex = p->grp_e[tid];
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
// its rows, column tiles and weights. Returns false when the item is done already: an
// expert without weights has zeroed its rows and set status bit 0. Uniform per workgroup.
template <int MODE>
__device__ bool staged_item(const RoutedGemm& g, const uint32_t* s_pref, uint32_t item, uint32_t n_ntiles,
                            uint32_t npi, uint32_t n_chunks, uint32_t out_per_nt, TileWork& t) {
    const Plan* p = g.plan;
    const uint32_t k = item / n_chunks, chunk = item - k * n_chunks;
    uint32_t lo = 0, hi = 512;
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (s_pref[mid] <= k) lo = mid;
        else hi = mid;
    }
    const uint32_t f = uint32_t(p->grp_start[lo]), e = uint32_t(p->grp_start[lo + 1]);
    const uint32_t ex = uint32_t(p->grp_e[lo]);
    t.nt_begin = chunk * npi;
    t.nt_end = t.nt_begin + npi < n_ntiles ? t.nt_begin + npi : n_ntiles;
    t.a0 = f + 64u * (k - s_pref[lo]);
    t.a1 = t.a0 + 64u < e ? t.a0 + 64u : e;
    const uint64_t* addr = g.addresses + 3u * ex;
    t.w0 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[0] : addr[2]);
    t.w1 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[1] : addr[2]);
    if (t.w0 == nullptr || t.w1 == nullptr) {
        if (threadIdx.x == 0) atomicOr(g.status, 1u);
        zero_cols<MODE>(g, t.a0, t.a1, t.nt_begin * out_per_nt, t.nt_end * out_per_nt, MODE == kDown);
        return false;
    }
    return true;
}

// Activation copy map of one 64 x 256 slab: wave instruction q = 4*wave + j (j = 0..3)
// fills chunk positions [64q, 64q + 64): row R = 2q + lane/32, swizzled chunk
// C = (lane & 31) ^ (R & 15). Rows past the tile's end repeat its last row.
__device__ __forceinline__ void slab_sources(const RoutedGemm& g, const TileWork& t, int wave, int lane,
                                             const _Float16* (&asrc)[4]) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t R = 2u * (4u * wave + j) + (uint32_t(lane) >> 5);
        const uint32_t C = (uint32_t(lane) & 31u) ^ (R & 15u);
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
// others are skipped. after_s(s) runs after k-step s: the staged kernel issues part s of
// the next step's copies there, so a wave never blocks on a long burst of memory
// instructions while it could be multiplying.
template <class Frag, int NF, int RB, class After>
__device__ __forceinline__ void slab_mma(const _Float16* buf, int n, int gq, const Frag (&c)[NF],
                                         float4v (&acc)[NF][4], After after_s) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        half8 b[NF];
#pragma unroll
        for (int f = 0; f < NF; ++f) b[f] = c[f].step(s);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const half8 a = *reinterpret_cast<const half8*>(buf + 8u * a_pos(16u * rb + n, 8u * gq + s));
#pragma unroll
            for (int f = 0; f < NF; ++f) acc[f][rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b[f], acc[f][rb], 0, 0, 0);
        }
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
                *reinterpret_cast<vecf*>(g.out_f + row * g.n_out + col0 + S::col(wave, n, 0)) = v;
            }
        }
#pragma unroll
    for (int f = 0; f < NF; ++f)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[f][rb] = float4v{0, 0, 0, 0};
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

// RESIDENT (K <= 512): both activation slabs are copied once and stay in LDS for all of
// the workgroup's column tiles, instead of being re-read from L2 for each of them.
template <class Frag, int MODE, int NF, bool RESIDENT>
__global__ __launch_bounds__(kV2Threads) void routed_gemm_staged_kernel(RoutedGemm g, uint32_t n_ntiles, uint32_t npi,
                                                                        uint32_t n_chunks) {
    using S = Staged<MODE, NF>;
    using WC = WeightCopy<Frag, MODE, NF>;
    constexpr int SB = SlabBytes<Frag>::value;
    constexpr int WBUF = StagedBuffers<Frag, NF>::kWBuf;
    __shared__ __attribute__((aligned(1024))) _Float16 sa[2][64 * kSlab];
    __shared__ __attribute__((aligned(1024))) uint8_t sw[WBUF][StagedBuffers<Frag, NF>::kImage];
    __shared__ uint32_t s_dst[64];  // down: destination row of each tile row
    __shared__ uint32_t s_pref[513], s_wsum[8], s_flag;
    const uint32_t flag = scan_small_tiles(g, s_pref, s_wsum, &s_flag);
    if (flag & 2u) {  // invalid plan or permutation: every tile slot writes zeros
        for (uint32_t slot = blockIdx.x; slot < g.tile_capacity * n_chunks; slot += gridDim.x) {
            const uint32_t ti = slot / n_chunks, ch = slot % n_chunks;
            const uint32_t nb = ch * npi, ne = nb + npi < n_ntiles ? nb + npi : n_ntiles;
            zero_cols<MODE>(g, ti * 64u, ti * 64u + 64u, nb * S::kOut, ne * S::kOut, false);
        }
        return;
    }
    // Persistent: XCD x (workgroups b with b % 8 == x) takes the contiguous item range
    // [x * per, (x + 1) * per), so the column chunks of a tile share that XCD's L2.
    const uint32_t items = s_pref[512] * n_chunks;
    const uint32_t per = (items + 7u) >> 3, x = blockIdx.x & 7u, P = gridDim.x >> 3;
    const uint32_t i_end = (x + 1u) * per < items ? (x + 1u) * per : items;
    for (uint32_t item = x * per + (blockIdx.x >> 3); item < i_end; item += P) {
    __syncthreads();  // the previous item's reads of LDS are done
    TileWork t;
    if (!staged_item<MODE>(g, s_pref, item, n_ntiles, npi, n_chunks, S::kOut, t)) continue;
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
    auto issue_part = [&](uint32_t step, int p) {
        const uint32_t nt = t.nt_begin + step / n_slabs, sb = step % n_slabs;
        if (!RESIDENT && p < 4) issue_slab_part(asrc, sb * kSlab, sa[step & 1u], wave, p);
        uint8_t* wb = sw[WBUF == 2 ? (step & 1u) : 0u];
#pragma unroll
        for (uint32_t j = uint32_t(p); j < WC::kPerWave; j += 8u) wc.issue(g, t, nt, sb, wb, wave, j);
    };
    if (RESIDENT)
        for (uint32_t sb = 0; sb < n_slabs; ++sb) issue_slab(asrc, sb * kSlab, sa[sb], wave);
#pragma unroll
    for (int p = 0; p < 8; ++p) issue_part(0, p);
    // The step loop, specialised on the number of 16-row blocks holding entries.
    auto run = [&](auto rb_const) {
        constexpr int RB = decltype(rb_const)::value;
        float4v acc[NF][4];
#pragma unroll
        for (int f = 0; f < NF; ++f)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) acc[f][rb] = float4v{0, 0, 0, 0};
        for (uint32_t step = 0; step < n_steps; ++step) {
            __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this step's copies ...
            __syncthreads();                                       // ... from every wave
            const bool more = step + 1 < n_steps;
            const uint8_t* wb = sw[WBUF == 2 ? (step & 1u) : 0u];
            Frag c[NF];
#pragma unroll
            for (int f = 0; f < NF; ++f) c[f].template load<FromLds>(wb + S::image_row(wave, n, f) * SB, gq);
            // A barrier waits for every outstanding load of the wave, so with one weight image
            // the next step's copies start only after the second barrier.
            if (WBUF == 1) __syncthreads();  // every wave holds its fragments: the image may be refilled
#pragma unroll
            for (int f = 0; f < NF; ++f) c[f].prepare();
            const uint32_t sb = step % n_slabs;
            slab_mma<Frag, NF, RB>(sa[RESIDENT ? sb : (step & 1u)], n, gq, c, acc, [&](int p) {
                if (more) issue_part(step + 1, p);
            });
            if (sb == n_slabs - 1u) {  // column tile complete
                const uint32_t nt = t.nt_begin + step / n_slabs;
                staged_epilogue<MODE, NF, RB>(g, s_dst, t.a0, t.a1, nt * S::kOut, wave, n, gq, acc);
            }
        }
    };
    switch ((t.a1 - t.a0 + 15u) / 16u) {  // workgroup-uniform
        case 1: run(std::integral_constant<int, 1>()); break;
        case 2: run(std::integral_constant<int, 2>()); break;
        case 3: run(std::integral_constant<int, 3>()); break;
        default: run(std::integral_constant<int, 4>()); break;
    }
    }
}

// Dense (shared-expert) products: rows are tokens in 64-row tiles.
template <class Frag, int MODE>
__global__ __launch_bounds__(256) void dense_gemm_kernel(DenseGemm g, uint32_t n_ntiles, uint32_t total) {
    __shared__ __attribute__((aligned(16))) _Float16 sa[kRows * kLdsRow];
    const uint32_t w = xcd_remap(blockIdx.x, total);
    if (w >= total) return;
    const uint32_t mt = w / n_ntiles, nt = w % n_ntiles;
    const uint32_t r0 = mt * 64u;
    const uint32_t r1 = r0 + 64u < g.rows ? r0 + 64u : g.rows;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n = lane & 15, gq = lane >> 4;
    uint32_t col0, col1;
    const uint8_t *w0, *w1;
    if (MODE == kGateUp) {
        col0 = nt * 64u + 16u * wave + n; col1 = col0; w0 = g.w0; w1 = g.w1;
    } else {
        col0 = nt * 128u + 32u * wave + n; col1 = col0 + 16u; w0 = g.w0; w1 = g.w0;
    }
    float4v acc0[4], acc1[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) { acc0[rb] = float4v{0, 0, 0, 0}; acc1[rb] = float4v{0, 0, 0, 0}; }
    tile_mma<Frag, true>(g.a, r0, r1 - 1u, g.k, (r1 - r0 + 15u) / 16u, w0 + uint64_t(col0) * g.row_bytes,
                   w1 + uint64_t(col1) * g.row_bytes, sa, acc0, acc1);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t r = r0 + 16u * rb + 4u * gq + i;
            if (r >= r1) continue;
            if (MODE == kGateUp) {
                g.out_h[uint64_t(r) * g.n_out + col0] = half_sat(silu_fast(acc0[rb][i]) * acc1[rb][i]);
            } else {
                g.out_f[uint64_t(r) * g.n_out + col0] = acc0[rb][i];
                g.out_f[uint64_t(r) * g.n_out + col1] = acc1[rb][i];
            }
        }
}

// gl[t] = sum_k x[t,k] * gv[k]: one wave per token; each lane takes 8 consecutive values
// per 16-byte load into two F32 partial sums, reduced by a fixed xor butterfly.
template <bool BF16>
__global__ __launch_bounds__(256) void gate_logit_kernel(const _Float16* __restrict__ x,
                                                         const uint16_t* __restrict__ gv,
                                                         float* __restrict__ gl, uint32_t rows, uint32_t d) {
    const uint32_t t = (blockIdx.x * 256u + threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63u;
    if (t >= rows) return;
    float s0 = 0.0f, s1 = 0.0f;
    for (uint32_t k = 8u * lane; k < d; k += 512u) {
        const half8 xv = ld_global<half8>(x + uint64_t(t) * d + k);
        const u32x4 wv = ld_global<u32x4>(gv + k);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t pair = wv[i];
            const float w0 = BF16 ? __builtin_bit_cast(float, pair << 16) : f16_lo(pair);
            const float w1 = BF16 ? __builtin_bit_cast(float, pair & 0xffff0000u) : f16_hi(pair);
            s0 = __builtin_fmaf(float(xv[2 * i]), w0, s0);
            s1 = __builtin_fmaf(float(xv[2 * i + 1]), w1, s1);
        }
    }
    float s = s0 + s1;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) s = s + __shfl_xor(s, off);
    if (lane == 0) gl[t] = s;
}

// Compute units of the current device (queried once; 256 if the query fails).
uint32_t device_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
            cus = v;
        else
            cus = 256;
    }
    return uint32_t(cus);
}

template <class Frag, int MODE, int NF>
hipError_t launch_staged(const RoutedGemm& g, hipStream_t s) {
    const uint32_t n_ntiles = g.n_out / Staged<MODE, NF>::kOut;
    // About 8 (column tile, slab) steps per workgroup; with the activation tile resident
    // (K <= 512) every column tile of a row tile goes to one workgroup, so the tile is read
    // once rather than once per workgroup.
    const uint32_t n_slabs = g.k / kSlab;
    uint32_t npi = n_slabs <= 2 ? n_ntiles : (n_slabs >= 8 ? 1u : 8u / n_slabs);
    if (npi > n_ntiles) npi = n_ntiles;
    const uint32_t n_chunks = (n_ntiles + npi - 1) / npi;
    // Persistent: one workgroup per CU (each holds about 130 KB of LDS), never more than the
    // tile slots, in whole groups of 8 (one per XCD).
    uint32_t blocks = (g.tile_capacity * n_chunks + 7u) & ~7u;
    const uint32_t cap = device_cus() & ~7u;
    if (blocks > cap) blocks = cap;
    if (blocks < 8u) blocks = 8u;
    if (n_slabs <= 2)
        routed_gemm_staged_kernel<Frag, MODE, NF, true><<<blocks, kV2Threads, 0, s>>>(g, n_ntiles, npi, n_chunks);
    else
        routed_gemm_staged_kernel<Frag, MODE, NF, false><<<blocks, kV2Threads, 0, s>>>(g, n_ntiles, npi, n_chunks);
    return hipGetLastError();
}

template <class Frag, int MODE>
hipError_t launch_routed(Fmt fmt, const RoutedGemm& g, hipStream_t s) {
    if (g.wide_min != ~0u) {
        const hipError_t e = launch_wide(fmt, MODE == kGateUp, g, s);
        if (e != hipSuccess) return e;
    }
    // Two fragments per wave: four (twice the multiplies per activation slab) measured no
    // faster on gfx950 and needs more than 256 VGPRs for Q4_K/Q2_K.
    if (g.k % kSlab == 0 && g.n_out % Staged<MODE, 2>::kOut == 0) return launch_staged<Frag, MODE, 2>(g, s);
    const uint32_t n_ntiles = MODE == kGateUp ? g.n_out / 64u : g.n_out / 128u;
    const uint32_t total = g.tile_capacity * n_ntiles;
    const uint32_t blocks = (total + 7u) & ~7u;
    if (g.k % kSlab == 0) routed_gemm_kernel<Frag, MODE, true><<<blocks, 256, 0, s>>>(g, n_ntiles, total);
    else routed_gemm_kernel<Frag, MODE, false><<<blocks, 256, 0, s>>>(g, n_ntiles, total);
    return hipGetLastError();
}

template <class Frag, int MODE>
hipError_t launch_dense(const DenseGemm& g, hipStream_t s) {
    const uint32_t n_ntiles = MODE == kGateUp ? g.n_out / 64u : g.n_out / 128u;
    const uint32_t total = ((g.rows + 63u) / 64u) * n_ntiles;
    const uint32_t blocks = (total + 7u) & ~7u;
    dense_gemm_kernel<Frag, MODE><<<blocks, 256, 0, s>>>(g, n_ntiles, total);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gate_up(Fmt fmt, const RoutedGemm& g, hipStream_t s) {
    switch (fmt) {
        case Fmt::Q8_0: return launch_routed<FragQ80, kGateUp>(fmt, g, s);
        case Fmt::Q4_K: return launch_routed<FragQ4K, kGateUp>(fmt, g, s);
        case Fmt::Q2_K: return launch_routed<FragQ2K, kGateUp>(fmt, g, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_down(Fmt fmt, const RoutedGemm& g, hipStream_t s) {
    switch (fmt) {
        case Fmt::Q8_0: return launch_routed<FragQ80, kDown>(fmt, g, s);
        case Fmt::Q4_K: return launch_routed<FragQ4K, kDown>(fmt, g, s);
        case Fmt::Q2_K: return launch_routed<FragQ2K, kDown>(fmt, g, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dense_gate_up(Fmt fmt, const DenseGemm& g, hipStream_t s) {
    if (wide_dense_fits(fmt, true, g.rows, g.k, g.n_out)) return launch_wide_dense(fmt, true, g, s);
    switch (fmt) {
        case Fmt::F16: return launch_dense<FragF16, kGateUp>(g, s);
        case Fmt::BF16: return launch_dense<FragBF16, kGateUp>(g, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_dense_down(Fmt fmt, const DenseGemm& g, hipStream_t s) {
    if (wide_dense_fits(fmt, false, g.rows, g.k, g.n_out)) return launch_wide_dense(fmt, false, g, s);
    switch (fmt) {
        case Fmt::F16: return launch_dense<FragF16, kDown>(g, s);
        case Fmt::BF16: return launch_dense<FragBF16, kDown>(g, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_decode_rows(Fmt fmt, const uint8_t* w, uint32_t rows, uint32_t k, uint64_t row_bytes,
                              uint16_t* out, hipStream_t s) {
    const dim3 grid((rows + 15u) / 16u, (k + kSlab - 1) / kSlab);
    switch (fmt) {
        case Fmt::Q8_0: decode_rows_kernel<FragQ80><<<grid, 64, 0, s>>>(w, rows, k, row_bytes, out); break;
        case Fmt::Q4_K: decode_rows_kernel<FragQ4K><<<grid, 64, 0, s>>>(w, rows, k, row_bytes, out); break;
        case Fmt::Q2_K: decode_rows_kernel<FragQ2K><<<grid, 64, 0, s>>>(w, rows, k, row_bytes, out); break;
        case Fmt::F16: decode_rows_kernel<FragF16><<<grid, 64, 0, s>>>(w, rows, k, row_bytes, out); break;
        case Fmt::BF16: decode_rows_kernel<FragBF16><<<grid, 64, 0, s>>>(w, rows, k, row_bytes, out); break;
    }
    return hipGetLastError();
}

hipError_t launch_gate_logit(Fmt fmt, const _Float16* x, const uint8_t* gv, float* gl, uint32_t rows,
                             uint32_t d, hipStream_t s) {
    const uint32_t blocks = (rows + 3u) / 4u;
    const uint16_t* v = reinterpret_cast<const uint16_t*>(gv);
    if (fmt == Fmt::BF16) gate_logit_kernel<true><<<blocks, 256, 0, s>>>(x, v, gl, rows, d);
    else gate_logit_kernel<false><<<blocks, 256, 0, s>>>(x, v, gl, rows, d);
    return hipGetLastError();
}

}  // namespace sm
