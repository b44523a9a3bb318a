// Routed expert products for large groups on gfx950: 256-row units x 256 weight rows.
//
// A group with at least `wide_min` entries is cut into ceil(size / 256) units of consecutive
// grouped rows, as even as whole 32-row blocks allow (a group of 300 rows: 160 + 140, not
// 256 + 44); the 64-row tile kernels skip such groups. One unit times one column tile is an
// item. A wave multiplies only the 32-row blocks of its row half that hold entries, so a unit
// of 160 rows costs five blocks of MFMA work, not eight. The kernel is persistent: each workgroup (512 threads, one
// per CU) walks its share of the items, so no workgroup slot is spent on idle tiles.
//
// Per 64-value K step, both operands sit in LDS:
//   A: 256 rows x 64 halves (32 KB), copied global -> LDS by LDS-DMA (global_load_lds);
//   B: 256 weight rows x 64 values (32 KB), decoded from the block format once per
//      workgroup by all 512 threads (two per weight row) and written as F16,
// each double buffered, so the copy and the decode of step j+1 run under the multiplies of
// step j. Decoding once per 256 rows, instead of once per 64-row tile, is what moves these
// products from decode-bound to MFMA-bound.
// Wave w multiplies rows [128 * (w >> 2), +128) by B rows of column quarter q = w & 3 with
// 32x32x16 MFMAs: up to 4 row blocks x 2 column blocks of 32x32 F32 accumulators (128 VGPRs):
//   gate/up: column block 0 = gate rows [32q, +32), block 1 = the up rows [128 + 32q, +32)
//            of the same hidden columns, so the SwiGLU epilogue pairs values of one lane;
//   down:    output columns [64q, +64).
// Each 16-value K slice's operands are read from LDS while the previous slice multiplies.
// The two waves of a SIMD (w and w + 4) take different row halves.
// Items are spread XCD-aware: XCD x (workgroup b runs on XCD b % 8) takes a contiguous eighth
// of the units, so the units of one expert share its weight rows in one L2, and the column
// tiles of a unit are neighbours in that XCD's item order, so they run together and share the
// unit's activation rows.
#include <type_traits>

#include "sm_device.h"
#include "sm_launch.h"
#include "sm_tiles.h"

namespace sm {
namespace {

constexpr int kWideThreads = 512;
constexpr uint32_t kUnitRows = 256;
constexpr uint32_t kStepK = 64;
constexpr uint32_t kStageBytes = 256u * kStepK * 2u;  // one operand stage: 256 rows x 64 halves

typedef float float16v __attribute__((ext_vector_type(16)));

// 16-byte chunk slot of logical chunk c (0..7) of row r in a stage of 8-chunk rows. The 16
// rows one operand read touches (same c) land in 16 distinct 4-bank groups: rows of one
// parity differ in (r >> 1) & 7, and the two parities sit 32 banks apart.
__device__ __forceinline__ uint32_t slot(uint32_t r, uint32_t c) { return r * 8u + (c ^ ((r >> 1) & 7u)); }

__device__ __forceinline__ void compiler_fence() { __asm__ volatile("" ::: "memory"); }

// Waits until no memory operation of this wave is outstanding, then joins the workgroup
// barrier. The wait is the s_waitcnt builtin (vmcnt = expcnt = lgkmcnt = 0), which the
// compiler's own wait insertion takes into account, so registers loaded before it need no
// further wait; the memory fences keep every memory operation on its side.
__device__ __forceinline__ void wait_barrier() {
    compiler_fence();
    __builtin_amdgcn_s_waitcnt(0);
    __asm__ volatile("s_barrier" ::: "memory");
}

template <class T>
__device__ __forceinline__ T lds_ld(const uint8_t* p) {
    return *(const __attribute__((address_space(3))) T*)(p);
}
template <class T>
__device__ __forceinline__ void lds_st(uint8_t* p, T v) {
    *(__attribute__((address_space(3))) T*)(p) = v;
}

// Weight producers. Two threads share a weight row: for the 64-value group g of a 256-value
// slab, thread b (0/1) decodes four of its eight chunks (8 values each) in parts s = 0..3,
// part s landing at chunk ChunkIndex::of(s, b). For the nibble and 2-bit formats those are
// the values coded by bytes [16b, 16b + 16) of the group's code bytes (chunks 2b, 2b+1 of
// the low bit plane, 4+2b, 5+2b of the high one); for Q8_0, block 2g + b (chunks 4b..4b+3).
// Both threads run the same code (b only moves addresses and shifts). The arithmetic is the
// fragment decoders' own (the same fma / conversion sequence per value), so every value is
// bit-identical to the 64-row tile kernels'.

// Q4_K: header (d, dmin, scales) and 16 code bytes; low nibbles use pair 2g, high 2g + 1.
struct ProdQ4K {
    static constexpr int kSlab = 144;
    u32x4 hdr, qs;
    float d_lo, m_lo, d_hi, m_hi;
    uint32_t g;
    __device__ __forceinline__ void load(const uint8_t* sb, uint32_t grp, uint32_t b) {
        g = grp;
        hdr = ld_global<u32x4>(sb);
        qs = ld_global<u32x4>(sb + 16 + 32 * grp + 16 * b);
    }
    __device__ __forceinline__ void prepare() { q4k_pair_scales(hdr, g, d_lo, m_lo, d_hi, m_hi); }
    __device__ __forceinline__ half8 chunk(int s) const {
        const int w = 2 * (s & 1);
        if (s < 2) return decode8_nib(qs[w] & 0x0F0F0F0Fu, qs[w + 1] & 0x0F0F0F0Fu, d_lo, m_lo);
        return decode8_nib((qs[w] >> 4) & 0x0F0F0F0Fu, (qs[w + 1] >> 4) & 0x0F0F0F0Fu, d_hi, m_hi);
    }
};

// Q8_0: block 2g + b. Nine dwords from the 4-aligned pair offset 68g + 32b hold it: b = 0
// puts d at byte 0 and the codes at byte 2, b = 1 puts d at byte 2 and the codes at byte 4,
// so a 64-bit funnel shift by 16 + 16b bits aligns either case.
struct ProdQ80 {
    static constexpr int kSlab = 272;
    u32x4 wa, wb;  // dwords 0-3, 4-7 (vector members keep the set in registers)
    uint32_t w8, sh;
    __device__ __forceinline__ void load(const uint8_t* sb, uint32_t g, uint32_t b) {
        const uint8_t* p = sb + 68u * g + 32u * b;
        // 16-byte loads at 4-byte-aligned addresses (allowed on this part): three loads per
        // lane instead of nine dword loads, each one cache access per lane.
        wa = ld_global<u32x4>(p);
        wb = ld_global<u32x4>(p + 16);
        w8 = ld_global<uint32_t>(p + 32);
        sh = 16u * b;
    }
    __device__ __forceinline__ void prepare() {}
    __device__ __forceinline__ uint32_t word(int i) const { return i < 4 ? wa[i] : i < 8 ? wb[i - 4] : w8; }
    __device__ __forceinline__ uint32_t code(int i) const {
        const uint64_t pair = (uint64_t(word(i + 1)) << 32) | word(i);
        return uint32_t(pair >> (16u + sh));
    }
    // Part s: codes 8s .. 8s+7 of the block.
    __device__ __forceinline__ half8 chunk(int s) const {
        const uint32_t x0 = code(2 * s) ^ 0x80808080u, x1 = code(2 * s + 1) ^ 0x80808080u;
        const _Float16 d = bits_f16(uint16_t(wa[0] >> sh));
        const half2v dd{d, d};
        const half2v p0 = q80_pair(x0, 0x04010400u, dd), p1 = q80_pair(x0, 0x04030402u, dd);
        const half2v p2 = q80_pair(x1, 0x04010400u, dd), p3 = q80_pair(x1, 0x04030402u, dd);
        return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
};

// Q2_K: group g covers n = g / 2 and planes jbase = 2 (g % 2), jbase + 1; value
// 128n + 32j + w uses bits 2j of code q[32n + w] and scale byte 8n + 2j + (w >= 16). Thread
// b holds codes w in [16b, 16b + 16) (both planes), the scale dword at 8n + 2 jbase, d/dmin.
struct ProdQ2K {
    static constexpr int kSlab = 84;
    u32x4 qs;
    uint32_t sc, dd, g, b;
    float d, dmin;
    __device__ __forceinline__ void load(const uint8_t* sb, uint32_t grp, uint32_t bb) {
        g = grp;
        b = bb;
        const uint32_t n = grp >> 1, jbase = 2u * (grp & 1u);
        // One 16-byte load at a 4-byte-aligned address (unaligned vector loads are allowed on
        // this part), not four dword loads: each is one cache access per lane.
        qs = ld_global<u32x4>(sb + 16 + 32 * n + 16 * bb);
        sc = ld_global<uint32_t>(sb + 8 * n + 2 * jbase);
        dd = ld_global<uint32_t>(sb + 80);
    }
    __device__ __forceinline__ void prepare() {
        d = f16_lo(dd);
        dmin = f16_hi(dd);
    }
    // Part s: plane jbase + (s >> 1), codes 16b + 8 (s & 1) .. +7.
    __device__ __forceinline__ half8 chunk(int s) const {
        const uint32_t jj = uint32_t(s >> 1);
        const uint32_t shift = 2u * (2u * (g & 1u) + jj);
        const uint32_t scb = (sc >> (8u * (2u * jj + b))) & 0xffu;
        const Q2Table t = q2_table(d * float(scb & 0xFu), -(dmin * float(scb >> 4)));
        const int w = 2 * (s & 1);
        const uint32_t x0 = (qs[w] >> shift) & 0x03030303u;
        const uint32_t x1 = (qs[w + 1] >> shift) & 0x03030303u;
        return lookup8(x0, x1, t);
    }
};

// F16 rows (dense weights): the chunks are copied as they are.
struct ProdF16 {
    static constexpr int kSlab = 512;
    half8 v[4];
    __device__ __forceinline__ void load(const uint8_t* sb, uint32_t g, uint32_t b) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            v[s] = ld_global<half8>(sb + 128u * g + 16u * (4u * uint32_t(s >> 1) + 2u * b + uint32_t(s & 1)));
    }
    __device__ __forceinline__ void prepare() {}
    __device__ __forceinline__ half8 chunk(int s) const { return v[s]; }
};

// BF16 rows (dense weights): widened exactly to F32 and rounded once to F16, as FragBF16.
struct ProdBF16 {
    static constexpr int kSlab = 512;
    u32x4 v[4];
    __device__ __forceinline__ void load(const uint8_t* sb, uint32_t g, uint32_t b) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            v[s] = ld_global<u32x4>(sb + 128u * g + 16u * (4u * uint32_t(s >> 1) + 2u * b + uint32_t(s & 1)));
    }
    __device__ __forceinline__ void prepare() {}
    __device__ __forceinline__ half8 chunk(int s) const {
        half8 h;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = v[s][i];
            h[2 * i] = _Float16(__builtin_bit_cast(float, w << 16));
            h[2 * i + 1] = _Float16(__builtin_bit_cast(float, w & 0xffff0000u));
        }
        return h;
    }
};

// Chunk (0..7) of the 64-value step that producer part s of thread b writes.
template <class Prod> struct ChunkIndex {
    static __device__ __forceinline__ uint32_t of(int s, uint32_t b) {
        return 4u * uint32_t(s >> 1) + 2u * b + uint32_t(s & 1);
    }
};
template <> struct ChunkIndex<ProdQ80> {
    static __device__ __forceinline__ uint32_t of(int s, uint32_t b) { return 4u * b + uint32_t(s); }
};

struct Unit {
    uint32_t a0, a1, ex;
};

// Rows per unit of a group of `size` entries: its ceil(size / 256) units are as even as whole
// 32-row blocks allow (at most 256; every unit holds at least one row).
__device__ __forceinline__ uint32_t unit_rows(uint32_t size) {
    const uint32_t nu = (size + kUnitRows - 1u) / kUnitRows;
    return 32u * ((size + 32u * nu - 1u) / (32u * nu));
}

template <int MODE>
__device__ void zero_item(const RoutedGemm& g, const Unit& u, uint32_t ct, const int32_t* s_dst) {
    const uint32_t width = MODE == kGateUp ? 128u : 256u, c0 = ct * width, rows = u.a1 - u.a0;
    for (uint32_t i = threadIdx.x; i < rows * width; i += kWideThreads) {
        const uint32_t r = i / width, c = c0 + i % width, a = u.a0 + r;
        if (MODE == kGateUp) {
            g.out_h[uint64_t(a) * g.n_out + c] = _Float16(0.0f);
        } else {
            const uint32_t d = uint32_t(s_dst[r]);
            if (d < g.n_entries) g.out_f[uint64_t(d) * g.n_out + c] = 0.0f;
            else atomicOr(g.status, 2u);
        }
    }
}

// LDS of the wide phase of the routed stage kernel: double-buffered activation and
// decoded-weight stages and the unit's destination rows (down).
struct WideSmem {
    int32_t s_dst[kUnitRows];
    uint8_t s_a[2][kStageBytes] __attribute__((aligned(1024)));
    uint8_t s_b[2][kStageBytes] __attribute__((aligned(1024)));
};

// Unit enumeration (512 threads, once per workgroup): groups with >= wide_min entries,
// ceil(size / 256) units each; s_pref[gi] = units of the groups before gi, s_pref[512] = all.
// With s_tiles (the routed stage kernel) the same pass also enumerates the small groups'
// 64-row tiles as scan_small_tiles does (an unusable group sets status bit 1). Group fields
// are loaded without waiting for n_groups (thread gi < 512 reads inside the plan's arrays), so
// the pass costs one round trip. Returns the status word read at start.
__device__ __forceinline__ uint32_t scan_wide_units(const RoutedGemm& g, uint32_t* s_pref, uint32_t* s_wsum, uint32_t* s_flag,
                                                    uint32_t* s_tiles = nullptr, uint32_t* s_tsum = nullptr,
                                                    int32_t* s_grp = nullptr) {
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const Plan* p = g.plan;
    if (tid == 0) *s_flag = __hip_atomic_load(g.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t ng_raw = p->n_groups;
    const int32_t f = p->grp_start[tid], e = p->grp_start[tid + 1], ex = p->grp_e[tid];
    if (s_grp != nullptr) stash_groups(s_grp, tid, f, e, ex);
    const uint32_t ng = ng_raw < 512u ? ng_raw : 512u;
    uint32_t units = 0, tiles = 0;
    if (tid < ng) {
        if (f >= 0 && e > f && uint32_t(e) <= g.n_entries && ex >= 0 && uint32_t(ex) < g.n_experts) {
            if (uint32_t(e - f) >= g.wide_min) units = (uint32_t(e - f) + kUnitRows - 1u) / kUnitRows;
            else tiles = (uint32_t(e - f) + 63u) / 64u;
        } else if (s_tiles != nullptr) {
            atomicOr(g.status, 2u);
        }
    }
    uint32_t incl = units, incl_t = tiles;
#pragma unroll
    for (uint32_t off = 1; off < 64u; off <<= 1) {
        const uint32_t y = __shfl_up(incl, off), yt = __shfl_up(incl_t, off);
        if (lane >= off) {
            incl += y;
            incl_t += yt;
        }
    }
    if (lane == 63u) {
        s_wsum[wave] = incl;
        if (s_tiles != nullptr) s_tsum[wave] = incl_t;
    }
    __syncthreads();
    uint32_t base = 0, base_t = 0;
    for (uint32_t w = 0; w < wave; ++w) {
        base += s_wsum[w];
        if (s_tiles != nullptr) base_t += s_tsum[w];
    }
    s_pref[tid + 1] = base + incl;
    if (tid == 0) s_pref[0] = 0;
    if (s_tiles != nullptr) {
        s_tiles[tid + 1] = base_t + incl_t;
        if (tid == 0) s_tiles[0] = 0;
    }
    __syncthreads();
    return *s_flag;
}

// The workgroup's share of the U units' items (unit x column tile). DENSE: the rows are the
// n_entries activation rows themselves (the shared expert), in units of 256 consecutive rows;
// the weights are dw0/dw1 and the down output row is the unit row.
// DYN (a phase that starts at different times on different workgroups): the items of XCD x's
// range are drawn from counter x of g.counters (zeroed by the stage's plan check) instead of
// the static order; thread 0 draws the next item when it starts the current one and publishes
// it in *s_next at the end, so the atomic's round trip overlaps the item.
template <class Prod, int MODE, bool DENSE, bool DYN = false>
__device__ __forceinline__ void wide_items(const RoutedGemm& g, const uint8_t* dw0, const uint8_t* dw1, uint32_t n_ct, uint32_t U,
                           const uint32_t* s_pref, uint8_t (&s_a)[2][kStageBytes], uint8_t (&s_b)[2][kStageBytes],
                           int32_t* s_dst, uint32_t* s_next = nullptr, const int32_t* s_grp = nullptr) {
    constexpr int SB = Prod::kSlab;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
    const Plan* p = g.plan;

    // ---- per-thread constant roles ----
    const uint32_t wave_u = uint32_t(__builtin_amdgcn_readfirstlane(int(wave)));
    const uint32_t rh = wave_u >> 2, cq = wave_u & 3u;
    // LDS byte offset of this lane's operand read for K slice t (16 values) within a stage:
    // row (or B row) 32 * block + (lane & 31), logical chunk 2t + lane / 32. Every block
    // starts at a multiple of 16 rows, so the swizzle depends on the lane alone and each
    // block is a constant 4 KB further.
    const uint32_t r32 = lane & 31u, kh = lane >> 5, swz = (r32 >> 1) & 7u;
    uint32_t lo[4];
#pragma unroll
    for (uint32_t t = 0; t < 4u; ++t) lo[t] = 16u * (8u * r32 + ((2u * t + kh) ^ swz));
    // B column blocks of this wave (first B row): gate/up {32q, 128 + 32q}; down 64q + 32cb.
    const uint32_t bofs0 = MODE == kGateUp ? 128u * 32u * cq : 128u * 64u * cq;
    const uint32_t bofs1 = MODE == kGateUp ? 128u * (128u + 32u * cq) : 128u * (64u * cq + 32u);
    const uint32_t prow = tid >> 1, pb = tid & 1u;  // producer: B row and byte half

    const uint32_t x = blockIdx.x & 7u, l = blockIdx.x >> 3, P = gridDim.x >> 3;
    // XCD x takes the contiguous unit range [x U / 8, (x + 1) U / 8): the units of one expert
    // (consecutive unit indices) then share its weight rows in one XCD's L2 instead of every
    // XCD reading the whole expert.
    const uint32_t u_begin = uint32_t((uint64_t(x) * U) >> 3), u_end = uint32_t((uint64_t(x + 1u) * U) >> 3);
    const uint32_t vx = u_end - u_begin;
    const uint32_t n_items = vx * n_ct;
    const uint32_t nK = g.k / kStepK;
    uint32_t* counter = g.counters + x;
    if (DYN && tid == 0) *s_next = atomicAdd(counter, 1u);
    for (uint32_t m_static = l;; m_static += P) {
        __syncthreads();  // the previous item's last reads of LDS are done; *s_next is visible
        const uint32_t m = DYN ? *s_next : m_static;
        if (m >= n_items) break;
        uint32_t next = 0;
        if (DYN && tid == 0) next = atomicAdd(counter, 1u);
        const uint32_t v = m / n_ct, ct = m - v * n_ct, uidx = u_begin + v;
        Unit u;
        if (DENSE) {
            u.a0 = kUnitRows * uidx;
            u.a1 = u.a0 + kUnitRows < g.n_entries ? u.a0 + kUnitRows : g.n_entries;
            u.ex = 0;
        } else {
            uint32_t lo_g = 0, hi_g = 512;
            while (hi_g - lo_g > 1u) {
                const uint32_t mid = (lo_g + hi_g) >> 1;
                if (s_pref[mid] <= uidx) lo_g = mid;
                else hi_g = mid;
            }
            uint32_t f, e, ex;
            group_fields(p, s_grp, lo_g, f, e, ex);
            const uint32_t usz = unit_rows(e - f);
            u.a0 = f + usz * (uidx - s_pref[lo_g]);
            u.a1 = u.a0 + usz < e ? u.a0 + usz : e;
            u.ex = ex;
        }
        const uint32_t nrows = u.a1 - u.a0;
        if (!DENSE && MODE == kDown && tid < kUnitRows) s_dst[tid] = tid < nrows ? g.dst[u.a0 + tid] : -1;
        const uint8_t* w0 = dw0;
        const uint8_t* w1 = dw1;
        if (!DENSE) {
            const uint64_t* addr = g.addresses + 3u * u.ex;
            w0 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[0] : addr[2]);
            w1 = reinterpret_cast<const uint8_t*>(MODE == kGateUp ? addr[1] : addr[2]);
        }
        const uint32_t fault = DENSE ? 0u : weight_fault(w0, w1);
        if (fault != 0u) {
            __syncthreads();
            if (tid == 0) atomicOr(g.status, fault);
            zero_item<MODE>(g, u, ct, s_dst);
            if (DYN && tid == 0) *s_next = next;
            continue;
        }

        // A copy sources: wave instruction q = 4 * wave + j fills slots [64q, 64q + 64):
        // row R = 8q + lane / 8, logical chunk (lane & 7) ^ swizzle(R). Rows past the unit's
        // end repeat its last row (their products are never stored).
        const _Float16* asrc[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t q = 4u * wave + uint32_t(j);
            const uint32_t R = 8u * q + (lane >> 3);
            const uint32_t c = (lane & 7u) ^ ((R >> 1) & 7u);
            const uint32_t row = u.a0 + (R < nrows ? R : nrows - 1u);
            asrc[j] = g.a + uint64_t(row) * g.k + 8u * c;
        }
        // Wave w copies rows [32 w, 32 w + 32): nothing for a block past the unit's rows.
        const bool copies = 32u * wave_u < nrows;
        auto copy_a = [&](uint32_t step, uint32_t buf) {
            if (!copies) return;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                __builtin_amdgcn_global_load_lds(
                    reinterpret_cast<const __attribute__((address_space(1))) void*>(
                        reinterpret_cast<uintptr_t>(asrc[j] + kStepK * step)),
                    reinterpret_cast<__attribute__((address_space(3))) void*>(
                        reinterpret_cast<uintptr_t>(&s_a[buf][(4u * wave_u + uint32_t(j)) * 1024u])),
                    16, 0, 0);
        };
        // Producer: B row prow of this column tile.
        const uint8_t* wrow;
        if (MODE == kGateUp) {
            wrow = prow < 128u ? w0 + uint64_t(128u * ct + prow) * g.row_bytes
                               : w1 + uint64_t(128u * ct + prow - 128u) * g.row_bytes;
        } else {
            wrow = w0 + uint64_t(256u * ct + prow) * g.row_bytes;
        }
        // Raw weight registers, double buffered: fr[i] holds steps i mod 2, so the prefetch two
        // steps ahead is issued at the top of a step, under the same wait as the activation
        // copy, while the other set is decoded.
        Prod fr[2];
        auto prefetch = [&](Prod& f, uint32_t step) { f.load(wrow + uint64_t(step >> 2) * SB, step & 3u, pb); };
        auto produce = [&](const Prod& f, uint8_t* bstage, int s) {
            lds_st<half8>(bstage + 16u * slot(prow, ChunkIndex<Prod>::of(s, pb)), f.chunk(s));
        };
        float16v acc[4][2];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int i = 0; i < 16; ++i) acc[rb][cb][i] = 0.0f;

        // Per K step: wait for this step's operands (and everything issued before them),
        // prefetch the raw weights of step + 2, start the activation copy of step + 1, then
        // multiply while decoding step + 1's weights into the other B stage. The loop body is
        // the same for every step (the last steps repeat the final step's copy and decode into
        // stages nobody reads), so it has no branches and the compiler's own waits for the
        // prefetched registers count exactly the copies issued since. Rows past a partial
        // unit's end hold repeated rows; their products are dropped.
        // NB: the 32-row blocks of this wave's row half that hold entries (0..4, wave-uniform);
        // the others are neither read nor multiplied.
        auto k_step = [&](uint32_t step, auto par_c, auto nb_c) {
            constexpr uint32_t PAR = decltype(par_c)::value;  // step & 1 == buffer index
            constexpr int NB = decltype(nb_c)::value;
            const uint32_t last = nK - 1u;
            wait_barrier();
            prefetch(fr[PAR], step + 2u < last ? step + 2u : last);
            compiler_fence();
            copy_a(step + 1u < last ? step + 1u : last, PAR ^ 1u);
            compiler_fence();
            Prod& fn = fr[PAR ^ 1u];
            const uint8_t* sa = s_a[PAR] + 16384u * rh;
            const uint8_t* sb = s_b[PAR];
            uint8_t* nb = s_b[PAR ^ 1u];
            half8 a[2][4], b[2][2];
            auto load_ops = [&](uint32_t t, int z) {
#pragma unroll
                for (int rb = 0; rb < NB; ++rb) a[z][rb] = lds_ld<half8>(sa + 4096u * uint32_t(rb) + lo[t]);
                if constexpr (NB > 0) {
                    b[z][0] = lds_ld<half8>(sb + bofs0 + lo[t]);
                    b[z][1] = lds_ld<half8>(sb + bofs1 + lo[t]);
                }
            };
            // Scheduling regions (nothing moves across a sched_barrier): slice t's region holds
            // its 8 MFMAs, the operand reads of slice t + 1 and one chunk of the next step's
            // decode, so operand reads run a slice (8 MFMAs) ahead of their use and the decode
            // fills the MFMA shadow.
            load_ops(0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (uint32_t t = 0; t < 4u; ++t) {
                const int z = int(t & 1u);
                if (t + 1u < 4u) load_ops(t + 1u, z ^ 1);
#pragma unroll
                for (int rb = 0; rb < NB; ++rb)
#pragma unroll
                    for (int cb = 0; cb < 2; ++cb)
                        acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[z][rb], b[z][cb], acc[rb][cb], 0, 0, 0);
                if (t == 0u) fn.prepare();
                produce(fn, nb, int(t));
                // Two MFMAs, the next slice's reads, the other MFMAs with the decode, then the
                // chunk's LDS write: the next region's first wait then finds those reads done.
                if constexpr (NB > 0) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, NB + 2, 0);
#pragma unroll
                    for (int i = 0; i < 2 * NB - 2; ++i) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                        __builtin_amdgcn_sched_group_barrier(0x002, 8, 0);
                    }
                    __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        };

        prefetch(fr[0], 0);
        compiler_fence();
        copy_a(0, 0);
        compiler_fence();
        fr[0].prepare();
#pragma unroll
        for (int s = 0; s < 4; ++s) produce(fr[0], s_b[0], s);
        compiler_fence();
        prefetch(fr[1], 1);  // nK >= 2
        // Blocks of this wave's row half holding entries (wave-uniform); every variant runs the
        // same barriers, copies and decode, so the waves of the workgroup stay in step.
        const uint32_t half_rows = nrows > 128u * rh ? nrows - 128u * rh : 0u;
        const uint32_t nb_rows = (half_rows + 31u) / 32u;
        auto k_loop = [&](auto nb_c) {
            for (uint32_t step = 0; step < nK; step += 2u) {
                k_step(step, std::integral_constant<uint32_t, 0>(), nb_c);
                k_step(step + 1u, std::integral_constant<uint32_t, 1>(), nb_c);
            }
        };
        switch (nb_rows < 4u ? nb_rows : 4u) {
            case 0: k_loop(std::integral_constant<int, 0>()); break;
            case 1: k_loop(std::integral_constant<int, 1>()); break;
            case 2: k_loop(std::integral_constant<int, 2>()); break;
            case 3: k_loop(std::integral_constant<int, 3>()); break;
            default: k_loop(std::integral_constant<int, 4>()); break;
        }
        wait_barrier();  // the repeated copies of the last step have landed

        // ---- epilogue: lane holds column (lane & 31) of each 32-column block, rows
        // 32 rb + 8 (i / 4) + 4 (lane / 32) + i % 4 of the wave's 128. Full units (the common
        // case) store without row checks; the down stage ORs its destination checks over the
        // item and reports a bad destination (status bit 1) once. ----
        const uint64_t n_out = g.n_out;
        const uint32_t col0 = MODE == kGateUp ? 128u * ct + 32u * cq + r32 : 256u * ct + 64u * cq + r32;
        bool any_bad = false;
        auto store_rows = [&](auto full_c) {
            constexpr bool FULL = decltype(full_c)::value;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t r = 128u * rh + 32u * uint32_t(rb) + 8u * uint32_t(i >> 2) + 4u * kh + uint32_t(i & 3);
                    if (!FULL && r >= nrows) continue;
                    const uint32_t a = u.a0 + r;
                    if (MODE == kGateUp) {
                        g.out_h[uint64_t(a) * n_out + col0] = half_sat(silu_fast(acc[rb][0][i]) * acc[rb][1][i]);
                    } else {
                        const uint32_t d = DENSE ? a : uint32_t(s_dst[r]);
                        const bool good = DENSE || d < g.n_entries;
                        any_bad = any_bad || !good;
                        float* out = g.out_f + uint64_t(good ? d : a) * n_out + col0;
                        __builtin_nontemporal_store(good ? acc[rb][0][i] : 0.0f, out);  // write-once rows
                        __builtin_nontemporal_store(good ? acc[rb][1][i] : 0.0f, out + 32);
                    }
                }
        };
        if (nrows == kUnitRows) store_rows(std::true_type());  // workgroup-uniform
        else store_rows(std::false_type());
        if (!DENSE && MODE == kDown && any_bad) atomicOr(g.status, 2u);
        if (DYN && tid == 0) *s_next = next;  // every thread read *s_next before the item's first barrier
    }
}

template <class Prod, int MODE, bool DENSE>
__global__ __launch_bounds__(kWideThreads) void wide_gemm_kernel(RoutedGemm g, const uint8_t* dw0, const uint8_t* dw1,
                                                                 uint32_t n_ct) {
    __shared__ __attribute__((aligned(1024))) uint8_t s_a[2][kStageBytes];
    __shared__ __attribute__((aligned(1024))) uint8_t s_b[2][kStageBytes];
    __shared__ uint32_t s_pref[513], s_wsum[8], s_flag;
    __shared__ int32_t s_dst[kUnitRows];
    uint32_t U;
    if (DENSE) {
        U = (g.n_entries + kUnitRows - 1u) / kUnitRows;
    } else {
        // An invalid plan or permutation: the 64-row tile kernel zeroes every slot.
        if (scan_wide_units(g, s_pref, s_wsum, &s_flag) & 2u) return;
        U = s_pref[512];
    }
    wide_items<Prod, MODE, DENSE>(g, dw0, dw1, n_ct, U, s_pref, s_a, s_b, s_dst);
}

// A whole routed stage in one launch. gate/up: each workgroup first takes its share of the
// wide units' items (as the wide kernel), then draws 64-row tile items of the smaller groups
// from the per-XCD counters, so workgroups with one wide item fewer take more tiles and the
// tiles fill the wide units' last round (without wide units the tiles are taken in the static
// order). Down: the tiles first, in the static order, then the wide units, drawn from the
// per-XCD counters (workgroups leave the tile phase at different times). A down tile item
// streams its expert's whole weight matrix through L2, which would evict the activation rows
// that concurrently running wide units share across column tiles; taken first, the tiles
// overlap the wide units only at the boundary.
template <class Prod, class Frag, int MODE, bool RESIDENT>
__global__ __launch_bounds__(kWideThreads) void routed_stage_kernel(RoutedGemm g, uint32_t n_ct, uint32_t n_ntiles,
                                                                    uint32_t npi, uint32_t n_chunks) {
    static_assert(kWideThreads == kV2Threads, "one workgroup shape for both phases");
    __shared__ union Smem {
        WideSmem w;
        TileSmem<Frag, 2> t;
    } sm;
    __shared__ uint32_t s_pref_w[513], s_pref_t[513], s_wsum[8], s_tsum[8], s_flag, s_next_w;
    __shared__ int32_t s_grp[kGrpWords];
    const uint32_t flag = scan_wide_units(g, s_pref_w, s_wsum, &s_flag, s_pref_t, s_tsum, s_grp);
    if (flag & 2u) {
        zero_tile_slots<MODE, 2>(g, n_ntiles, npi, n_chunks);
        return;
    }
    const uint32_t U = s_pref_w[512];
    // Without wide units (U == 0, workgroup-uniform) the wide phase is skipped whole: its setup
    // (per-thread constants, some of them spilled at entry) would run for nothing.
    if (MODE == kGateUp) {
        if (U > 0u) {
            wide_items<Prod, MODE, false>(g, nullptr, nullptr, n_ct, U, s_pref_w, sm.w.s_a, sm.w.s_b, sm.w.s_dst, nullptr,
                                          s_grp);
            __syncthreads();  // the wide phase's LDS is free
            tile_items<Frag, MODE, 2, RESIDENT, true>(g, sm.t, s_pref_t, n_ntiles, npi, n_chunks, s_grp);
        } else {
            tile_items<Frag, MODE, 2, RESIDENT, false>(g, sm.t, s_pref_t, n_ntiles, npi, n_chunks, s_grp);
        }
    } else {
        tile_items<Frag, MODE, 2, RESIDENT, false>(g, sm.t, s_pref_t, n_ntiles, npi, n_chunks, s_grp);
        if (U > 0u) {
            __syncthreads();  // the tile phase's LDS is free
            // Workgroups leave the tile phase at different times: the wide items are drawn.
            wide_items<Prod, MODE, false, true>(g, nullptr, nullptr, n_ct, U, s_pref_w, sm.w.s_a, sm.w.s_b,
                                                sm.w.s_dst, &s_next_w, s_grp);
        }
    }
}

uint32_t wide_cus() {
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

// Persistent grid: one workgroup per CU (each holds about 133 KB of LDS), at most one per
// item, in whole groups of 8 (one per XCD).
uint32_t wide_blocks(uint64_t max_items) {
    uint64_t blocks = (max_items + 7u) & ~uint64_t(7);
    const uint64_t cap = uint64_t(wide_cus()) & ~uint64_t(7);
    if (blocks > cap) blocks = cap;
    if (blocks < 8) blocks = 8;
    return uint32_t(blocks);
}

template <class Prod, int MODE>
hipError_t launch_wide_t(const RoutedGemm& g, hipStream_t s) {
    const uint32_t n_ct = MODE == kGateUp ? g.n_out / 128u : g.n_out / 256u;
    // Units are at most n_entries / wide_min (each covers >= wide_min / 2 rows of a group of
    // at least wide_min entries, wide_min >= 128), so small layers launch fewer workgroups.
    const uint32_t blocks = wide_blocks(uint64_t(g.n_entries / g.wide_min + 1u) * n_ct);
    wide_gemm_kernel<Prod, MODE, false><<<blocks, kWideThreads, 0, s>>>(g, nullptr, nullptr, n_ct);
    return hipGetLastError();
}

template <class Prod, class Frag, int MODE>
hipError_t launch_stage_t(const RoutedGemm& g, hipStream_t s) {
    const uint32_t n_ct = MODE == kGateUp ? g.n_out / 128u : g.n_out / 256u;
    const TilePlan tp = tile_plan<MODE, 2>(g.k, g.n_out);
    const uint32_t blocks = wide_blocks(uint64_t(g.tile_capacity) * tp.n_chunks);
    if (tp.resident)
        routed_stage_kernel<Prod, Frag, MODE, true><<<blocks, kWideThreads, 0, s>>>(g, n_ct, tp.n_ntiles, tp.npi,
                                                                                   tp.n_chunks);
    else
        routed_stage_kernel<Prod, Frag, MODE, false><<<blocks, kWideThreads, 0, s>>>(g, n_ct, tp.n_ntiles, tp.npi,
                                                                                    tp.n_chunks);
    return hipGetLastError();
}

template <class Prod, int MODE>
hipError_t launch_dense_t(const DenseGemm& d, hipStream_t s) {
    RoutedGemm g{};
    g.a = d.a;
    g.out_h = d.out_h;
    g.out_f = d.out_f;
    g.n_entries = d.rows;
    g.k = d.k;
    g.n_out = d.n_out;
    g.row_bytes = d.row_bytes;
    const uint32_t n_ct = MODE == kGateUp ? g.n_out / 128u : g.n_out / 256u;
    const uint32_t blocks = wide_blocks(uint64_t((d.rows + kUnitRows - 1u) / kUnitRows) * n_ct);
    wide_gemm_kernel<Prod, MODE, true><<<blocks, kWideThreads, 0, s>>>(g, d.w0, MODE == kGateUp ? d.w1 : d.w0, n_ct);
    return hipGetLastError();
}

}  // namespace

bool wide_fits(Fmt fmt, bool gate_up, uint32_t k, uint32_t n_out) {
    if (fmt != Fmt::Q8_0 && fmt != Fmt::Q4_K && fmt != Fmt::Q2_K) return false;
    return k % (2u * kStepK) == 0 && n_out % (gate_up ? 128u : 256u) == 0;
}

bool wide_dense_fits(Fmt fmt, bool gate_up, uint32_t rows, uint32_t k, uint32_t n_out) {
    if (fmt != Fmt::F16 && fmt != Fmt::BF16) return false;
    if (k % (2u * kStepK) != 0 || n_out % (gate_up ? 128u : 256u) != 0) return false;
    // Worth it once the units keep at least half of the CUs busy.
    const uint64_t items = uint64_t((rows + kUnitRows - 1u) / kUnitRows) * (gate_up ? n_out / 128u : n_out / 256u);
    return items * 2u >= wide_cus();
}

hipError_t launch_wide_dense(Fmt fmt, bool gate_up, const DenseGemm& d, hipStream_t s) {
    switch (fmt) {
        case Fmt::F16: return gate_up ? launch_dense_t<ProdF16, kGateUp>(d, s) : launch_dense_t<ProdF16, kDown>(d, s);
        case Fmt::BF16: return gate_up ? launch_dense_t<ProdBF16, kGateUp>(d, s) : launch_dense_t<ProdBF16, kDown>(d, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_stage(Fmt fmt, bool gate_up, const RoutedGemm& g, hipStream_t s) {
    switch (fmt) {
        case Fmt::Q8_0:
            return gate_up ? launch_stage_t<ProdQ80, FragQ80, kGateUp>(g, s) : launch_stage_t<ProdQ80, FragQ80, kDown>(g, s);
        case Fmt::Q4_K:
            return gate_up ? launch_stage_t<ProdQ4K, FragQ4K, kGateUp>(g, s) : launch_stage_t<ProdQ4K, FragQ4K, kDown>(g, s);
        case Fmt::Q2_K:
            return gate_up ? launch_stage_t<ProdQ2K, FragQ2K, kGateUp>(g, s) : launch_stage_t<ProdQ2K, FragQ2K, kDown>(g, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_wide(Fmt fmt, bool gate_up, const RoutedGemm& g, hipStream_t s) {
    switch (fmt) {
        case Fmt::Q8_0: return gate_up ? launch_wide_t<ProdQ80, kGateUp>(g, s) : launch_wide_t<ProdQ80, kDown>(g, s);
        case Fmt::Q4_K: return gate_up ? launch_wide_t<ProdQ4K, kGateUp>(g, s) : launch_wide_t<ProdQ4K, kDown>(g, s);
        case Fmt::Q2_K: return gate_up ? launch_wide_t<ProdQ2K, kGateUp>(g, s) : launch_wide_t<ProdQ2K, kDown>(g, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace sm
