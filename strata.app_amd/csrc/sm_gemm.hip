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
#include "sm_tiles.h"

namespace sm {
namespace {

constexpr int kRows = 64;
constexpr int kLdsRow = kSlab + 8;  // halves

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
    if (const uint32_t fault = weight_fault(w0, w1)) {
        if (threadIdx.x == 0) atomicOr(g.status, fault);
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
    const TilePlan p = tile_plan<MODE, NF>(g.k, g.n_out);
    // Persistent: one workgroup per CU (each holds about 130 KB of LDS), never more than the
    // tile slots, in whole groups of 8 (one per XCD).
    uint32_t blocks = (g.tile_capacity * p.n_chunks + 7u) & ~7u;
    const uint32_t cap = device_cus() & ~7u;
    if (blocks > cap) blocks = cap;
    if (blocks < 8u) blocks = 8u;
    if (p.resident)
        routed_gemm_staged_kernel<Frag, MODE, NF, true><<<blocks, kV2Threads, 0, s>>>(g, p.n_ntiles, p.npi, p.n_chunks);
    else
        routed_gemm_staged_kernel<Frag, MODE, NF, false><<<blocks, kV2Threads, 0, s>>>(g, p.n_ntiles, p.npi, p.n_chunks);
    return hipGetLastError();
}

template <class Frag, int MODE>
hipError_t launch_tiles(const RoutedGemm& g, hipStream_t s) {
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

// A stage with wide units: one launch of the routed stage kernel (wide units and the small
// groups' tiles) where the tiles fit the staged kernel, else the wide kernel and then the
// plain tile kernel.
template <class Frag, int MODE>
hipError_t launch_routed(Fmt fmt, const RoutedGemm& g, hipStream_t s) {
    if (g.wide_min == ~0u) return launch_tiles<Frag, MODE>(g, s);
    if (g.k % kSlab == 0 && g.n_out % Staged<MODE, 2>::kOut == 0) return launch_stage(fmt, MODE == kGateUp, g, s);
    const hipError_t e = launch_wide(fmt, MODE == kGateUp, g, s);
    return e != hipSuccess ? e : launch_tiles<Frag, MODE>(g, s);
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
