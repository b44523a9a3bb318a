// Device numerics and ggml block decoders for the gfx950 Prefill MoE kernels.
//
// Everything here is a fixed sequence of correctly rounded IEEE operations (explicit fma,
// round-to-nearest-even conversions), so each result is a function of its inputs alone.
// The library is compiled with -ffp-contract=off; fusion happens only where written.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sm {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));

// Loads through address-space-1 pointers compile to global_load (vmcnt only). Weight
// pointers read from the expert address table would otherwise be generic (flat) pointers,
// whose loads also count against lgkmcnt and are then waited on by every LDS barrier.
template <class T>
__device__ __forceinline__ T ld_global(const void* p) {
    return *reinterpret_cast<const __attribute__((address_space(1))) T*>(reinterpret_cast<uintptr_t>(p));
}
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Where a fragment is read from: global memory, or a copy staged in LDS (generic pointers
// into the workgroup's shared arrays, read through address space 3 as ds_read).
struct FromGlobal {
    template <class T>
    __device__ __forceinline__ static T ld(const uint8_t* p) { return ld_global<T>(p); }
};
struct FromLds {
    template <class T>
    __device__ __forceinline__ static T ld(const uint8_t* p) {
        return *(const __attribute__((address_space(3))) T*)(p);
    }
};

// exp(x): Cody & Waite reduction x = n*ln2 + r with a two-part ln2, a degree-7 Taylor
// polynomial in r evaluated by Horner with fma, and an exact scale by 2^n (v_ldexp_f32).
// Branch-free: the polynomial runs on x clamped into [-104, 88.72...] (the identity inside it),
// and the special cases are selected afterwards (NaN -> x, above -> +inf, below -> 0).
__device__ __forceinline__ float exp_cw(float x) {
    const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 88.72283935546875f);
    const float n = __builtin_rintf(xc * 1.44269502162933349609375f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, xc);
    r = __builtin_fmaf(-n, 1.428606765330187045e-06f, r);
    float p = 1.98412698412698412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    float e = __builtin_amdgcn_ldexpf(p, int(n));
    e = x < -104.0f ? 0.0f : e;
    e = x > 88.72283935546875f ? __builtin_inff() : e;
    return __builtin_isnan(x) ? x : e;
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + exp_cw(-x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + exp_cw(-x)); }

// silu for the fused product epilogues, whose F32 inputs already carry accumulation-order
// rounding: exp2 and the reciprocal come from the hardware (v_exp_f32, v_rcp_f32, each
// within 1 ulp), a few F32 ulps from silu() above before the result is rounded to F16.
// Limits match silu(): +inf -> +inf, -inf -> NaN, large negative x -> -0.
__device__ __forceinline__ float silu_fast(float x) {
    const float e = __builtin_amdgcn_exp2f(x * -1.44269502162933349609375f);
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

__device__ __forceinline__ uint16_t f16_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }
__device__ __forceinline__ _Float16 bits_f16(uint16_t u) { return __builtin_bit_cast(_Float16, u); }
__device__ __forceinline__ float f16_lo(uint32_t w) { return float(bits_f16(uint16_t(w & 0xffffu))); }
__device__ __forceinline__ float f16_hi(uint32_t w) { return float(bits_f16(uint16_t(w >> 16))); }

// half_sat: F32 subnormals -> +0, NaN -> 0x7e00, otherwise clamp to +-65504 and round
// to nearest even (the reference's common/math.h:33-40).
__device__ __forceinline__ _Float16 half_sat(float x) {
    const uint32_t b = __builtin_bit_cast(uint32_t, x);
    if ((b & 0x7f800000u) == 0u && (b & 0x007fffffu) != 0u) return bits_f16(0);
    if (__builtin_isnan(x)) return bits_f16(0x7e00);
    return _Float16(__builtin_fminf(__builtin_fmaxf(x, -65504.0f), 65504.0f));
}

// Status bits an expert's weight pair raises, as the address snapshot holds it: a null
// address (status bit 0, a missing expert), or an address tagged in bit 0 (status bit 2, a
// tiered slot address no live lease pins; real addresses are at least 4-byte aligned). The
// expert's rows are written as zeros either way.
__device__ __forceinline__ uint32_t weight_fault(const uint8_t* w0, const uint8_t* w1) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(w0), b = reinterpret_cast<uintptr_t>(w1);
    if (a == 0 || b == 0) return 1u;
    return ((a | b) & 1u) ? 4u : 0u;
}

// Byte j (0..3) of a dword as an exact float (selected as v_cvt_f32_ubyte{j}).
__device__ __forceinline__ float ubyte(uint32_t w, int j) { return float((w >> (8 * j)) & 0xffu); }

typedef float float2v __attribute__((ext_vector_type(2)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

// Two F32 values rounded to nearest-even F16 as one packed pair (v_cvt_pk_f16_f32).
__device__ __forceinline__ half2v cvt_pk_f16(float a, float b) {
    return __builtin_convertvector(float2v{a, b}, half2v);
}

// A code byte b <= 15 read as an OCP E4M3 value is exactly b * 2^-9 (b < 8: the subnormal
// b/8 * 2^-6; 8 <= b <= 15: (1 + (b - 8)/8) * 2^-6), so one v_cvt_pk_f32_fp8 turns two code
// bytes into exact F32 values, where v_cvt_f32_ubyte{j} takes one instruction per byte.
__device__ __forceinline__ float2v nib_pair(uint32_t w, bool hi_word) {
    return hi_word ? __builtin_amdgcn_cvt_pk_f32_fp8(int(w), true) : __builtin_amdgcn_cvt_pk_f32_fp8(int(w), false);
}

// Eight values fma(scale, q_j, bias) from the code bytes q_j <= 15 of two dwords, rounded to
// F32 and then to F16 in pairs (v_fma_f32, then v_cvt_pk_f16_f32: two separate roundings),
// given scale512 = 512 * scale (exact: a power-of-two factor on a normal F32). The product
// 512 scale * (q 2^-9) is scale * q exactly, and with scale carrying <= 17 significant bits
// and q < 2^4 it is exact in F32, so this equals the reference's `scale * q - bias` in F32,
// then F16.
__device__ __forceinline__ half8 decode8_nib(uint32_t w0, uint32_t w1, float scale512, float bias) {
    const float2v q[4] = {nib_pair(w0, false), nib_pair(w0, true), nib_pair(w1, false), nib_pair(w1, true)};
    half2v p[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        p[i] = cvt_pk_f16(__builtin_fmaf(scale512, q[i][0], bias), __builtin_fmaf(scale512, q[i][1], bias));
    return half8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
}

// 2-bit codes by table: a 16-value group of one scale byte takes only the four values
// fma(dl, q, ml), q = 0..3, each rounded to F32 and then F16 as decode8_nib rounds it. The
// table holds their low bytes in `lo` and high bytes in `hi` (byte q of each). A dword of four
// codes (one per byte, each <= 3) is itself a v_perm_b32 selector into either half, so two
// permutes give the four values' low and high bytes and two more interleave them into F16
// pairs.
struct Q2Table {
    uint32_t lo, hi;
};
__device__ __forceinline__ Q2Table q2_table(float dl, float ml) {
    const uint32_t p01 = __builtin_bit_cast(uint32_t, cvt_pk_f16(__builtin_fmaf(dl, 0.0f, ml), __builtin_fmaf(dl, 1.0f, ml)));
    const uint32_t p23 = __builtin_bit_cast(uint32_t, cvt_pk_f16(__builtin_fmaf(dl, 2.0f, ml), __builtin_fmaf(dl, 3.0f, ml)));
    return {__builtin_amdgcn_perm(p23, p01, 0x06040200u), __builtin_amdgcn_perm(p23, p01, 0x07050301u)};
}
// Eight values from the codes (one per byte, each <= 3) of two dwords.
__device__ __forceinline__ half8 lookup8(uint32_t x0, uint32_t x1, const Q2Table& t) {
    half2v p[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t x = i == 0 ? x0 : x1;
        const uint32_t lo = __builtin_amdgcn_perm(0u, t.lo, x), hi = __builtin_amdgcn_perm(0u, t.hi, x);
        p[2 * i] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(hi, lo, 0x05010400u));
        p[2 * i + 1] = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(hi, lo, 0x07030602u));
    }
    return half8{p[0][0], p[0][1], p[1][0], p[1][1], p[2][0], p[2][1], p[3][0], p[3][1]};
}

// ---------------------------------------------------------------------------------------
// Per-lane weight fragments. A 256-value K slab ("superblock") of one weight row is split
// over the four lane groups g = lane/16 of a wave: group g owns values [64g, 64g+64), and
// MFMA step s (0..7) feeds it values 64g + 8s + i, i = 0..7. The A operand uses the same
// mapping, so the product covers every K value exactly once.
// ---------------------------------------------------------------------------------------

// Scale and bias of Q4_K pairs 2g (low nibbles) and 2g + 1 (high nibbles) from a block's first
// 16 bytes: f16 d, f16 dmin, scales[12] = bytes b0..b11 (hdr[1..3]). Pair j < 4: scale =
// b[j] & 63, min = b[j+4] & 63; pair j >= 4: scale = (b[j+4] & 15) | (b[j-4] >> 6) << 4, min =
// (b[j+4] >> 4) | (b[j] >> 6) << 4 (dequant.hpp:157-190). The four 6-bit fields land in the
// bytes of one dword {scale 2g, scale 2g+1, min 2g, min 2g+1}: a byte permute gathers
// X = {b[2g], b[2g+1], b[2g+4], b[2g+5]} (g < 2) or {b[2g+4], b[2g+5]} twice (g >= 2) and
// Y = {b[2g-4], b[2g-3], b[2g], b[2g+1]}; then V = (X & m1) | ((X >> 4) & m3) | ((Y >> 2) & m2)
// with (m1, m3, m2) = (0x3F3F3F3F, 0, 0) for g < 2 and (0x0F0F, 0x0F0F0000, 0x30303030) for
// g >= 2, since (y >> 2) & 0x30 == (y >> 6) << 4 for a byte y. The scales are returned
// premultiplied by 512 for decode8_nib (exact: d * scale is 0 or at least 2^-24).
__device__ __forceinline__ void q4k_pair_scales(const u32x4& hdr, uint32_t g, float& d_lo, float& m_lo, float& d_hi,
                                                float& m_hi) {
    const float d = f16_lo(hdr[0]), dmin = f16_hi(hdr[0]);
    const bool hi_pairs = g >= 2u;
    const uint32_t sel_lo = (g & 1u) ? 0x07060302u : 0x05040100u;   // bytes of {hdr[2], hdr[1]}
    const uint32_t sel_x = hi_pairs ? ((g & 1u) ? 0x03020302u : 0x01000100u) : sel_lo;
    const uint32_t x = __builtin_amdgcn_perm(hi_pairs ? hdr[3] : hdr[2], hi_pairs ? hdr[3] : hdr[1], sel_x);
    const uint32_t y = __builtin_amdgcn_perm(hdr[2], hdr[1], sel_lo);
    const uint32_t v = (x & (hi_pairs ? 0x00000F0Fu : 0x3F3F3F3Fu)) | ((x >> 4) & (hi_pairs ? 0x0F0F0000u : 0u)) |
                       ((y >> 2) & (hi_pairs ? 0x30303030u : 0u));
    d_lo = d * ubyte(v, 0) * 512.0f;
    d_hi = d * ubyte(v, 1) * 512.0f;
    m_lo = -(dmin * ubyte(v, 2));
    m_hi = -(dmin * ubyte(v, 3));
}

// Q4_K (144 B / 256): f16 d, f16 dmin, scales[12] (6-bit scale/min pairs), q[128] nibbles.
// Values 64g..64g+31 are the low nibbles of q[32g..32g+31] with pair 2g; values
// 64g+32..64g+63 the high nibbles with pair 2g+1 (dequant.hpp:157-190).
struct FragQ4K {
    u32x4 hdr, qa, qb;
    float d_lo, m_lo, d_hi, m_hi;
    int g;
    template <class M = FromGlobal>
    __device__ __forceinline__ void load(const uint8_t* sb, int grp) {
        g = grp;
        hdr = M::template ld<u32x4>(sb);
        qa = M::template ld<u32x4>(sb + 16 + 32 * grp);
        qb = M::template ld<u32x4>(sb + 32 + 32 * grp);
    }
    __device__ __forceinline__ void prepare() { q4k_pair_scales(hdr, uint32_t(g), d_lo, m_lo, d_hi, m_hi); }
    __device__ __forceinline__ uint32_t q(int i) const { return i < 4 ? qa[i] : qb[i - 4]; }
    __device__ __forceinline__ half8 step(int s) const {
        if (s < 4) return decode8_nib(q(2 * s) & 0x0F0F0F0Fu, q(2 * s + 1) & 0x0F0F0F0Fu, d_lo, m_lo);
        return decode8_nib((q(2 * s - 8) >> 4) & 0x0F0F0F0Fu, (q(2 * s - 7) >> 4) & 0x0F0F0F0Fu, d_hi, m_hi);
    }
};

// Q8_0 (34 B / 32): f16 d, int8 q[32]. A 256-value slab is 8 blocks (272 B); group g owns
// blocks 2g and 2g+1 (68 B at a 4-byte-aligned offset). The value is d*q rounded to F16
// (dequant.hpp:81-86); d*q is exact in F32 (11 x 8 bits), so one F16 rounding of the exact
// product is the same value. Decoding runs on packed F16 pairs: the byte, biased by 128, is
// placed under the exponent of 1024 (0x6400 | u = 1024 + u exactly), 1152 is subtracted
// (exact, giving q), and v_pk_mul_f16 rounds q*d once. A zero code keeps the sign of d.
__device__ __forceinline__ half2v q80_pair(uint32_t u, uint32_t sel, half2v dd) {
    const uint32_t biased = __builtin_amdgcn_perm(0x64646464u, u, sel);  // bytes {u_a, 0x64, u_b, 0x64}
    const half2v q = __builtin_bit_cast(half2v, biased) + half2v{_Float16(-1152.0f), _Float16(-1152.0f)};
    return q * dd;
}
struct FragQ80 {
    uint32_t w[17];
    template <class M = FromGlobal>
    __device__ __forceinline__ void load(const uint8_t* slab, int g) {
        const uint8_t* p = slab + 68 * g;
        if constexpr (__is_same(M, FromGlobal)) {  // four dword-aligned 16-byte loads and a dword
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32x4 v = M::template ld<u32x4>(p + 16 * i);
#pragma unroll
                for (int j = 0; j < 4; ++j) w[4 * i + j] = v[j];
            }
            w[16] = M::template ld<uint32_t>(p + 64);
        } else {
#pragma unroll
            for (int i = 0; i < 17; ++i) w[i] = M::template ld<uint32_t>(p + 4 * i);
        }
    }
    __device__ __forceinline__ void prepare() {}
    // Block b (0/1) occupies bytes 34b .. 34b+33 of the 68: d at 34b, q at 34b+2.
    __device__ __forceinline__ half8 step(int s) const {
        const int b = s >> 2;          // block
        const int o = 34 * b + 2 + 8 * (s & 3);  // byte offset of the 8 quants
        const int wi = o >> 2;
        const int sh = (o & 3) * 8;    // 0 or 16
        const uint32_t x0 = (sh ? __builtin_amdgcn_alignbyte(w[wi + 1], w[wi], 2) : w[wi]) ^ 0x80808080u;
        const uint32_t x1 = (sh ? __builtin_amdgcn_alignbyte(w[wi + 2], w[wi + 1], 2) : w[wi + 1]) ^ 0x80808080u;
        const uint32_t dw = w[(34 * b) >> 2];
        const _Float16 d = bits_f16(uint16_t(b == 0 ? (dw & 0xffffu) : (dw >> 16)));
        const half2v dd{d, d};
        const half2v p0 = q80_pair(x0, 0x04010400u, dd), p1 = q80_pair(x0, 0x04030402u, dd);
        const half2v p2 = q80_pair(x1, 0x04010400u, dd), p3 = q80_pair(x1, 0x04030402u, dd);
        return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
    }
};

// Q2_K (84 B / 256): scales[16] (low nibble scale, high nibble min), q[64] (2-bit codes,
// four planes per byte), f16 d, f16 dmin. Value e = 128n + 32j + w uses bits 2j of
// q[32n + w] and scale byte 8n + 2j + (w >= 16) (ggml's dequantize_row_q2_K). Group g
// owns n = g/2, j in {2(g%2), 2(g%2)+1}.
struct FragQ2K {
    u32x4 qa, qb;
    uint32_t sc, dd;
    float d, dmin;
    int jbase;
    template <class M = FromGlobal>
    __device__ __forceinline__ void load(const uint8_t* sb, int g) {
        const int n = g >> 1;
        jbase = 2 * (g & 1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // dword reads: an 84-byte slab staged in LDS is only 4-byte aligned
            qa[i] = M::template ld<uint32_t>(sb + 16 + 32 * n + 4 * i);
            qb[i] = M::template ld<uint32_t>(sb + 32 + 32 * n + 4 * i);
        }
        sc = M::template ld<uint32_t>(sb + 8 * n + 2 * jbase);
        dd = M::template ld<uint32_t>(sb + 80);
    }
    __device__ __forceinline__ void prepare() {
        d = f16_lo(dd);
        dmin = f16_hi(dd);
    }
    __device__ __forceinline__ uint32_t q(int i) const { return i < 4 ? qa[i] : qb[i - 4]; }
    __device__ __forceinline__ half8 step(int s) const {
        const int jj = s >> 2;                 // 0/1 -> plane j = jbase + jj
        const int w0 = 8 * (s & 3);            // first w of the 8
        const int shift = 2 * (jbase + jj);
        const uint32_t scb = (sc >> (8 * (2 * jj + (w0 >= 16 ? 1 : 0)))) & 0xffu;
        const Q2Table t = q2_table(d * float(scb & 0xFu), -(dmin * float(scb >> 4)));
        const uint32_t x0 = (q(w0 >> 2) >> shift) & 0x03030303u;
        const uint32_t x1 = (q((w0 >> 2) + 1) >> shift) & 0x03030303u;
        return lookup8(x0, x1, t);
    }
};

// F16 rows: group g owns values [64g, 64g+64) as 8 x 16-byte fragments.
struct FragF16 {
    half8 v[8];
    template <class M = FromGlobal>
    __device__ __forceinline__ void load(const uint8_t* slab, int g) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = M::template ld<half8>(slab + 128 * g + 16 * i);
    }
    __device__ __forceinline__ void prepare() {}
    __device__ __forceinline__ half8 step(int s) const { return v[s]; }
};

// BF16 rows, widened exactly to F32 and rounded once to F16.
struct FragBF16 {
    u32x4 v[8];
    template <class M = FromGlobal>
    __device__ __forceinline__ void load(const uint8_t* slab, int g) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = M::template ld<u32x4>(slab + 128 * g + 16 * i);
    }
    __device__ __forceinline__ void prepare() {}
    __device__ __forceinline__ half8 step(int s) const {
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

// Bytes of one 256-value slab per format (Q8_0: eight 34-byte blocks).
template <class F> struct SlabBytes;
template <> struct SlabBytes<FragQ4K> { static constexpr int value = 144; };
template <> struct SlabBytes<FragQ80> { static constexpr int value = 272; };
template <> struct SlabBytes<FragQ2K> { static constexpr int value = 84; };
template <> struct SlabBytes<FragF16> { static constexpr int value = 512; };
template <> struct SlabBytes<FragBF16> { static constexpr int value = 512; };

}  // namespace sm
