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
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// exp(x): Cody & Waite reduction x = n*ln2 + r with a two-part ln2, a degree-7 Taylor
// polynomial in r evaluated by Horner with fma, and an exact scale by 2^n (v_ldexp_f32).
__device__ __forceinline__ float exp_cw(float x) {
    if (__builtin_isnan(x)) return x;
    if (x > 88.72283935546875f) return __builtin_inff();
    if (x < -104.0f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269502162933349609375f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.428606765330187045e-06f, r);
    float p = 1.98412698412698412698e-4f;
    p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f);
    p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f);
    p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f);
    p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    return __builtin_amdgcn_ldexpf(p, int(n));
}

__device__ __forceinline__ float silu(float x) { return x / (1.0f + exp_cw(-x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.0f / (1.0f + exp_cw(-x)); }

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

// Byte j (0..3) of a dword as an exact float (selected as v_cvt_f32_ubyte{j}).
__device__ __forceinline__ float ubyte(uint32_t w, int j) { return float((w >> (8 * j)) & 0xffu); }

// Eight values fma(scale, byte_j, bias) from the four bytes of two dwords, rounded once
// to F16. With every byte < 2^8 and scale carrying <= 17 significant bits the product is
// exact, so this equals the reference's `scale * q - bias` rounded to F32 then to F16.
__device__ __forceinline__ half8 decode8(uint32_t w0, uint32_t w1, float scale, float bias) {
    half8 h;
    h[0] = _Float16(__builtin_fmaf(scale, ubyte(w0, 0), bias));
    h[1] = _Float16(__builtin_fmaf(scale, ubyte(w0, 1), bias));
    h[2] = _Float16(__builtin_fmaf(scale, ubyte(w0, 2), bias));
    h[3] = _Float16(__builtin_fmaf(scale, ubyte(w0, 3), bias));
    h[4] = _Float16(__builtin_fmaf(scale, ubyte(w1, 0), bias));
    h[5] = _Float16(__builtin_fmaf(scale, ubyte(w1, 1), bias));
    h[6] = _Float16(__builtin_fmaf(scale, ubyte(w1, 2), bias));
    h[7] = _Float16(__builtin_fmaf(scale, ubyte(w1, 3), bias));
    return h;
}

// ---------------------------------------------------------------------------------------
// Per-lane weight fragments. A 256-value K slab ("superblock") of one weight row is split
// over the four lane groups g = lane/16 of a wave: group g owns values [64g, 64g+64), and
// MFMA step s (0..7) feeds it values 64g + 8s + i, i = 0..7. The A operand uses the same
// mapping, so the product covers every K value exactly once.
// ---------------------------------------------------------------------------------------

// Q4_K (144 B / 256): f16 d, f16 dmin, scales[12] (6-bit scale/min pairs), q[128] nibbles.
// Values 64g..64g+31 are the low nibbles of q[32g..32g+31] with pair 2g; values
// 64g+32..64g+63 the high nibbles with pair 2g+1 (dequant.hpp:157-190).
struct FragQ4K {
    uint32_t q[8];
    float d_lo, m_lo, d_hi, m_hi;
    __device__ __forceinline__ void load(const uint8_t* sb, int g) {
        const u32x4 hdr = *reinterpret_cast<const u32x4*>(sb);
        const u32x4 a = *reinterpret_cast<const u32x4*>(sb + 16 + 32 * g);
        const u32x4 b = *reinterpret_cast<const u32x4*>(sb + 32 + 32 * g);
        q[0] = a[0]; q[1] = a[1]; q[2] = a[2]; q[3] = a[3];
        q[4] = b[0]; q[5] = b[1]; q[6] = b[2]; q[7] = b[3];
        const float d = f16_lo(hdr[0]);
        const float dmin = f16_hi(hdr[0]);
        // scales[12] = bytes 4..15 of the block = hdr[1..3].
        const uint32_t s0 = hdr[1], s1 = hdr[2], s2 = hdr[3];
        auto byte = [&](int i) -> uint32_t {
            const uint32_t w = i < 4 ? s0 : (i < 8 ? s1 : s2);
            return (w >> (8 * (i & 3))) & 0xffu;
        };
        uint32_t sc_lo, mn_lo, sc_hi, mn_hi;
        const int j0 = 2 * g, j1 = 2 * g + 1;
        if (j0 < 4) {
            sc_lo = byte(j0) & 63u; mn_lo = byte(j0 + 4) & 63u;
            sc_hi = byte(j1) & 63u; mn_hi = byte(j1 + 4) & 63u;
        } else {
            sc_lo = (byte(j0 + 4) & 0xFu) | ((byte(j0 - 4) >> 6) << 4);
            mn_lo = (byte(j0 + 4) >> 4) | ((byte(j0) >> 6) << 4);
            sc_hi = (byte(j1 + 4) & 0xFu) | ((byte(j1 - 4) >> 6) << 4);
            mn_hi = (byte(j1 + 4) >> 4) | ((byte(j1) >> 6) << 4);
        }
        d_lo = d * float(sc_lo); m_lo = -(dmin * float(mn_lo));
        d_hi = d * float(sc_hi); m_hi = -(dmin * float(mn_hi));
    }
    __device__ __forceinline__ half8 step(int s) const {
        if (s < 4) return decode8(q[2 * s] & 0x0F0F0F0Fu, q[2 * s + 1] & 0x0F0F0F0Fu, d_lo, m_lo);
        return decode8((q[2 * s - 8] >> 4) & 0x0F0F0F0Fu, (q[2 * s - 7] >> 4) & 0x0F0F0F0Fu, d_hi, m_hi);
    }
};

// Q8_0 (34 B / 32): f16 d, int8 q[32]. A 256-value slab is 8 blocks (272 B); group g owns
// blocks 2g and 2g+1 (68 B at a 4-byte-aligned offset). Bytes are biased by 128 so the
// unsigned byte converters apply: d*(u - 128) = fma(d, u, -128 d), exact (dequant.hpp:81-86).
struct FragQ80 {
    uint32_t w[17];
    __device__ __forceinline__ void load(const uint8_t* slab, int g) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(slab + 68 * g);
#pragma unroll
        for (int i = 0; i < 17; ++i) w[i] = p[i];
    }
    // Block b (0/1) occupies bytes 34b .. 34b+33 of the 68: d at 34b, q at 34b+2.
    __device__ __forceinline__ half8 step(int s) const {
        const int b = s >> 2;          // block
        const int o = 34 * b + 2 + 8 * (s & 3);  // byte offset of the 8 quants
        const int wi = o >> 2;
        const int sh = (o & 3) * 8;    // 0 or 16
        const uint32_t x0 = sh ? __builtin_amdgcn_alignbyte(w[wi + 1], w[wi], 2) : w[wi];
        const uint32_t x1 = sh ? __builtin_amdgcn_alignbyte(w[wi + 2], w[wi + 1], 2) : w[wi + 1];
        const uint32_t dw = w[(34 * b) >> 2];
        const float d = b == 0 ? f16_lo(dw) : f16_hi(dw);
        return decode8(x0 ^ 0x80808080u, x1 ^ 0x80808080u, d, -128.0f * d);
    }
};

// Q2_K (84 B / 256): scales[16] (low nibble scale, high nibble min), q[64] (2-bit codes,
// four planes per byte), f16 d, f16 dmin. Value e = 128n + 32j + w uses bits 2j of
// q[32n + w] and scale byte 8n + 2j + (w >= 16) (ggml's dequantize_row_q2_K). Group g
// owns n = g/2, j in {2(g%2), 2(g%2)+1}.
struct FragQ2K {
    uint32_t q[8];
    uint32_t sc;
    float d, dmin;
    int jbase;
    __device__ __forceinline__ void load(const uint8_t* sb, int g) {
        const int n = g >> 1;
        jbase = 2 * (g & 1);
        const u32x4 a = *reinterpret_cast<const u32x4*>(sb + 16 + 32 * n);
        const u32x4 b = *reinterpret_cast<const u32x4*>(sb + 32 + 32 * n);
        q[0] = a[0]; q[1] = a[1]; q[2] = a[2]; q[3] = a[3];
        q[4] = b[0]; q[5] = b[1]; q[6] = b[2]; q[7] = b[3];
        sc = *reinterpret_cast<const uint32_t*>(sb + 8 * n + 2 * jbase);
        const uint32_t dd = *reinterpret_cast<const uint32_t*>(sb + 80);
        d = f16_lo(dd);
        dmin = f16_hi(dd);
    }
    __device__ __forceinline__ half8 step(int s) const {
        const int jj = s >> 2;                 // 0/1 -> plane j = jbase + jj
        const int w0 = 8 * (s & 3);            // first w of the 8
        const int shift = 2 * (jbase + jj);
        const uint32_t scb = (sc >> (8 * (2 * jj + (w0 >= 16 ? 1 : 0)))) & 0xffu;
        const float dl = d * float(scb & 0xFu);
        const float ml = -(dmin * float(scb >> 4));
        const uint32_t x0 = (q[w0 >> 2] >> shift) & 0x03030303u;
        const uint32_t x1 = (q[(w0 >> 2) + 1] >> shift) & 0x03030303u;
        return decode8(x0, x1, dl, ml);
    }
};

// F16 rows: group g owns values [64g, 64g+64) as 8 x 16-byte fragments.
struct FragF16 {
    half8 v[8];
    __device__ __forceinline__ void load(const uint8_t* slab, int g) {
        const half8* p = reinterpret_cast<const half8*>(slab + 128 * g);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = p[i];
    }
    __device__ __forceinline__ half8 step(int s) const { return v[s]; }
};

// BF16 rows, widened exactly to F32 and rounded once to F16.
struct FragBF16 {
    u32x4 v[8];
    __device__ __forceinline__ void load(const uint8_t* slab, int g) {
        const u32x4* p = reinterpret_cast<const u32x4*>(slab + 128 * g);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = p[i];
    }
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
