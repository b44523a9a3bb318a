// Deterministic synthetic inputs and block quantizers (host side).
//
// Every value is a pure function of (seed, stream, index): one SplitMix64 hash per index
// pair gives two uniforms and the Box-Muller transform two N(0,1) draws, so results do not
// depend on the thread count. The quantizers produce valid ggml block layouts (Q8_0, Q4_K, Q2_K);
// they need not match ggml's reference quantizers bit for bit because the GPU path and the
// CPU checker consume the same bytes.
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/strata_moe.h"

namespace {

inline uint64_t splitmix(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

// Draw i of a (seed, stream) sequence: pair j = i/2 takes one 64-bit hash, split into two
// 32-bit uniforms u1 in (0,1], u2 in [0,1); Box-Muller gives r*cos (even i) and r*sin (odd i).
inline double normal_at(uint64_t seed, uint64_t stream, uint64_t i) {
    const uint64_t key = splitmix(seed ^ splitmix(stream + 0x5EEDull));
    const uint64_t h = splitmix(key + (i >> 1));
    const double u1 = (double((h >> 32) + 1)) * 0x1.0p-32;
    const double u2 = double(h & 0xffffffffull) * 0x1.0p-32;
    const double r = std::sqrt(-2.0 * std::log(u1));
    const double a = 6.283185307179586 * u2;
    return (i & 1) ? r * std::sin(a) : r * std::cos(a);
}

// Fills out[0..n) of the sequence, computing each pair's radius and angle once.
template <class Store>
void normal_fill(uint64_t seed, uint64_t stream, uint64_t b, uint64_t e, Store store) {
    const uint64_t key = splitmix(seed ^ splitmix(stream + 0x5EEDull));
    uint64_t i = b;
    if (i < e && (i & 1)) { store(i, normal_at(seed, stream, i)); ++i; }
    for (; i + 1 < e; i += 2) {
        const uint64_t h = splitmix(key + (i >> 1));
        const double u1 = (double((h >> 32) + 1)) * 0x1.0p-32;
        const double u2 = double(h & 0xffffffffull) * 0x1.0p-32;
        const double r = std::sqrt(-2.0 * std::log(u1));
        const double a = 6.283185307179586 * u2;
        store(i, r * std::cos(a));
        store(i + 1, r * std::sin(a));
    }
    if (i < e) store(i, normal_at(seed, stream, i));
}

uint32_t fbits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

uint16_t to_f16(float f) {  // round to nearest even
    const uint32_t x = fbits(f);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return uint16_t(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);
    if (ax >= 0x38800000u) {
        uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
        const uint32_t rem = ax & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
        return uint16_t(sign | h);
    }
    if (ax <= 0x33000000u) return sign;
    const uint32_t e = ax >> 23, mant = (ax & 0x7fffffu) | 0x800000u, shift = 126u - e;
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return uint16_t(sign | h);
}

float from_f16(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    uint32_t u;
    if (e == 0) {
        const float v = std::ldexp(float(m), -24);
        return sign ? -v : v;
    }
    if (e == 31) u = sign | 0x7f800000u | (m << 13);
    else u = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

uint16_t to_bf16(float f) {
    const uint32_t b = fbits(f);
    if ((b & 0x7fffffffu) > 0x7f800000u) return uint16_t((b >> 16) | 64u);
    return uint16_t((b + ((b >> 16) & 1u) + 0x7fffu) >> 16);
}

template <class F>
void parallel_for(uint64_t n, F f) {
    unsigned nt = std::thread::hardware_concurrency();
    if (nt == 0) nt = 1;
    if (nt > 32) nt = 32;
    if (n < 65536) nt = 1;
    std::vector<std::thread> th;
    const uint64_t chunk = (n + nt - 1) / nt;
    for (unsigned t = 0; t < nt; ++t) {
        const uint64_t b = t * chunk, e = std::min<uint64_t>(n, b + chunk);
        if (b >= e) break;
        th.emplace_back([=] { f(b, e); });
    }
    for (auto& x : th) x.join();
}

inline int nearest(float x) { return int(std::lrint(x)); }

// Q8_0: d = absmax/127, q = round(x/d).
void quant_q8_0(const float* x, uint8_t* out) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = std::fmax(amax, std::fabs(x[i]));
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    const uint16_t dh = to_f16(d);
    std::memcpy(out, &dh, 2);
    for (int i = 0; i < 32; ++i) {
        int q = nearest(x[i] * id);
        q = q < -127 ? -127 : (q > 127 ? 127 : q);
        out[2 + i] = uint8_t(int8_t(q));
    }
}

// Q4_K: per 32-value sub-block an affine (scale, min) fit, 6-bit scale/min codes under
// F16 super-scales, 4-bit codes.
void quant_q4_k(const float* x, uint8_t* out) {
    float sc[8], mn[8];
    for (int j = 0; j < 8; ++j) {
        float lo = x[32 * j], hi = x[32 * j];
        for (int i = 1; i < 32; ++i) { lo = std::fmin(lo, x[32 * j + i]); hi = std::fmax(hi, x[32 * j + i]); }
        if (lo > 0.0f) lo = 0.0f;
        sc[j] = (hi - lo) / 15.0f;
        mn[j] = -lo;
    }
    float msc = 0.0f, mmn = 0.0f;
    for (int j = 0; j < 8; ++j) { msc = std::fmax(msc, sc[j]); mmn = std::fmax(mmn, mn[j]); }
    const uint16_t dh = to_f16(msc / 63.0f), mh = to_f16(mmn / 63.0f);
    const float d = from_f16(dh), dmin = from_f16(mh);
    uint8_t ls[8], lm[8];
    for (int j = 0; j < 8; ++j) {
        int a = d > 0.0f ? nearest(sc[j] / d) : 0;
        int b = dmin > 0.0f ? nearest(mn[j] / dmin) : 0;
        ls[j] = uint8_t(a < 0 ? 0 : (a > 63 ? 63 : a));
        lm[j] = uint8_t(b < 0 ? 0 : (b > 63 ? 63 : b));
    }
    std::memcpy(out, &dh, 2);
    std::memcpy(out + 2, &mh, 2);
    uint8_t* s = out + 4;
    for (int j = 0; j < 4; ++j) {
        s[j] = uint8_t((ls[j] & 63) | ((ls[j + 4] >> 4) << 6));
        s[j + 4] = uint8_t((lm[j] & 63) | ((lm[j + 4] >> 4) << 6));
        s[j + 8] = uint8_t((ls[j + 4] & 0xF) | ((lm[j + 4] & 0xF) << 4));
    }
    uint8_t* q = out + 16;
    std::memset(q, 0, 128);
    for (int j = 0; j < 8; ++j) {
        const float dl = d * float(ls[j]), ml = dmin * float(lm[j]);
        for (int i = 0; i < 32; ++i) {
            int v = dl > 0.0f ? nearest((x[32 * j + i] + ml) / dl) : 0;
            v = v < 0 ? 0 : (v > 15 ? 15 : v);
            const int e = 32 * j + i, g = e / 64, w = e % 64;
            q[32 * g + (w % 32)] |= uint8_t(w < 32 ? v : (v << 4));
        }
    }
}

// Q2_K: per 16-value sub-block an affine fit with 4-bit scale/min codes, 2-bit codes.
void quant_q2_k(const float* x, uint8_t* out) {
    float sc[16], mn[16];
    for (int j = 0; j < 16; ++j) {
        float lo = x[16 * j], hi = x[16 * j];
        for (int i = 1; i < 16; ++i) { lo = std::fmin(lo, x[16 * j + i]); hi = std::fmax(hi, x[16 * j + i]); }
        if (lo > 0.0f) lo = 0.0f;
        sc[j] = (hi - lo) / 3.0f;
        mn[j] = -lo;
    }
    float msc = 0.0f, mmn = 0.0f;
    for (int j = 0; j < 16; ++j) { msc = std::fmax(msc, sc[j]); mmn = std::fmax(mmn, mn[j]); }
    const uint16_t dh = to_f16(msc / 15.0f), mh = to_f16(mmn / 15.0f);
    const float d = from_f16(dh), dmin = from_f16(mh);
    std::memset(out, 0, 84);
    for (int j = 0; j < 16; ++j) {
        int a = d > 0.0f ? nearest(sc[j] / d) : 0;
        int b = dmin > 0.0f ? nearest(mn[j] / dmin) : 0;
        a = a < 0 ? 0 : (a > 15 ? 15 : a);
        b = b < 0 ? 0 : (b > 15 ? 15 : b);
        out[j] = uint8_t(a | (b << 4));
        const float dl = d * float(a), ml = dmin * float(b);
        for (int i = 0; i < 16; ++i) {
            int v = dl > 0.0f ? nearest((x[16 * j + i] + ml) / dl) : 0;
            v = v < 0 ? 0 : (v > 3 ? 3 : v);
            const int e = 16 * j + i, n = e / 128, r = e % 128, jj = r / 32, w = r % 32;
            out[16 + 32 * n + w] |= uint8_t(v << (2 * jj));
        }
    }
    std::memcpy(out + 80, &dh, 2);
    std::memcpy(out + 82, &mh, 2);
}

uint64_t block_values(int fmt) { return fmt == SM_FMT_Q8_0 ? 32 : 256; }
uint64_t block_bytes(int fmt) {
    switch (fmt) {
        case SM_FMT_Q8_0: return 34;
        case SM_FMT_Q4_K: return 144;
        case SM_FMT_Q2_K: return 84;
    }
    return 0;
}

void quant_block(int fmt, const float* x, uint8_t* out) {
    if (fmt == SM_FMT_Q8_0) quant_q8_0(x, out);
    else if (fmt == SM_FMT_Q4_K) quant_q4_k(x, out);
    else quant_q2_k(x, out);
}

}  // namespace

extern "C" {

void sm_synth_normal_f32(uint64_t seed, uint64_t stream, float sigma, float* out, uint64_t n) {
    parallel_for(n, [=](uint64_t b, uint64_t e) {
        normal_fill(seed, stream, b, e, [&](uint64_t i, double z) { out[i] = float(z * sigma); });
    });
}

void sm_synth_normal_f16(uint64_t seed, uint64_t stream, float sigma, uint16_t* out, uint64_t n) {
    parallel_for(n, [=](uint64_t b, uint64_t e) {
        normal_fill(seed, stream, b, e, [&](uint64_t i, double z) { out[i] = to_f16(float(z * sigma)); });
    });
}

void sm_synth_normal_bf16(uint64_t seed, uint64_t stream, float sigma, uint16_t* out, uint64_t n) {
    parallel_for(n, [=](uint64_t b, uint64_t e) {
        normal_fill(seed, stream, b, e, [&](uint64_t i, double z) { out[i] = to_bf16(float(z * sigma)); });
    });
}

sm_status sm_quantize(sm_format fmt, const float* in, uint64_t rows, uint64_t k, uint8_t* out) {
    const uint64_t bv = block_values(fmt), bb = block_bytes(fmt);
    if (!in || !out || bb == 0 || k % bv != 0) return SM_E_ARGUMENT;
    const uint64_t blocks = rows * (k / bv);
    parallel_for(blocks, [=](uint64_t b, uint64_t e) {
        for (uint64_t i = b; i < e; ++i) quant_block(fmt, in + i * bv, out + i * bb);
    });
    return SM_OK;
}

sm_status sm_synth_quantized(sm_format fmt, uint64_t seed, uint64_t stream, float sigma, uint64_t rows,
                             uint64_t k, uint8_t* out) {
    const uint64_t bv = block_values(fmt), bb = block_bytes(fmt);
    if (!out || bb == 0 || k % bv != 0) return SM_E_ARGUMENT;
    const uint64_t blocks = rows * (k / bv);
    parallel_for(blocks, [=](uint64_t b, uint64_t e) {
        float x[256];
        for (uint64_t i = b; i < e; ++i) {
            normal_fill(seed, stream, i * bv, (i + 1) * bv,
                        [&](uint64_t j, double z) { x[j - i * bv] = float(z * sigma); });
            quant_block(fmt, x, out + i * bb);
        }
    });
    return SM_OK;
}

}  // extern "C"
