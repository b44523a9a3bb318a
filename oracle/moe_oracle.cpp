// CPU oracle for the Prefill MoE layer — TEST INFRASTRUCTURE ONLY (see moe_oracle.h).
//
// Compiled with -ffp-contract=off: every fused multiply-add below is an explicit std::fma,
// and every other float operation rounds separately, so the results are a fixed function of
// the inputs that the GPU kernels must reproduce bit for bit where the stage is integer/exact.
#include "moe_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <limits>
#include <vector>

namespace {

inline uint32_t fbits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }
inline float bitsf(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint16_t rd16(const uint8_t* p) { return uint16_t(p[0] | (p[1] << 8)); }

constexpr uint32_t kWave = 32;            // reference SIMD-group width (moe.metal:17)
constexpr float kWeightFloor = 6.103515625e-5f;  // 2^-14, params.h:52, moe.metal:80
constexpr uint32_t kCountTile = 256;      // grouping count tile, prefill_moe.metal:52
constexpr uint32_t kExpertTile = 64;      // expert tile rows, prefill_moe.metal:171-173
constexpr uint32_t kPlanExperts = 512;    // PfPlan arrays, prefill_moe.metal:23-33
constexpr size_t kPlanSlotBytes = 6400;   // prefill_moe_grouping.hpp:17

struct Plan {  // PfPlan, prefill_moe.metal:23-33 (6180 bytes)
    uint32_t n_groups, n_entries, n_miss, skip, n_tiles, bad, pad[2];
    int32_t grp_e[kPlanExperts];
    int32_t grp_res[kPlanExperts];
    int32_t grp_start[kPlanExperts + 1];
};
static_assert(sizeof(Plan) == 6180, "PfPlan host layout");
static_assert(offsetof(Plan, grp_e) == 32 && offsetof(Plan, grp_res) == 2080 &&
              offsetof(Plan, grp_start) == 4128, "PfPlan field offsets");

// ---------------------------------------------------------------------------------------
// exp: Cody & Waite argument reduction (two-constant ln 2 split) followed by a degree-7
// Taylor polynomial on |r| <= ln2/2, evaluated by Horner with explicit fma, then an exact
// power-of-two scale. Every step is a correctly rounded IEEE operation.
// ---------------------------------------------------------------------------------------
float exp_cw(float x) {
    if (std::isnan(x)) return x;
    if (x > 88.72283935546875f) return std::numeric_limits<float>::infinity();
    if (x < -104.0f) return 0.0f;
    const float n = std::nearbyint(x * 1.44269502162933349609375f);  // log2(e) rounded to f32
    float r = std::fma(-n, 0.693145751953125f, x);       // ln2 high part (exact in 16 bits)
    r = std::fma(-n, 1.428606765330187045e-06f, r);      // ln2 low part
    float p = 1.98412698412698412698e-4f;                // 1/5040
    p = std::fma(p, r, 1.38888888888888888889e-3f);      // 1/720
    p = std::fma(p, r, 8.33333333333333333333e-3f);      // 1/120
    p = std::fma(p, r, 4.16666666666666666667e-2f);      // 1/24
    p = std::fma(p, r, 1.66666666666666666667e-1f);      // 1/6
    p = std::fma(p, r, 0.5f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    return std::ldexp(p, int(n));
}

uint16_t f32_to_f16(float f) {  // IEEE binary16, round to nearest even
    const uint32_t x = fbits(f);
    const uint16_t sign = uint16_t((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return uint16_t(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return uint16_t(sign | 0x7c00u);  // >= 65520 rounds to inf
    if (ax >= 0x38800000u) {  // normal half
        uint32_t h = ((((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13));
        const uint32_t rem = ax & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
        return uint16_t(sign | h);
    }
    if (ax <= 0x33000000u) return sign;  // <= 2^-25 rounds to zero (tie to even)
    const uint32_t e = ax >> 23;
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return uint16_t(sign | h);
}

float f16_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bitsf(sign);
        return (sign ? -1.0f : 1.0f) * std::ldexp(float(m), -24);
    }
    if (e == 31) return bitsf(sign | 0x7f800000u | (m << 13));
    return bitsf(sign | ((e + 112u) << 23) | (m << 13));
}

float bf16_to_f32(uint16_t b) { return bitsf(uint32_t(b) << 16); }

// half_sat, common/math.h:33-40: F32 subnormals -> +0, NaN -> 0x7e00, clamp to +-65504.
uint16_t half_sat(float x) {
    const uint32_t b = fbits(x);
    if ((b & 0x7f800000u) == 0u && (b & 0x007fffffu) != 0u) return 0;
    if (std::isnan(x)) return 0x7e00;
    return f32_to_f16(std::fmin(std::fmax(x, -65504.0f), 65504.0f));
}

float silu(float x) { return x / (1.0f + exp_cw(-x)); }        // math.h:10-12
float sigmoid(float x) { return 1.0f / (1.0f + exp_cw(-x)); }  // math.h:6-8

// Q4_K 6-bit scale/min unpacking, dequant.hpp:162-170.
inline void scale_min_k4(int j, const uint8_t* q, uint8_t& d, uint8_t& m) {
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = uint8_t((q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4));
        m = uint8_t((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

// One dequantized value (F32, before the single F16 rounding) at index k of a row.
float value_f32(int fmt, const uint8_t* row, uint64_t k) {
    switch (fmt) {
        case OR_FMT_Q8_0: {  // dequant.hpp:81-86: d * q
            const uint8_t* b = row + (k / 32) * 34;
            return f16_to_f32(rd16(b)) * float(int8_t(b[2 + k % 32]));
        }
        case OR_FMT_Q4_K: {  // dequant.hpp:172-190: d*sc*q - dmin*m
            const uint8_t* b = row + (k / 256) * 144;
            const uint32_t e = uint32_t(k % 256), g = e / 64, w = e % 64;
            const uint8_t byte = b[16 + g * 32 + (w % 32)];
            const uint32_t q = w < 32 ? (byte & 0x0Fu) : (byte >> 4);
            uint8_t sc, m;
            scale_min_k4(int(2 * g + (w >= 32 ? 1 : 0)), b + 4, sc, m);
            const float d1 = f16_to_f32(rd16(b)) * float(sc);
            const float m1 = f16_to_f32(rd16(b + 2)) * float(m);
            return d1 * float(q) - m1;
        }
        case OR_FMT_Q2_K: {  // ggml dequantize_row_q2_K: d*(sc&15)*q - dmin*(sc>>4)
            const uint8_t* b = row + (k / 256) * 84;
            const uint32_t e = uint32_t(k % 256), n = e / 128, r = e % 128, j = r / 32, w = r % 32;
            const uint32_t q = (b[16 + n * 32 + w] >> (2 * j)) & 3u;
            const uint8_t sc = b[n * 8 + 2 * j + (w >= 16 ? 1 : 0)];
            const float dl = f16_to_f32(rd16(b + 80)) * float(sc & 0xF);
            const float ml = f16_to_f32(rd16(b + 82)) * float(sc >> 4);
            return dl * float(q) - ml;
        }
        case OR_FMT_F16:
            return f16_to_f32(rd16(row + 2 * k));
        case OR_FMT_BF16:
            return bf16_to_f32(rd16(row + 2 * k));
    }
    return std::numeric_limits<float>::quiet_NaN();
}

// F16-rounded dequantized value as a float (the operand the expert tiles multiply).
inline float value_h(int fmt, const uint8_t* row, uint64_t k) {
    return f16_to_f32(f32_to_f16(value_f32(fmt, row, k)));
}

uint64_t row_bytes(int fmt, uint64_t k) {
    switch (fmt) {
        case OR_FMT_Q8_0: return k % 32 ? 0 : k / 32 * 34;
        case OR_FMT_Q4_K: return k % 256 ? 0 : k / 256 * 144;
        case OR_FMT_Q2_K: return k % 256 ? 0 : k / 256 * 84;
        case OR_FMT_F16:
        case OR_FMT_BF16: return 2 * k;
    }
    return 0;
}

void dequant_matrix(int fmt, const uint8_t* base, uint32_t rows, uint32_t k, float* out) {
    const uint64_t rb = row_bytes(fmt, k);
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t c = 0; c < k; ++c) out[uint64_t(r) * k + c] = value_h(fmt, base + r * rb, c);
}

int plan_group_of(const Plan& p, uint32_t a) {
    // grp_start is ascending; the group is the last start <= a.
    int lo = 0, hi = int(p.n_groups) - 1;
    if (p.n_groups == 0 || a >= uint32_t(p.grp_start[p.n_groups])) return -1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) / 2;
        if (uint32_t(p.grp_start[mid]) <= a) lo = mid; else hi = mid - 1;
    }
    return lo;
}

}  // namespace

extern "C" {

float or_exp(float x) { return exp_cw(x); }
uint16_t or_f32_to_f16(float x) { return f32_to_f16(x); }
float or_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
uint16_t or_half_sat(float x) { return half_sat(x); }
float or_silu(float x) { return silu(x); }
float or_sigmoid(float x) { return sigmoid(x); }
uint64_t or_row_bytes(int fmt, uint64_t k) { return row_bytes(fmt, k); }

int or_dequant(int fmt, const uint8_t* blocks, uint64_t n, uint16_t* out) {
    if (row_bytes(fmt, n) == 0) return -1;
    for (uint64_t i = 0; i < n; ++i) out[i] = f32_to_f16(value_f32(fmt, blocks, i));
    return 0;
}

// Route: softmax over E in the reference's 32-lane order, then k rounds of a lane-local
// strict-greater scan and a 5-step xor butterfly where the larger value wins and equal
// values go to the lower expert id (moe.metal:28-86). Generalised to any E <= 512 by
// padding lane slots past E; pads take no part in the sums and are never selectable.
int or_route(const float* logits, uint32_t rows, uint32_t E, uint32_t K, int divide,
             int32_t* ids, float* weights) {
    if (rows == 0 || E == 0 || E > 512 || K == 0 || K > 32 || K > E) return -1;
    const uint32_t nv = (E + kWave - 1) / kWave;
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < int64_t(rows); ++t) {
        const float* row = logits + uint64_t(t) * E;
        float v[kWave][16];
        float lane_max[kWave];
        for (uint32_t L = 0; L < kWave; ++L) {
            float m = -std::numeric_limits<float>::infinity();
            for (uint32_t i = 0; i < nv; ++i) {
                const uint32_t idx = L + kWave * i;
                v[L][i] = idx < E ? row[idx] : -std::numeric_limits<float>::infinity();
                m = std::fmax(m, v[L][i]);
            }
            lane_max[L] = m;
        }
        for (uint32_t off = 16; off; off >>= 1) {
            float prev[kWave];
            std::memcpy(prev, lane_max, sizeof prev);
            for (uint32_t L = 0; L < kWave; ++L) lane_max[L] = std::fmax(prev[L], prev[L ^ off]);
        }
        const float mx = lane_max[0];
        float lane_sum[kWave];
        for (uint32_t L = 0; L < kWave; ++L) {
            float s = 0.0f;
            for (uint32_t i = 0; i < nv; ++i) {
                if (L + kWave * i >= E) continue;
                v[L][i] = exp_cw(v[L][i] - mx);
                s = s + v[L][i];
            }
            lane_sum[L] = s;
        }
        for (uint32_t off = 16; off; off >>= 1) {
            float prev[kWave];
            std::memcpy(prev, lane_sum, sizeof prev);
            for (uint32_t L = 0; L < kWave; ++L) lane_sum[L] = prev[L] + prev[L ^ off];
        }
        const float recip = 1.0f / lane_sum[0];
        for (uint32_t L = 0; L < kWave; ++L)
            for (uint32_t i = 0; i < nv; ++i) {
                if (L + kWave * i >= E) { v[L][i] = -std::numeric_limits<float>::infinity(); continue; }
                v[L][i] = v[L][i] * recip;
                if (std::isnan(v[L][i])) v[L][i] = -std::numeric_limits<float>::max();
            }
        float sel_sum[kWave] = {};
        float selected[kWave] = {};
        for (uint32_t rank = 0; rank < K; ++rank) {
            float best[kWave];
            int32_t who[kWave];
            for (uint32_t L = 0; L < kWave; ++L) {
                best[L] = v[L][0];
                who[L] = int32_t(L);
                for (uint32_t i = 1; i < nv; ++i)
                    if (v[L][i] > best[L]) { best[L] = v[L][i]; who[L] = int32_t(L + kWave * i); }
            }
            for (uint32_t off = 16; off; off >>= 1) {
                float pb[kWave];
                int32_t pw[kWave];
                std::memcpy(pb, best, sizeof pb);
                std::memcpy(pw, who, sizeof pw);
                for (uint32_t L = 0; L < kWave; ++L) {
                    const float o = pb[L ^ off];
                    const int32_t oe = pw[L ^ off];
                    if (o > pb[L] || (o == pb[L] && oe < pw[L])) { best[L] = o; who[L] = oe; }
                    else { best[L] = pb[L]; who[L] = pw[L]; }
                }
            }
            const uint32_t e = uint32_t(who[0]);
            ids[uint64_t(t) * K + rank] = int32_t(e);
            v[e & 31u][e / kWave] = -std::numeric_limits<float>::infinity();
            sel_sum[e & 31u] = sel_sum[e & 31u] + best[0];
            selected[rank] = best[0];
        }
        for (uint32_t off = 16; off; off >>= 1) {
            float prev[kWave];
            std::memcpy(prev, sel_sum, sizeof prev);
            for (uint32_t L = 0; L < kWave; ++L) sel_sum[L] = prev[L] + prev[L ^ off];
        }
        const float ssum = std::fmax(sel_sum[0], kWeightFloor);
        const float inv = 1.0f / ssum;
        for (uint32_t r = 0; r < K; ++r)
            weights[uint64_t(t) * K + r] = divide ? selected[r] / ssum : selected[r] * inv;
    }
    return 0;
}

// Grouping: counts -> exclusive prefix in expert-id order -> stable fill in entry order;
// a histogram row is the fill cursor at its 256-entry tile's start; groups are the
// experts with a non-zero count in ascending id order; tiles are 64-entry chunks of each
// group (pf_sort_eq_host_grouping.mm:192-253).
int or_grouping(const int32_t* ids, uint32_t rows, uint32_t K, uint32_t E, uint32_t* hist,
                uint8_t* plan_slot, uint32_t* tiles, uint32_t* n_tiles_out, int32_t* src,
                int32_t* dst) {
    if (rows == 0 || K == 0 || E == 0 || E > kPlanExperts) return -1;
    const uint64_t N = uint64_t(rows) * K;
    if (N > 0x7fffffffu) return -1;
    const uint64_t n_count_tiles = (N + kCountTile - 1) / kCountTile;
    std::vector<uint32_t> count(E, 0);
    uint32_t bad = 0;
    for (uint64_t i = 0; i < N; ++i) {
        if (ids[i] >= 0 && uint32_t(ids[i]) < E) ++count[uint32_t(ids[i])]; else ++bad;
    }
    std::vector<uint32_t> first(E);
    uint32_t total = 0;
    for (uint32_t e = 0; e < E; ++e) { first[e] = total; total += count[e]; }
    std::vector<uint32_t> cursor = first;
    for (uint64_t i = 0; i < N; ++i) { src[i] = -1; dst[i] = -1; }
    for (uint64_t tile = 0; tile < n_count_tiles; ++tile) {
        for (uint32_t e = 0; e < E; ++e) hist[tile * E + e] = cursor[e];
        const uint64_t end = std::min<uint64_t>(N, (tile + 1) * kCountTile);
        for (uint64_t i = tile * kCountTile; i < end; ++i) {
            if (ids[i] < 0 || uint32_t(ids[i]) >= E) continue;
            const uint32_t slot = cursor[uint32_t(ids[i])]++;
            src[slot] = int32_t(i / K);
            dst[slot] = int32_t(i);
        }
    }
    std::memset(plan_slot, 0, kPlanSlotBytes);
    Plan p;
    std::memset(&p, 0, sizeof p);
    for (uint32_t g = 0; g < kPlanExperts; ++g) { p.grp_e[g] = -1; p.grp_res[g] = -1; }
    p.n_entries = uint32_t(N);
    p.bad = bad;
    uint32_t nt = 0;
    for (uint32_t e = 0; e < E; ++e) {
        if (count[e] == 0) continue;
        const uint32_t g = p.n_groups++;
        p.grp_e[g] = int32_t(e);
        p.grp_res[g] = 1;  // full residency: every group is resident
        p.grp_start[g] = int32_t(first[e]);
        for (uint32_t j = 0; j < (count[e] + kExpertTile - 1) / kExpertTile; ++j) {
            tiles[2 * nt] = g;
            tiles[2 * nt + 1] = first[e] + kExpertTile * j;
            ++nt;
        }
    }
    p.grp_start[p.n_groups] = int32_t(total);
    p.n_tiles = nt;
    p.n_miss = 0;
    p.skip = 1;
    std::memcpy(plan_slot, &p, sizeof p);
    if (n_tiles_out) *n_tiles_out = nt;
    return 0;
}

int or_gather(const uint16_t* x, uint32_t rows, uint32_t d, const int32_t* src, uint32_t n_valid,
              uint16_t* xs) {
    for (uint32_t a = 0; a < n_valid; ++a) {
        if (src[a] < 0 || uint32_t(src[a]) >= rows) return -1;
        std::memcpy(xs + uint64_t(a) * d, x + uint64_t(src[a]) * d, size_t(d) * 2);
    }
    return 0;
}

int or_router_ref(const uint16_t* x, const float* w, uint32_t rows, uint32_t d, uint32_t E,
                  double* logits) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < int64_t(rows); ++t) {
        std::vector<double> xr(d);
        for (uint32_t k = 0; k < d; ++k) xr[k] = f16_to_f32(x[uint64_t(t) * d + k]);
        for (uint32_t e = 0; e < E; ++e) {
            double s = 0.0;
            const float* wr = w + uint64_t(e) * d;
            for (uint32_t k = 0; k < d; ++k) s += xr[k] * double(wr[k]);
            logits[uint64_t(t) * E + e] = s;
        }
    }
    return 0;
}

int or_gate_up_ref(int fmt, const uint16_t* xs, uint32_t d, uint32_t I, const uint8_t* plan_slot,
                   const uint8_t* w_gate, const uint8_t* w_up, uint64_t stride,
                   const uint32_t* entries, uint32_t n_sel, double* g, double* u, uint16_t* eh) {
    Plan p;
    std::memcpy(&p, plan_slot, sizeof p);
    const uint64_t rb = row_bytes(fmt, d);
    if (rb == 0) return -1;
    std::vector<int> expert(n_sel);
    for (uint32_t s = 0; s < n_sel; ++s) {
        const int grp = plan_group_of(p, entries[s]);
        if (grp < 0) return -2;
        expert[s] = p.grp_e[grp];
    }
    std::vector<int> experts_used(expert);
    std::sort(experts_used.begin(), experts_used.end());
    experts_used.erase(std::unique(experts_used.begin(), experts_used.end()), experts_used.end());
#pragma omp parallel for schedule(dynamic)
    for (int64_t ui = 0; ui < int64_t(experts_used.size()); ++ui) {
        const int e = experts_used[ui];
        std::vector<float> wg(uint64_t(I) * d), wu(uint64_t(I) * d);
        dequant_matrix(fmt, w_gate + uint64_t(e) * stride, I, d, wg.data());
        dequant_matrix(fmt, w_up + uint64_t(e) * stride, I, d, wu.data());
        std::vector<double> xr(d);
        for (uint32_t s = 0; s < n_sel; ++s) {
            if (expert[s] != e) continue;
            for (uint32_t k = 0; k < d; ++k) xr[k] = f16_to_f32(xs[uint64_t(entries[s]) * d + k]);
            for (uint32_t j = 0; j < I; ++j) {
                double sg = 0.0, su = 0.0;
                const float* gr = wg.data() + uint64_t(j) * d;
                const float* ur = wu.data() + uint64_t(j) * d;
                for (uint32_t k = 0; k < d; ++k) { sg += xr[k] * double(gr[k]); su += xr[k] * double(ur[k]); }
                g[uint64_t(s) * I + j] = sg;
                u[uint64_t(s) * I + j] = su;
                eh[uint64_t(s) * I + j] = half_sat(silu(float(sg)) * float(su));
            }
        }
    }
    return 0;
}

int or_down_ref(int fmt, const uint16_t* eh, uint32_t d, uint32_t I, const uint8_t* plan_slot,
                const uint8_t* w_down, uint64_t stride, const uint32_t* entries, uint32_t n_sel,
                double* out) {
    Plan p;
    std::memcpy(&p, plan_slot, sizeof p);
    if (row_bytes(fmt, I) == 0) return -1;
    std::vector<int> expert(n_sel);
    for (uint32_t s = 0; s < n_sel; ++s) {
        const int grp = plan_group_of(p, entries[s]);
        if (grp < 0) return -2;
        expert[s] = p.grp_e[grp];
    }
    std::vector<int> experts_used(expert);
    std::sort(experts_used.begin(), experts_used.end());
    experts_used.erase(std::unique(experts_used.begin(), experts_used.end()), experts_used.end());
#pragma omp parallel for schedule(dynamic)
    for (int64_t ui = 0; ui < int64_t(experts_used.size()); ++ui) {
        const int e = experts_used[ui];
        std::vector<float> wd(uint64_t(d) * I);
        dequant_matrix(fmt, w_down + uint64_t(e) * stride, d, I, wd.data());
        std::vector<double> hr(I);
        for (uint32_t s = 0; s < n_sel; ++s) {
            if (expert[s] != e) continue;
            for (uint32_t j = 0; j < I; ++j) hr[j] = f16_to_f32(eh[uint64_t(entries[s]) * I + j]);
            for (uint32_t c = 0; c < d; ++c) {
                double acc = 0.0;
                const float* wr = wd.data() + uint64_t(c) * I;
                for (uint32_t j = 0; j < I; ++j) acc += hr[j] * double(wr[j]);
                out[uint64_t(s) * d + c] = acc;
            }
        }
    }
    return 0;
}

int or_shared_ref(int fmt, const uint16_t* x, uint32_t d, uint32_t Is, const uint8_t* w_gate,
                  const uint8_t* w_up, const uint8_t* w_down, const uint8_t* gate_vec,
                  const uint32_t* tokens, uint32_t n_sel, uint16_t* hidden, double* out,
                  double* gl) {
    if (fmt != OR_FMT_F16 && fmt != OR_FMT_BF16) return -1;
    std::vector<float> wg(uint64_t(Is) * d), wu(uint64_t(Is) * d), wd(uint64_t(d) * Is), gv(d);
    dequant_matrix(fmt, w_gate, Is, d, wg.data());
    dequant_matrix(fmt, w_up, Is, d, wu.data());
    dequant_matrix(fmt, w_down, d, Is, wd.data());
    dequant_matrix(fmt, gate_vec, 1, d, gv.data());
#pragma omp parallel for schedule(dynamic)
    for (int64_t s = 0; s < int64_t(n_sel); ++s) {
        std::vector<double> xr(d), hr(Is);
        for (uint32_t k = 0; k < d; ++k) xr[k] = f16_to_f32(x[uint64_t(tokens[s]) * d + k]);
        double sgl = 0.0;
        for (uint32_t k = 0; k < d; ++k) sgl += xr[k] * double(gv[k]);
        gl[s] = sgl;
        for (uint32_t j = 0; j < Is; ++j) {
            double sg = 0.0, su = 0.0;
            for (uint32_t k = 0; k < d; ++k) {
                sg += xr[k] * double(wg[uint64_t(j) * d + k]);
                su += xr[k] * double(wu[uint64_t(j) * d + k]);
            }
            const uint16_t h = half_sat(silu(float(sg)) * float(su));
            hidden[uint64_t(s) * Is + j] = h;
            hr[j] = f16_to_f32(h);
        }
        for (uint32_t c = 0; c < d; ++c) {
            double acc = 0.0;
            for (uint32_t j = 0; j < Is; ++j) acc += hr[j] * double(wd[uint64_t(c) * Is + j]);
            out[uint64_t(s) * d + c] = acc;
        }
    }
    return 0;
}

// SwiGLU pair, prefill_moe.metal:1185-1199: half_sat(silu(g) * u).
int or_swiglu(const float* gate, const float* up, uint64_t n, uint16_t* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = half_sat(silu(gate[i]) * up[i]);
    return 0;
}

// Combine, prefill_moe.metal:1213-1221: rank-ordered fma from s = 0, then the gated
// shared term as one more fma.
int or_combine(const float* parts, const float* w, const float* shared, const float* gl,
               uint32_t rows, uint32_t K, uint32_t d, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t t = 0; t < int64_t(rows); ++t) {
        const float gate = (shared && gl) ? sigmoid(gl[t]) : 0.0f;
        for (uint32_t c = 0; c < d; ++c) {
            float s = 0.0f;
            for (uint32_t r = 0; r < K; ++r)
                s = std::fma(w[uint64_t(t) * K + r], parts[(uint64_t(t) * K + r) * d + c], s);
            out[uint64_t(t) * d + c] = (shared && gl) ? std::fma(shared[uint64_t(t) * d + c], gate, s) : s;
        }
    }
    return 0;
}

}  // extern "C"

// Internal entry points for the timed CPU baseline (cpu_baseline.cpp).
namespace oracle_internal {
void dequant_matrix_f32(int fmt, const uint8_t* base, uint32_t rows, uint32_t k, float* out) {
    dequant_matrix(fmt, base, rows, k, out);
}
float silu_f(float x) { return silu(x); }
uint16_t half_sat_f(float x) { return half_sat(x); }
float f16_f(uint16_t h) { return f16_to_f32(h); }
}  // namespace oracle_internal

// =========================================================================================
// Decode-side MoE (the reference's Window MoE over T <= 8 rows).
// =========================================================================================
namespace {

struct DecodePlanLayout {  // MoePlan, moe.metal:101-111 (1620 bytes)
    uint32_t n_groups, n_entries, n_miss, skip;
    int32_t grp_e[80], grp_res[80], grp_start[81], ent_tok[80], ent_dst[80];
};
static_assert(sizeof(DecodePlanLayout) == 1620, "MoePlan host layout");

constexpr uint32_t kQ81 = 36;  // half d, half sum, int8 q[32] (types.h:128-131)

// Sum of 32 lanes as the butterfly leaves it in lane 0: after each xor offset o (16 .. 1) lane
// l holds v[l] + v[l ^ o] of the previous level.
float butterfly32(const float* x) {
    float v[32];
    std::memcpy(v, x, sizeof v);
    for (uint32_t o = 16; o; o >>= 1) {
        float nv[32];
        for (uint32_t l = 0; l < 32; ++l) nv[l] = v[l] + v[l ^ o];
        std::memcpy(v, nv, sizeof v);
    }
    return v[0];
}

// One 32-value weight block b of a row as integer codes and its scales: value i of the block
// is d*sc[i/16]*q[i] - dmin*mn[i/16] (Q8_0: sc = 1, dmin = 0).
struct WBlock {
    int q[32];
    double d, dmin;
    int sc[2], mn[2];
};

void weight_block(int fmt, const uint8_t* row, uint32_t b, WBlock& w) {
    switch (fmt) {
        case OR_FMT_Q8_0: {  // dequant.hpp:81-86
            const uint8_t* p = row + 34u * b;
            w.d = f16_to_f32(rd16(p));
            w.dmin = 0.0;
            w.sc[0] = w.sc[1] = 1;
            w.mn[0] = w.mn[1] = 0;
            for (int i = 0; i < 32; ++i) w.q[i] = int8_t(p[2 + i]);
            break;
        }
        case OR_FMT_Q4_K: {  // dequant.hpp:157-190: sub-block j = values 32j .. 32j+31
            const uint8_t* p = row + 144u * (b / 8);
            const uint32_t j = b % 8;
            uint8_t sc, m;
            scale_min_k4(int(j), p + 4, sc, m);
            w.d = f16_to_f32(rd16(p));
            w.dmin = f16_to_f32(rd16(p + 2));
            w.sc[0] = w.sc[1] = sc;
            w.mn[0] = w.mn[1] = m;
            for (int i = 0; i < 32; ++i) {
                const uint8_t byte = p[16 + 32 * (j / 2) + i];
                w.q[i] = (j & 1) ? byte >> 4 : byte & 0x0F;
            }
            break;
        }
        case OR_FMT_Q2_K: {  // ggml-common.h:298-309 layout, dequantize_row_q2_K values
            const uint8_t* p = row + 84u * (b / 8);
            const uint32_t e0 = 32u * (b % 8), n = e0 / 128, j = (e0 % 128) / 32;
            w.d = f16_to_f32(rd16(p + 80));
            w.dmin = f16_to_f32(rd16(p + 82));
            for (int h = 0; h < 2; ++h) {
                const uint8_t s = p[8 * n + 2 * j + h];
                w.sc[h] = s & 0xF;
                w.mn[h] = s >> 4;
            }
            for (int i = 0; i < 32; ++i) w.q[i] = (p[16 + 32 * n + i] >> (2 * j)) & 3;
            break;
        }
        default:
            std::memset(&w, 0, sizeof w);
    }
}

}  // namespace

extern "C" {

// The decode expert plan (moe.metal:123-210): groups in order of each expert's first
// appearance among the n = rows*top_k route entries; a group's entries are its expert's
// entries in index order, packed after the previous groups'. Built here by walking each first
// appearance's members.
int or_moe_plan(const int32_t* ids, uint32_t rows, uint32_t top_k, uint32_t n_experts,
                const int32_t* resident, float* usage, uint8_t* plan_out) {
    const uint32_t n = rows * top_k;
    if (rows == 0 || top_k == 0 || n > 80 || n_experts == 0) return -1;
    DecodePlanLayout p;
    std::memset(&p, 0, sizeof p);
    bool bad = false;
    for (uint32_t i = 0; i < n; ++i) bad = bad || ids[i] < 0 || uint32_t(ids[i]) >= n_experts;
    if (bad) {  // an empty plan (this build's status bit 1; the reference does not check)
        p.skip = 1;
        std::memcpy(plan_out, &p, sizeof p);
        return 1;
    }
    uint32_t entry = 0;
    for (uint32_t j = 0; j < n; ++j) {
        bool seen = false;
        for (uint32_t i = 0; i < j && !seen; ++i) seen = ids[i] == ids[j];
        if (seen) continue;
        const uint32_t g = p.n_groups++;
        const bool res = resident == nullptr || resident[ids[j]] >= 0;
        p.grp_e[g] = ids[j];
        p.grp_start[g] = int32_t(entry);
        p.grp_res[g] = res ? 1 : 0;
        p.n_miss += res ? 0 : 1;
        for (uint32_t i = j; i < n; ++i)
            if (ids[i] == ids[j]) {
                p.ent_dst[entry] = int32_t(i);
                p.ent_tok[entry] = int32_t(i / top_k);
                ++entry;
            }
    }
    p.grp_start[p.n_groups] = int32_t(entry);
    p.n_entries = n;
    p.skip = p.n_miss == 0 ? 1 : 0;
    if (usage != nullptr)
        for (uint32_t i = 0; i < n; ++i) usage[ids[i]] += 1.0f;
    std::memcpy(plan_out, &p, sizeof p);
    return 0;
}

// The precise Q8_1 quantizer (quantize_q8_1.metal; tests/metal/oracles/q8_1.cpp:56-124): per
// 32-value block, amax = max |x|, d = amax / 127 in F32 and q = round(x / d), half away from
// zero, clamped to +-127 when d is subnormal. Where d rounds to zero although amax is not
// zero, q = round(127 x / amax) of the exact ratio (half away from zero, at most 127). The
// block stores f16(d) and f16 of the values' butterfly sum.
// The F32 quotient is formed in double and rounded once to float: for a quotient of two
// floats that equals the correctly rounded F32 quotient (53 >= 2*24 + 2 bits), so the result
// does not depend on the host's denormal mode.
int or_quantize_q8_1(const float* x, uint32_t rows, uint32_t n, uint8_t* out) {
    if (rows == 0 || n == 0 || n % 32 != 0) return -1;
    const uint32_t nb = n / 32;
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t b = 0; b < nb; ++b) {
            const float* v = x + uint64_t(r) * n + 32u * b;
            uint8_t* blk = out + (uint64_t(r) * nb + b) * kQ81;
            float amax = 0.0f;
            for (int i = 0; i < 32; ++i) {
                if (!std::isfinite(v[i])) return -2;
                amax = std::fmax(amax, std::fabs(v[i]));
            }
            const float d = float(double(amax) / 127.0);
            const uint32_t db = fbits(d);
            const uint16_t hd = f32_to_f16(d), hs = f32_to_f16(butterfly32(v));
            blk[0] = uint8_t(hd);
            blk[1] = uint8_t(hd >> 8);
            blk[2] = uint8_t(hs);
            blk[3] = uint8_t(hs >> 8);
            for (int i = 0; i < 32; ++i) {
                double q = 0.0;
                if (amax != 0.0f) {
                    if (db == 0u) {
                        q = std::min(std::round(127.0 * std::fabs(double(v[i])) / double(amax)), 127.0);
                        if (std::signbit(v[i])) q = -q;
                    } else {
                        q = std::round(double(float(double(v[i]) / double(d))));
                        if ((db & 0x7f800000u) == 0u) q = std::min(std::max(q, -127.0), 127.0);
                    }
                }
                blk[4 + i] = uint8_t(int8_t(int(q)));
            }
        }
    return 0;
}

// Grouped decode mat-vec value in FP64: out[c][r] = sum over the 32-value blocks of row r of
// dx * (d * sum_h sc_h * sum(qw * qx) - dmin * sum_h mn_h * sum(qx)), the exact product of
// the dequantized weights (d*sc*q - dmin*mn) with the Q8_1 codes times dx
// (q8_0_mv.cpp:21-33, q4_k_mv.cpp:26-70 for the split). mag[c][r] (optional) sums the two
// terms' magnitudes per block: the scale of the F32 rounding a GPU accumulation may add.
int or_q81_matvec(int fmt, const uint8_t* w, uint32_t n_out, uint32_t k, const uint8_t* act,
                  uint32_t nc, double* out, double* mag) {
    const uint64_t rb = row_bytes(fmt, k);
    if (rb == 0 || k % 32 != 0 || n_out == 0 || nc == 0 || fmt == OR_FMT_F16 || fmt == OR_FMT_BF16) return -1;
    const uint32_t nb = k / 32;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < int64_t(n_out); ++r) {
        const uint8_t* row = w + uint64_t(r) * rb;
        std::vector<double> acc(nc, 0.0), am(nc, 0.0);
        WBlock wb;
        for (uint32_t b = 0; b < nb; ++b) {
            weight_block(fmt, row, b, wb);
            for (uint32_t c = 0; c < nc; ++c) {
                const uint8_t* ab = act + (uint64_t(c) * nb + b) * kQ81;
                const double dx = f16_to_f32(rd16(ab));
                int64_t s[2] = {0, 0}, t[2] = {0, 0};
                for (int i = 0; i < 32; ++i) {
                    const int qx = int8_t(ab[4 + i]);
                    s[i / 16] += int64_t(wb.q[i]) * qx;
                    t[i / 16] += qx;
                }
                const double sd = wb.d * double(wb.sc[0] * s[0] + wb.sc[1] * s[1]);
                const double sm = wb.dmin * double(wb.mn[0] * t[0] + wb.mn[1] * t[1]);
                acc[c] += dx * (sd - sm);
                am[c] += std::fabs(dx) * (std::fabs(sd) + std::fabs(sm));
            }
        }
        for (uint32_t c = 0; c < nc; ++c) {
            out[uint64_t(c) * n_out + r] = acc[c];
            if (mag) mag[uint64_t(c) * n_out + r] = am[c];
        }
    }
    return 0;
}

// The decode SwiGLU, moe.metal:213-221: silu(g) * u in F32.
int or_swiglu_f32(const float* gate, const float* up, uint64_t n, float* out) {
    for (uint64_t i = 0; i < n; ++i) out[i] = silu(gate[i]) * up[i];
    return 0;
}

// The decode combine, moe.metal:253-274: the first rank's product, fma over the other ranks
// in order, then the gated shared term added as a separately rounded product.
int or_combine_decode(const float* parts, const float* w, const float* shared, const float* gl,
                      uint32_t rows, uint32_t K, uint32_t d, float* out) {
    if (rows == 0 || K == 0 || d == 0) return -1;
    for (uint32_t t = 0; t < rows; ++t) {
        const float* p = parts + uint64_t(t) * K * d;
        const float* wt = w + uint64_t(t) * K;
        const float gs = shared ? sigmoid(gl[t]) : 0.0f;
        for (uint32_t c = 0; c < d; ++c) {
            float s = p[c] * wt[0];
            for (uint32_t r = 1; r < K; ++r) s = std::fma(p[uint64_t(r) * d + c], wt[r], s);
            if (shared) {
                const float term = shared[uint64_t(t) * d + c] * gs;
                s = s + term;
            }
            out[uint64_t(t) * d + c] = s;
        }
    }
    return 0;
}

}  // extern "C"
