// The softmax top-k of one token per wave or half-wave (gfx950): the body shared by the route
// kernel and the decode layer's front launch.
#pragma once

#include "sm_device.h"
#include "sm_launch.h"

namespace sm {
namespace {

constexpr float kNegInf = -__builtin_inff();
constexpr float kWeightFloor = 6.103515625e-5f;  // 2^-14

// ---------------------------------------------------------------------------------------
// Softmax top-k. The values are the reference's (moe.metal:28-86): its 32-lane SIMD group
// gives lane L the experts L + 32i, sums each lane's exponentials in order of i, and
// finishes the sums by xor butterflies 16..1; each round's argmax prefers the larger value
// and, on equal values, the lower expert id. Two layouts replay it:
//   WAVE (one token per wave, for few tokens: half the serial work per token): the lower
//     half-wave (h = 0) holds slots i < NV of its lane L and the upper half slots NV + i, so
//     lane L's ordered sum is its own NV terms followed by those of lane L + 32;
//   half-wave (two tokens per wave, for many tokens: half the instructions per token):
//     lane L of each half holds all NV slots of its token.
// The butterflies run in each half in the reference's order. The maximum and the argmax do
// not depend on the combination order: a round takes the token's maximum m, then the
// minimum over its lanes' lowest ids holding m. Slots past E are padding: they take no part
// in the sums and hold -inf, so they are never selected (top_k <= E); any NV whose slots cover
// E gives the same results.
// ---------------------------------------------------------------------------------------
// One step of an order-free reduction within 16-lane rows by DPP (CTRL: quad_perm [1,0,3,2]
// = 0xB1, quad_perm [2,3,0,1] = 0x4E, row_ror:4 = 0x124, row_ror:8 = 0x128; after all four
// every lane of a row holds the row's result). Used only where the result does not depend
// on the combination order (the maximum and the minimum).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Lane exchanges without the LDS crossbar: xor 16 swaps the two 16-lane rows of each half-wave
// (v_permlane16_swap), xor 32 the two half-waves (v_permlane32_swap), and xor 4 picks lane
// n ^ 4 from the two row rotations by 4. Which output holds the partner is decided by
// applying the same exchange to the lane numbers once per thread (XorSel), so the result does
// not rest on a reading of the operand order.
struct XorSel {
    bool x16_first, x32_first, x4_ror4;
};
__device__ __forceinline__ XorSel xor_sel(uint32_t lane) {
    const auto r = __builtin_amdgcn_permlane16_swap(lane, lane, false, false);
    const auto q = __builtin_amdgcn_permlane32_swap(lane, lane, false, false);
    const uint32_t ror4 = uint32_t(__builtin_amdgcn_mov_dpp(int(lane), 0x124, 0xF, 0xF, false));
    return XorSel{r[0] == (lane ^ 16u), q[0] == (lane ^ 32u), ror4 == (lane ^ 4u)};
}
__device__ __forceinline__ float xor16(float v, const XorSel& s) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, s.x16_first ? r[0] : r[1]);
}
__device__ __forceinline__ float xor32(float v, const XorSel& s) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, s.x32_first ? r[0] : r[1]);
}
__device__ __forceinline__ float xor4(float v, const XorSel& s) {
    const float a = dpp_f<0x124>(v), b = dpp_f<0x12C>(v);  // row_ror:4, row_ror:12
    return s.x4_ror4 ? a : b;
}
// Butterfly sum over each half-wave's 32 lanes in the reference's xor order.
__device__ __forceinline__ float half_sum(float v, const XorSel& s) {
    v = v + xor16(v, s);
    v = v + dpp_f<0x128>(v);  // xor 8 (row_ror:8)
    v = v + xor4(v, s);
    v = v + dpp_f<0x4E>(v);   // xor 2
    v = v + dpp_f<0xB1>(v);   // xor 1
    return v;
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
    return uint32_t(__builtin_amdgcn_mov_dpp(int(v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ uint32_t xor16(uint32_t v, const XorSel& s) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return s.x16_first ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t xor32(uint32_t v, const XorSel& s) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return s.x32_first ? r[0] : r[1];
}

// Token t of the route (t uniform over its wave, WAVE, or half-wave). ids_lds (may be null)
// receives the token's ids as well, at the same route-order index.
template <int NV, bool WAVE>
__device__ __forceinline__ void topk_token(const float* __restrict__ logits, int32_t* __restrict__ ids,
                                           float* __restrict__ weights, uint32_t rows, uint32_t E, uint32_t K,
                                           int divide, uint32_t* __restrict__ hist, uint32_t t, int32_t* ids_lds) {
    const uint32_t lane = threadIdx.x & 63u, L = lane & 31u, h = WAVE ? lane >> 5 : 0u;
    const uint32_t r = WAVE ? lane : L;  // the token's lane index (round r's id and value)
    const bool live = t < rows;
    const XorSel xs = xor_sel(lane);
    // Expert of slot i of this lane; every load is issued, clamped into the row (a dead token
    // reads row 0), so the loads go out together; padding is set to -inf afterwards.
    auto expert = [&](int i) { return L + 32u * (h * uint32_t(NV) + uint32_t(i)); };
    auto tok_max = [&](float m) {
        m = __builtin_fmaxf(m, dpp_f<0xB1>(m));
        m = __builtin_fmaxf(m, dpp_f<0x4E>(m));
        m = __builtin_fmaxf(m, dpp_f<0x124>(m));
        m = __builtin_fmaxf(m, dpp_f<0x128>(m));
        m = __builtin_fmaxf(m, xor16(m, xs));
        return WAVE ? __builtin_fmaxf(m, xor32(m, xs)) : m;
    };
    auto tok_min = [&](uint32_t m) {
        m = __builtin_elementwise_min(m, dpp_u<0xB1>(m));
        m = __builtin_elementwise_min(m, dpp_u<0x4E>(m));
        m = __builtin_elementwise_min(m, dpp_u<0x124>(m));
        m = __builtin_elementwise_min(m, dpp_u<0x128>(m));
        m = __builtin_elementwise_min(m, xor16(m, xs));
        return WAVE ? __builtin_elementwise_min(m, xor32(m, xs)) : m;
    };
    const float* row = logits + uint64_t(live ? t : 0u) * E;
    float v[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) v[i] = row[expert(i) < E ? expert(i) : E - 1u];
    float mx = kNegInf;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        if (expert(i) >= E) v[i] = kNegInf;
        mx = __builtin_fmaxf(mx, v[i]);
    }
    mx = tok_max(mx);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const float e = exp_cw(v[i] - mx);
        v[i] = expert(i) < E ? e : v[i];
    }
    // Lane L's terms in slot order (WAVE: then lane L + 32's, which hold the later slots).
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) sum = expert(i) < E ? sum + v[i] : sum;
    if (WAVE) {
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const float up = xor32(v[i], xs);
            sum = L + 32u * uint32_t(NV + i) < E ? sum + up : sum;
        }
    }
    sum = half_sum(sum, xs);
    if (WAVE) sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sum)));
    const float recip = 1.0f / sum;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        float p = v[i] * recip;
        if (__builtin_isnan(p)) p = -3.40282346638528859812e+38f;
        v[i] = expert(i) < E ? p : kNegInf;
    }
    // K rounds. Lane r keeps round r's id and value; lane L (both halves in WAVE) adds the
    // winners of its residue L in round order to its share of the selected sum.
    float selected = 0.0f, sel_sum = 0.0f;
    int32_t chosen = -1;
    for (uint32_t rank = 0; rank < K; ++rank) {
        float m = v[0];
#pragma unroll
        for (int i = 1; i < NV; ++i) m = __builtin_fmaxf(m, v[i]);
        m = tok_max(m);
        // The lowest id holding m (m is one of the token's values, so some lane matches).
        uint32_t who = 0xffffffffu;
#pragma unroll
        for (int i = NV - 1; i >= 0; --i) who = v[i] == m ? expert(i) : who;
        who = tok_min(who);
#pragma unroll
        for (int i = 0; i < NV; ++i) v[i] = expert(i) == who ? kNegInf : v[i];
        sel_sum = (who & 31u) == L ? sel_sum + m : sel_sum;
        if (rank == r) {
            selected = m;
            chosen = int32_t(who);
        }
    }
    sel_sum = half_sum(sel_sum, xs);
    const float ssum = __builtin_fmaxf(sel_sum, kWeightFloor);
    const float inv = 1.0f / ssum;
    if (live && r < K) {
        const uint64_t entry = uint64_t(t) * K + r;
        ids[entry] = chosen;
        if (ids_lds != nullptr) ids_lds[entry] = chosen;
        weights[entry] = divide ? selected / ssum : selected * inv;
        if (hist != nullptr && uint32_t(chosen) < E) atomicAdd(&hist[(entry / kCountTile) * E + uint32_t(chosen)], 1u);
    }
}

}  // namespace
}  // namespace sm
