// Timed CPU baseline of the Prefill MoE layer — TEST/BENCH INFRASTRUCTURE ONLY.
//
// The reference has no CPU Prefill-MoE path, so the baseline is this restatement of the
// same stages: F32 accumulation over the same F16-rounded dequantized weights, OpenMP over
// tokens (router, shared, combine) and experts (gate/up, down). This file is compiled with
// -ffast-math so the dot products vectorise; the exact numerics (route, grouping, combine)
// come from moe_oracle.cpp, which is compiled without it.
#include "moe_oracle.h"

#include <omp.h>

#include <chrono>
#include <cstring>
#include <vector>

namespace oracle_internal {
void dequant_matrix_f32(int fmt, const uint8_t* base, uint32_t rows, uint32_t k, float* out);
float silu_f(float x);
uint16_t half_sat_f(float x);
float f16_f(uint16_t h);
}  // namespace oracle_internal

namespace {

using clk = std::chrono::steady_clock;
double us_since(clk::time_point t0) {
    return std::chrono::duration<double, std::micro>(clk::now() - t0).count();
}

// Y[m][n] = X[m][k] . W[n][k]^T for a block of up to 4 rows of X sharing each W row.
inline void dot_rows(const float* X, int m, const float* W, int n, int k, float* Y, int ldy) {
    for (int r0 = 0; r0 < m; r0 += 4) {
        const int rm = m - r0 < 4 ? m - r0 : 4;
        const float* x0 = X + size_t(r0) * k;
        const float* x1 = rm > 1 ? x0 + k : x0;
        const float* x2 = rm > 2 ? x0 + 2 * size_t(k) : x0;
        const float* x3 = rm > 3 ? x0 + 3 * size_t(k) : x0;
        for (int j = 0; j < n; ++j) {
            const float* w = W + size_t(j) * k;
            float s0 = 0, s1 = 0, s2 = 0, s3 = 0;
            for (int i = 0; i < k; ++i) {
                const float wi = w[i];
                s0 += x0[i] * wi; s1 += x1[i] * wi; s2 += x2[i] * wi; s3 += x3[i] * wi;
            }
            float s[4] = {s0, s1, s2, s3};
            for (int r = 0; r < rm; ++r) Y[size_t(r0 + r) * ldy + j] = s[r];
        }
    }
}

}  // namespace

extern "C" int or_cpu_layer(uint32_t T, uint32_t d, uint32_t E, uint32_t K, uint32_t I,
                            uint32_t Is, int fmt_gu, int fmt_dn, int fmt_sh, const uint16_t* x,
                            const float* w_router, const uint8_t* w_gate, const uint8_t* w_up,
                            uint64_t gu_stride, const uint8_t* w_down, uint64_t dn_stride,
                            const uint8_t* w_sg, const uint8_t* w_su, const uint8_t* w_sd,
                            const uint8_t* g_vec, int n_threads, float* out, double* stage_us) {
    using namespace oracle_internal;
    if (n_threads > 0) omp_set_num_threads(n_threads);
    const int threads = omp_get_max_threads();
    const uint64_t N = uint64_t(T) * K;

    // 0: router GEMM (F16 activations widened to F32, F32 weights).
    auto t0 = clk::now();
    std::vector<float> xf(uint64_t(T) * d), logits(uint64_t(T) * E);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < int64_t(T) * d; ++i) xf[i] = f16_f(x[i]);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t t0b = 0; t0b < int64_t(T); t0b += 16) {
        const int m = int(T - t0b < 16 ? T - t0b : 16);
        dot_rows(xf.data() + t0b * d, m, w_router, int(E), int(d), logits.data() + t0b * E, int(E));
    }
    stage_us[0] = us_since(t0);

    // 1: softmax top-k, divide-mode weights.
    t0 = clk::now();
    std::vector<int32_t> ids(N);
    std::vector<float> rw(N);
    if (or_route(logits.data(), T, E, K, 1, ids.data(), rw.data()) != 0) return -1;
    stage_us[1] = us_since(t0);

    // 2: stable grouping and F16 gather.
    t0 = clk::now();
    std::vector<uint32_t> hist(((N + 255) / 256) * E), tiles(2 * ((N + 63) / 64 + E));
    std::vector<uint8_t> plan(6400);
    std::vector<int32_t> src(N), dst(N);
    uint32_t n_tiles = 0;
    if (or_grouping(ids.data(), T, K, E, hist.data(), plan.data(), tiles.data(), &n_tiles,
                    src.data(), dst.data()) != 0)
        return -2;
    uint32_t n_groups, bad;
    std::memcpy(&n_groups, plan.data(), 4);
    std::memcpy(&bad, plan.data() + 20, 4);
    const uint32_t n_valid = uint32_t(N) - bad;
    std::vector<uint16_t> xs(uint64_t(N) * d);
    if (or_gather(x, T, d, src.data(), n_valid, xs.data()) != 0) return -3;
    stage_us[2] = us_since(t0);
    const int32_t* grp_e = reinterpret_cast<const int32_t*>(plan.data() + 32);
    const int32_t* grp_start = reinterpret_cast<const int32_t*>(plan.data() + 4128);

    // 3: shared expert FFN and its sigmoid-gate logit.
    t0 = clk::now();
    std::vector<float> sh, gl;
    if (Is > 0) {
        sh.assign(uint64_t(T) * d, 0.0f);
        gl.assign(T, 0.0f);
        std::vector<float> wg(uint64_t(Is) * d), wu(uint64_t(Is) * d), wd(uint64_t(d) * Is), gv(d);
        dequant_matrix_f32(fmt_sh, w_sg, Is, d, wg.data());
        dequant_matrix_f32(fmt_sh, w_su, Is, d, wu.data());
        dequant_matrix_f32(fmt_sh, w_sd, d, Is, wd.data());
        dequant_matrix_f32(fmt_sh, g_vec, 1, d, gv.data());
#pragma omp parallel for schedule(dynamic, 1)
        for (int64_t tb = 0; tb < int64_t(T); tb += 16) {
            const int m = int(T - tb < 16 ? T - tb : 16);
            std::vector<float> g(size_t(m) * Is), u(size_t(m) * Is), h(size_t(m) * Is);
            dot_rows(xf.data() + tb * d, m, wg.data(), int(Is), int(d), g.data(), int(Is));
            dot_rows(xf.data() + tb * d, m, wu.data(), int(Is), int(d), u.data(), int(Is));
            for (size_t i = 0; i < g.size(); ++i) h[i] = f16_f(half_sat_f(silu_f(g[i]) * u[i]));
            dot_rows(h.data(), m, wd.data(), int(d), int(Is), sh.data() + tb * d, int(d));
            dot_rows(xf.data() + tb * d, m, gv.data(), 1, int(d), gl.data() + tb, 1);
        }
    }
    stage_us[3] = us_since(t0);

    // 4: routed gate/up with SwiGLU, one expert group per task.
    t0 = clk::now();
    std::vector<uint16_t> eh(uint64_t(n_valid) * I);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t grp = 0; grp < int64_t(n_groups); ++grp) {
        const int e = grp_e[grp];
        const uint32_t a0 = uint32_t(grp_start[grp]), a1 = uint32_t(grp_start[grp + 1]);
        std::vector<float> wg(uint64_t(I) * d), wu(uint64_t(I) * d);
        dequant_matrix_f32(fmt_gu, w_gate + uint64_t(e) * gu_stride, I, d, wg.data());
        dequant_matrix_f32(fmt_gu, w_up + uint64_t(e) * gu_stride, I, d, wu.data());
        std::vector<float> xa(size_t(16) * d), g(size_t(16) * I), u(size_t(16) * I);
        for (uint32_t a = a0; a < a1; a += 16) {
            const int m = int(a1 - a < 16 ? a1 - a : 16);
            for (size_t i = 0; i < size_t(m) * d; ++i) xa[i] = f16_f(xs[uint64_t(a) * d + i]);
            dot_rows(xa.data(), m, wg.data(), int(I), int(d), g.data(), int(I));
            dot_rows(xa.data(), m, wu.data(), int(I), int(d), u.data(), int(I));
            for (size_t i = 0; i < size_t(m) * I; ++i)
                eh[uint64_t(a) * I + i] = half_sat_f(silu_f(g[i]) * u[i]);
        }
    }
    stage_us[4] = us_since(t0);

    // 5: routed down, rows stored back in route order through dst.
    t0 = clk::now();
    std::vector<float> parts(N * d, 0.0f);
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t grp = 0; grp < int64_t(n_groups); ++grp) {
        const int e = grp_e[grp];
        const uint32_t a0 = uint32_t(grp_start[grp]), a1 = uint32_t(grp_start[grp + 1]);
        std::vector<float> wd(uint64_t(d) * I);
        dequant_matrix_f32(fmt_dn, w_down + uint64_t(e) * dn_stride, d, I, wd.data());
        std::vector<float> ha(size_t(16) * I), o(size_t(16) * d);
        for (uint32_t a = a0; a < a1; a += 16) {
            const int m = int(a1 - a < 16 ? a1 - a : 16);
            for (size_t i = 0; i < size_t(m) * I; ++i) ha[i] = f16_f(eh[uint64_t(a) * I + i]);
            dot_rows(ha.data(), m, wd.data(), int(d), int(I), o.data(), int(d));
            for (int r = 0; r < m; ++r)
                std::memcpy(parts.data() + uint64_t(dst[a + r]) * d, o.data() + size_t(r) * d, d * 4);
        }
    }
    stage_us[5] = us_since(t0);

    // 6: ordered combine plus gated shared expert.
    t0 = clk::now();
    or_combine(parts.data(), rw.data(), Is ? sh.data() : nullptr, Is ? gl.data() : nullptr, T, K,
               d, out);
    stage_us[6] = us_since(t0);
    return threads;
}
