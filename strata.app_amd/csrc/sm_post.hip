// Post-ops for gfx950: the SwiGLU pair and the deterministic weighted combine.
#include "sm_device.h"
#include "sm_launch.h"

namespace sm {
namespace {

// out = half_sat(silu(gate) * up), elementwise (prefill_moe.metal:1185-1199).
__global__ __launch_bounds__(256) void swiglu_kernel(const float* __restrict__ gate, const float* __restrict__ up,
                                                     _Float16* __restrict__ out, uint64_t n) {
    const uint64_t i = uint64_t(blockIdx.x) * 256u + threadIdx.x;
    if (i < n) out[i] = half_sat(silu(gate[i]) * up[i]);
}

// out[t,c] = fma(shared[t,c], sigmoid(gl[t]), s) with s = 0 then s = fma(w[t,r], parts[t,r,c], s)
// for r = 0..k-1 in rank order (prefill_moe.metal:1201-1222): a per-token gather-reduce in a
// fixed order, no atomics. Each thread owns four consecutive columns of one token. KC > 0: the
// top-k is KC, and every rank's 16 bytes are loaded before the first fma, so a thread keeps KC
// loads in flight; KC = 0: any top-k, one rank at a time.
template <int KC>
__global__ __launch_bounds__(256) void combine_kernel(const float4v* __restrict__ parts,
                                                      const float* __restrict__ weights,
                                                      const float4v* __restrict__ shared,
                                                      const float* __restrict__ gl,
                                                      float4v* __restrict__ out, uint32_t rows,
                                                      uint32_t K, uint32_t v4) {
    const uint64_t idx = uint64_t(blockIdx.x) * 256u + threadIdx.x;
    if (idx >= uint64_t(rows) * v4) return;
    const uint32_t t = uint32_t(idx / v4), c = uint32_t(idx % v4);
    float4v s = {0.0f, 0.0f, 0.0f, 0.0f};
    const float4v* prow = parts + uint64_t(t) * K * v4 + c;
    auto add = [&](float w, const float4v& p) {
        s[0] = __builtin_fmaf(w, p[0], s[0]);
        s[1] = __builtin_fmaf(w, p[1], s[1]);
        s[2] = __builtin_fmaf(w, p[2], s[2]);
        s[3] = __builtin_fmaf(w, p[3], s[3]);
    };
    if constexpr (KC > 0) {
        float4v p[KC];
        float w[KC];
#pragma unroll
        for (int r = 0; r < KC; ++r) p[r] = __builtin_nontemporal_load(prow + uint64_t(r) * v4);
#pragma unroll
        for (int r = 0; r < KC; ++r) w[r] = weights[uint64_t(t) * KC + r];
#pragma unroll
        for (int r = 0; r < KC; ++r) add(w[r], p[r]);
    } else {
        for (uint32_t r = 0; r < K; ++r) add(weights[uint64_t(t) * K + r], prow[uint64_t(r) * v4]);
    }
    if (shared != nullptr) {
        const float gate = sigmoid(gl[t]);
        const float4v sh = shared[idx];
        s[0] = __builtin_fmaf(sh[0], gate, s[0]);
        s[1] = __builtin_fmaf(sh[1], gate, s[1]);
        s[2] = __builtin_fmaf(sh[2], gate, s[2]);
        s[3] = __builtin_fmaf(sh[3], gate, s[3]);
    }
    out[idx] = s;
}

}  // namespace

hipError_t launch_swiglu(const float* gate, const float* up, _Float16* out, uint64_t n, hipStream_t s) {
    const uint64_t blocks = (n + 255) / 256;
    swiglu_kernel<<<dim3(uint32_t(blocks)), 256, 0, s>>>(gate, up, out, n);
    return hipGetLastError();
}

hipError_t launch_combine(const float* parts, const float* weights, const float* shared, const float* gl,
                          float* out, uint32_t rows, uint32_t K, uint32_t d, hipStream_t s) {
    const uint32_t v4 = d / 4;
    const uint64_t blocks = (uint64_t(rows) * v4 + 255) / 256;
    const auto* p = reinterpret_cast<const float4v*>(parts);
    const auto* sh = reinterpret_cast<const float4v*>(shared);
    auto* o = reinterpret_cast<float4v*>(out);
    const dim3 grid(static_cast<uint32_t>(blocks));
    switch (K) {  // the benchmark layers' top-k values
        case 8: combine_kernel<8><<<grid, 256, 0, s>>>(p, weights, sh, gl, o, rows, K, v4); break;
        case 10: combine_kernel<10><<<grid, 256, 0, s>>>(p, weights, sh, gl, o, rows, K, v4); break;
        default: combine_kernel<0><<<grid, 256, 0, s>>>(p, weights, sh, gl, o, rows, K, v4); break;
    }
    return hipGetLastError();
}

}  // namespace sm
