// C-ABI shim over the reference's own CPU twins (tests/metal/oracles/*.cpp in the
// reference checkout), compiled where they lie into oracle/_ref/ by build_ref.sh.
// TEST INFRASTRUCTURE ONLY: tests use it to cross-check this repo's oracle; nothing in the
// product loads it. The twins hard-code k=10, width 2560, E in {256,512}, rows<=8 (combine);
// the mat-vec twins take nc in {1, 2, 4, 8} activation rows.
#include "oracles/moe_combine.hpp"
#include "oracles/moe_route.hpp"
#include "oracles/moe_swiglu.hpp"
#include "oracles/q4_k_mv.hpp"
#include "oracles/q8_0_mv.hpp"
#include "oracles/q8_1.hpp"

#include <cstring>

#include <cstdint>
#include <span>
#include <string>
#include <vector>

extern "C" {

// moe_route_reference (moe_route.cpp:27-159). Writes ids [rows*10] and weight values.
int ref_route(const float* logits, uint32_t rows, uint32_t experts, int divide, int32_t* ids,
              float* weights) {
    std::vector<int32_t> out_ids;
    std::vector<twin::tf> out_w;
    std::string err;
    if (!twin::moe_route_reference(std::span<const float>(logits, size_t(rows) * experts), rows,
                                   experts, divide != 0, out_ids, out_w, err))
        return -1;
    for (size_t i = 0; i < out_ids.size(); ++i) { ids[i] = out_ids[i]; weights[i] = out_w[i].value; }
    return 0;
}

// moe_combine_reference (moe_combine.cpp:8-57): parts [rows][10][2560], out [rows][2560].
int ref_combine(const float* parts, const float* weights, const float* shared, const float* gate,
                uint32_t rows, float* out) {
    std::vector<twin::tf> o;
    std::string err;
    if (!twin::moe_combine_reference(std::span<const float>(parts, size_t(rows) * 10 * 2560),
                                     std::span<const float>(weights, size_t(rows) * 10),
                                     std::span<const float>(shared, size_t(rows) * 2560),
                                     std::span<const float>(gate, rows), rows, o, err))
        return -1;
    for (size_t i = 0; i < o.size(); ++i) out[i] = o[i].value;
    return 0;
}

// moe_swiglu_reference (moe_swiglu.cpp:8-34): n must be a multiple of 640.
int ref_swiglu(const float* gate, const float* up, uint64_t n, float* out) {
    std::vector<twin::tf> o;
    std::string err;
    if (!twin::moe_swiglu_reference(std::span<const float>(gate, n), std::span<const float>(up, n),
                                    o, err))
        return -1;
    for (size_t i = 0; i < o.size(); ++i) out[i] = o[i].value;
    return 0;
}

// quantize_q8_1_reference (q8_1.cpp:56-124): rows x n floats to 36-byte blocks.
int ref_q8_1(const float* x, uint32_t n, uint32_t rows, uint8_t* out) {
    std::vector<Q81> o;
    std::string err;
    if (!twin::quantize_q8_1_reference(std::span<const float>(x, size_t(rows) * n), n, rows, o, err)) return -1;
    std::memcpy(out, o.data(), o.size() * sizeof(Q81));
    return 0;
}

// q8_0_matvec_reference (q8_0_mv.cpp:37-109): out [nc][n_out].
int ref_q80_mv(const uint8_t* w, const uint8_t* act, uint32_t n_in, uint32_t n_out, uint32_t nc, float* out) {
    std::vector<float> o;
    std::string err;
    const size_t nb = n_in / 32;
    if (!twin::q8_0_matvec_reference(std::span<const block_q8_0>(reinterpret_cast<const block_q8_0*>(w), nb * n_out),
                                     std::span<const Q81>(reinterpret_cast<const Q81*>(act), nb * nc), n_in, n_out,
                                     nc, nc, o, err))
        return -1;
    std::memcpy(out, o.data(), o.size() * sizeof(float));
    return 0;
}

// q4_k_matvec_reference (q4_k_mv.cpp:86-158): out [nc][n_out].
int ref_q4k_mv(const uint8_t* w, const uint8_t* act, uint32_t n_in, uint32_t n_out, uint32_t nc, float* out) {
    std::vector<float> o;
    std::string err;
    const size_t nb = n_in / 256;
    if (!twin::q4_k_matvec_reference(std::span<const block_q4_K>(reinterpret_cast<const block_q4_K*>(w), nb * n_out),
                                     std::span<const Q81>(reinterpret_cast<const Q81*>(act), nb * 8 * nc), n_in,
                                     n_out, nc, nc, o, err))
        return -1;
    std::memcpy(out, o.data(), o.size() * sizeof(float));
    return 0;
}
}
