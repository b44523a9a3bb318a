/*
 * CPU oracle for the Prefill MoE layer — TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, on the host, every stage of the reference's Prefill MoE path
 * so that tests can check the HIP implementation against it. Only tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load it; the
 * product library never links or calls it.
 *
 * Reference files followed (paths relative to the reference checkout):
 *   route / top-k ......... src/metal/kernels/safe/moe.metal:17-86,
 *                           tests/metal/oracles/moe_route.cpp:27-159
 *   grouping .............. tests/metal/pf_sort_eq_host_grouping.mm:184-253,
 *                           src/metal/kernels/safe/prefill_moe.metal:61-269
 *   gather ................ src/metal/kernels/safe/prefill_moe.metal:271-323
 *   gate/up + SwiGLU ...... src/metal/kernels/safe/prefill_moe.metal:771-997
 *   down .................. src/metal/kernels/safe/prefill_moe.metal:999-1183
 *   SwiGLU / half_sat ..... src/metal/kernels/safe/prefill_moe.metal:1185-1199,
 *                           src/metal/kernels/common/math.h:6-40
 *   combine ............... src/metal/kernels/safe/prefill_moe.metal:1201-1222,
 *                           tests/metal/oracles/moe_combine.cpp:8-57
 *   decode plan ........... src/metal/kernels/safe/moe.metal:101-210
 *   Q8_1 quantizer ........ src/metal/kernels/safe/quantize_q8_1.metal,
 *                           tests/metal/oracles/q8_1.cpp:56-124
 *   Q8_1 mat-vecs ......... tests/metal/oracles/q8_0_mv.cpp:21-106, q4_k_mv.cpp:26-154
 *   decode SwiGLU/combine . src/metal/kernels/safe/moe.metal:213-274
 *   dequant Q8_0 / Q4_K ... include/strata/artifact/dequant.hpp:80-86,157-190,
 *                           src/metal/kernels/prefill_dequant.metal:12-56,341-361
 *   dequant Q2_K .......... third_party/ggml/ggml-common.h:298-309 (layout only; the value
 *                           formula is ggml's published dequantize_row_q2_K at 3cf03257,
 *                           which the reference does not vendor)
 *
 * Parity pins (each function's independent check lives in tests/):
 *   or_exp ........ double-precision exp, <= 2 ulp over a dense sweep; special cases.
 *   or_route ...... reference golden weight bits and tie patterns
 *                   (tests/metal/metal_moe_test.mm:124-141,270-309,605-652), brute-force sort,
 *                   and the reference's own moe_route.cpp built into oracle/_ref.
 *   or_grouping ... reference pattern generators (pf_sort_eq_host_grouping.mm:126-178),
 *                   std::stable_sort, permutation/stability invariants, plan offsets.
 *   or_dequant .... hand-computed known-answer blocks and brute-force code sweeps.
 *   or_combine / or_swiglu ... the reference's moe_combine.cpp / moe_swiglu.cpp in oracle/_ref,
 *                   and a double-precision formula.
 *   GEMM refs ..... FP64 sums of exact products; checked against numpy float64 matmul.
 *   or_moe_plan ... brute-force plan invariants (each entry once, contiguous groups in
 *                   first-appearance order, ascending members) and hand-worked plans.
 *   or_quantize_q8_1 ... the reference's q8_1.cpp in oracle/_ref, bit for bit, over random,
 *                   subnormal, zero and huge blocks.
 *   or_q81_matvec . the reference's q8_0_mv.cpp / q4_k_mv.cpp in oracle/_ref (F32 twins, within
 *                   their rounding) and, exactly, FP64 dots of or_dequant values on weights
 *                   whose dequantized values are exact in F16 (Q8_0, Q4_K, Q2_K).
 *   or_swiglu_f32 / or_combine_decode ... moe_swiglu.cpp / moe_combine.cpp in oracle/_ref.
 *
 * All arrays are host memory. F16 values are passed as their uint16 bit patterns.
 * Functions return 0 on success and a negative value on a shape error.
 */
#ifndef STRATA_MOE_ORACLE_H
#define STRATA_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Weight formats; values match sm_format in include/strata_moe.h. */
enum { OR_FMT_Q8_0 = 1, OR_FMT_Q4_K = 2, OR_FMT_Q2_K = 3, OR_FMT_F16 = 4, OR_FMT_BF16 = 5 };

/* ---- numerics ---- */
float or_exp(float x);
uint16_t or_f32_to_f16(float x);
float or_f16_to_f32(uint16_t h);
uint16_t or_half_sat(float x);
float or_silu(float x);
float or_sigmoid(float x);

/* ---- block formats ---- */
/* Bytes of one weight row of `k` values in `fmt` (0 if k is not a multiple of the block). */
uint64_t or_row_bytes(int fmt, uint64_t k);
/* Dequantize `n_values` consecutive values to F16 bits (values rounded once from F32). */
int or_dequant(int fmt, const uint8_t* blocks, uint64_t n_values, uint16_t* out_f16);

/* ---- route / top-k (moe.metal:17-86) ---- */
int or_route(const float* logits, uint32_t rows, uint32_t n_experts, uint32_t top_k,
             int divide_weights, int32_t* ids, float* weights);

/* ---- grouping (pf_sort_eq_host_grouping.mm:192-253) ----
 * hist: [ceil(N/256)][n_experts] cursor at each 256-entry tile start (u32)
 * plan: 6400-byte slot (PfPlan layout; bytes past 6180 are zero)
 * tiles: uint32 pairs {group, first_entry}; capacity ceil(N/64) + n_experts pairs
 * src/dst: int32 [N]; entries past the valid count are set to -1. */
int or_grouping(const int32_t* ids, uint32_t rows, uint32_t top_k, uint32_t n_experts,
                uint32_t* hist, uint8_t* plan, uint32_t* tiles, uint32_t* n_tiles_out,
                int32_t* src, int32_t* dst);

/* Xs[a,:] = X[src[a],:] for a < n_valid (F16 bits, row width d). */
int or_gather(const uint16_t* x, uint32_t rows, uint32_t d, const int32_t* src,
              uint32_t n_valid, uint16_t* xs);

/* ---- F32 router GEMM reference: logits[t,e] = sum_k x[t,k]*W[e,k] in double ---- */
int or_router_ref(const uint16_t* x, const float* w, uint32_t rows, uint32_t d,
                  uint32_t n_experts, double* logits);

/* ---- grouped expert products, FP64 over F16-rounded dequantized weights ----
 * Weights are stacked per expert: expert e's gate rows start at w_gate + e*expert_stride.
 * gate/up rows are [I][d]; down rows are [d][I].
 * `entries` lists the grouped entry indices a to evaluate (n_sel of them); the expert of
 * entry a is grp_e of the plan group containing a.
 * gate/up: g,u (double, [n_sel][I]) and eh (F16 bits, [n_sel][I]) =
 *          half_sat(silu(float(g)) * float(u)).
 * down:    out (double, [n_sel][d]) = sum_j eh[a,j] * Wd[c,j]. */
int or_gate_up_ref(int fmt, const uint16_t* xs, uint32_t d, uint32_t inter,
                   const uint8_t* plan, const uint8_t* w_gate, const uint8_t* w_up,
                   uint64_t expert_stride, const uint32_t* entries, uint32_t n_sel,
                   double* g, double* u, uint16_t* eh);
int or_down_ref(int fmt, const uint16_t* eh, uint32_t d, uint32_t inter,
                const uint8_t* plan, const uint8_t* w_down, uint64_t expert_stride,
                const uint32_t* entries, uint32_t n_sel, double* out);

/* Dense shared expert on selected tokens:
 * hidden (F16 bits, [n_sel][Is]) = half_sat(silu(float(x.Gs)) * float(x.Us)) with FP64 dots,
 * out (double, [n_sel][d]) = hidden . Ds, gl (double, [n_sel]) = x . g. */
int or_shared_ref(int fmt, const uint16_t* x, uint32_t d, uint32_t shared_ff,
                  const uint8_t* w_gate, const uint8_t* w_up, const uint8_t* w_down,
                  const uint8_t* gate_vec, const uint32_t* tokens, uint32_t n_sel,
                  uint16_t* hidden, double* out, double* gl);

/* ---- post-ops (exact float restatements) ---- */
int or_swiglu(const float* gate, const float* up, uint64_t n, uint16_t* out);
/* out[t,c] = fma(shared[t,c], sigmoid(gl[t]), sum_r fma(w[t,r], parts[t*k+r,c], .))
 * shared/gl may be NULL (no shared expert): out = ordered sum. */
int or_combine(const float* parts, const float* weights, const float* shared, const float* gl,
               uint32_t rows, uint32_t top_k, uint32_t d, float* out);

/* ---- decode-side MoE (the Window MoE, T <= 8 rows; moe.metal:101-275) ----
 * or_moe_plan: the 1620-byte MoePlan of n = rows*top_k <= 80 entries. resident (per expert,
 *   >= 0 means resident) and usage (+1 per entry) may be NULL. Returns 1 and an empty plan
 *   (skip = 1, everything else zero) when an id is outside [0, n_experts).
 * or_quantize_q8_1: rows x n F32 values (n % 32 == 0, finite) to 36-byte Q8_1 blocks.
 * or_q81_matvec: out/mag [nc][n_out] in FP64 for n_out rows of k values in fmt (Q8_0, Q4_K,
 *   Q2_K) against nc Q8_1 activation rows of k values; mag may be NULL.
 * or_swiglu_f32: out = silu(g) * u in F32. or_combine_decode: the decode combine; shared/gl
 *   may be NULL. */
int or_moe_plan(const int32_t* ids, uint32_t rows, uint32_t top_k, uint32_t n_experts,
                const int32_t* resident, float* usage, uint8_t* plan_out);
int or_quantize_q8_1(const float* x, uint32_t rows, uint32_t n, uint8_t* out);
int or_q81_matvec(int fmt, const uint8_t* w, uint32_t n_out, uint32_t k, const uint8_t* act,
                  uint32_t nc, double* out, double* mag);
int or_swiglu_f32(const float* gate, const float* up, uint64_t n, float* out);
int or_combine_decode(const float* parts, const float* w, const float* shared, const float* gl,
                      uint32_t rows, uint32_t top_k, uint32_t d, float* out);

/* ---- timed CPU baseline of the whole layer (F32 accumulation, OpenMP) ----
 * Stages, in order of stage_us[]: 0 router GEMM, 1 top-k, 2 grouping+gather, 3 shared FFN,
 * 4 gate/up, 5 down, 6 combine. Returns the thread count used (> 0) or < 0 on error.
 * The shared expert is skipped when shared_ff == 0 (then w_sg.. may be NULL). */
int or_cpu_layer(uint32_t rows, uint32_t d, uint32_t n_experts, uint32_t top_k,
                 uint32_t inter, uint32_t shared_ff, int fmt_gu, int fmt_dn, int fmt_sh,
                 const uint16_t* x, const float* w_router,
                 const uint8_t* w_gate, const uint8_t* w_up, uint64_t gu_stride,
                 const uint8_t* w_down, uint64_t dn_stride,
                 const uint8_t* w_sg, const uint8_t* w_su, const uint8_t* w_sd,
                 const uint8_t* g_vec, int n_threads, float* out, double* stage_us);

#ifdef __cplusplus
}
#endif
#endif
