/*
 * strata_moe.h — C ABI of the MI355X Prefill MoE layer (libstrata_moe.so).
 *
 * Drop-in boundary for the reference's Prefill MoE coordinators
 * (namespace strata::metal in the reference checkout). Each reference coordinator has two
 * forms; both are kept:
 *   - a SEGMENT form: sm_encode_*(segment, ...) validates and records launches into an open
 *     segment (the reference's caller-owned `Encoder&` overload). On failure it returns a
 *     non-zero status, records the message, and poisons the segment: the caller must
 *     propagate the failure and call sm_segment_abort(), exactly as the reference requires
 *     callers to propagate `false` so the whole segment is discarded
 *     (include/strata/metal/prefill_moe_full_pipeline.hpp:64-67).
 *   - a STANDALONE form: sm_submit_*(context, stream, ..., err, err_cap) begins a segment,
 *     encodes, then commits or aborts (the reference's `CommandBuffer&` overload,
 *     prefill_moe_full_pipeline.hpp:75-82; encoder.mm:165-231).
 * Nothing reaches the GPU unless every stage of the segment validated: launches are
 * deferred until sm_segment_commit().
 *
 * Buffers are caller-owned device allocations registered with the context (the reference's
 * "owned by this Context" check, context.hpp:405-413). A view is {buffer handle, byte
 * offset, byte length} (the reference's BufferRef, context.hpp:136-233). The library never
 * allocates device memory on the layer path.
 *
 * Status words (u32 in caller device memory) keep the reference's bits
 * (prefill_moe_expert_dispatch.hpp:46-50): bit0 an active expert's weight address is null,
 * bit1 the grouping plan / tile list / destination permutation is invalid. Failing tiles
 * write zeros. The plan's `bad` field counts route ids outside [0, n_experts)
 * (prefill_moe_grouping.hpp:40-41); callers check both after completion.
 *
 * No C++ exception crosses this ABI. All functions are thread-compatible: one segment is
 * used by one thread at a time; distinct segments may be encoded concurrently.
 */
#ifndef STRATA_MOE_H
#define STRATA_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SM_ABI_VERSION 2u

/* Error classes; each maps onto a class of reference validation message
 * (prefill_moe_grouping_dispatch.mm:84-254, prefill_moe_full_pipeline.cpp:451-475). */
typedef enum sm_status {
    SM_OK = 0,
    SM_E_ARGUMENT = 1,  /* null pointer / unknown enum                                   */
    SM_E_SHAPE = 2,     /* unsupported rows, experts, top-k or widths                       */
    SM_E_VIEW = 3,      /* "view is undersized or misaligned"                              */
    SM_E_OWNERSHIP = 4, /* "view is not owned by this context"                              */
    SM_E_ALIAS = 5,     /* "<output> overlaps active <range>"                               */
    SM_E_SEGMENT = 6,   /* segment already failed / committed                               */
    SM_E_FORMAT = 7,    /* weight format not supported for this role                        */
    SM_E_ADDRESS = 8,   /* expert weight address outside declared storage or misaligned    */
    SM_E_DEVICE = 9,    /* HIP runtime error                                                */
    SM_E_FILE = 10      /* model file missing, truncated or malformed                       */
} sm_status;

/* Weight formats (ggml block layouts, third_party/ggml/ggml-common.h:252-338). */
typedef enum sm_format {
    SM_FMT_Q8_0 = 1, /* 34 B / 32 values: f16 d, int8 q[32]                                 */
    SM_FMT_Q4_K = 2, /* 144 B / 256: f16 d, f16 dmin, scales[12], q[128]                   */
    SM_FMT_Q2_K = 3, /* 84 B / 256: scales[16], q[64], f16 d, f16 dmin                     */
    SM_FMT_F16 = 4,  /* shared expert only                                                  */
    SM_FMT_BF16 = 5  /* shared expert only                                                  */
} sm_format;

typedef struct sm_context sm_context;
typedef struct sm_segment sm_segment;

/* A byte range of a registered device allocation; buffer == 0 is the null view. */
typedef struct sm_view {
    uint64_t buffer;
    uint64_t offset;
    uint64_t length;
} sm_view;

/* Layer geometry (the reference hard-codes d=2560, k=10, I=640; here they are parameters).
 * rows: tokens T in this chunk (1..SM_MAX_ROWS); hidden: d (multiple of 256);
 * n_experts: E (1..512); top_k: k (1..min(E,32)); expert_ff: I (multiple of 256 when the
 * down weights are K-quants, else of 64); shared_ff: I_s (0 = no shared expert). */
typedef struct sm_moe_shape {
    uint32_t rows;
    uint32_t hidden;
    uint32_t n_experts;
    uint32_t top_k;
    uint32_t expert_ff;
    uint32_t shared_ff;
} sm_moe_shape;

#define SM_MAX_ROWS 419430u       /* prefill.hpp:15 (kPrefillMaxShaderRows)               */
#define SM_MAX_EXPERTS 512u       /* PfPlan arrays, prefill_moe.metal:23-33              */
#define SM_MAX_TOP_K 32u
#define SM_PLAN_BYTES 6180u       /* prefill_moe_grouping.hpp:18                          */
#define SM_PLAN_SLOT_BYTES 6400u  /* prefill_moe_grouping.hpp:17                          */
#define SM_COUNT_TILE 256u        /* grouping histogram tile, prefill_moe.metal:52        */
#define SM_EXPERT_TILE 64u        /* entries per tile-list tile, prefill_moe.metal:171-173 */

/* Scratch sizes a caller must provide (bytes), given the shape. */
uint64_t sm_histogram_bytes(const sm_moe_shape* shape); /* (ceil(T*k/256) + 1) * E * 4 */
uint64_t sm_tiles_bytes(const sm_moe_shape* shape);     /* (ceil(T*k/64) + E) * 8    */
uint64_t sm_format_row_bytes(sm_format fmt, uint64_t values);

/* ---- context, buffers, segments -------------------------------------------------------- */
sm_status sm_context_create(int device, sm_context** out);
void sm_context_destroy(sm_context* ctx);
/* Registers a device allocation [ptr, ptr+bytes); returns a non-zero handle. */
sm_status sm_buffer_register(sm_context* ctx, void* device_ptr, uint64_t bytes, uint64_t* handle);
sm_status sm_buffer_unregister(sm_context* ctx, uint64_t handle);

sm_status sm_segment_begin(sm_context* ctx, sm_segment** out);
/* Launches every recorded step in order on `hip_stream` (a hipStream_t; NULL = default
 * stream) and frees the segment. Refused (and the segment freed) if any encode failed, and
 * with SM_E_ARGUMENT (nothing launched) if `hip_stream` is capturing a graph: the expert
 * address tables are copied from the context's reusable pinned host ring when the launches
 * run, so a captured graph would replay whatever tables a later commit left there. */
sm_status sm_segment_commit(sm_segment* seg, void* hip_stream);
/* Measurement form of sm_segment_commit (no counterpart in the reference, whose command
 * buffers report GPU start/end times instead): brackets every launch with HIP events on
 * `hip_stream`, waits for the stream, and writes each launch's milliseconds, in recording
 * order, to ms[0..n) and its static label to labels[i] (labels may be NULL). Refused with
 * SM_E_ARGUMENT (segment freed, nothing ran) when cap < sm_segment_launches(seg). */
sm_status sm_segment_commit_timed(sm_segment* seg, void* hip_stream, float* ms, const char** labels, uint32_t cap,
                                  uint32_t* n_launches);
/* Discards every recorded step; nothing ran. Frees the segment. */
void sm_segment_abort(sm_segment* seg);
/* Message of the first failure recorded in the segment ("" if none). */
const char* sm_segment_error(const sm_segment* seg);
uint32_t sm_segment_launches(const sm_segment* seg);

/* ---- stage buffers (mirror the reference's *Buffers structs) ---------------------------- */

/* encode_moe_route (moe_dispatch.cpp:345-379, moe.metal:17-86): logits F32 [T,E] ->
 * ids I32 [T,k], weights F32 [T,k]. */
typedef struct sm_route_buffers {
    sm_view logits;
    sm_view ids;
    sm_view weights;
} sm_route_buffers;

/* PrefillMoeGroupingBuffers (prefill_moe_grouping.hpp:21-39), full residency. */
typedef struct sm_grouping_buffers {
    sm_view ids;              /* I32 [T*k] route ids, token-major                         */
    sm_view mixed_h;          /* F16 [T,d], 16-byte aligned                               */
    sm_view histogram;        /* U32 [ceil(T*k/256) + 1][E]: tile cursors + first slots   */
    sm_view plan;             /* 6400-byte PfPlan slot (tail: stage counters, arrival) */
    sm_view tiles;            /* U32x2 [ceil(T*k/64)+E] {group, first_entry}              */
    sm_view source_rows;      /* I32 [T*k]: grouped entry -> token                        */
    sm_view destination_rows; /* I32 [T*k]: grouped entry -> route index t*k+r            */
    sm_view gathered_rows;    /* F16 [T*k,d]                                              */
    sm_view resident;         /* I32 [layer][E] residency table (tiered mode); null = all resident */
    uint32_t layer;           /* the layer's row of `resident`                             */
} sm_grouping_buffers;

/* PrefillMoeRouteGatherBuffers (prefill_moe_pipeline.hpp:21-33): router GEMM + top-k +
 * grouping + gather. The router is F32 weights [E,d] against F16 activations. */
typedef struct sm_route_gather_buffers {
    sm_view mixed_h;          /* F16 [T,d]                                                */
    sm_view router_weights;   /* F32 [E,d]                                                */
    sm_view logits;           /* F32 [T,E]                                                */
    sm_view route_ids;        /* I32 [T,k]                                                */
    sm_view route_weights;    /* F32 [T,k], divide mode                                   */
    sm_view histogram;
    sm_view plan;
    sm_view tiles;
    sm_view source_rows;
    sm_view destination_rows;
    sm_view gathered_rows;
    sm_view router_bias;      /* F32 [E] added to the logits; null view = none            */
    sm_view resident;         /* as in sm_grouping_buffers                                 */
    uint32_t layer;
} sm_route_gather_buffers;

/* Routed expert weights: a host copy of the model's [layer][E][3] device-address table
 * (gate, up, down; 0 = missing), as the reference keeps it (prefill_moe_expert_dispatch.hpp:
 * 21-22). `layer` selects row layer*E*3 of the n_layers rows, as the reference's `layer`
 * argument does (prefill_moe_expert_dispatch.mm:259-266); that row is validated against the
 * declared storage views (prefill_moe_expert_dispatch.mm:377-448) and copied at commit into
 * `address_snapshot` (device, E*3*8 bytes) before the kernels. */
typedef struct sm_lease_set sm_lease_set;
typedef struct sm_expert_weights {
    const uint64_t* addresses;
    uint32_t n_layers;          /* rows of `addresses` (layer < n_layers)                   */
    uint32_t layer;
    sm_view address_snapshot;
    const sm_view* storage;
    uint32_t n_storage;
    /* Tiered mode (prefill_moe_expert_dispatch.hpp:36-37): addresses inside `slot_arena` are
     * expert-store slots and must be pinned by `leases` for `layer`; an unpinned one makes the
     * kernels report status bit 2 for that expert and zero its rows. Null view / NULL = none. */
    sm_view slot_arena;
    const sm_lease_set* leases;
} sm_expert_weights;

/* PrefillMoeExpertTileBuffers (prefill_moe_expert_dispatch.hpp:20-51). */
typedef struct sm_gate_up_buffers {
    sm_expert_weights weights;
    sm_view gathered_rows;    /* F16 [T*k,d]                                              */
    sm_view plan;
    sm_view tiles;
    sm_view hidden;           /* F16 [T*k,I] = half_sat(silu(x.Wg) * (x.Wu))              */
    sm_view status;           /* U32, cleared on the GPU before use                       */
} sm_gate_up_buffers;

/* PrefillMoeDownTileBuffers (prefill_moe_down_dispatch.hpp:12-38). */
typedef struct sm_down_buffers {
    sm_expert_weights weights;
    sm_view hidden;           /* F16 [T*k,I]                                              */
    sm_view plan;
    sm_view tiles;
    sm_view destinations;     /* I32 [T*k]                                                */
    sm_view parts;            /* F32 [T*k,d] in route order                               */
    sm_view status;           /* U32, distinct from the gate/up status                    */
} sm_down_buffers;

/* PrefillMoeSharedFFNBuffers (prefill_moe_shared_pipeline.hpp:29-42). The gate/up SwiGLU is
 * fused into the projection epilogue, so no F32 gate/up or dequant scratch is needed. */
typedef struct sm_shared_buffers {
    sm_view mixed_h;          /* F16 [T,d]                                                */
    sm_view gate_weights;     /* [I_s][d] in the shared format                            */
    sm_view up_weights;       /* [I_s][d]                                                 */
    sm_view down_weights;     /* [d][I_s]                                                 */
    sm_view gate_vector;      /* [d] sigmoid-gate weights, shared format, 16-byte aligned */
    sm_view hidden;           /* F16 [T,I_s]                                              */
    sm_view output;           /* F32 [T,d]                                                */
    sm_view gate_logit;       /* F32 [T]                                                  */
} sm_shared_buffers;

/* PrefillMoeSwiGLUBuffers / PrefillMoeCombineBuffers (prefill_moe_post.hpp:15-27). */
typedef struct sm_swiglu_buffers {
    sm_view gate;             /* F32 [rows*width]                                         */
    sm_view up;
    sm_view output;           /* F16                                                      */
} sm_swiglu_buffers;

typedef struct sm_combine_buffers {
    sm_view parts;            /* F32 [T,k,d]                                              */
    sm_view weights;          /* F32 [T,k]                                                */
    sm_view shared;           /* F32 [T,d]; null view when shared_ff == 0                 */
    sm_view gate;             /* F32 [T];   null view when shared_ff == 0                 */
    sm_view output;           /* F32 [T,d]                                                */
} sm_combine_buffers;

typedef struct sm_layer_formats {
    sm_format gate_up;        /* Q8_0, Q4_K, Q2_K                                          */
    sm_format down;           /* Q8_0, Q4_K, Q2_K                                          */
    sm_format shared;         /* F16, BF16 (ignored when shared_ff == 0)                   */
} sm_layer_formats;

/* PrefillMoeFullPipelineBuffers (prefill_moe_full_pipeline.hpp:43-56). */
typedef struct sm_layer_buffers {
    sm_route_gather_buffers route_gather;
    sm_shared_buffers shared;
    sm_gate_up_buffers gate_up;
    sm_down_buffers down;
    sm_combine_buffers combine;
} sm_layer_buffers;

/* ---- coordinators: segment form ------------------------------------------------------- */
/* encode_moe_route(divide_weights) — moe_dispatch.cpp:1500-1518. */
sm_status sm_encode_route(sm_segment* seg, const sm_moe_shape* shape, int divide_weights,
                          const sm_route_buffers* b);
/* encode_prefill_moe_grouping — prefill_moe_grouping.hpp:50-53. */
sm_status sm_encode_grouping(sm_segment* seg, const sm_moe_shape* shape,
                             const sm_grouping_buffers* b);
/* encode_prefill_moe_full_mode_route_gather — prefill_moe_pipeline.hpp:51-55. */
sm_status sm_encode_route_gather(sm_segment* seg, const sm_moe_shape* shape,
                                 const sm_route_gather_buffers* b);
/* encode_prefill_moe_shared_ffn — prefill_moe_shared_pipeline.hpp:54-58. */
sm_status sm_encode_shared_ffn(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt,
                               const sm_shared_buffers* b);
/* encode_prefill_moe_gu_<fmt> — prefill_moe_expert_dispatch.hpp:55-99. */
sm_status sm_encode_gate_up(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt,
                            const sm_gate_up_buffers* b);
/* encode_prefill_moe_down_<fmt> — prefill_moe_down_dispatch.hpp:40-49. */
sm_status sm_encode_down(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt,
                         const sm_down_buffers* b);
/* encode_prefill_moe_swiglu — prefill_moe_post.hpp:31-34. */
sm_status sm_encode_swiglu(sm_segment* seg, uint32_t rows, uint32_t width,
                           const sm_swiglu_buffers* b);
/* encode_prefill_moe_combine — prefill_moe_post.hpp:46-49. */
sm_status sm_encode_combine(sm_segment* seg, const sm_moe_shape* shape,
                            const sm_combine_buffers* b);
/* encode_prefill_dequant_<fmt> — prefill_dequant_dispatch.hpp:13-26: expands n_out
 * row-major weight rows of k values (`weights`) to K-major F16 [k][n_out] (`k_major_f16`),
 * with the same per-value decoders the expert products use. */
sm_status sm_encode_dequant(sm_segment* seg, sm_format fmt, uint32_t n_out, uint32_t k, sm_view weights,
                            sm_view k_major_f16);
/* encode_prefill_moe_full_mode_layer — prefill_moe_full_pipeline.hpp:68-73. */
sm_status sm_encode_full_layer(sm_segment* seg, const sm_moe_shape* shape,
                               const sm_layer_formats* formats, const sm_layer_buffers* b);

/* ---- decode-side MoE (the reference's Window MoE over T = 1..8 rows) -----------------------
 * The step after prefill on the same layer (include/strata/metal/moe_dispatch.hpp:13-372,
 * src/metal/kernels/safe/moe.metal:101-275, docs/mac/04-metal-kernels.md sections 5.8, 5.10):
 * a first-appearance expert plan, Q8_1 activations, grouped mat-vecs that read each active
 * expert's weights once per group, an F32 SwiGLU and the decode combine. The expert formats
 * are this library's block formats (Q8_0, Q4_K, Q2_K) over the same [layer][E][3] address
 * table as prefill. hidden is a multiple of 256 and expert_ff of 64, both at most 4096 (K-quant down weights need
 * expert_ff in whole 256-value super-blocks; the reference model's 2560 / 640 fit); rows * top_k <= 80.
 * Status word (one per coordinator call, cleared on the GPU first): bit 0 an active expert's
 * address is null, bit 1 the plan is unusable (an id outside [0, E), a malformed header or
 * entry, a group of more than T entries), bit 2 an active expert's tiered slot is not leased.
 * Failing groups write zeros. */
#define SM_DECODE_MAX_ROWS 8u
#define SM_DECODE_MAX_WIDTH 4096u       /* hidden and expert_ff of the decode mat-vecs          */
#define SM_MOE_PLAN_BYTES 1620u       /* MoePlan, moe.metal:101-111 (TieredMoePlan, tiered.hpp:24-36) */
#define SM_MOE_PLAN_MAX_ENTRIES 80u   /* T * k <= 8 * 10                                        */
#define SM_Q8_1_BLOCK_BYTES 36u       /* Q81 {half d, half sum; int8 q[32]}, types.h:128-131     */

/* MoePlanBuffers (moe_dispatch.hpp:19-24). The plan, residency and usage views start at layer 0
 * and contain the selected layer: plan `plans + layer * 1620`, rows `layer * E` of the I32
 * residency and F32 usage tables (tiered mode: usage += 1 per routed entry; null views = full
 * mode, every group resident). */
typedef struct sm_moe_plan_buffers {
    sm_view ids;                /* I32 [T*k] route ids, token-major                         */
    sm_view resident;           /* I32 [layer+1][E] or null                                 */
    sm_view usage;              /* F32 [layer+1][E] or null                                 */
    sm_view plans;              /* MoePlan [layer+1]                                        */
    sm_view status;             /* U32 or null                                              */
    uint32_t layer;
} sm_moe_plan_buffers;

/* MoeGroupedExpertBuffers (moe_dispatch.hpp:37-51): gate and up, F32, in grouped entry order. */
typedef struct sm_moe_expert_buffers {
    sm_expert_weights weights;  /* layer = the plan's layer                                 */
    sm_view activations;        /* Q8_1 [T][d/32]                                           */
    sm_view plans;              /* MoePlan table from layer 0                               */
    sm_view gate;               /* F32 [T*k][I]                                             */
    sm_view up;                 /* F32 [T*k][I]                                             */
    sm_view status;             /* U32                                                      */
} sm_moe_expert_buffers;

/* MoeGroupedDownBuffers (moe_dispatch.hpp:54-63): parts F32 in route order. */
typedef struct sm_moe_down_buffers {
    sm_expert_weights weights;
    sm_view activations;        /* Q8_1 [T*k][I/32], grouped entry order                   */
    sm_view plans;
    sm_view parts;              /* F32 [T*k][d], row t*k + rank                             */
    sm_view status;
} sm_moe_down_buffers;

/* MoeSwiGLUBuffers (moe_dispatch.hpp:82-86): F32 silu(gate) * up. */
typedef struct sm_moe_swiglu_buffers {
    sm_view gate;
    sm_view up;
    sm_view output;
} sm_moe_swiglu_buffers;

/* MoeRoutedFFNBuffers (moe_dispatch.hpp:65-80): gate/up, SwiGLU, Q8_1, down in one segment. */
typedef struct sm_moe_routed_ffn_buffers {
    sm_expert_weights gate_up_weights;
    sm_expert_weights down_weights;
    sm_view input_activations;  /* Q8_1 [T][d/32]                                           */
    sm_view plans;
    sm_view gate;               /* F32 [T*k][I] scratch                                     */
    sm_view up;
    sm_view hidden;
    sm_view down_activations;   /* Q8_1 [T*k][I/32] scratch                                 */
    sm_view parts;              /* F32 [T*k][d]                                             */
    sm_view status;
} sm_moe_routed_ffn_buffers;

/* MoeSharedFFNBuffers (moe_dispatch.hpp:101-135): the shared expert over T <= 8 rows, then the
 * decode combine with the routed parts. This library's shared weights are F16/BF16 [Is][d]
 * (down [d][Is]) read by dense mat-vecs; shared.hidden is F32 [T][Is] = silu(x.Wg) * (x.Wu). */
typedef struct sm_moe_shared_ffn_buffers {
    sm_shared_buffers shared;   /* hidden F32 [T][Is]; output F32 [T][d]; gate_logit F32 [T] */
    sm_view routed_parts;       /* F32 [T*k][d], route order                                */
    sm_view route_weights;      /* F32 [T,k]                                                */
    sm_view output;             /* F32 [T,d]                                                */
} sm_moe_shared_ffn_buffers;

/* One decode layer: router GEMM, top-k in multiply mode (the Window's route, moe_dispatch.hpp:
 * 161-168), plan (+ both address snapshots), Q8_1 of the input, the routed FFN, the shared
 * expert (F16/BF16 mat-vecs on mixed_h, as sm_encode_moe_shared_ffn) and the decode combine, as
 * six launches on the commit's stream: router with the shared gate/up; top-k, plan, Q8_1 input
 * and shared down; routed gate/up; SwiGLU + Q8_1; routed down; combine. */
typedef struct sm_decode_layer_buffers {
    sm_view mixed_h;            /* F16 [T,d]                                                */
    sm_view router_weights;     /* F32 [E,d]                                                */
    sm_view router_bias;        /* F32 [E] or null                                          */
    sm_view logits;             /* F32 [T,E]                                                */
    sm_view route_ids;          /* I32 [T,k]                                                */
    sm_view route_weights;      /* F32 [T,k]                                                */
    sm_view resident;           /* tiered mode, as in sm_moe_plan_buffers (or null)         */
    sm_view usage;
    sm_view plans;
    uint32_t layer;
    sm_view input_activations;  /* Q8_1 [T][d/32] scratch                                   */
    sm_moe_routed_ffn_buffers routed;  /* its input_activations and plans views are ignored  */
    sm_shared_buffers shared;   /* shared_ff == 0: ignored; mixed_h must equal mixed_h; hidden F32 [T][Is] */
    sm_view output;             /* F32 [T,d]                                                */
} sm_decode_layer_buffers;

/* encode_moe_plan — moe_dispatch.hpp:184-188. */
sm_status sm_encode_moe_plan(sm_segment* seg, const sm_moe_shape* shape, const sm_moe_plan_buffers* b);
/* strata_q_q8_1 — 04-metal-kernels.md section 5.8 (quantize_q8_1.metal): rows x n values
 * (n a multiple of 32; F16 input, or F32 when f32_input != 0) to Q8_1 blocks. */
sm_status sm_encode_quantize_q8_1(sm_segment* seg, uint32_t rows, uint32_t n, int f32_input, sm_view input,
                                  sm_view output);
/* encode_moe_experts — moe_dispatch.hpp:203-208. */
sm_status sm_encode_moe_experts(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt,
                                const sm_moe_expert_buffers* b);
/* encode_moe_down — moe_dispatch.hpp:223-228. */
sm_status sm_encode_moe_down(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt,
                             const sm_moe_down_buffers* b);
/* encode_moe_swiglu — moe_dispatch.hpp:264-267: rows x width F32 values. */
sm_status sm_encode_moe_swiglu(sm_segment* seg, uint32_t rows, uint32_t width, const sm_moe_swiglu_buffers* b);
/* encode_moe_routed_ffn — moe_dispatch.hpp:244-250. */
sm_status sm_encode_moe_routed_ffn(sm_segment* seg, const sm_moe_shape* shape, sm_format gate_up_fmt,
                                   sm_format down_fmt, const sm_moe_routed_ffn_buffers* b);
/* encode_moe_combine — moe_dispatch.hpp:277-280 (the decode combine: the first rank a product,
 * the others fma, the gated shared output added last; moe.metal:253-274). */
sm_status sm_encode_moe_combine(sm_segment* seg, const sm_moe_shape* shape, const sm_combine_buffers* b);
/* encode_moe_shared_ffn — moe_dispatch.hpp:287-308: shared gate/up + F32 SwiGLU (with the
 * sigmoid gate logit in the same launch), down, then the decode combine (3 launches). */
sm_status sm_encode_moe_shared_ffn(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt,
                                   const sm_moe_shared_ffn_buffers* b);
/* The Window MoE FFN of one layer (moe_dispatch.hpp:339-372's composition, with the route and
 * plan in front): see sm_decode_layer_buffers. */
sm_status sm_encode_moe_decode_layer(sm_segment* seg, const sm_moe_shape* shape, const sm_layer_formats* formats,
                                     const sm_decode_layer_buffers* b);
sm_status sm_submit_moe_decode_layer(sm_context* ctx, void* hip_stream, const sm_moe_shape* shape,
                                     const sm_layer_formats* formats, const sm_decode_layer_buffers* b, char* err,
                                     size_t err_cap);

/* ---- chunk driver (the reference's Prefill::run chunk loop) ------------------------------ */
/* PrefillChunkSchedule (include/strata/metal/prefill.hpp:47-72): a prompt of token_count
 * tokens starting at cell pos0, split into contiguous, unpadded ranges of at most chunk_rows. */
typedef struct sm_chunk_schedule {
    uint32_t pos0;
    uint32_t chunk_rows;
    uint64_t token_count;
} sm_chunk_schedule;
/* PrefillChunkRange (prefill.hpp:40-45). */
typedef struct sm_chunk_range {
    uint64_t token_offset;
    uint32_t pos0;
    uint32_t rows;
} sm_chunk_range;
/* build_prefill_chunk_schedule (prefill.hpp:74-88, src/metal/engine/prefill.cpp:57-83):
 * chunk_rows must be 1..SM_MAX_ROWS and the prompt's positions must fit a signed 32-bit
 * StepRow; an empty prompt gives an empty schedule. `out` is unchanged on failure. */
sm_status sm_build_chunk_schedule(uint32_t pos0, uint64_t token_count, uint32_t chunk_rows,
                                  sm_chunk_schedule* out, char* err, size_t cap);
/* PrefillChunkSchedule::chunk_count (prefill.hpp:53-57). */
uint64_t sm_chunk_count(const sm_chunk_schedule* schedule);
/* PrefillChunkSchedule::range_at (prefill.cpp:39-55): 1 and the range, or 0 with `out`
 * unchanged for an index past the last range. */
int sm_chunk_range_at(const sm_chunk_schedule* schedule, uint64_t index, sm_chunk_range* out);

/* The MoE layer over a whole prompt, one full-mode layer call per range of `schedule`, in
 * order, in one segment (Prefill::run's per-chunk MoE, 04-metal-kernels.md:3701-3891):
 * chunk k reads rows [token_offset, token_offset + rows) of `input` (F16 [token_count][d])
 * and writes the same rows of `output` (F32 [token_count][d]). Every other view of `b` is
 * chunk scratch sized for shape->rows == schedule->chunk_rows rows and reused by every chunk;
 * stream order serialises the chunks. b->route_gather.mixed_h, b->shared.mixed_h and
 * b->combine.output are not used (the chunk slices of `input` and `output` replace them).
 * The two status words are cleared before the first chunk only, so after completion they
 * hold the OR over every chunk (a route id outside [0, E) in any chunk shows as bit 1); the
 * plan slot's `bad` field is the last chunk's. */
sm_status sm_encode_prefill_moe_chunks(sm_segment* seg, const sm_chunk_schedule* schedule,
                                       const sm_moe_shape* shape, const sm_layer_formats* formats,
                                       sm_view input, sm_view output, const sm_layer_buffers* b);

/* ---- coordinators: standalone transactional form ---------------------------------------- */
sm_status sm_submit_route(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                          int divide_weights, const sm_route_buffers* b, char* err, size_t cap);
sm_status sm_submit_grouping(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                             const sm_grouping_buffers* b, char* err, size_t cap);
sm_status sm_submit_route_gather(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                                 const sm_route_gather_buffers* b, char* err, size_t cap);
sm_status sm_submit_shared_ffn(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                               sm_format fmt, const sm_shared_buffers* b, char* err, size_t cap);
sm_status sm_submit_gate_up(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                            sm_format fmt, const sm_gate_up_buffers* b, char* err, size_t cap);
sm_status sm_submit_down(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                         sm_format fmt, const sm_down_buffers* b, char* err, size_t cap);
sm_status sm_submit_swiglu(sm_context* ctx, void* stream, uint32_t rows, uint32_t width,
                           const sm_swiglu_buffers* b, char* err, size_t cap);
sm_status sm_submit_combine(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                            const sm_combine_buffers* b, char* err, size_t cap);
sm_status sm_submit_dequant(sm_context* ctx, void* stream, sm_format fmt, uint32_t n_out, uint32_t k,
                            sm_view weights, sm_view k_major_f16, char* err, size_t cap);
sm_status sm_submit_full_layer(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                               const sm_layer_formats* formats, const sm_layer_buffers* b,
                               char* err, size_t cap);
/* The full-mode layer (as sm_submit_full_layer) with its workspace in the library's fixed
 * per-GPU scratch instead of caller views. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (tight serving loops, harnesses that forbid hipMalloc); it
 * allocates nothing. Like every commit it refuses a capturing stream (SM_E_ARGUMENT): the expert
 * address tables are copied from the context's reusable pinned host ring when the launches run,
 * so a captured graph would replay stale tables. b->route_gather.histogram,
 * b->gate_up.weights.address_snapshot and b->down.weights.address_snapshot must be null views:
 * the histogram ((ceil(T*k/256) + 1) * E * 4 bytes, at most SM_FIXED_SCRATCH_HISTOGRAM_BYTES,
 * else SM_E_SHAPE) and both snapshots live in the scratch. Every call on a GPU uses that GPU's
 * one copy, so calls that overlap on one GPU race; calls ordered on one stream do not. */
#define SM_FIXED_SCRATCH_HISTOGRAM_BYTES (1u << 20)
sm_status sm_submit_full_layer_fixed_scratch(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                                             const sm_layer_formats* formats, const sm_layer_buffers* b,
                                             char* err, size_t cap);
sm_status sm_submit_prefill_moe_chunks(sm_context* ctx, void* stream, const sm_chunk_schedule* schedule,
                                       const sm_moe_shape* shape, const sm_layer_formats* formats,
                                       sm_view input, sm_view output, const sm_layer_buffers* b, char* err,
                                       size_t cap);

/* ---- model file: GGUF expert tensors -> device storage + address table ------------------ */
/* The reference's full-mode layout (src/metal/engine/window.cpp:128-270): every layer's routed
 * experts are the GGUF tensors blk.<l>.ffn_{gate,up,down}_exps.weight, ne = [d, I, E] for gate
 * and up (one type) and [I, d, E] for down (docs/mac/03-model-reference.md:292-297), each
 * expert a contiguous slab; the [layer][E][3] table holds each slab's device address. */
typedef struct sm_gguf sm_gguf;
typedef struct sm_gguf_tensor {
    uint32_t ggml_type;      /* ggml type id (0 F32, 1 F16, 8 Q8_0, 10 Q2_K, 12 Q4_K, 30 BF16, ...) */
    uint32_t n_dims;
    uint64_t ne[4];          /* ne[0] varies fastest; unused dimensions are 1                  */
    uint64_t offset;         /* absolute file offset of the data                               */
    uint64_t bytes;          /* data bytes (0 for a type without a known block layout)         */
} sm_gguf_tensor;
#define SM_GGUF_MAX_LAYERS 64u
typedef struct sm_expert_layout {
    uint32_t n_layers, n_experts, hidden, expert_ff;
    sm_format gate_up, down;
    uint64_t total_bytes;                      /* device bytes for every expert tensor          */
    uint64_t offsets[SM_GGUF_MAX_LAYERS][3];   /* each tensor's offset in that storage (256-aligned) */
} sm_expert_layout;
/* Opens a GGUF v2/v3 file and validates its header, metadata and tensor directory (every
 * tensor's data inside the file, aligned to general.alignment). SM_E_FILE on a bad file. */
sm_status sm_gguf_open(const char* path, sm_gguf** out, char* err, size_t cap);
void sm_gguf_close(sm_gguf* gguf);
uint64_t sm_gguf_tensor_count(const sm_gguf* gguf);
/* SM_E_ARGUMENT when the tensor does not exist. */
sm_status sm_gguf_find(const sm_gguf* gguf, const char* name, sm_gguf_tensor* out);
/* The expert tensors of layers 0..n_layers-1: every one present, 3-D, Q8_0/Q4_K/Q2_K, shapes and
 * types equal across layers, expert slabs aligned for the kernels; and where each goes in one
 * device allocation of total_bytes. */
sm_status sm_gguf_expert_layout(const sm_gguf* gguf, uint32_t n_layers, sm_expert_layout* out, char* err,
                                size_t cap);
/* Copies every expert tensor of `layout` from the file into `storage` (a registered device view
 * of at least layout->total_bytes, 256-byte aligned) through pinned chunks on `stream`, waits
 * for the copies, and writes the host [n_layers][E][3] address table (n_addresses >=
 * n_layers * E * 3) for sm_expert_weights.addresses (with n_layers and the selected layer). */
sm_status sm_gguf_load_experts(sm_gguf* gguf, sm_context* ctx, void* stream, const sm_expert_layout* layout,
                               sm_view storage, uint64_t* addresses, uint64_t n_addresses, char* err,
                               size_t cap);

/* ---- tiered residency: expert store, slot leases and the per-layer handshake ------------- */
/* The reference's ExpertStore / ExpertLeaseSet (include/strata/metal/experts.hpp:18-90) and the
 * layer handshake (docs/mac/06-engine-host-port.md section 9.3): when the experts do not all
 * fit in HBM, the grouping marks each group resident or not from the layer's residency-table
 * row (PfPlan grp_res, n_miss, skip); the host then resolves the misses into slots of a device
 * arena before the expert stages run. Here the handshake is host-driven between segments: the
 * routing segment is committed, sm_expert_store_resolve_layer waits for it, reads the plan,
 * brings each missing expert from the cold tier (the model's GGUF file) into a slot of half
 * layer % 2 (least recently used unpinned slot, or a cached one), writes the slot addresses
 * into the layer's address-table row and pins them in the lease set; then the expert segment is
 * encoded with that table, the arena and the lease set. */
typedef struct sm_expert_store sm_expert_store;
typedef struct sm_store_stats {
    uint64_t hits, lookups, file_reads, file_bytes;   /* ExpertLayerStats (experts.hpp:45-51) */
} sm_store_stats;
/* Bytes of one slot: the gate, up and down slabs of one expert, each 256-byte aligned. */
uint64_t sm_expert_slot_bytes(const sm_expert_layout* layout);
/* A store over the experts of `layout` in `gguf` (the cold tier) with `slot_arena` (a registered
 * device view of at least 2 * slots_per_half * sm_expert_slot_bytes bytes) as two halves. */
sm_status sm_expert_store_create(sm_context* ctx, sm_gguf* gguf, const sm_expert_layout* layout, sm_view slot_arena,
                                 uint32_t slots_per_half, sm_expert_store** out, char* err, size_t cap);
void sm_expert_store_destroy(sm_expert_store* store);
/* A lease set for one command sequence (prepare_command_buffer): its pins keep slots from
 * being reused until they are retired or the set is destroyed, which the caller does only
 * after the GPU work that reads the slots has completed. */
sm_status sm_lease_set_create(sm_expert_store* store, sm_lease_set** out);
void sm_lease_set_destroy(sm_lease_set* leases);
void sm_lease_set_retire_layer(sm_lease_set* leases, uint32_t layer);
/* ExpertLeaseSet::pins (experts.hpp:30-31): 1 if a pin of `layer` covers [address, +bytes). */
int sm_lease_set_pins(const sm_lease_set* leases, uint32_t layer, uint64_t address, uint64_t bytes);
/* resolve_layer_after_plan (experts.hpp:74-85): waits for `stream` (the grouping that wrote
 * `plan` is committed on it), retires the lease set's pins of earlier layers, reads the plan
 * (only the header when skip is set; n_miss must match the groups marked non-resident), resolves
 * every non-resident group's expert into a slot and writes its three slot addresses into
 * table[(layer * E + e) * 3 + role] (n_table >= (layer + 1) * E * 3). Misses are read from the
 * file by up to 8 host threads (kExpertFetchWorkers, experts.hpp:14) and copied into their slots
 * asynchronously on `stream`: the expert segment must be committed on `stream` (or on a stream
 * that waits for it). On failure nothing of the layer is pinned, the slots it was filling are
 * emptied and the table row may be partly written. */
sm_status sm_expert_store_resolve_layer(sm_expert_store* store, void* stream, uint32_t layer, sm_view plan,
                                        sm_lease_set* leases, uint64_t* table, uint64_t n_table,
                                        sm_store_stats* stats, char* err, size_t cap);
/* prefetch_layer / prefetch_experts (experts.hpp:90-94): warms experts of `layer` into slots of
 * half layer % 2 ahead of its plan, so that a later resolve of the layer finds them cached
 * (stats.hits). experts: n_experts expert ids, or NULL for every expert of the layer in id
 * order. Cached experts count as hits; the others are read as in resolve and copied
 * asynchronously on `stream` into free or least recently used unpinned slots, never evicting a
 * slot this call filled, and the call stops (successfully) when no such slot is left. Pins
 * nothing. */
sm_status sm_expert_store_prefetch(sm_expert_store* store, void* stream, uint32_t layer, const int32_t* experts,
                                   uint32_t n_experts, sm_store_stats* stats, char* err, size_t cap);

/* ---- after completion ----------------------------------------------------------------- */
/* Synchronises `stream`, then reads the plan's `bad` count and up to two status words
 * (null views are skipped and read as 0). The reference's caller contract
 * (prefill_moe_full_pipeline.hpp:44-46). */
sm_status sm_read_layer_status(sm_context* ctx, void* stream, sm_view plan, sm_view gate_up_status,
                               sm_view down_status, uint32_t* bad, uint32_t* gate_up_bits,
                               uint32_t* down_bits);

/* ---- synthetic inputs (host, deterministic; used by tests and the benchmark) ------------ */
/* out[i] = N(0, sigma) from SplitMix64(seed, stream, i) + Box-Muller, as F32. */
void sm_synth_normal_f32(uint64_t seed, uint64_t stream, float sigma, float* out, uint64_t n);
/* Same values rounded to F16 (RNE) / BF16 (RNE). */
void sm_synth_normal_f16(uint64_t seed, uint64_t stream, float sigma, uint16_t* out, uint64_t n);
void sm_synth_normal_bf16(uint64_t seed, uint64_t stream, float sigma, uint16_t* out, uint64_t n);
/* Quantizes rows*k F32 values (row-major [rows][k]) to `fmt` blocks. */
sm_status sm_quantize(sm_format fmt, const float* in, uint64_t rows, uint64_t k, uint8_t* out);
/* Generates N(0, sigma) weights for `rows` rows of `k` and quantizes them directly. */
sm_status sm_synth_quantized(sm_format fmt, uint64_t seed, uint64_t stream, float sigma,
                             uint64_t rows, uint64_t k, uint8_t* out);

/* Library build identity. */
uint32_t sm_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* STRATA_MOE_H */
