// Internal launch interface between the host coordinators (sm_runtime.cpp) and the gfx950
// kernels. Plain pointers and sizes only; every launcher assumes its arguments were
// validated by the coordinator (shapes, extents, alignment) and checks nothing itself.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sm {

// PfPlan (the reference's prefill_moe.metal:23-33): 6180 bytes inside a 6400-byte slot.
struct Plan {
    uint32_t n_groups, n_entries, n_miss, skip, n_tiles, bad, pad[2];
    int32_t grp_e[512];
    int32_t grp_res[512];
    int32_t grp_start[513];
};
static_assert(sizeof(Plan) == 6180, "PfPlan layout");

constexpr uint32_t kCountTile = 256;   // histogram tile (entries)
constexpr uint32_t kExpertTile = 64;   // tile-list tile (entries)
constexpr uint32_t kPlanSlotBytes = 6400;
// The 64-row tile kernels take their work items from per-XCD counters kept in the plan slot's
// padding after the PfPlan fields: 8 words for gate/up, then 8 for down. Each stage's plan
// check zeroes them before the stage runs.
constexpr uint32_t kCounterBytes = 6208;
constexpr uint32_t kCounterWords = 8;
static_assert(sizeof(Plan) <= kCounterBytes && kCounterBytes + 2 * 4 * kCounterWords <= kPlanSlotBytes,
              "counters in the plan slot's padding");
// The grouping's column-scan workgroups count themselves in at this word of the slot (the
// count kernel zeroes it, or in a route/gather composition the router; the plan fill that
// follows leaves it zero).
constexpr uint32_t kArriveBytes = kCounterBytes + 2 * 4 * kCounterWords;
static_assert(kArriveBytes + 4 <= kPlanSlotBytes, "arrival word inside the plan slot");

enum class Fmt : int { Q8_0 = 1, Q4_K = 2, Q2_K = 3, F16 = 4, BF16 = 5 };

// ---- route ----
// Duty of the router in a route/gather composition (null: none): it zeroes the grouping
// histogram's first `hist_words` words (the per-tile counts) and the plan's arrival word, so
// that top-k counts the routed entries straight into the histogram (launch_route_topk with
// hist) and the grouping skips its count kernel (launch_grouping with counted).
struct RouterPrep {
    uint32_t* hist = nullptr;
    uint32_t hist_words = 0;
    uint32_t* arrive = nullptr;
};
// bias (F32 [E]) may be null.
hipError_t launch_router_gemm(const _Float16* x, const float* w, const float* bias, float* logits,
                              uint32_t rows, uint32_t d, uint32_t n_experts, hipStream_t s,
                              const RouterPrep* prep = nullptr);
// hist (may be null): per-tile counts (tiles of kCountTile route-order entries) that each
// selected entry is added to.
hipError_t launch_route_topk(const float* logits, int32_t* ids, float* weights, uint32_t rows,
                             uint32_t n_experts, uint32_t top_k, int divide, hipStream_t s,
                             uint32_t* hist = nullptr);

// ---- grouping ----
// hist has ceil(N/256) + 1 rows of n_experts u32; the extra last row holds each expert's
// first grouped slot.
// Full-layer duties of the grouping's scan workgroup: the expert stages' status words and the
// destination bitset are zeroed before the gather's checks (launch_gather_checked) run.
struct GroupPrep {
    uint32_t* status = nullptr;
    uint32_t* status2 = nullptr;
    uint32_t* clear = nullptr;
    uint32_t clear_words = 0;
};
// resident (may be null: full residency): the selected layer's row of the I32 [layer][E]
// residency table; a group's grp_res is resident[e] >= 0, n_miss counts the other groups and
// skip = (n_miss == 0).
// counted: top-k has already counted the entries into hist (RouterPrep), so the count
// kernel is skipped.
hipError_t launch_grouping(const int32_t* ids, uint32_t rows, uint32_t top_k, uint32_t n_experts,
                           uint32_t* hist, Plan* plan, uint32_t* tiles, int32_t* src, int32_t* dst,
                           const GroupPrep* prep, const int32_t* resident, hipStream_t s,
                           bool counted = false);
// The gather runs after the grouping of the same ids and histogram (it recomputes each entry's
// grouped slot from them); d % 256 == 0.
hipError_t launch_gather(const _Float16* x, uint32_t d, const int32_t* ids, const uint32_t* hist, uint32_t top_k,
                         uint32_t n_experts, const Plan* plan, uint32_t n_entries, _Float16* xs, hipStream_t s);

// ---- expert stage validation (the reference's plan/destination validators) ----
// One plan check for up to two expert stages. The check's verdict goes to `status` and, when
// set, `status2` (both cleared first). The kernel also copies each stage's validated
// expert-address table (`snap_words` u64 from pinned host memory `snap_src`, which may be
// null) into its device snapshot, and zeroes `clear_words` u32 at `clear` (a destination
// bitset), so a full layer validates its shared plan once for the gate/up and down stages.
struct PlanCheck {
    const Plan* plan;
    const uint32_t* tiles;
    uint32_t* status;
    uint32_t* status2;
    uint32_t n_entries, n_experts, tile_capacity;
    const uint64_t* snap_src;
    uint64_t* snap_dst;
    uint32_t snap_words;
    const uint64_t* snap_src2;
    uint64_t* snap_dst2;
    uint32_t snap_words2;
    uint32_t* clear;
    uint32_t clear_words;
    uint32_t* counters;         // tile-kernel work counters to zero (may be null)
    uint32_t n_counters;
    uint32_t keep_status;       // non-zero: the status words are not cleared first (they
                                // accumulate over the chunks of one prompt)
};
hipError_t launch_plan_validate(const PlanCheck& c, hipStream_t s);
// The gather of a full layer with both expert stages' checks in the same launch: one extra
// workgroup runs the plan check `c` (its `clear` and status clearing are not used: the
// grouping's GroupPrep zeroed both status words and the bitset `bits`), and every gather
// workgroup marks its share of `dst` in `bits`, setting bit 1 of `c.status2` for an entry
// outside [0, n_entries) or a repeated one.
hipError_t launch_gather_checked(const _Float16* x, uint32_t d, const int32_t* ids, const uint32_t* hist,
                                 uint32_t top_k, uint32_t n_experts, const Plan* plan, uint32_t n_entries,
                                 _Float16* xs, const PlanCheck& c, const int32_t* dst, uint32_t* bits,
                                 hipStream_t s);
// Checks that `dst` is a permutation of [0, n_entries) with a bitset (zeroed first unless
// `bitset_clear` is false because a PlanCheck cleared it).
hipError_t launch_destination_validate(const int32_t* dst, uint32_t* bitset, uint32_t* status,
                                       uint32_t n_entries, bool bitset_clear, hipStream_t s);

// ---- grouped expert products ----
enum Mode { kGateUp = 0, kDown = 1 };

struct RoutedGemm {
    const uint64_t* addresses;  // device [E][3] (gate, up, down)
    const _Float16* a;          // grouped rows [N][K]
    const Plan* plan;
    const uint32_t* tiles;      // {group, first_entry} pairs
    const int32_t* dst;         // down only
    _Float16* out_h;            // gate/up: [N][I]
    float* out_f;               // down: [N][d] route order
    uint32_t* status;
    uint32_t n_entries, n_experts, tile_capacity;
    uint32_t k;                 // reduction length (d for gate/up, I for down)
    uint32_t n_out;             // output columns (I for gate/up, d for down)
    uint64_t row_bytes;         // bytes of one weight row of k values
    // Groups with at least this many entries run in 256-row units on the wide kernel and are
    // skipped by the 64-row tile kernels; ~0u: every group runs in 64-row tiles.
    uint32_t wide_min;
    uint32_t* counters;         // kCounterWords per-XCD item counters, zeroed by the plan check
};
// Groups of at least g.wide_min entries run on the wide kernel, the others on the 64-row
// tile kernels; both run in one launch where they fit (the routed stage kernel).
hipError_t launch_gate_up(Fmt fmt, const RoutedGemm& g, hipStream_t s);
hipError_t launch_down(Fmt fmt, const RoutedGemm& g, hipStream_t s);
// Whether the wide kernel supports a stage: a block format, K a multiple of 64, and whole
// 256-row column tiles (gate/up: 128 hidden columns, down: 256 output columns).
bool wide_fits(Fmt fmt, bool gate_up, uint32_t k, uint32_t n_out);
hipError_t launch_wide(Fmt fmt, bool gate_up, const RoutedGemm& g, hipStream_t s);
// One launch for a whole routed stage: wide units (groups >= g.wide_min) and the other
// groups' 64-row tiles in the staged form (K a multiple of 256, whole column tiles).
hipError_t launch_stage(Fmt fmt, bool gate_up, const RoutedGemm& g, hipStream_t s);
constexpr uint32_t kWideMin = 128;

struct DenseGemm {
    const _Float16* a;          // [rows][k]
    const uint8_t* w0;          // gate/up: gate [n][k]; down: W [n_out][k]
    const uint8_t* w1;          // gate/up: up   [n][k]
    _Float16* out_h;            // gate/up output [rows][n]
    float* out_f;               // down output [rows][n_out]
    uint32_t rows, k, n_out;
    uint64_t row_bytes;
};
hipError_t launch_dense_gate_up(Fmt fmt, const DenseGemm& g, hipStream_t s);
hipError_t launch_dense_down(Fmt fmt, const DenseGemm& g, hipStream_t s);
// The dense products on the wide kernel (256-row units of the activation rows): F16/BF16
// weights, K a multiple of 128, whole column tiles, and enough units for half of the CUs.
bool wide_dense_fits(Fmt fmt, bool gate_up, uint32_t rows, uint32_t k, uint32_t n_out);
hipError_t launch_wide_dense(Fmt fmt, bool gate_up, const DenseGemm& g, hipStream_t s);
// gl[t] = sum_k x[t,k] * gv[k] (F16 or BF16 gate vector), F32 accumulation.
hipError_t launch_gate_logit(Fmt fmt, const _Float16* x, const uint8_t* gv, float* gl, uint32_t rows,
                             uint32_t d, hipStream_t s);

// Decode `rows` weight rows of `k` values to K-major F16 bits [k][rows], through the
// products' own per-lane fragment decoders.
hipError_t launch_decode_rows(Fmt fmt, const uint8_t* w, uint32_t rows, uint32_t k, uint64_t row_bytes,
                              uint16_t* out, hipStream_t s);

// ---- decode-side MoE (T <= 8 rows) ----
// The first-appearance plan (MoePlan, 1620 bytes) of rows * top_k <= 80 entries; the launch
// also copies up to two validated address tables (pinned host ring -> device snapshot).
struct DecodePlanArgs {
    const int32_t* ids;         // [rows * top_k]
    const int32_t* resident;    // the layer's [E] residency row; null = full residency
    float* usage;               // the layer's [E] usage row (tiered mode); null = none
    uint8_t* plan;              // the layer's MoePlan
    uint32_t* status;           // bit 1 on an id outside [0, E) (may be null)
    uint32_t rows, top_k, n_experts;
    // launch_decode_front only (may be null): the route's logits [rows][E]; the launch's plan
    // workgroup then runs the top-k (multiply mode) first, into route_ids (the buffer `ids`
    // names) and route_weights.
    const float* logits;
    int32_t* route_ids;
    float* route_weights;
};
hipError_t launch_decode_plan(const DecodePlanArgs& a, hipStream_t s);
// hidden = silu(gate) * up (F32, rows x n, n a multiple of 32) and its Q8_1 blocks y, one launch.
hipError_t launch_swiglu_q8_1(const float* gate, const float* up, float* hidden, uint8_t* y, uint32_t n, uint32_t rows,
                              hipStream_t s);
// A standalone expert stage's snapshot copy (src may be null: nothing copied); clears *status.
hipError_t launch_snapshot_copy(const uint64_t* src, uint64_t* dst, uint32_t words, uint32_t* status, hipStream_t s);
// Q8_1 blocks (36 B: half d, half sum, int8 q[32]) of rows x n values (F16 or F32 input).
hipError_t launch_quantize_q8_1(const void* x, bool f32_input, uint8_t* y, uint32_t n, uint32_t rows, hipStream_t s);
// Grouped mat-vec of one stage over a MoePlan. gate/up: act = Q8_1 [rows][k/32] by token,
// out0/out1 = gate/up F32 [n_entries][out_width] by grouped entry; down: act = Q8_1
// [n_entries][k/32] by grouped entry, out0 = parts F32 [n_entries][out_width] by route index.
struct DecodeMatvec {
    const uint64_t* addresses;  // device [E][3]
    const uint8_t* act;
    const uint8_t* plan;
    float* out0;
    float* out1;
    uint32_t* status;
    uint32_t n_entries, n_experts, act_rows;
    uint32_t k, out_width;
    uint64_t row_bytes;
    uint32_t max_group;  // entries a group may hold (T: one per token); larger groups are a bad plan
    uint32_t iters;      // set by the launcher: row slices per workgroup
};
hipError_t launch_decode_matvec(Fmt fmt, bool gate_up, const DecodeMatvec& m, hipStream_t s);
hipError_t launch_swiglu_f32(const float* gate, const float* up, float* out, uint64_t n, hipStream_t s);
// The shared expert of a decode layer over F16/BF16 weights [n_out][k]. gate/up (w0 gate, w1 up,
// x F16 [rows][k]): out = hidden F32 [rows][n_out] = silu(x.Wg) * (x.Wu). down (w0, x F32 hidden
// [rows][k]): out F32 [rows][n_out] = x.Wd. k is a multiple of 64; rows <= 8.
struct DenseDecode {
    const uint8_t* w0;
    const uint8_t* w1;
    const void* x;
    const float* bias;  // router only (may be null)
    float* out;
    uint32_t rows, k, n_out;
    const uint8_t* gv;  // gate/up only: the sigmoid-gate vector [k] (may be null) ...
    float* gl;          // ... and its logits [rows], computed by one more workgroup of the launch
    // router only: address tables to copy into their snapshots (words may be 0)
    const uint64_t* snap_src;
    uint64_t* snap_dst;
    uint32_t snap_words;
    const uint64_t* snap_src2;
    uint64_t* snap_dst2;
    uint32_t snap_words2;
    uint32_t row_blocks;  // set by the launcher
};
struct SnapshotCopy {
    const uint64_t* src;
    uint64_t* dst;
    uint32_t words;
    const uint64_t* src2;
    uint64_t* dst2;
    uint32_t words2;
};
hipError_t launch_dense_decode(Fmt fmt, bool gate_up, const DenseDecode& m, hipStream_t s);
// The router of a decode layer (T <= 8 rows): logits[t][e] = x_t . W_e + bias[e] with F32
// weights [E][d] and F32 accumulation (d a multiple of 64).
// The launch also copies the validated address tables of `snap` into their device snapshots.
hipError_t launch_router_decode(const _Float16* x, const float* w, const float* bias, float* logits, uint32_t rows,
                                uint32_t d, uint32_t E, const SnapshotCopy& snap, hipStream_t s);
// The router above and the shared expert's gate/up (launch_dense_decode with gate_up, x the same
// F16 rows) in one launch.
hipError_t launch_router_shared_decode(const _Float16* x, const float* w, const float* bias, float* logits,
                                       uint32_t rows, uint32_t d, uint32_t E, const SnapshotCopy& snap, Fmt shared_fmt,
                                       const DenseDecode& shared_gate_up, hipStream_t s);
// The plan (after the top-k when a.logits is given), the Q8_1 quantization of rows x n F16 input
// values (n a multiple of 32) and, when shared_down is given, the shared expert's down mat-vec
// (launch_dense_decode, down) in one launch. E <= 512.
hipError_t launch_decode_front(const DecodePlanArgs& a, const _Float16* x, uint8_t* y, uint32_t n, uint32_t rows,
                               Fmt shared_fmt, const DenseDecode* shared_down, hipStream_t s);
// out = (p_0 w_0 + sum_r fma) + shared * sigmoid(gl); shared == null: no shared term.
hipError_t launch_combine_decode(const float* parts, const float* w, const float* shared, const float* gl, float* out,
                                 uint32_t rows, uint32_t top_k, uint32_t d, hipStream_t s);

// ---- post ops ----
hipError_t launch_swiglu(const float* gate, const float* up, _Float16* out, uint64_t n,
                         hipStream_t s);
hipError_t launch_combine(const float* parts, const float* weights, const float* shared,
                          const float* gl, float* out, uint32_t rows, uint32_t top_k, uint32_t d,
                          hipStream_t s);

}  // namespace sm
