// Host runtime and coordinators behind the C ABI in include/strata_moe.h.
//
// A segment is an ordered list of validated launches. Every coordinator first validates
// all of its views (ownership, extent, alignment, aliasing) and only then appends its
// launches; a failure poisons the segment so that commit refuses it and nothing reaches
// the GPU — the reference's transactional encoder (encoder.mm:165-231,
// context.mm:623-680), built on deferred launches because a HIP launch cannot be revoked.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <functional>
#include <limits>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/strata_moe.h"
#include "sm_internal.h"
#include "sm_launch.h"

struct sm_context {
    int device = 0;
    bool has_device = false;
    std::mutex mu;
    struct Alloc { uintptr_t ptr; uint64_t bytes; };
    std::map<uint64_t, Alloc> buffers;
    // Pinned host ring for validated expert-address tables. Allocated once at context
    // creation; a slot is reused only after the event recorded behind the kernel that read
    // it has completed.
    static constexpr uint32_t kRingSlots = 64;
    static constexpr uint32_t kSlotWords = 3 * 512;
    uint64_t* ring = nullptr;
    hipEvent_t ring_ev[kRingSlots] = {};
    bool ring_pending[kRingSlots] = {};
    bool ring_claimed[kRingSlots] = {};  // filled by an encode whose segment is not committed yet
    // A step that reads two slots records one event, into its first slot's; the second slot
    // (ring_alias = the first) is free once its partner is not pending. Every step that reads
    // a ring slot runs on the commit's own stream, so a partner re-recorded later in the same
    // commit completes after the earlier record, and one re-recorded by a later commit was
    // claimed, and its earlier record waited on, first.
    int ring_alias[kRingSlots] = {};
    uint32_t ring_next = 0;
    std::mutex ring_mu;
    // Second stream (default priority) for launches off the critical path of a full layer (the
    // shared expert): a side launch waits for the latest fork event, recorded on the caller's
    // stream before a step marked `fork_before` (or, if none came yet, right before the side
    // launch itself); a later step marked `join` waits for the side launches. side_mu keeps
    // one commit's event records and waits together.
    hipStream_t side = nullptr;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
    std::mutex side_mu;
    uintptr_t fixed_scratch = 0;  // this device's copy of the fixed scratch array (0: none)
};

namespace {
// Handles are unique across every context of the process, so a view from another context
// never resolves in this one's registry (the reference's "owned by this Context" check).
std::atomic<uint64_t> g_next_handle{1};

// ---- fixed scratch of sm_submit_full_layer_fixed_scratch ----------------------------------
// The workspace of the allocation-free full layer lives in this array, one copy per GPU in
// the code object's device globals: the grouping histogram (kFixedHistBytes), then the gate/up
// and the down address snapshots (kFixedSnapBytes each). Host code never takes the array's
// name as an address (on the host it is only a stand-in for the symbol): each device's copy
// is resolved once, with that device current, by hipGetSymbolAddress, and that pointer is
// what the kernels receive.
constexpr uint64_t kFixedHistBytes = SM_FIXED_SCRATCH_HISTOGRAM_BYTES;
constexpr uint64_t kFixedSnapBytes = 3ull * SM_MAX_EXPERTS * 8;
static __device__ __align__(256) uint8_t scratch[kFixedHistBytes + 2 * kFixedSnapBytes];

std::mutex g_scratch_mu;
std::map<int, uintptr_t> g_scratch_ptr;  // device -> its copy of `scratch`

// The device's copy of the fixed scratch (device current); 0 if it cannot be resolved.
uintptr_t fixed_scratch_of(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    auto it = g_scratch_ptr.find(device);
    if (it != g_scratch_ptr.end()) return it->second;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return 0;
    g_scratch_ptr[device] = reinterpret_cast<uintptr_t>(p);
    return reinterpret_cast<uintptr_t>(p);
}

// Where the allocation-free layer's workspace lies (all 0 on a context without a device,
// which still validates).
struct FixedScratch {
    uintptr_t hist = 0, snap_gu = 0, snap_dn = 0;
};
}  // namespace

struct sm_segment {
    sm_context* ctx = nullptr;
    // ring_slot >= 0: the step reads that pinned ring slot; an event is recorded after it.
    struct Step {
        const char* label;
        std::function<hipError_t(hipStream_t)> run;
        int ring_slot = -1, ring_slot2 = -1;
        bool side = false;         // runs on the context's side stream (untimed commits)
        bool join = false;         // waits for every side launch recorded before it
        bool fork_before = false;  // later side launches wait for the steps before this one
    };
    std::vector<Step> steps;
    bool failed = false;
    std::string error;
};

namespace {

using sm::Fmt;

// ---- small helpers --------------------------------------------------------------------

bool mul_ok(std::initializer_list<uint64_t> f, uint64_t& out) {
    out = 1;
    for (uint64_t v : f) {
        if (v != 0 && out > std::numeric_limits<uint64_t>::max() / v) return false;
        out *= v;
    }
    return true;
}

uint64_t ceil_div(uint64_t a, uint64_t b) { return a / b + (a % b != 0 ? 1 : 0); }

uint64_t fmt_row_bytes(int fmt, uint64_t k) {
    switch (fmt) {
        case SM_FMT_Q8_0: return k % 32 ? 0 : k / 32 * 34;
        case SM_FMT_Q4_K: return k % 256 ? 0 : k / 256 * 144;
        case SM_FMT_Q2_K: return k % 256 ? 0 : k / 256 * 84;
        case SM_FMT_F16:
        case SM_FMT_BF16: return 2 * k;
    }
    return 0;
}

bool routed_fmt(int f) { return f == SM_FMT_Q8_0 || f == SM_FMT_Q4_K || f == SM_FMT_Q2_K; }
bool dense_fmt(int f) { return f == SM_FMT_F16 || f == SM_FMT_BF16; }

// K granularity of the expert kernels: whole 256-value slabs for the K-quants and dense
// rows; 64-value lane groups for Q8_0.
bool k_ok(int fmt, uint64_t k) {
    if (fmt == SM_FMT_Q8_0) return k % 64 == 0 && k > 0;
    return k % 256 == 0 && k > 0;
}

uint64_t weight_align(int fmt) { return fmt == SM_FMT_Q8_0 ? 4 : 16; }

// One active byte range taking part in alias checks.
struct Range {
    uintptr_t ptr = 0;
    uint64_t bytes = 0;
    std::string name;
    bool writable = false;
    int stage = 0;
};

bool overlap(const Range& a, const Range& b) {
    if (a.bytes == 0 || b.bytes == 0) return false;
    return a.ptr < b.ptr + b.bytes && b.ptr < a.ptr + a.bytes;
}

// Validation context of one coordinator call.
struct Check {
    sm_context* ctx;
    std::string prefix;  // e.g. "Prefill MoE grouping"
    int stage = 0;
    const FixedScratch* fixed = nullptr;  // the histogram and snapshots come from the fixed scratch
    std::vector<Range> inputs, outputs;
    std::string err;
    sm_status st = SM_OK;

    bool fail(sm_status s, const std::string& msg) {
        if (st == SM_OK) { st = s; err = msg; }
        return false;
    }

    // Resolves a view to a device address after the ownership/extent/alignment checks.
    bool view(const sm_view& v, uint64_t need, uint64_t align, const char* name, bool writable,
              uintptr_t& out) {
        if (st != SM_OK) return false;
        sm_context::Alloc a{};
        {
            std::lock_guard<std::mutex> lk(ctx->mu);
            auto it = ctx->buffers.find(v.buffer);
            if (v.buffer == 0 || it == ctx->buffers.end())
                return fail(SM_E_OWNERSHIP, prefix + " " + name + " view is not owned by this context");
            a = it->second;
        }
        uint64_t end = v.offset + v.length;
        if (end < v.offset || end > a.bytes)
            return fail(SM_E_VIEW, prefix + " " + name + " view is undersized or misaligned");
        const uintptr_t p = a.ptr + v.offset;
        if (v.length < need || align == 0 || p % align != 0)
            return fail(SM_E_VIEW, prefix + " " + name + " view is undersized or misaligned");
        Range r{p, need, std::string(name), writable, stage};
        (writable ? outputs : inputs).push_back(r);
        out = p;
        return true;
    }

    // An expert stage's plan view: the PfPlan fields are read, and the stage's work-item
    // counters in the slot's padding (`words` u32 at byte `counter_off`) are written, so the
    // view is registered as a read-only PfPlan range and a writable counter range.
    bool plan_view(const sm_view& v, uint32_t counter_off, uint32_t words, uintptr_t& out) {
        if (!view(v, SM_PLAN_SLOT_BYTES, 4, "PfPlan slot", false, out)) return false;
        inputs.back().bytes = sm::kCounterBytes;
        outputs.push_back({out + counter_off, 4ull * words, "work counters", true, stage});
        return true;
    }

    // Outputs must be disjoint from every input and from each other
    // (prefill_moe_grouping_dispatch.mm:234-252).
    bool aliases() {
        if (st != SM_OK) return false;
        for (const auto& o : outputs)
            for (const auto& i : inputs)
                if (overlap(o, i)) return fail(SM_E_ALIAS, prefix + " " + o.name + " overlaps active " + i.name);
        for (size_t i = 0; i < outputs.size(); ++i)
            for (size_t j = i + 1; j < outputs.size(); ++j)
                if (overlap(outputs[i], outputs[j]))
                    return fail(SM_E_ALIAS, prefix + " " + outputs[i].name + " overlaps active " + outputs[j].name);
        return true;
    }
};

sm_status shape_check(const sm_moe_shape* s, const char* prefix, std::string& err, bool need_ff) {
    if (s == nullptr) { err = std::string(prefix) + " shape is null"; return SM_E_ARGUMENT; }
    if (s->rows == 0 || s->rows > SM_MAX_ROWS) {
        err = std::string(prefix) + " row count exceeds the supported range";
        return SM_E_SHAPE;
    }
    if (s->n_experts == 0 || s->n_experts > SM_MAX_EXPERTS) {
        err = std::string(prefix) + " supports 1..512 experts";
        return SM_E_SHAPE;
    }
    if (s->top_k == 0 || s->top_k > SM_MAX_TOP_K || s->top_k > s->n_experts) {
        err = std::string(prefix) + " top-k must be 1..min(experts, 32)";
        return SM_E_SHAPE;
    }
    if (s->hidden == 0 || s->hidden % 256 != 0) {
        err = std::string(prefix) + " hidden width must be a positive multiple of 256";
        return SM_E_SHAPE;
    }
    if (need_ff && (s->expert_ff == 0 || s->expert_ff % 64 != 0)) {
        err = std::string(prefix) + " expert width must be a positive multiple of 64";
        return SM_E_SHAPE;
    }
    return SM_OK;
}

sm_status record_fail(sm_segment* seg, sm_status st, const std::string& err) {
    if (!seg->failed) { seg->failed = true; seg->error = err; }
    return st;
}

void add_step(sm_segment* seg, const char* label, std::function<hipError_t(hipStream_t)> fn, bool side = false,
              bool join = false) {
    seg->steps.push_back({label, std::move(fn)});
    seg->steps.back().side = side;
    seg->steps.back().join = join;
}

// ---- stage encoders (validation + deferred launches) --------------------------------

struct RouteRes { uintptr_t logits, ids, weights; };
bool check_route(Check& c, const sm_moe_shape& s, const sm_route_buffers& b, RouteRes& r, bool logits_input) {
    uint64_t lb, ob;
    if (!mul_ok({s.rows, s.n_experts, 4}, lb) || !mul_ok({s.rows, s.top_k, 4}, ob))
        return c.fail(SM_E_SHAPE, c.prefix + " buffer size overflows");
    // Logits are an input of the route stage alone, and an output of route/gather.
    bool ok = c.view(b.logits, lb, 4, "logits", !logits_input, r.logits);
    ok = ok && c.view(b.ids, ob, 4, "route IDs", true, r.ids) && c.view(b.weights, ob, 4, "route weights", true, r.weights);
    return ok;
}

// hist (0: none): the grouping histogram that top-k counts its entries into (route/gather).
void encode_route_launch(sm_segment* seg, const sm_moe_shape& s, int divide, const RouteRes& r, uintptr_t hist = 0) {
    const auto rows = s.rows, E = s.n_experts, K = s.top_k;
    add_step(seg, "route top-k", [=](hipStream_t st) {
        return sm::launch_route_topk(reinterpret_cast<const float*>(r.logits), reinterpret_cast<int32_t*>(r.ids),
                                     reinterpret_cast<float*>(r.weights), rows, E, K, divide, st,
                                     reinterpret_cast<uint32_t*>(hist));
    });
}

struct GroupRes { uintptr_t ids, mixed, hist, plan, tiles, src, dst, gathered, resident; };

// The grouping histogram: the caller's view, or the fixed scratch (its view must then be null).
bool hist_view(Check& c, const sm_view& v, uint64_t bytes, uintptr_t& out) {
    if (c.fixed == nullptr) return c.view(v, bytes, 4, "histogram", true, out);
    if (v.buffer != 0) return c.fail(SM_E_ARGUMENT, c.prefix + " histogram view must be null: the fixed scratch holds it");
    if (bytes > kFixedHistBytes) {
        char msg[160];
        std::snprintf(msg, sizeof msg, " histogram needs %llu bytes, more than the fixed scratch's %llu",
                      (unsigned long long)bytes, (unsigned long long)kFixedHistBytes);
        return c.fail(SM_E_SHAPE, c.prefix + msg);
    }
    out = c.fixed->hist;
    return true;
}
// The residency table of tiered mode (prefill_moe_grouping.hpp:21-39): I32 [layer][E]; the
// grouping reads row `layer` (pre-offset here). A null view is full residency.
bool resident_view(Check& c, const sm_moe_shape& s, const sm_grouping_buffers& b, GroupRes& r) {
    r.resident = 0;
    if (b.resident.buffer == 0) return true;
    uint64_t need;
    if (!mul_ok({uint64_t(b.layer) + 1, s.n_experts, 4}, need))
        return c.fail(SM_E_SHAPE, c.prefix + " buffer size overflows");
    uintptr_t p;
    if (!c.view(b.resident, need, 4, "residency table", false, p)) return false;
    r.resident = p + uint64_t(b.layer) * s.n_experts * 4;
    return true;
}

bool check_grouping(Check& c, const sm_moe_shape& s, const sm_grouping_buffers& b, GroupRes& r) {
    const uint64_t N = uint64_t(s.rows) * s.top_k;
    if (N > 0x7fffffffull) return c.fail(SM_E_SHAPE, c.prefix + " entry count exceeds kernel indexing");
    uint64_t hist_b, tiles_b, route_b, mixed_b, gath_b;
    if (!mul_ok({ceil_div(N, SM_COUNT_TILE) + 1, s.n_experts, 4}, hist_b) ||
        !mul_ok({ceil_div(N, SM_EXPERT_TILE) + s.n_experts, 8}, tiles_b) || !mul_ok({N, 4}, route_b) ||
        !mul_ok({s.rows, s.hidden, 2}, mixed_b) || !mul_ok({N, s.hidden, 2}, gath_b))
        return c.fail(SM_E_SHAPE, c.prefix + " buffer size overflows");
    return c.view(b.ids, route_b, 4, "route IDs", false, r.ids) &&
           c.view(b.mixed_h, mixed_b, 16, "mixed activation", false, r.mixed) &&
           hist_view(c, b.histogram, hist_b, r.hist) &&
           c.view(b.plan, SM_PLAN_SLOT_BYTES, 4, "PfPlan slot", true, r.plan) &&
           c.view(b.tiles, tiles_b, 8, "tile list", true, r.tiles) &&
           c.view(b.source_rows, route_b, 4, "source rows", true, r.src) &&
           c.view(b.destination_rows, route_b, 4, "destination rows", true, r.dst) &&
           c.view(b.gathered_rows, gath_b, 16, "gathered rows", true, r.gathered) && resident_view(c, s, b, r);
}

// A full layer whose expert stages share one plan and tile list folds their checks into the
// grouping and the gather: the grouping's scan workgroup zeroes both status words and the
// destination bitset, and the gather launch runs the plan check (with the address-table
// snapshots from the two ring slots) and the destination marks.
struct LayerChecks {
    sm::GroupPrep prep;
    sm::PlanCheck check;
    const int32_t* dst;
    uint32_t* bits;
    int slot1, slot2;
};

// counted: top-k has counted the entries into the histogram already (route/gather).
void encode_grouping_launch(sm_segment* seg, const sm_moe_shape& s, const GroupRes& r,
                            const LayerChecks* lc = nullptr, bool counted = false) {
    const auto rows = s.rows, E = s.n_experts, K = s.top_k, d = s.hidden;
    const bool fused = lc != nullptr;
    const sm::GroupPrep prep = fused ? lc->prep : sm::GroupPrep{};
    add_step(seg, "grouping", [=](hipStream_t st) {
        return sm::launch_grouping(reinterpret_cast<const int32_t*>(r.ids), rows, K, E,
                                   reinterpret_cast<uint32_t*>(r.hist), reinterpret_cast<sm::Plan*>(r.plan),
                                   reinterpret_cast<uint32_t*>(r.tiles), reinterpret_cast<int32_t*>(r.src),
                                   reinterpret_cast<int32_t*>(r.dst), fused ? &prep : nullptr,
                                   reinterpret_cast<const int32_t*>(r.resident), st, counted);
    });
    if (!fused) {
        add_step(seg, "gather", [=](hipStream_t st) {
            return sm::launch_gather(reinterpret_cast<const _Float16*>(r.mixed), d,
                                     reinterpret_cast<const int32_t*>(r.ids),
                                     reinterpret_cast<const uint32_t*>(r.hist), K, E,
                                     reinterpret_cast<const sm::Plan*>(r.plan), rows * K,
                                     reinterpret_cast<_Float16*>(r.gathered), st);
        });
        return;
    }
    const LayerChecks l = *lc;
    add_step(seg, "gather + expert checks", [=](hipStream_t st) {
        return sm::launch_gather_checked(reinterpret_cast<const _Float16*>(r.mixed), d,
                                         reinterpret_cast<const int32_t*>(r.ids),
                                         reinterpret_cast<const uint32_t*>(r.hist), K, E,
                                         reinterpret_cast<const sm::Plan*>(r.plan), rows * K,
                                         reinterpret_cast<_Float16*>(r.gathered), l.check, l.dst, l.bits, st);
    });
    seg->steps.back().ring_slot = l.slot1;
    seg->steps.back().ring_slot2 = l.slot2;
}

struct RouterRes { uintptr_t x, w, bias, logits; };

// Expert weight table: validates every non-null address of the used roles against the
// declared storage (prefill_moe_expert_dispatch.mm:377-448) and snapshots the table.
struct WeightsRes { uintptr_t snapshot; std::vector<uint64_t> table; };
bool check_weights(Check& c, const sm_moe_shape& s, const sm_expert_weights& w, int fmt, bool gate_up,
                   WeightsRes& r) {
    if (w.addresses == nullptr) return c.fail(SM_E_ARGUMENT, c.prefix + " address table is null");
    if (w.layer >= w.n_layers)
        return c.fail(SM_E_ARGUMENT, c.prefix + " layer is outside the address table");
    const uint64_t E = s.n_experts;
    if (c.fixed != nullptr) {
        if (w.address_snapshot.buffer != 0)
            return c.fail(SM_E_ARGUMENT, c.prefix + " address snapshot view must be null: the fixed scratch holds it");
        r.snapshot = gate_up ? c.fixed->snap_gu : c.fixed->snap_dn;
    } else if (!c.view(w.address_snapshot, E * 3 * 8, 8, "address snapshot", true, r.snapshot)) {
        return false;
    }
    const uint64_t per_row = gate_up ? fmt_row_bytes(fmt, s.hidden) : fmt_row_bytes(fmt, s.expert_ff);
    uint64_t expert_bytes;
    if (!mul_ok({per_row, gate_up ? uint64_t(s.expert_ff) : uint64_t(s.hidden)}, expert_bytes) || per_row == 0)
        return c.fail(SM_E_SHAPE, c.prefix + " expert weight extent is invalid");
    std::vector<Range> storage;
    for (uint32_t i = 0; i < w.n_storage; ++i) {
        uintptr_t p;
        const sm_view& v = w.storage[i];
        if (!c.view(v, v.length, 1, "weight storage", false, p)) return false;
        storage.push_back({p, v.length, "weight storage", false, c.stage});
    }
    // Tiered mode: the expert store's slot arena is storage too, but a slot address counts only
    // while the lease set pins it for this layer (prefill_moe_expert_dispatch.mm:425-440).
    Range arena{};
    if (w.slot_arena.buffer != 0) {
        uintptr_t p;
        if (!c.view(w.slot_arena, w.slot_arena.length, 1, "slot arena", false, p)) return false;
        arena = {p, w.slot_arena.length, "slot arena", false, c.stage};
        storage.push_back(arena);
    }
    const uint64_t* row = w.addresses + uint64_t(w.layer) * E * 3;  // the selected layer's [E][3]
    r.table.assign(row, row + E * 3);
    const uint64_t align = weight_align(fmt);
    for (uint64_t e = 0; e < E; ++e) {
        for (int role = 0; role < 3; ++role) {
            if (gate_up ? role == 2 : role != 2) continue;
            const uint64_t a = r.table[e * 3 + role];
            if (a == 0) continue;  // reported on the GPU (status bit 0) if the expert is active
            bool inside = false;
            for (const auto& st : storage)
                if (a >= st.ptr && a - st.ptr <= st.bytes && expert_bytes <= st.bytes - (a - st.ptr)) inside = true;
            if (!inside || a % align != 0) {
                char msg[160];
                std::snprintf(msg, sizeof msg, " expert %llu %s address is outside declared storage or misaligned",
                              (unsigned long long)e, role == 0 ? "gate" : (role == 1 ? "up" : "down"));
                return c.fail(SM_E_ADDRESS, c.prefix + msg);
            }
            // An unpinned slot address is tagged in bit 0: the kernels then report status
            // bit 2 for the expert (if it is active) and zero its rows instead of reading it.
            if (arena.bytes != 0 && a >= arena.ptr && a - arena.ptr < arena.bytes &&
                !(w.leases != nullptr && sm_lease_set_pins(w.leases, w.layer, a, expert_bytes)))
                r.table[e * 3 + role] |= 1u;
        }
    }
    return true;
}

// Copies a validated table into a pinned ring slot; the plan-validation kernel of the
// stage copies it on to the device snapshot. Returns the slot (-1 without a device).
// Returns -2 when every slot belongs to a segment that has not been committed or aborted,
// -3 when waiting for a slot's previous copy failed.
int claim_ring_slot(sm_context* ctx, const std::vector<uint64_t>& table) {
    if (ctx->ring == nullptr) return -1;
    std::lock_guard<std::mutex> lk(ctx->ring_mu);
    for (uint32_t tries = 0; tries < sm_context::kRingSlots; ++tries) {
        const uint32_t slot = ctx->ring_next++ % sm_context::kRingSlots;
        if (ctx->ring_claimed[slot]) continue;
        if (ctx->ring_pending[slot]) {
            int waited = slot;
            if (ctx->ring_alias[slot] >= 0) {
                const int a = ctx->ring_alias[slot];
                waited = ctx->ring_pending[a] ? a : -1;
            }
            if (waited >= 0) {
                if (hipEventSynchronize(ctx->ring_ev[waited]) != hipSuccess) return -3;
                ctx->ring_pending[waited] = false;
            }
            ctx->ring_pending[slot] = false;
        }
        ctx->ring_claimed[slot] = true;
        std::memcpy(ctx->ring + uint64_t(slot) * sm_context::kSlotWords, table.data(), table.size() * 8);
        return int(slot);
    }
    return -2;
}

void release_ring_slots(sm_segment* seg) {
    std::lock_guard<std::mutex> lk(seg->ctx->ring_mu);
    for (const auto& step : seg->steps)
        for (const int slot : {step.ring_slot, step.ring_slot2})
            if (slot >= 0) seg->ctx->ring_claimed[slot] = false;
}

struct GateUpRes { WeightsRes w; uintptr_t xs, plan, tiles, hidden, status; };
bool check_gate_up(Check& c, const sm_moe_shape& s, int fmt, const sm_gate_up_buffers& b, GateUpRes& r) {
    if (!routed_fmt(fmt)) return c.fail(SM_E_FORMAT, c.prefix + " weight format is not a supported block format");
    if (!k_ok(fmt, s.hidden) || s.expert_ff % 64 != 0)
        return c.fail(SM_E_SHAPE, c.prefix + " widths do not fit the weight format's blocks");
    const uint64_t N = uint64_t(s.rows) * s.top_k;
    uint64_t xs_b, h_b, tiles_b;
    if (!mul_ok({N, s.hidden, 2}, xs_b) || !mul_ok({N, s.expert_ff, 2}, h_b) ||
        !mul_ok({ceil_div(N, SM_EXPERT_TILE) + s.n_experts, 8}, tiles_b))
        return c.fail(SM_E_SHAPE, c.prefix + " buffer size overflows");
    return check_weights(c, s, b.weights, fmt, true, r.w) &&
           c.view(b.gathered_rows, xs_b, 16, "gathered rows", false, r.xs) &&
           c.plan_view(b.plan, sm::kCounterBytes, sm::kCounterWords, r.plan) &&
           c.view(b.tiles, tiles_b, 8, "tile list", false, r.tiles) &&
           c.view(b.hidden, h_b, 16, "hidden", true, r.hidden) &&
           c.view(b.status, 4, 4, "status", true, r.status);
}

sm::RoutedGemm gate_up_gemm(const sm_moe_shape& s, int fmt, const GateUpRes& r) {
    const uint32_t N = s.rows * s.top_k;
    sm::RoutedGemm g{};
    g.addresses = reinterpret_cast<const uint64_t*>(r.w.snapshot);
    g.a = reinterpret_cast<const _Float16*>(r.xs);
    g.plan = reinterpret_cast<const sm::Plan*>(r.plan);
    g.tiles = reinterpret_cast<const uint32_t*>(r.tiles);
    g.out_h = reinterpret_cast<_Float16*>(r.hidden);
    g.status = reinterpret_cast<uint32_t*>(r.status);
    g.n_entries = N;
    g.n_experts = s.n_experts;
    g.tile_capacity = uint32_t(ceil_div(N, SM_EXPERT_TILE) + s.n_experts);
    g.k = s.hidden;
    g.n_out = s.expert_ff;
    g.row_bytes = fmt_row_bytes(fmt, s.hidden);
    g.wide_min = sm::wide_fits(Fmt(fmt), true, g.k, g.n_out) ? sm::kWideMin : ~0u;
    g.counters = reinterpret_cast<uint32_t*>(r.plan + sm::kCounterBytes);
    return g;
}

// Plan check of one stage, with its snapshot copy from ring slot `slot` (-1: none).
sm::PlanCheck stage_check(sm_context* ctx, const sm::RoutedGemm& g, int slot, uintptr_t snapshot, uint32_t words) {
    sm::PlanCheck c{};
    c.plan = g.plan;
    c.tiles = g.tiles;
    c.status = g.status;
    c.n_entries = g.n_entries;
    c.n_experts = g.n_experts;
    c.tile_capacity = g.tile_capacity;
    c.snap_src = slot >= 0 ? ctx->ring + uint64_t(slot) * sm_context::kSlotWords : nullptr;
    c.snap_dst = reinterpret_cast<uint64_t*>(snapshot);
    c.snap_words = words;
    c.counters = g.counters;
    c.n_counters = sm::kCounterWords;
    return c;
}

sm_status claim_status(int slot) { return slot == -2 ? SM_E_SEGMENT : slot == -3 ? SM_E_DEVICE : SM_OK; }

// The chunks of one prompt (sm_encode_prefill_moe_chunks) run the same layer over the same
// weights: the first chunk claims the pinned ring slots of the address tables and the later
// chunks read the same slots, and only the first chunk clears the status words.
struct ChunkCtl {
    bool keep_status = false;
    int slot_gu = -9, slot_dn = -9;  // -9: not claimed yet
};

// A ring slot for one expert stage: the chunk's slot when it has one, else a new claim
// (recorded in the chunk control for the later chunks).
int stage_slot(sm_segment* seg, const std::vector<uint64_t>& table, int* chunk_slot) {
    if (chunk_slot != nullptr && *chunk_slot != -9) return *chunk_slot;
    const int slot = claim_ring_slot(seg->ctx, table);
    if (chunk_slot != nullptr && claim_status(slot) == SM_OK) *chunk_slot = slot;
    return slot;
}

sm_status encode_gate_up_launch(sm_segment* seg, const sm_moe_shape& s, int fmt, const GateUpRes& r,
                                ChunkCtl* ctl = nullptr) {
    const int slot = stage_slot(seg, r.w.table, ctl ? &ctl->slot_gu : nullptr);
    if (claim_status(slot) != SM_OK) return claim_status(slot);
    const sm::RoutedGemm g = gate_up_gemm(s, fmt, r);
    sm::PlanCheck c = stage_check(seg->ctx, g, slot, r.w.snapshot, uint32_t(r.w.table.size()));
    c.keep_status = ctl && ctl->keep_status ? 1u : 0u;
    add_step(seg, "gate/up plan validate", [=](hipStream_t st) { return sm::launch_plan_validate(c, st); });
    seg->steps.back().ring_slot = slot;
    add_step(seg, "gate/up tiles", [=](hipStream_t st) { return sm::launch_gate_up(Fmt(fmt), g, st); });
    return SM_OK;
}

struct DownRes { WeightsRes w; uintptr_t hidden, plan, tiles, dst, parts, status; };
bool check_down(Check& c, const sm_moe_shape& s, int fmt, const sm_down_buffers& b, DownRes& r) {
    if (!routed_fmt(fmt)) return c.fail(SM_E_FORMAT, c.prefix + " weight format is not a supported block format");
    if (!k_ok(fmt, s.expert_ff) || s.hidden % 128 != 0)
        return c.fail(SM_E_SHAPE, c.prefix + " widths do not fit the weight format's blocks");
    const uint64_t N = uint64_t(s.rows) * s.top_k;
    uint64_t h_b, p_b, tiles_b;
    if (!mul_ok({N, s.expert_ff, 2}, h_b) || !mul_ok({N, s.hidden, 4}, p_b) ||
        !mul_ok({ceil_div(N, SM_EXPERT_TILE) + s.n_experts, 8}, tiles_b))
        return c.fail(SM_E_SHAPE, c.prefix + " buffer size overflows");
    return check_weights(c, s, b.weights, fmt, false, r.w) &&
           c.view(b.hidden, h_b, 16, "hidden", false, r.hidden) &&
           c.plan_view(b.plan, sm::kCounterBytes + 4 * sm::kCounterWords, sm::kCounterWords, r.plan) &&
           c.view(b.tiles, tiles_b, 8, "tile list", false, r.tiles) &&
           c.view(b.destinations, N * 4, 4, "destinations", false, r.dst) &&
           c.view(b.parts, p_b, 16, "parts", true, r.parts) &&
           c.view(b.status, 4, 4, "status", true, r.status);
}

sm::RoutedGemm down_gemm(const sm_moe_shape& s, int fmt, const DownRes& r) {
    const uint32_t N = s.rows * s.top_k;
    sm::RoutedGemm g{};
    g.addresses = reinterpret_cast<const uint64_t*>(r.w.snapshot);
    g.a = reinterpret_cast<const _Float16*>(r.hidden);
    g.plan = reinterpret_cast<const sm::Plan*>(r.plan);
    g.tiles = reinterpret_cast<const uint32_t*>(r.tiles);
    g.dst = reinterpret_cast<const int32_t*>(r.dst);
    g.out_f = reinterpret_cast<float*>(r.parts);
    g.status = reinterpret_cast<uint32_t*>(r.status);
    g.n_entries = N;
    g.n_experts = s.n_experts;
    g.tile_capacity = uint32_t(ceil_div(N, SM_EXPERT_TILE) + s.n_experts);
    g.k = s.expert_ff;
    g.n_out = s.hidden;
    g.row_bytes = fmt_row_bytes(fmt, s.expert_ff);
    g.wide_min = sm::wide_fits(Fmt(fmt), false, g.k, g.n_out) ? sm::kWideMin : ~0u;
    g.counters = reinterpret_cast<uint32_t*>(r.plan + sm::kCounterBytes + 4 * sm::kCounterWords);
    return g;
}

// The destination bitset borrows the head of `parts`, which the down tiles overwrite
// (the reference's prefill_moe_down_dispatch.mm:470-520 does the same).
void add_down_tail(sm_segment* seg, int fmt, const sm::RoutedGemm& g, bool bitset_clear) {
    add_step(seg, "down destination validate", [=](hipStream_t st) {
        return sm::launch_destination_validate(g.dst, reinterpret_cast<uint32_t*>(g.out_f), g.status, g.n_entries,
                                               bitset_clear, st);
    });
    add_step(seg, "down tiles", [=](hipStream_t st) { return sm::launch_down(Fmt(fmt), g, st); });
}

sm_status encode_down_launch(sm_segment* seg, const sm_moe_shape& s, int fmt, const DownRes& r,
                             ChunkCtl* ctl = nullptr) {
    const int slot = stage_slot(seg, r.w.table, ctl ? &ctl->slot_dn : nullptr);
    if (claim_status(slot) != SM_OK) return claim_status(slot);
    const sm::RoutedGemm g = down_gemm(s, fmt, r);
    sm::PlanCheck c = stage_check(seg->ctx, g, slot, r.w.snapshot, uint32_t(r.w.table.size()));
    c.keep_status = ctl && ctl->keep_status ? 1u : 0u;
    add_step(seg, "down plan validate", [=](hipStream_t st) { return sm::launch_plan_validate(c, st); });
    seg->steps.back().ring_slot = slot;
    add_down_tail(seg, fmt, g, true);
    return SM_OK;
}

// Both expert stages on one plan and tile list: the plan is checked once, for both status
// words, and the same launch copies both address snapshots and clears the destination
// bitset. Claims the two ring slots (released again if the second claim fails).
struct ExpertsPlan {
    sm::RoutedGemm g, d;
    sm::PlanCheck check;
    int slot1, slot2;
};
sm_status prepare_experts(sm_segment* seg, const sm_moe_shape& s, int fmt_gu, const GateUpRes& gu, int fmt_dn,
                          const DownRes& dn, ExpertsPlan& x, ChunkCtl* ctl = nullptr) {
    const bool had_gu = ctl != nullptr && ctl->slot_gu != -9;
    x.slot1 = stage_slot(seg, gu.w.table, ctl ? &ctl->slot_gu : nullptr);
    if (claim_status(x.slot1) != SM_OK) return claim_status(x.slot1);
    x.slot2 = stage_slot(seg, dn.w.table, ctl ? &ctl->slot_dn : nullptr);
    if (claim_status(x.slot2) != SM_OK) {
        if (x.slot1 >= 0 && !had_gu) {
            std::lock_guard<std::mutex> lk(seg->ctx->ring_mu);
            seg->ctx->ring_claimed[x.slot1] = false;
        }
        return claim_status(x.slot2);
    }
    x.g = gate_up_gemm(s, fmt_gu, gu);
    x.d = down_gemm(s, fmt_dn, dn);
    sm::PlanCheck& c = x.check;
    c = stage_check(seg->ctx, x.g, x.slot1, gu.w.snapshot, uint32_t(gu.w.table.size()));
    const sm::PlanCheck c2 = stage_check(seg->ctx, x.d, x.slot2, dn.w.snapshot, uint32_t(dn.w.table.size()));
    c.status2 = x.d.status;
    c.snap_src2 = c2.snap_src;
    c.snap_dst2 = c2.snap_dst;
    c.snap_words2 = c2.snap_words;
    c.clear = reinterpret_cast<uint32_t*>(x.d.out_f);
    c.clear_words = uint32_t(ceil_div(x.d.n_entries, 32));
    c.n_counters = 2 * sm::kCounterWords;  // gate/up's counters, then down's
    c.keep_status = ctl && ctl->keep_status ? 1u : 0u;
    return SM_OK;
}

// Stages with distinct plan or tile views are encoded separately.
sm_status encode_experts_launch(sm_segment* seg, const sm_moe_shape& s, int fmt_gu, const GateUpRes& gu, int fmt_dn,
                                const DownRes& dn, ChunkCtl* ctl = nullptr) {
    if (gu.plan != dn.plan || gu.tiles != dn.tiles) {
        sm_status st = encode_gate_up_launch(seg, s, fmt_gu, gu, ctl);
        return st != SM_OK ? st : encode_down_launch(seg, s, fmt_dn, dn, ctl);
    }
    ExpertsPlan x;
    const sm_status st = prepare_experts(seg, s, fmt_gu, gu, fmt_dn, dn, x, ctl);
    if (st != SM_OK) return st;
    const sm::PlanCheck c = x.check;
    const sm::RoutedGemm g = x.g;
    add_step(seg, "expert plan validate", [=](hipStream_t st) { return sm::launch_plan_validate(c, st); });
    seg->steps.back().ring_slot = x.slot1;
    seg->steps.back().ring_slot2 = x.slot2;
    add_step(seg, "gate/up tiles", [=](hipStream_t st) { return sm::launch_gate_up(Fmt(fmt_gu), g, st); });
    add_down_tail(seg, fmt_dn, x.d, false);
    return SM_OK;
}

struct SharedRes { uintptr_t x, wg, wu, wd, gv, hidden, out, gl; };
bool check_shared(Check& c, const sm_moe_shape& s, int fmt, const sm_shared_buffers& b, SharedRes& r) {
    if (!dense_fmt(fmt)) return c.fail(SM_E_FORMAT, c.prefix + " shared expert format must be F16 or BF16");
    const uint64_t Is = s.shared_ff;
    if (Is == 0 || Is % 256 != 0 || s.hidden % 128 != 0)
        return c.fail(SM_E_SHAPE, c.prefix + " shared expert width must be a positive multiple of 256");
    uint64_t x_b, w_b, h_b, o_b;
    if (!mul_ok({s.rows, s.hidden, 2}, x_b) || !mul_ok({Is, s.hidden, 2}, w_b) || !mul_ok({s.rows, Is, 2}, h_b) ||
        !mul_ok({s.rows, s.hidden, 4}, o_b))
        return c.fail(SM_E_SHAPE, c.prefix + " buffer size overflows");
    return c.view(b.mixed_h, x_b, 16, "mixed activation", false, r.x) &&
           c.view(b.gate_weights, w_b, 16, "gate weights", false, r.wg) &&
           c.view(b.up_weights, w_b, 16, "up weights", false, r.wu) &&
           c.view(b.down_weights, w_b, 16, "down weights", false, r.wd) &&
           c.view(b.gate_vector, uint64_t(s.hidden) * 2, 16, "gate vector", false, r.gv) &&
           c.view(b.hidden, h_b, 16, "hidden", true, r.hidden) &&
           c.view(b.output, o_b, 16, "output", true, r.out) &&
           c.view(b.gate_logit, uint64_t(s.rows) * 4, 4, "gate logit", true, r.gl);
}

// side: the launches go to the context's side stream (a full layer, where nothing before
// them in the segment writes what they read).
void encode_shared_launch(sm_segment* seg, const sm_moe_shape& s, int fmt, const SharedRes& r, bool side = false) {
    sm::DenseGemm gu{};
    gu.a = reinterpret_cast<const _Float16*>(r.x);
    gu.w0 = reinterpret_cast<const uint8_t*>(r.wg);
    gu.w1 = reinterpret_cast<const uint8_t*>(r.wu);
    gu.out_h = reinterpret_cast<_Float16*>(r.hidden);
    gu.rows = s.rows;
    gu.k = s.hidden;
    gu.n_out = s.shared_ff;
    gu.row_bytes = 2ull * s.hidden;
    sm::DenseGemm dn{};
    dn.a = reinterpret_cast<const _Float16*>(r.hidden);
    dn.w0 = reinterpret_cast<const uint8_t*>(r.wd);
    dn.out_f = reinterpret_cast<float*>(r.out);
    dn.rows = s.rows;
    dn.k = s.shared_ff;
    dn.n_out = s.hidden;
    dn.row_bytes = 2ull * s.shared_ff;
    const auto rows = s.rows, d = s.hidden;
    const uintptr_t x = r.x, gv = r.gv, gl = r.gl;
    add_step(seg, "shared gate/up", [=](hipStream_t st) { return sm::launch_dense_gate_up(Fmt(fmt), gu, st); }, side);
    add_step(seg, "shared down", [=](hipStream_t st) { return sm::launch_dense_down(Fmt(fmt), dn, st); }, side);
    add_step(seg, "shared gate logit", [=](hipStream_t st) {
        return sm::launch_gate_logit(Fmt(fmt), reinterpret_cast<const _Float16*>(x), reinterpret_cast<const uint8_t*>(gv),
                                     reinterpret_cast<float*>(gl), rows, d, st);
    }, side);
}

struct CombineRes { uintptr_t parts, weights, shared, gate, out; };
bool check_combine(Check& c, const sm_moe_shape& s, const sm_combine_buffers& b, CombineRes& r) {
    if (s.hidden % 4 != 0) return c.fail(SM_E_SHAPE, c.prefix + " hidden width must be a multiple of 4");
    uint64_t p_b, w_b, o_b;
    if (!mul_ok({s.rows, s.top_k, s.hidden, 4}, p_b) || !mul_ok({s.rows, s.top_k, 4}, w_b) ||
        !mul_ok({s.rows, s.hidden, 4}, o_b))
        return c.fail(SM_E_SHAPE, c.prefix + " buffer size overflows");
    r.shared = r.gate = 0;
    bool ok = c.view(b.parts, p_b, 16, "parts", false, r.parts) && c.view(b.weights, w_b, 4, "weights", false, r.weights);
    if (ok && s.shared_ff != 0)
        ok = c.view(b.shared, o_b, 16, "shared", false, r.shared) &&
             c.view(b.gate, uint64_t(s.rows) * 4, 4, "gate", false, r.gate);
    return ok && c.view(b.output, o_b, 16, "output", true, r.out);
}

void encode_combine_launch(sm_segment* seg, const sm_moe_shape& s, const CombineRes& r, bool join = false) {
    const auto rows = s.rows, K = s.top_k, d = s.hidden;
    add_step(seg, "combine", [=](hipStream_t st) {
        return sm::launch_combine(reinterpret_cast<const float*>(r.parts), reinterpret_cast<const float*>(r.weights),
                                  reinterpret_cast<const float*>(r.shared), reinterpret_cast<const float*>(r.gate),
                                  reinterpret_cast<float*>(r.out), rows, K, d, st);
    }, false, join);
}

const char* const kRingFull =
    "Prefill MoE expert stage: 64 expert stages are encoded but neither committed nor aborted";
const char* const kRingWait = "Prefill MoE expert stage: waiting for an address-table copy failed";

sm_status ring_fail(sm_segment* seg, sm_status st) {
    return record_fail(seg, st, st == SM_E_DEVICE ? kRingWait : kRingFull);
}

sm_status begin_check(sm_segment* seg, const char* prefix, Check& c) {
    if (seg == nullptr) return SM_E_ARGUMENT;
    c.ctx = seg->ctx;
    c.prefix = prefix;
    if (seg->failed) return SM_E_SEGMENT;
    return SM_OK;
}

sm_status finish(sm_segment* seg, Check& c) {
    if (c.st != SM_OK) return record_fail(seg, c.st, c.err);
    return SM_OK;
}

// Cross-stage dataflow edges a full layer may alias (prefill_moe_full_pipeline.cpp:109-162):
// a writer and a reader of a later stage may share memory only on these edges, and only
// when they start at the same address and the reader lies inside the writer.
bool expected_edge(const Range& w, const Range& r) {
    static const char* const edges[][2] = {
        {"route.gathered rows", "gate_up.gathered rows"}, {"route.PfPlan slot", "gate_up.PfPlan slot"},
        {"route.PfPlan slot", "down.PfPlan slot"},       {"route.tile list", "gate_up.tile list"},
        {"route.tile list", "down.tile list"},           {"route.destination rows", "down.destinations"},
        {"route.route weights", "combine.weights"},      {"shared.output", "combine.shared"},
        {"shared.gate logit", "combine.gate"},           {"gate_up.hidden", "down.hidden"},
        {"down.parts", "combine.parts"},
    };
    if (!w.writable || w.stage >= r.stage) return false;
    // The expert stages' work counters lie in the padding of the plan slot the grouping
    // wrote; each stage owns its own words, so a later stage may write inside that range.
    static const char* const scratch[][2] = {
        {"route.PfPlan slot", "gate_up.work counters"}, {"route.PfPlan slot", "down.work counters"},
    };
    if (r.writable) {
        for (const auto& e : scratch)
            if (w.name == e[0] && r.name == e[1]) return r.ptr >= w.ptr && r.ptr + r.bytes <= w.ptr + w.bytes;
        return false;
    }
    for (const auto& e : edges)
        if (w.name == e[0] && r.name == e[1]) return w.ptr == r.ptr && r.bytes <= w.bytes;
    return false;
}

}  // namespace

extern "C" {

uint32_t sm_abi_version(void) { return SM_ABI_VERSION; }

sm_status sm_internal_make_current(sm_context* ctx) {
    if (!ctx || !ctx->has_device || hipSetDevice(ctx->device) != hipSuccess) return SM_E_DEVICE;
    return SM_OK;
}

sm_status sm_internal_resolve_view(sm_context* ctx, sm_view v, uint64_t need, uint64_t align, uintptr_t* out) {
    if (!ctx || !out || align == 0) return SM_E_ARGUMENT;
    sm_context::Alloc a{};
    {
        std::lock_guard<std::mutex> lk(ctx->mu);
        auto it = ctx->buffers.find(v.buffer);
        if (v.buffer == 0 || it == ctx->buffers.end()) return SM_E_OWNERSHIP;
        a = it->second;
    }
    const uint64_t end = v.offset + v.length;
    const uintptr_t p = a.ptr + v.offset;
    if (end < v.offset || end > a.bytes || v.length < need || p % align != 0) return SM_E_VIEW;
    *out = p;
    return SM_OK;
}

uint64_t sm_histogram_bytes(const sm_moe_shape* s) {
    if (!s) return 0;
    const uint64_t N = uint64_t(s->rows) * s->top_k;
    return (ceil_div(N, SM_COUNT_TILE) + 1) * s->n_experts * 4;
}
uint64_t sm_tiles_bytes(const sm_moe_shape* s) {
    if (!s) return 0;
    const uint64_t N = uint64_t(s->rows) * s->top_k;
    return (ceil_div(N, SM_EXPERT_TILE) + s->n_experts) * 8;
}
uint64_t sm_format_row_bytes(sm_format fmt, uint64_t values) { return fmt_row_bytes(fmt, values); }

sm_status sm_context_create(int device, sm_context** out) {
    if (out == nullptr || device < 0) return SM_E_ARGUMENT;
    // A context without a visible device still validates and encodes (host-only use,
    // e.g. preflight tests); commit then reports SM_E_DEVICE.
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    if (n > 0 && device >= n) return SM_E_DEVICE;
    auto* c = new (std::nothrow) sm_context();
    if (!c) return SM_E_DEVICE;
    c->device = device;
    c->has_device = n > 0;
    if (c->has_device) {
        bool ok = hipSetDevice(device) == hipSuccess &&
                  hipHostMalloc(reinterpret_cast<void**>(&c->ring),
                                sizeof(uint64_t) * sm_context::kSlotWords * sm_context::kRingSlots,
                                hipHostMallocDefault) == hipSuccess;
        for (uint32_t i = 0; ok && i < sm_context::kRingSlots; ++i) {
            c->ring_alias[i] = -1;
            ok = hipEventCreateWithFlags(&c->ring_ev[i], hipEventDisableTiming) == hipSuccess;
        }
        ok = ok && hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking) == hipSuccess &&
             hipEventCreateWithFlags(&c->fork_ev, hipEventDisableTiming) == hipSuccess &&
             hipEventCreateWithFlags(&c->join_ev, hipEventDisableTiming) == hipSuccess;
        if (ok) c->fixed_scratch = fixed_scratch_of(device);  // device is current here
        if (!ok) {
            sm_context_destroy(c);
            return SM_E_DEVICE;
        }
    }
    *out = c;
    return SM_OK;
}

void sm_context_destroy(sm_context* ctx) {
    if (!ctx) return;
    // Teardown is best effort: a failed wait or release leaves nothing the caller can act on.
    for (uint32_t i = 0; i < sm_context::kRingSlots; ++i) {
        if (ctx->ring_ev[i] == nullptr) continue;
        if (ctx->ring_pending[i] && ctx->ring_alias[i] < 0) (void)hipEventSynchronize(ctx->ring_ev[i]);
        (void)hipEventDestroy(ctx->ring_ev[i]);
    }
    if (ctx->ring) (void)hipHostFree(ctx->ring);
    if (ctx->side) {
        (void)hipStreamSynchronize(ctx->side);
        (void)hipStreamDestroy(ctx->side);
    }
    if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
    if (ctx->join_ev) (void)hipEventDestroy(ctx->join_ev);
    delete ctx;
}

sm_status sm_buffer_register(sm_context* ctx, void* ptr, uint64_t bytes, uint64_t* handle) {
    if (!ctx || !ptr || !handle || bytes == 0) return SM_E_ARGUMENT;
    std::lock_guard<std::mutex> lk(ctx->mu);
    const uint64_t h = g_next_handle.fetch_add(1);
    ctx->buffers[h] = {reinterpret_cast<uintptr_t>(ptr), bytes};
    *handle = h;
    return SM_OK;
}

sm_status sm_buffer_unregister(sm_context* ctx, uint64_t handle) {
    if (!ctx) return SM_E_ARGUMENT;
    std::lock_guard<std::mutex> lk(ctx->mu);
    return ctx->buffers.erase(handle) ? SM_OK : SM_E_OWNERSHIP;
}

sm_status sm_segment_begin(sm_context* ctx, sm_segment** out) {
    if (!ctx || !out) return SM_E_ARGUMENT;
    auto* s = new (std::nothrow) sm_segment();
    if (!s) return SM_E_DEVICE;
    s->ctx = ctx;
    *out = s;
    return SM_OK;
}

namespace {

// Runs the recorded launches in order on `stream`. With `ev` (two events per launch), each
// launch is bracketed by event records for sm_segment_commit_timed, and every launch runs
// on `stream`. Without it, side steps run on the context's side stream: it waits for a fork
// event recorded on `stream` before the first launch, and `stream` waits for a join event
// recorded on the side stream before each join step and, if side launches follow the last
// join, at the end, so the caller's stream orders after all of the segment's work.
sm_status run_segment(sm_segment* seg, hipStream_t stream, hipEvent_t* ev) {
    sm_status st = SM_OK;
    sm_context* ctx = seg->ctx;
    if (!ctx->has_device || hipSetDevice(ctx->device) != hipSuccess) st = SM_E_DEVICE;
    // The expert address tables reach the GPU from the context's pinned host ring, whose slots
    // are reused once the launch that read them has run. A captured graph would copy from its
    // slot again at every replay, after later commits rewrote it, so no segment runs on a
    // stream that is capturing.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (st == SM_OK && (hipStreamIsCapturing(stream, &capture) != hipSuccess || capture != hipStreamCaptureStatusNone))
        st = SM_E_ARGUMENT;
    bool use_side = false;
    for (const auto& step : seg->steps) use_side = use_side || (step.side && ev == nullptr);
    std::unique_lock<std::mutex> side_lk(ctx->side_mu, std::defer_lock);
    if (use_side) side_lk.lock();
    bool side_open = false;     // side launches not yet joined
    bool forked = false;        // the side stream waits for some point of this segment
    bool fork_pending = false;  // a fork event the next side launch must wait for
    auto fork = [&]() {
        if (st == SM_OK && hipEventRecord(ctx->fork_ev, stream) != hipSuccess) st = SM_E_DEVICE;
        fork_pending = true;
    };
    // Also after a failed launch: the caller's stream must not run ahead of side launches
    // already queued (a caller may free the buffers they write once its stream is idle).
    // If the join itself cannot be recorded, the side stream is drained instead.
    auto join = [&]() {
        if (hipEventRecord(ctx->join_ev, ctx->side) != hipSuccess ||
            hipStreamWaitEvent(stream, ctx->join_ev, 0) != hipSuccess) {
            (void)hipStreamSynchronize(ctx->side);  // best effort; the failure is reported below
            st = SM_E_DEVICE;
        }
        side_open = false;
    };
    for (size_t i = 0; i < seg->steps.size(); ++i) {
        auto& step = seg->steps[i];
        if (st != SM_OK) break;
        if (step.join && side_open) join();
        if (st != SM_OK) break;
        if (use_side && step.fork_before) fork();
        const hipStream_t hs = use_side && step.side ? ctx->side : stream;
        if (hs != stream) {
            if (!forked && !fork_pending) fork();
            if (st == SM_OK && fork_pending && hipStreamWaitEvent(ctx->side, ctx->fork_ev, 0) != hipSuccess)
                st = SM_E_DEVICE;
            fork_pending = false;
            forked = true;
        }
        side_open = side_open || hs != stream;
        if (st == SM_OK && ev && hipEventRecord(ev[2 * i], hs) != hipSuccess) st = SM_E_DEVICE;
        if (st == SM_OK && step.run(hs) != hipSuccess) st = SM_E_DEVICE;
        if (st == SM_OK && ev && hipEventRecord(ev[2 * i + 1], hs) != hipSuccess) st = SM_E_DEVICE;
        const int s1 = step.ring_slot >= 0 ? step.ring_slot : step.ring_slot2;
        const int s2 = step.ring_slot >= 0 ? step.ring_slot2 : -1;
        if (s1 >= 0) {
            std::lock_guard<std::mutex> lk(ctx->ring_mu);
            if (hipEventRecord(ctx->ring_ev[s1], hs) == hipSuccess) {
                ctx->ring_pending[s1] = true;
                ctx->ring_alias[s1] = -1;
                if (s2 >= 0) {
                    ctx->ring_pending[s2] = true;
                    ctx->ring_alias[s2] = s1;
                }
            } else {
                st = SM_E_DEVICE;
            }
        }
    }
    if (side_open) join();
    release_ring_slots(seg);
    return st;
}

}  // namespace

sm_status sm_segment_commit(sm_segment* seg, void* stream) {
    if (!seg) return SM_E_ARGUMENT;
    if (seg->failed) { release_ring_slots(seg); delete seg; return SM_E_SEGMENT; }
    const sm_status st = run_segment(seg, reinterpret_cast<hipStream_t>(stream), nullptr);
    delete seg;
    return st;
}

sm_status sm_segment_commit_timed(sm_segment* seg, void* stream, float* ms, const char** labels, uint32_t cap,
                                  uint32_t* n_launches) {
    if (!seg) return SM_E_ARGUMENT;
    if (seg->failed || !ms || !n_launches || cap < seg->steps.size()) {
        const bool failed = seg->failed;
        release_ring_slots(seg);
        delete seg;
        return failed ? SM_E_SEGMENT : SM_E_ARGUMENT;
    }
    const size_t n = seg->steps.size();
    std::vector<hipEvent_t> ev(2 * n, nullptr);
    sm_status st = SM_OK;
    if (!seg->ctx->has_device || hipSetDevice(seg->ctx->device) != hipSuccess) st = SM_E_DEVICE;
    for (size_t i = 0; i < ev.size() && st == SM_OK; ++i)
        if (hipEventCreate(&ev[i]) != hipSuccess) st = SM_E_DEVICE;
    const hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
    if (st == SM_OK) st = run_segment(seg, hs, ev.data());
    else release_ring_slots(seg);
    if (st == SM_OK && hipStreamSynchronize(hs) != hipSuccess) st = SM_E_DEVICE;
    for (size_t i = 0; i < n && st == SM_OK; ++i) {
        if (hipEventElapsedTime(&ms[i], ev[2 * i], ev[2 * i + 1]) != hipSuccess) st = SM_E_DEVICE;
        if (labels) labels[i] = seg->steps[i].label;
    }
    *n_launches = st == SM_OK ? uint32_t(n) : 0u;
    for (hipEvent_t e : ev)
        if (e) (void)hipEventDestroy(e);  // best effort: nothing to report to the caller
    delete seg;
    return st;
}

void sm_segment_abort(sm_segment* seg) {
    if (!seg) return;
    release_ring_slots(seg);
    delete seg;
}

const char* sm_segment_error(const sm_segment* seg) { return seg ? seg->error.c_str() : ""; }
uint32_t sm_segment_launches(const sm_segment* seg) { return seg ? uint32_t(seg->steps.size()) : 0; }

sm_status sm_encode_route(sm_segment* seg, const sm_moe_shape* shape, int divide, const sm_route_buffers* b) {
    Check c;
    sm_status st = begin_check(seg, "MoE route", c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = shape_check(shape, "MoE route", err, false)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, "MoE route buffers are null");
    RouteRes r{};
    if (!check_route(c, *shape, *b, r, true) || !c.aliases()) return finish(seg, c);
    encode_route_launch(seg, *shape, divide, r);
    return SM_OK;
}

sm_status sm_encode_grouping(sm_segment* seg, const sm_moe_shape* shape, const sm_grouping_buffers* b) {
    Check c;
    sm_status st = begin_check(seg, "Prefill MoE grouping", c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = shape_check(shape, "Prefill MoE grouping", err, false)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, "Prefill MoE grouping buffers are null");
    GroupRes r{};
    if (!check_grouping(c, *shape, *b, r) || !c.aliases()) return finish(seg, c);
    encode_grouping_launch(seg, *shape, r);
    return SM_OK;
}

namespace {
// Validates the route+gather composition and returns its ranges (stage-tagged "route.").
bool check_route_gather(Check& c, const sm_moe_shape& s, const sm_route_gather_buffers& b, RouterRes& rr,
                        RouteRes& ro, GroupRes& gr) {
    uint64_t x_b, w_b;
    if (!mul_ok({s.rows, s.hidden, 2}, x_b) || !mul_ok({s.n_experts, s.hidden, 4}, w_b))
        return c.fail(SM_E_SHAPE, c.prefix + " buffer size overflows");
    if (!c.view(b.mixed_h, x_b, 16, "mixed activation", false, rr.x) ||
        !c.view(b.router_weights, w_b, 16, "router weights", false, rr.w))
        return false;
    rr.bias = 0;
    if (b.router_bias.buffer != 0 && !c.view(b.router_bias, uint64_t(s.n_experts) * 4, 4, "router bias", false, rr.bias))
        return false;
    sm_route_buffers rb{b.logits, b.route_ids, b.route_weights};
    if (!check_route(c, s, rb, ro, false)) return false;
    rr.logits = ro.logits;
    // Grouping reads the IDs the route step writes; validate its other views.
    sm_grouping_buffers gb{b.route_ids, b.mixed_h, b.histogram, b.plan, b.tiles, b.source_rows,
                           b.destination_rows, b.gathered_rows, b.resident, b.layer};
    const size_t n_in = c.inputs.size();
    if (!check_grouping(c, s, gb, gr)) return false;
    // Drop the duplicate input entries (route IDs and mixed activation are produced or
    // already listed by this composition).
    c.inputs.erase(c.inputs.begin() + n_in, c.inputs.begin() + n_in + 2);
    return true;
}

void encode_route_gather_launch(sm_segment* seg, const sm_moe_shape& s, const RouterRes& rr, const RouteRes& ro,
                                const GroupRes& gr, const LayerChecks* lc = nullptr) {
    const auto rows = s.rows, d = s.hidden, E = s.n_experts;
    // The router clears the histogram's counts and the arrival word, top-k counts its entries
    // into the histogram, and the grouping starts at its scan: one launch fewer.
    const uint32_t n_tiles = uint32_t((uint64_t(rows) * s.top_k + sm::kCountTile - 1) / sm::kCountTile);
    const sm::RouterPrep rp{reinterpret_cast<uint32_t*>(gr.hist), n_tiles * E,
                            reinterpret_cast<uint32_t*>(gr.plan + sm::kArriveBytes)};
    add_step(seg, "router GEMM", [=](hipStream_t st) {
        return sm::launch_router_gemm(reinterpret_cast<const _Float16*>(rr.x), reinterpret_cast<const float*>(rr.w),
                                      reinterpret_cast<const float*>(rr.bias), reinterpret_cast<float*>(rr.logits),
                                      rows, d, E, st, &rp);
    });
    encode_route_launch(seg, s, 1, ro, gr.hist);
    encode_grouping_launch(seg, s, gr, lc, true);
}
}  // namespace

sm_status sm_encode_route_gather(sm_segment* seg, const sm_moe_shape* shape, const sm_route_gather_buffers* b) {
    Check c;
    const char* P = "Prefill MoE route/gather";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = shape_check(shape, P, err, false)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    RouterRes rr{};
    RouteRes ro{};
    GroupRes gr{};
    if (!check_route_gather(c, *shape, *b, rr, ro, gr) || !c.aliases()) return finish(seg, c);
    encode_route_gather_launch(seg, *shape, rr, ro, gr);
    return SM_OK;
}

sm_status sm_encode_shared_ffn(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt, const sm_shared_buffers* b) {
    Check c;
    const char* P = "Prefill MoE shared FFN";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = shape_check(shape, P, err, false)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    SharedRes r{};
    if (!check_shared(c, *shape, fmt, *b, r) || !c.aliases()) return finish(seg, c);
    encode_shared_launch(seg, *shape, fmt, r);
    return SM_OK;
}

sm_status sm_encode_gate_up(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt, const sm_gate_up_buffers* b) {
    Check c;
    const char* P = "Prefill MoE gate/up";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = shape_check(shape, P, err, true)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    GateUpRes r{};
    if (!check_gate_up(c, *shape, fmt, *b, r) || !c.aliases()) return finish(seg, c);
    if ((st = encode_gate_up_launch(seg, *shape, fmt, r)) != SM_OK) return ring_fail(seg, st);
    return SM_OK;
}

sm_status sm_encode_down(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt, const sm_down_buffers* b) {
    Check c;
    const char* P = "Prefill MoE down";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = shape_check(shape, P, err, true)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    DownRes r{};
    if (!check_down(c, *shape, fmt, *b, r) || !c.aliases()) return finish(seg, c);
    if ((st = encode_down_launch(seg, *shape, fmt, r)) != SM_OK) return ring_fail(seg, st);
    return SM_OK;
}

sm_status sm_encode_swiglu(sm_segment* seg, uint32_t rows, uint32_t width, const sm_swiglu_buffers* b) {
    Check c;
    const char* P = "Prefill MoE SwiGLU";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    if (rows == 0 || rows > SM_MAX_ROWS || width == 0)
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " row count exceeds the supported range");
    uint64_t n, f_b, h_b;
    if (!mul_ok({rows, width}, n) || !mul_ok({n, 4}, f_b) || !mul_ok({n, 2}, h_b))
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " buffer size overflows");
    uintptr_t g, u, o;
    // Read-only inputs may alias each other; the output must be disjoint from both.
    if (!c.view(b->gate, f_b, 4, "gate", false, g) || !c.view(b->up, f_b, 4, "up", false, u) ||
        !c.view(b->output, h_b, 2, "output", true, o) || !c.aliases())
        return finish(seg, c);
    add_step(seg, "swiglu", [=](hipStream_t s) {
        return sm::launch_swiglu(reinterpret_cast<const float*>(g), reinterpret_cast<const float*>(u),
                                 reinterpret_cast<_Float16*>(o), n, s);
    });
    return SM_OK;
}

sm_status sm_encode_combine(sm_segment* seg, const sm_moe_shape* shape, const sm_combine_buffers* b) {
    Check c;
    const char* P = "Prefill MoE combine";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = shape_check(shape, P, err, false)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    CombineRes r{};
    if (!check_combine(c, *shape, *b, r) || !c.aliases()) return finish(seg, c);
    encode_combine_launch(seg, *shape, r);
    return SM_OK;
}

sm_status sm_encode_dequant(sm_segment* seg, sm_format fmt, uint32_t n_out, uint32_t k, sm_view weights,
                            sm_view out) {
    Check c;
    const char* P = "Prefill dequant";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    if (!routed_fmt(fmt) && !dense_fmt(fmt)) return record_fail(seg, SM_E_FORMAT, std::string(P) + " format is not supported");
    if (n_out == 0 || !k_ok(fmt, k)) return record_fail(seg, SM_E_SHAPE, std::string(P) + " widths do not fit the format's blocks");
    uint64_t w_b, o_b;
    if (!mul_ok({n_out, fmt_row_bytes(fmt, k)}, w_b) || !mul_ok({n_out, k, 2}, o_b))
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " buffer size overflows");
    uintptr_t w, o;
    if (!c.view(weights, w_b, weight_align(fmt), "weights", false, w) || !c.view(out, o_b, 2, "K-major F16", true, o) ||
        !c.aliases())
        return finish(seg, c);
    const uint64_t rb = fmt_row_bytes(fmt, k);
    add_step(seg, "dequant", [=](hipStream_t s) {
        return sm::launch_decode_rows(Fmt(fmt), reinterpret_cast<const uint8_t*>(w), n_out, k, rb,
                                      reinterpret_cast<uint16_t*>(o), s);
    });
    return SM_OK;
}

// Where a full layer's shared expert forks off: beside the router GEMM (offset 0) or, for
// layers of at least 8192 tokens, after top-k (offset 2: the router and top-k run first).
// Measured on MI355X: at 2048 tokens the shared GEMMs fit in the router's and the
// grouping's idle CUs (forking after top-k was 8 us slower), at 8192 tokens they slow the
// larger router GEMM down (forking after top-k was 17 us faster).
static size_t shared_fork_offset(const sm_moe_shape& s) { return s.rows >= 8192 ? 2 : 0; }

namespace {
sm_status encode_full_layer_impl(sm_segment* seg, const sm_moe_shape* shape, const sm_layer_formats* f,
                                 const sm_layer_buffers* b, ChunkCtl* ctl, const FixedScratch* fixed = nullptr) {
    const char* P = "full-mode Prefill MoE";
    if (seg == nullptr) return SM_E_ARGUMENT;
    if (seg->failed) return SM_E_SEGMENT;
    std::string err;
    sm_status st = shape_check(shape, P, err, true);
    if (st != SM_OK) return record_fail(seg, st, err);
    if (!b || !f) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    const sm_moe_shape& s = *shape;
    const bool has_shared = s.shared_ff != 0;
    // Validate every stage before anything is recorded.
    Check cr, cs, cg, cd, cc;
    for (Check* c : {&cr, &cs, &cg, &cd, &cc}) { c->ctx = seg->ctx; c->prefix = P; c->fixed = fixed; }
    cr.stage = 0; cs.stage = 1; cg.stage = 2; cd.stage = 3; cc.stage = 4;
    RouterRes rr{};
    RouteRes ro{};
    GroupRes gr{};
    SharedRes sr{};
    GateUpRes gu{};
    DownRes dn{};
    CombineRes co{};
    const bool ok = check_route_gather(cr, s, b->route_gather, rr, ro, gr) && cr.aliases() &&
                    (!has_shared || (check_shared(cs, s, f->shared, b->shared, sr) && cs.aliases())) &&
                    check_gate_up(cg, s, f->gate_up, b->gate_up, gu) && cg.aliases() &&
                    check_down(cd, s, f->down, b->down, dn) && cd.aliases() &&
                    check_combine(cc, s, b->combine, co) && cc.aliases();
    if (!ok) {
        for (Check* c : {&cr, &cs, &cg, &cd, &cc})
            if (c->st != SM_OK) return record_fail(seg, c->st, c->err);
        return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " validation failed");
    }
    // Cross-stage aliasing: only the listed producer -> consumer edges.
    std::vector<Range> all;
    const char* names[] = {"route.", "shared.", "gate_up.", "down.", "combine."};
    for (Check* c : {&cr, &cs, &cg, &cd, &cc}) {
        for (auto r : c->inputs) { r.name = names[c->stage] + r.name; all.push_back(r); }
        for (auto r : c->outputs) { r.name = names[c->stage] + r.name; all.push_back(r); }
    }
    for (size_t i = 0; i < all.size(); ++i)
        for (size_t j = i + 1; j < all.size(); ++j) {
            const Range& a = all[i];
            const Range& bb = all[j];
            if (a.stage == bb.stage || !overlap(a, bb) || (!a.writable && !bb.writable)) continue;
            // Writer first: the earlier stage when both write.
            const bool a_first = a.writable && (!bb.writable || a.stage < bb.stage);
            const Range& w = a_first ? a : bb;
            const Range& r = a_first ? bb : a;
            if (expected_edge(w, r)) continue;
            return record_fail(seg, SM_E_ALIAS, std::string(P) + " " + w.name + " overlaps active " + r.name);
        }
    // The shared expert reads only the activations and its weights, which no earlier launch
    // writes (checked above), so it runs beside routing and the routed experts; combine joins.
    // The shared expert waits for the work recorded before this layer (in a segment of
    // several layers, the previous layer), not for this layer's routing.
    const size_t first = seg->steps.size();
    if (gu.plan == dn.plan && gu.tiles == dn.tiles) {
        // One plan for both expert stages: their checks ride on the grouping and the gather.
        ExpertsPlan x;
        if ((st = prepare_experts(seg, s, f->gate_up, gu, f->down, dn, x, ctl)) != SM_OK) return ring_fail(seg, st);
        LayerChecks lc{};
        if (!(ctl && ctl->keep_status)) {
            lc.prep.status = x.g.status;
            lc.prep.status2 = x.d.status;
        }
        lc.prep.clear = x.check.clear;
        lc.prep.clear_words = x.check.clear_words;
        lc.check = x.check;
        lc.check.clear = nullptr;
        lc.check.clear_words = 0;
        lc.dst = x.d.dst;
        lc.bits = x.check.clear;
        lc.slot1 = x.slot1;
        lc.slot2 = x.slot2;
        encode_route_gather_launch(seg, s, rr, ro, gr, &lc);
        seg->steps[first + shared_fork_offset(s)].fork_before = true;
        if (has_shared) encode_shared_launch(seg, s, f->shared, sr, true);
        const sm::RoutedGemm g = x.g, d = x.d;
        const int fg = f->gate_up, fd = f->down;
        add_step(seg, "gate/up tiles", [=](hipStream_t st) { return sm::launch_gate_up(Fmt(fg), g, st); });
        add_step(seg, "down tiles", [=](hipStream_t st) { return sm::launch_down(Fmt(fd), d, st); });
    } else {
        encode_route_gather_launch(seg, s, rr, ro, gr);
        seg->steps[first + shared_fork_offset(s)].fork_before = true;
        if (has_shared) encode_shared_launch(seg, s, f->shared, sr, true);
        if ((st = encode_experts_launch(seg, s, f->gate_up, gu, f->down, dn, ctl)) != SM_OK) return ring_fail(seg, st);
    }
    encode_combine_launch(seg, s, co, has_shared);
    return SM_OK;
}
}  // namespace

sm_status sm_encode_full_layer(sm_segment* seg, const sm_moe_shape* shape, const sm_layer_formats* f,
                               const sm_layer_buffers* b) {
    return encode_full_layer_impl(seg, shape, f, b, nullptr);
}

// ---- chunk driver ---------------------------------------------------------------------

sm_status sm_build_chunk_schedule(uint32_t pos0, uint64_t token_count, uint32_t chunk_rows, sm_chunk_schedule* out,
                                  char* err, size_t cap) {
    auto fail = [&](const char* msg) {
        if (err && cap) std::snprintf(err, cap, "%s", msg);
        return SM_E_SHAPE;
    };
    if (out == nullptr) return SM_E_ARGUMENT;
    if (chunk_rows == 0 || chunk_rows > SM_MAX_ROWS) return fail("Prefill chunk size must fit the shader row limit");
    // Every position p0 + t must fit a signed 32-bit StepRow (n_kv = pos + 1 included).
    const uint64_t max_step = uint64_t(std::numeric_limits<int32_t>::max());
    if (token_count != 0 && (pos0 >= max_step || token_count > max_step - pos0))
        return fail("Prefill prompt positions exceed the signed StepRow range");
    *out = sm_chunk_schedule{pos0, chunk_rows, token_count};
    if (err && cap) err[0] = 0;
    return SM_OK;
}

uint64_t sm_chunk_count(const sm_chunk_schedule* s) {
    if (s == nullptr || s->token_count == 0 || s->chunk_rows == 0) return 0;
    return 1 + (s->token_count - 1) / s->chunk_rows;
}

int sm_chunk_range_at(const sm_chunk_schedule* s, uint64_t index, sm_chunk_range* out) {
    if (s == nullptr || out == nullptr || index >= sm_chunk_count(s)) return 0;
    const uint64_t off = index * s->chunk_rows;
    const uint64_t rows = std::min<uint64_t>(s->token_count - off, s->chunk_rows);
    *out = sm_chunk_range{off, uint32_t(uint64_t(s->pos0) + off), uint32_t(rows)};
    return 1;
}

sm_status sm_encode_prefill_moe_chunks(sm_segment* seg, const sm_chunk_schedule* schedule, const sm_moe_shape* shape,
                                       const sm_layer_formats* f, sm_view input, sm_view output,
                                       const sm_layer_buffers* b) {
    const char* P = "Prefill MoE chunks";
    if (seg == nullptr) return SM_E_ARGUMENT;
    if (seg->failed) return SM_E_SEGMENT;
    if (!schedule || !shape || !f || !b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " arguments are null");
    if (schedule->chunk_rows == 0 || schedule->chunk_rows > SM_MAX_ROWS)
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " chunk size must fit the shader row limit");
    if (shape->rows != schedule->chunk_rows)
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " scratch rows must equal the schedule's chunk size");
    const uint64_t n = sm_chunk_count(schedule);
    if (n == 0) return SM_OK;
    // The whole prompt's input and output views: owned, large enough, output apart from input.
    Check c;
    c.ctx = seg->ctx;
    c.prefix = P;
    uint64_t in_b, out_b;
    if (!mul_ok({schedule->token_count, shape->hidden, 2}, in_b) || !mul_ok({schedule->token_count, shape->hidden, 4}, out_b))
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " buffer size overflows");
    uintptr_t pin, pout;
    if (!c.view(input, in_b, 16, "input rows", false, pin) || !c.view(output, out_b, 16, "output rows", true, pout) ||
        !c.aliases())
        return finish(seg, c);
    ChunkCtl ctl;
    for (uint64_t k = 0; k < n; ++k) {
        sm_chunk_range r{};
        sm_chunk_range_at(schedule, k, &r);
        sm_moe_shape cs = *shape;
        cs.rows = r.rows;
        sm_layer_buffers lb = *b;
        const sm_view xin{input.buffer, input.offset + r.token_offset * shape->hidden * 2, uint64_t(r.rows) * shape->hidden * 2};
        lb.route_gather.mixed_h = xin;
        lb.shared.mixed_h = xin;
        lb.combine.output = sm_view{output.buffer, output.offset + r.token_offset * shape->hidden * 4,
                                    uint64_t(r.rows) * shape->hidden * 4};
        ctl.keep_status = k > 0;
        const sm_status st = encode_full_layer_impl(seg, &cs, f, &lb, &ctl);
        if (st != SM_OK) return st;  // the segment is poisoned with the chunk's message
    }
    return SM_OK;
}

// ---- standalone transactional forms --------------------------------------------------

// What a failed commit reports (empty on success).
static const char* commit_message(sm_status st) {
    if (st == SM_OK) return "";
    if (st == SM_E_ARGUMENT)
        return "segment committed on a capturing stream: the expert address tables are read from the "
               "context's reusable host ring when the launches run, so segments run outside stream capture";
    return "HIP launch failed";
}

#define SM_SUBMIT_BODY(ENCODE_CALL)                                                   \
    sm_segment* seg = nullptr;                                                        \
    sm_status st = sm_segment_begin(ctx, &seg);                                       \
    if (st != SM_OK) return st;                                                       \
    st = ENCODE_CALL;                                                                 \
    if (st != SM_OK) {                                                                \
        if (err && cap) std::snprintf(err, cap, "%s", seg->error.c_str());            \
        sm_segment_abort(seg);                                                        \
        return st;                                                                    \
    }                                                                                 \
    st = sm_segment_commit(seg, stream);                                              \
    if (err && cap) std::snprintf(err, cap, "%s", commit_message(st));                \
    return st;

sm_status sm_submit_route(sm_context* ctx, void* stream, const sm_moe_shape* shape, int divide,
                          const sm_route_buffers* b, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_route(seg, shape, divide, b))
}
sm_status sm_submit_grouping(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                             const sm_grouping_buffers* b, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_grouping(seg, shape, b))
}
sm_status sm_submit_route_gather(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                                 const sm_route_gather_buffers* b, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_route_gather(seg, shape, b))
}
sm_status sm_submit_shared_ffn(sm_context* ctx, void* stream, const sm_moe_shape* shape, sm_format fmt,
                               const sm_shared_buffers* b, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_shared_ffn(seg, shape, fmt, b))
}
sm_status sm_submit_gate_up(sm_context* ctx, void* stream, const sm_moe_shape* shape, sm_format fmt,
                            const sm_gate_up_buffers* b, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_gate_up(seg, shape, fmt, b))
}
sm_status sm_submit_down(sm_context* ctx, void* stream, const sm_moe_shape* shape, sm_format fmt,
                         const sm_down_buffers* b, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_down(seg, shape, fmt, b))
}
sm_status sm_submit_swiglu(sm_context* ctx, void* stream, uint32_t rows, uint32_t width,
                           const sm_swiglu_buffers* b, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_swiglu(seg, rows, width, b))
}
sm_status sm_submit_combine(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                            const sm_combine_buffers* b, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_combine(seg, shape, b))
}
sm_status sm_submit_dequant(sm_context* ctx, void* stream, sm_format fmt, uint32_t n_out, uint32_t k,
                            sm_view weights, sm_view out, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_dequant(seg, fmt, n_out, k, weights, out))
}
sm_status sm_submit_full_layer(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                               const sm_layer_formats* formats, const sm_layer_buffers* b, char* err,
                               size_t cap) {
    SM_SUBMIT_BODY(sm_encode_full_layer(seg, shape, formats, b))
}

sm_status sm_submit_full_layer_fixed_scratch(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                                             const sm_layer_formats* formats, const sm_layer_buffers* b, char* err,
                                             size_t cap) {
    auto message = [&](const char* msg) {
        if (err && cap) std::snprintf(err, cap, "%s", msg);
    };
    if (ctx == nullptr) return SM_E_ARGUMENT;
    // Checked before anything is encoded (no ring slot is claimed): see run_segment.
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (ctx->has_device && hipSetDevice(ctx->device) == hipSuccess &&
        hipStreamIsCapturing(reinterpret_cast<hipStream_t>(stream), &capture) == hipSuccess &&
        capture != hipStreamCaptureStatusNone) {
        message(commit_message(SM_E_ARGUMENT));
        return SM_E_ARGUMENT;
    }
    FixedScratch fs;
    if (ctx->fixed_scratch != 0) {
        fs.hist = ctx->fixed_scratch;
        fs.snap_gu = fs.hist + kFixedHistBytes;
        fs.snap_dn = fs.snap_gu + kFixedSnapBytes;
    }
    sm_segment* seg = nullptr;
    sm_status st = sm_segment_begin(ctx, &seg);
    if (st != SM_OK) return st;
    st = encode_full_layer_impl(seg, shape, formats, b, nullptr, &fs);
    if (st != SM_OK) {
        message(seg->error.c_str());
        sm_segment_abort(seg);
        return st;
    }
    if (ctx->fixed_scratch == 0) {  // validated, but there is no device copy to run on
        message("full-mode Prefill MoE fixed scratch is not available on this context's device");
        sm_segment_abort(seg);
        return SM_E_DEVICE;
    }
    st = sm_segment_commit(seg, stream);
    message(commit_message(st));
    return st;
}

sm_status sm_submit_prefill_moe_chunks(sm_context* ctx, void* stream, const sm_chunk_schedule* schedule,
                                       const sm_moe_shape* shape, const sm_layer_formats* formats, sm_view input,
                                       sm_view output, const sm_layer_buffers* b, char* err, size_t cap) {
    SM_SUBMIT_BODY(sm_encode_prefill_moe_chunks(seg, schedule, shape, formats, input, output, b))
}

sm_status sm_read_layer_status(sm_context* ctx, void* stream, sm_view plan, sm_view gu, sm_view dn,
                               uint32_t* bad, uint32_t* gu_bits, uint32_t* dn_bits) {
    if (!ctx) return SM_E_ARGUMENT;
    if (hipSetDevice(ctx->device) != hipSuccess) return SM_E_DEVICE;
    if (hipStreamSynchronize(reinterpret_cast<hipStream_t>(stream)) != hipSuccess) return SM_E_DEVICE;
    auto read_word = [&](const sm_view& v, uint64_t off, uint32_t* out) -> sm_status {
        if (!out) return SM_OK;
        *out = 0;
        if (v.buffer == 0) return SM_OK;
        sm_context::Alloc a{};
        {
            std::lock_guard<std::mutex> lk(ctx->mu);
            auto it = ctx->buffers.find(v.buffer);
            if (it == ctx->buffers.end()) return SM_E_OWNERSHIP;
            a = it->second;
        }
        if (v.offset + off + 4 > a.bytes || v.length < off + 4) return SM_E_VIEW;
        if (hipMemcpy(out, reinterpret_cast<void*>(a.ptr + v.offset + off), 4, hipMemcpyDeviceToHost) != hipSuccess)
            return SM_E_DEVICE;
        return SM_OK;
    };
    sm_status st = read_word(plan, 20, bad);  // PfPlan.bad
    if (st == SM_OK) st = read_word(gu, 0, gu_bits);
    if (st == SM_OK) st = read_word(dn, 0, dn_bits);
    return st;
}

}  // extern "C"

// =========================================================================================
// Decode-side MoE (the reference's Window MoE over T = 1..8 rows; moe_dispatch.hpp:13-372).
// =========================================================================================
namespace {

// Rows and entries of the plan; widths as prefill (hidden a multiple of 256, the expert width of
// 64). A K-quant down stage needs the expert width in whole 256-value super-blocks, which the
// weight check reports.
sm_status decode_shape_check(const sm_moe_shape* s, const char* prefix, std::string& err, bool need_ff) {
    sm_status st = shape_check(s, prefix, err, need_ff);
    if (st != SM_OK) return st;
    if (s->rows > SM_DECODE_MAX_ROWS || uint64_t(s->rows) * s->top_k > SM_MOE_PLAN_MAX_ENTRIES) {
        err = std::string(prefix) + " requires T=1..8 rows and at most 80 routed entries";
        return SM_E_SHAPE;
    }
    if (s->hidden > SM_DECODE_MAX_WIDTH || (need_ff && s->expert_ff > SM_DECODE_MAX_WIDTH)) {
        err = std::string(prefix) + " widths above 4096 are not supported";
        return SM_E_SHAPE;
    }
    return SM_OK;
}

// The selected layer's slice of a table view that starts at layer 0: validated over
// [0, (layer + 1) * per_layer) and registered as the slice alone.
bool layer_slice(Check& c, const sm_view& v, uint32_t layer, uint64_t per_layer, uint64_t align, const char* name,
                 bool writable, uintptr_t& out) {
    uint64_t need;
    if (!mul_ok({uint64_t(layer) + 1u, per_layer}, need)) return c.fail(SM_E_SHAPE, c.prefix + " table size overflows");
    uintptr_t base;
    if (!c.view(v, need, align, name, writable, base)) return false;
    auto& r = writable ? c.outputs.back() : c.inputs.back();
    r.ptr = base + uint64_t(layer) * per_layer;
    r.bytes = per_layer;
    out = r.ptr;
    return true;
}

struct DecodePlanRes { uintptr_t ids = 0, resident = 0, usage = 0, plan = 0, status = 0; };
bool check_decode_plan(Check& c, const sm_moe_shape& s, const sm_moe_plan_buffers& b, DecodePlanRes& r, bool ids_view) {
    const uint64_t n = uint64_t(s.rows) * s.top_k, E = s.n_experts;
    if (ids_view && !c.view(b.ids, n * 4, 4, "route IDs", false, r.ids)) return false;
    if (!layer_slice(c, b.plans, b.layer, SM_MOE_PLAN_BYTES, 4, "MoePlan", true, r.plan)) return false;
    if (b.resident.buffer != 0 && !layer_slice(c, b.resident, b.layer, E * 4, 4, "residency table", false, r.resident))
        return false;
    if (b.usage.buffer != 0 && !layer_slice(c, b.usage, b.layer, E * 4, 4, "usage table", true, r.usage)) return false;
    if (b.status.buffer != 0 && !c.view(b.status, 4, 4, "status", true, r.status)) return false;
    return true;
}

// A read-only MoePlan of the selected layer.
bool decode_plan_input(Check& c, const sm_view& plans, uint32_t layer, uintptr_t& out) {
    return layer_slice(c, plans, layer, SM_MOE_PLAN_BYTES, 4, "MoePlan", false, out);
}

sm::DecodePlanArgs decode_plan_args(const sm_moe_shape& s, const DecodePlanRes& r) {
    sm::DecodePlanArgs a{};
    a.ids = reinterpret_cast<const int32_t*>(r.ids);
    a.resident = reinterpret_cast<const int32_t*>(r.resident);
    a.usage = reinterpret_cast<float*>(r.usage);
    a.plan = reinterpret_cast<uint8_t*>(r.plan);
    a.status = reinterpret_cast<uint32_t*>(r.status);
    a.rows = s.rows;
    a.top_k = s.top_k;
    a.n_experts = s.n_experts;
    return a;
}

uint64_t q81_bytes(uint64_t rows, uint64_t n) { return rows * (n / 32u) * SM_Q8_1_BLOCK_BYTES; }

// One grouped mat-vec stage over a validated expert table: the snapshot copy (from a pinned
// ring slot; it also clears the status word when `clear` is set) then the mat-vec. `slot` < -1
// means the copy happens elsewhere (a decode layer's plan launch).
struct DecodeStage { WeightsRes w; uintptr_t act = 0, plan = 0, out0 = 0, out1 = 0, status = 0; };
sm::DecodeMatvec decode_matvec(const sm_moe_shape& s, int fmt, bool gate_up, const DecodeStage& r) {
    sm::DecodeMatvec m{};
    m.addresses = reinterpret_cast<const uint64_t*>(r.w.snapshot);
    m.act = reinterpret_cast<const uint8_t*>(r.act);
    m.plan = reinterpret_cast<const uint8_t*>(r.plan);
    m.out0 = reinterpret_cast<float*>(r.out0);
    m.out1 = reinterpret_cast<float*>(r.out1);
    m.status = reinterpret_cast<uint32_t*>(r.status);
    m.n_entries = s.rows * s.top_k;
    m.n_experts = s.n_experts;
    m.act_rows = gate_up ? s.rows : s.rows * s.top_k;
    m.k = gate_up ? s.hidden : s.expert_ff;
    m.out_width = gate_up ? s.expert_ff : s.hidden;
    m.row_bytes = fmt_row_bytes(fmt, m.k);
    m.max_group = s.rows;
    return m;
}

sm_status encode_decode_stage(sm_segment* seg, const sm_moe_shape& s, int fmt, bool gate_up, const DecodeStage& r,
                              bool clear_status) {
    const int slot = claim_ring_slot(seg->ctx, r.w.table);
    if (claim_status(slot) != SM_OK) return ring_fail(seg, claim_status(slot));
    const uint64_t* src = slot >= 0 ? seg->ctx->ring + uint64_t(slot) * sm_context::kSlotWords : nullptr;
    uint64_t* dst = reinterpret_cast<uint64_t*>(r.w.snapshot);
    const uint32_t words = slot >= 0 ? uint32_t(r.w.table.size()) : 0u;
    uint32_t* status = clear_status ? reinterpret_cast<uint32_t*>(r.status) : nullptr;
    add_step(seg, gate_up ? "decode gate/up snapshot" : "decode down snapshot",
             [=](hipStream_t st) { return sm::launch_snapshot_copy(src, dst, words, status, st); });
    seg->steps.back().ring_slot = slot;
    const sm::DecodeMatvec m = decode_matvec(s, fmt, gate_up, r);
    add_step(seg, gate_up ? "decode gate/up" : "decode down",
             [=](hipStream_t st) { return sm::launch_decode_matvec(Fmt(fmt), gate_up, m, st); });
    return SM_OK;
}

bool check_decode_experts(Check& c, const sm_moe_shape& s, int fmt, const sm_expert_weights& w, const sm_view& act,
                          const sm_view& plans, const sm_view& gate, const sm_view& up, const sm_view& status,
                          DecodeStage& r, bool act_view, bool plan_view, bool status_view) {
    if (!routed_fmt(fmt)) return c.fail(SM_E_FORMAT, c.prefix + " weight format is not a supported block format");
    const uint64_t N = uint64_t(s.rows) * s.top_k;
    return check_weights(c, s, w, fmt, true, r.w) &&
           (!act_view || c.view(act, q81_bytes(s.rows, s.hidden), 4, "Q8_1 activations", false, r.act)) &&
           (!plan_view || decode_plan_input(c, plans, w.layer, r.plan)) &&
           c.view(gate, N * s.expert_ff * 4, 16, "gate", true, r.out0) &&
           c.view(up, N * s.expert_ff * 4, 16, "up", true, r.out1) &&
           (!status_view || c.view(status, 4, 4, "status", true, r.status));
}

bool check_decode_down(Check& c, const sm_moe_shape& s, int fmt, const sm_expert_weights& w, const sm_view& act,
                       const sm_view& plans, const sm_view& parts, const sm_view& status, DecodeStage& r, bool act_view,
                       bool plan_view, bool status_view) {
    if (!routed_fmt(fmt)) return c.fail(SM_E_FORMAT, c.prefix + " weight format is not a supported block format");
    const uint64_t N = uint64_t(s.rows) * s.top_k;
    return check_weights(c, s, w, fmt, false, r.w) &&
           (!act_view || c.view(act, q81_bytes(N, s.expert_ff), 4, "Q8_1 hidden", false, r.act)) &&
           (!plan_view || decode_plan_input(c, plans, w.layer, r.plan)) &&
           c.view(parts, N * s.hidden * 4, 16, "parts", true, r.out0) &&
           (!status_view || c.view(status, 4, 4, "status", true, r.status));
}

void encode_q81_launch(sm_segment* seg, uintptr_t in, bool f32, uintptr_t out, uint32_t n, uint32_t rows,
                       const char* label) {
    add_step(seg, label, [=](hipStream_t st) {
        return sm::launch_quantize_q8_1(reinterpret_cast<const void*>(in), f32, reinterpret_cast<uint8_t*>(out), n, rows, st);
    });
}

void encode_swiglu_f32_launch(sm_segment* seg, uintptr_t g, uintptr_t u, uintptr_t o, uint64_t n) {
    add_step(seg, "decode swiglu", [=](hipStream_t st) {
        return sm::launch_swiglu_f32(reinterpret_cast<const float*>(g), reinterpret_cast<const float*>(u),
                                     reinterpret_cast<float*>(o), n, st);
    });
}

void encode_combine_decode_launch(sm_segment* seg, const sm_moe_shape& s, const CombineRes& r) {
    const auto rows = s.rows, K = s.top_k, d = s.hidden;
    add_step(seg, "decode combine", [=](hipStream_t st) {
        return sm::launch_combine_decode(reinterpret_cast<const float*>(r.parts), reinterpret_cast<const float*>(r.weights),
                                         reinterpret_cast<const float*>(r.shared), reinterpret_cast<const float*>(r.gate),
                                         reinterpret_cast<float*>(r.out), rows, K, d, st);
    });
}

// The decode shared expert over F16/BF16 weights: the hidden view holds F32 [T][Is] (the
// reference's F32 shx SwiGLU output), Is a multiple of 64 (the reference model's 640 fits).
bool check_shared_decode(Check& c, const sm_moe_shape& s, int fmt, const sm_shared_buffers& b, SharedRes& r) {
    if (!dense_fmt(fmt)) return c.fail(SM_E_FORMAT, c.prefix + " shared expert format must be F16 or BF16");
    const uint64_t Is = s.shared_ff;
    if (Is == 0 || Is % 64 != 0) return c.fail(SM_E_SHAPE, c.prefix + " shared expert width must be a positive multiple of 64");
    uint64_t x_b, w_b, h_b, o_b;
    if (!mul_ok({s.rows, s.hidden, 2}, x_b) || !mul_ok({Is, s.hidden, 2}, w_b) || !mul_ok({s.rows, Is, 4}, h_b) ||
        !mul_ok({s.rows, s.hidden, 4}, o_b))
        return c.fail(SM_E_SHAPE, c.prefix + " buffer size overflows");
    return c.view(b.mixed_h, x_b, 16, "mixed activation", false, r.x) &&
           c.view(b.gate_weights, w_b, 16, "shared gate weights", false, r.wg) &&
           c.view(b.up_weights, w_b, 16, "shared up weights", false, r.wu) &&
           c.view(b.down_weights, w_b, 16, "shared down weights", false, r.wd) &&
           c.view(b.gate_vector, uint64_t(s.hidden) * 2, 16, "shared gate vector", false, r.gv) &&
           c.view(b.hidden, h_b, 16, "shared hidden", true, r.hidden) &&
           c.view(b.output, o_b, 16, "shared output", true, r.out) &&
           c.view(b.gate_logit, uint64_t(s.rows) * 4, 4, "shared gate logit", true, r.gl);
}

// The decode shared expert's two mat-vecs: gate/up (with the gate logit), then down.
struct SharedDecodeJobs { sm::DenseDecode gu, dn; };
SharedDecodeJobs shared_decode_jobs(const sm_moe_shape& s, const SharedRes& r) {
    sm::DenseDecode gu{};
    gu.w0 = reinterpret_cast<const uint8_t*>(r.wg);
    gu.w1 = reinterpret_cast<const uint8_t*>(r.wu);
    gu.x = reinterpret_cast<const void*>(r.x);
    gu.out = reinterpret_cast<float*>(r.hidden);
    gu.rows = s.rows;
    gu.k = s.hidden;
    gu.n_out = s.shared_ff;
    gu.gv = reinterpret_cast<const uint8_t*>(r.gv);
    gu.gl = reinterpret_cast<float*>(r.gl);
    sm::DenseDecode dn{};
    dn.w0 = reinterpret_cast<const uint8_t*>(r.wd);
    dn.x = reinterpret_cast<const void*>(r.hidden);
    dn.out = reinterpret_cast<float*>(r.out);
    dn.rows = s.rows;
    dn.k = s.shared_ff;
    dn.n_out = s.hidden;
    return {gu, dn};
}

void encode_shared_decode_launch(sm_segment* seg, const sm_moe_shape& s, int fmt, const SharedRes& r) {
    const SharedDecodeJobs j = shared_decode_jobs(s, r);
    const sm::DenseDecode gu = j.gu, dn = j.dn;
    add_step(seg, "decode shared gate/up", [=](hipStream_t st) { return sm::launch_dense_decode(Fmt(fmt), true, gu, st); });
    add_step(seg, "decode shared down", [=](hipStream_t st) { return sm::launch_dense_decode(Fmt(fmt), false, dn, st); });
}

// The routed FFN's scratch and output views (gate, up, hidden, Q8_1 hidden, parts, status).
struct RoutedFFNRes { DecodeStage gu, dn; uintptr_t hidden = 0, hq = 0; };
bool check_routed_ffn(Check& c, const sm_moe_shape& s, int fgu, int fdn, const sm_moe_routed_ffn_buffers& b,
                      RoutedFFNRes& r, bool own_inputs) {
    const uint64_t N = uint64_t(s.rows) * s.top_k;
    if (!check_decode_experts(c, s, fgu, b.gate_up_weights, b.input_activations, b.plans, b.gate, b.up, b.status, r.gu,
                              own_inputs, own_inputs, true))
        return false;
    if (!c.view(b.hidden, N * s.expert_ff * 4, 16, "hidden", true, r.hidden) ||
        !c.view(b.down_activations, q81_bytes(N, s.expert_ff), 4, "Q8_1 hidden", true, r.hq))
        return false;
    r.dn.act = r.hq;
    r.dn.plan = r.gu.plan;
    r.dn.status = r.gu.status;
    return check_decode_down(c, s, fdn, b.down_weights, b.down_activations, b.plans, b.parts, b.status, r.dn, false, false,
                             false);
}

// gate/up, SwiGLU, Q8_1, down. With snapshots_done, the plan launch has copied both address
// tables and cleared the status word already (a decode layer).
sm_status encode_routed_ffn_launch(sm_segment* seg, const sm_moe_shape& s, int fgu, int fdn, const RoutedFFNRes& r,
                                   bool snapshots_done) {
    const uint64_t N = uint64_t(s.rows) * s.top_k;
    if (snapshots_done) {
        const sm::DecodeMatvec m = decode_matvec(s, fgu, true, r.gu);
        add_step(seg, "decode gate/up", [=](hipStream_t st) { return sm::launch_decode_matvec(Fmt(fgu), true, m, st); });
    } else {
        const sm_status st = encode_decode_stage(seg, s, fgu, true, r.gu, true);
        if (st != SM_OK) return st;
    }
    const uintptr_t g = r.gu.out0, u = r.gu.out1, h = r.hidden, hq = r.hq;
    const uint32_t I = s.expert_ff, rows = uint32_t(N);
    add_step(seg, "decode swiglu + Q8_1", [=](hipStream_t st) {
        return sm::launch_swiglu_q8_1(reinterpret_cast<const float*>(g), reinterpret_cast<const float*>(u),
                                      reinterpret_cast<float*>(h), reinterpret_cast<uint8_t*>(hq), I, rows, st);
    });
    if (snapshots_done) {
        const sm::DecodeMatvec m = decode_matvec(s, fdn, false, r.dn);
        add_step(seg, "decode down", [=](hipStream_t st) { return sm::launch_decode_matvec(Fmt(fdn), false, m, st); });
        return SM_OK;
    }
    return encode_decode_stage(seg, s, fdn, false, r.dn, false);
}

}  // namespace

extern "C" {

sm_status sm_encode_moe_plan(sm_segment* seg, const sm_moe_shape* shape, const sm_moe_plan_buffers* b) {
    Check c;
    const char* P = "MoE plan";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = decode_shape_check(shape, P, err, false)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    DecodePlanRes r;
    if (!check_decode_plan(c, *shape, *b, r, true) || !c.aliases()) return finish(seg, c);
    const sm::DecodePlanArgs a = decode_plan_args(*shape, r);
    add_step(seg, "decode plan", [=](hipStream_t s) { return sm::launch_decode_plan(a, s); });
    return SM_OK;
}

sm_status sm_encode_quantize_q8_1(sm_segment* seg, uint32_t rows, uint32_t n, int f32_input, sm_view input,
                                  sm_view output) {
    Check c;
    const char* P = "Q8_1 quantize";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    if (rows == 0 || rows > SM_MOE_PLAN_MAX_ENTRIES * 8u || n == 0 || n % 32 != 0)
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " needs 1..640 rows of a positive multiple of 32 values");
    uintptr_t in, out;
    const uint64_t es = f32_input ? 4 : 2;
    if (!c.view(input, uint64_t(rows) * n * es, es, "input", false, in) ||
        !c.view(output, q81_bytes(rows, n), 4, "Q8_1 output", true, out) || !c.aliases())
        return finish(seg, c);
    encode_q81_launch(seg, in, f32_input != 0, out, n, rows, "Q8_1 quantize");
    return SM_OK;
}

sm_status sm_encode_moe_experts(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt,
                                const sm_moe_expert_buffers* b) {
    Check c;
    const char* P = "MoE experts";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = decode_shape_check(shape, P, err, true)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    DecodeStage r;
    if (!check_decode_experts(c, *shape, fmt, b->weights, b->activations, b->plans, b->gate, b->up, b->status, r, true,
                              true, true) ||
        !c.aliases())
        return finish(seg, c);
    return encode_decode_stage(seg, *shape, fmt, true, r, true);
}

sm_status sm_encode_moe_down(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt, const sm_moe_down_buffers* b) {
    Check c;
    const char* P = "MoE down";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = decode_shape_check(shape, P, err, true)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    DecodeStage r;
    if (!check_decode_down(c, *shape, fmt, b->weights, b->activations, b->plans, b->parts, b->status, r, true, true, true) ||
        !c.aliases())
        return finish(seg, c);
    return encode_decode_stage(seg, *shape, fmt, false, r, true);
}

sm_status sm_encode_moe_swiglu(sm_segment* seg, uint32_t rows, uint32_t width, const sm_moe_swiglu_buffers* b) {
    Check c;
    const char* P = "MoE SwiGLU";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    if (rows == 0 || rows > SM_MOE_PLAN_MAX_ENTRIES || width == 0)
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " needs 1..80 rows of a positive width");
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    const uint64_t n = uint64_t(rows) * width;
    uintptr_t g, u, o;
    if (!c.view(b->gate, n * 4, 4, "gate", false, g) || !c.view(b->up, n * 4, 4, "up", false, u) ||
        !c.view(b->output, n * 4, 4, "output", true, o) || !c.aliases())
        return finish(seg, c);
    encode_swiglu_f32_launch(seg, g, u, o, n);
    return SM_OK;
}

sm_status sm_encode_moe_routed_ffn(sm_segment* seg, const sm_moe_shape* shape, sm_format gate_up_fmt,
                                   sm_format down_fmt, const sm_moe_routed_ffn_buffers* b) {
    Check c;
    const char* P = "MoE routed FFN";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = decode_shape_check(shape, P, err, true)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    if (b->gate_up_weights.layer != b->down_weights.layer)
        return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " gate/up and down weights select different layers");
    RoutedFFNRes r;
    if (!check_routed_ffn(c, *shape, gate_up_fmt, down_fmt, *b, r, true) || !c.aliases()) return finish(seg, c);
    return encode_routed_ffn_launch(seg, *shape, gate_up_fmt, down_fmt, r, false);
}

sm_status sm_encode_moe_combine(sm_segment* seg, const sm_moe_shape* shape, const sm_combine_buffers* b) {
    Check c;
    const char* P = "MoE combine";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = decode_shape_check(shape, P, err, false)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    CombineRes r{};
    if (!check_combine(c, *shape, *b, r) || !c.aliases()) return finish(seg, c);
    encode_combine_decode_launch(seg, *shape, r);
    return SM_OK;
}

sm_status sm_encode_moe_decode_layer(sm_segment* seg, const sm_moe_shape* shape, const sm_layer_formats* f,
                                     const sm_decode_layer_buffers* b) {
    Check c;
    const char* P = "MoE decode layer";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = decode_shape_check(shape, P, err, true)) != SM_OK) return record_fail(seg, st, err);
    if (!b || !f) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers or formats are null");
    const sm_moe_shape& s = *shape;
    const sm_moe_routed_ffn_buffers& rb = b->routed;
    if (rb.gate_up_weights.layer != b->layer || rb.down_weights.layer != b->layer)
        return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " expert weights select a different layer than the plan");
    // Route: router GEMM into the logits, top-k in multiply mode.
    RouterRes rr{};
    uint64_t x_b, w_b;
    if (!mul_ok({s.rows, s.hidden, 2}, x_b) || !mul_ok({s.n_experts, s.hidden, 4}, w_b))
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " buffer size overflows");
    bool ok = c.view(b->mixed_h, x_b, 16, "mixed activation", false, rr.x) &&
              c.view(b->router_weights, w_b, 16, "router weights", false, rr.w);
    rr.bias = 0;
    if (ok && b->router_bias.buffer != 0)
        ok = c.view(b->router_bias, uint64_t(s.n_experts) * 4, 4, "router bias", false, rr.bias);
    RouteRes ro{};
    const sm_route_buffers rob{b->logits, b->route_ids, b->route_weights};
    ok = ok && check_route(c, s, rob, ro, false);
    rr.logits = ro.logits;
    // Plan (reads the route ids written above) and the Q8_1 input.
    DecodePlanRes pr;
    pr.ids = ro.ids;
    // (The status word is registered once, by the routed FFN below; the plan launch clears it.)
    const sm_moe_plan_buffers pb{b->route_ids, b->resident, b->usage, b->plans, sm_view{}, b->layer};
    ok = ok && check_decode_plan(c, s, pb, pr, false);
    uintptr_t xq = 0;
    ok = ok && c.view(b->input_activations, q81_bytes(s.rows, s.hidden), 4, "Q8_1 activations", true, xq);
    // Routed FFN over that plan and input; its status word is the plan's.
    RoutedFFNRes fr;
    ok = ok && check_routed_ffn(c, s, f->gate_up, f->down, rb, fr, false);
    fr.gu.act = xq;
    fr.gu.plan = fr.dn.plan = pr.plan;
    pr.status = fr.gu.status;
    // Shared expert (optional) and combine.
    SharedRes sr{};
    if (ok && s.shared_ff != 0) {
        if (b->shared.mixed_h.buffer != b->mixed_h.buffer || b->shared.mixed_h.offset != b->mixed_h.offset)
            return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " shared expert must read the layer's mixed activation");
        ok = check_shared_decode(c, s, f->shared, b->shared, sr);
    }
    CombineRes cr{};
    if (ok) {
        uint64_t o_b;
        if (!mul_ok({s.rows, s.hidden, 4}, o_b)) return record_fail(seg, SM_E_SHAPE, std::string(P) + " buffer size overflows");
        cr.parts = fr.dn.out0;
        cr.weights = ro.weights;
        cr.shared = s.shared_ff != 0 ? sr.out : 0;
        cr.gate = s.shared_ff != 0 ? sr.gl : 0;
        ok = c.view(b->output, o_b, 16, "output", true, cr.out);
    }
    if (!ok || !c.aliases()) return finish(seg, c);
    // Launches: the plan launch also copies both validated address tables.
    const int s_gu = claim_ring_slot(seg->ctx, fr.gu.w.table);
    if (claim_status(s_gu) != SM_OK) return ring_fail(seg, claim_status(s_gu));
    const int s_dn = claim_ring_slot(seg->ctx, fr.dn.w.table);
    if (claim_status(s_dn) != SM_OK) {
        if (s_gu >= 0) {
            std::lock_guard<std::mutex> lk(seg->ctx->ring_mu);
            seg->ctx->ring_claimed[s_gu] = false;
        }
        return ring_fail(seg, claim_status(s_dn));
    }
    const auto rows = s.rows, d = s.hidden, E = s.n_experts;
    // The router launch copies both validated address tables; the plan reads no table.
    sm::SnapshotCopy snap{};
    snap.src = s_gu >= 0 ? seg->ctx->ring + uint64_t(s_gu) * sm_context::kSlotWords : nullptr;
    snap.dst = reinterpret_cast<uint64_t*>(fr.gu.w.snapshot);
    snap.words = s_gu >= 0 ? uint32_t(fr.gu.w.table.size()) : 0u;
    snap.src2 = s_dn >= 0 ? seg->ctx->ring + uint64_t(s_dn) * sm_context::kSlotWords : nullptr;
    snap.dst2 = reinterpret_cast<uint64_t*>(fr.dn.w.snapshot);
    snap.words2 = s_dn >= 0 ? uint32_t(fr.dn.w.table.size()) : 0u;
    // The shared expert reads only the layer's input and its own weights, and only the combine
    // reads its outputs (the alias checks above), so its two mat-vecs ride in launches of the
    // routed chain: gate/up in the router's, down in the plan's. At the reference model's widths
    // this beats running them on a second stream beside the chain, whose fork and join cost more
    // than the overlap gains (T = 1: 48.0 -> 41.1 us per layer, T = 8: 104.4 -> 97.6 us).
    const bool fused = s.shared_ff != 0;
    const SharedDecodeJobs sj = fused ? shared_decode_jobs(s, sr) : SharedDecodeJobs{};
    const Fmt sfmt = Fmt(f->shared);
    add_step(seg, fused ? "decode router + shared gate/up" : "decode router", [=](hipStream_t st2) {
        const auto* x = reinterpret_cast<const _Float16*>(rr.x);
        const auto* w = reinterpret_cast<const float*>(rr.w);
        const auto* bias = reinterpret_cast<const float*>(rr.bias);
        auto* logits = reinterpret_cast<float*>(rr.logits);
        if (fused) return sm::launch_router_shared_decode(x, w, bias, logits, rows, d, E, snap, sfmt, sj.gu, st2);
        return sm::launch_router_decode(x, w, bias, logits, rows, d, E, snap, st2);
    });
    seg->steps.back().ring_slot = s_gu;
    seg->steps.back().ring_slot2 = s_dn;
    // The route (multiply mode, the Window's) runs in the plan's workgroup of the next launch.
    sm::DecodePlanArgs pa = decode_plan_args(s, pr);
    pa.logits = reinterpret_cast<const float*>(ro.logits);
    pa.route_ids = reinterpret_cast<int32_t*>(ro.ids);
    pa.route_weights = reinterpret_cast<float*>(ro.weights);
    const uintptr_t x = rr.x;
    add_step(seg, fused ? "decode top-k + plan + Q8_1 input + shared down" : "decode top-k + plan + Q8_1 input",
             [=](hipStream_t st2) {
        return sm::launch_decode_front(pa, reinterpret_cast<const _Float16*>(x), reinterpret_cast<uint8_t*>(xq), d, rows,
                                       sfmt, fused ? &sj.dn : nullptr, st2);
    });
    if ((st = encode_routed_ffn_launch(seg, s, f->gate_up, f->down, fr, true)) != SM_OK) return st;
    encode_combine_decode_launch(seg, s, cr);
    return SM_OK;
}

sm_status sm_encode_moe_shared_ffn(sm_segment* seg, const sm_moe_shape* shape, sm_format fmt,
                                   const sm_moe_shared_ffn_buffers* b) {
    Check c;
    const char* P = "MoE shared FFN";
    sm_status st = begin_check(seg, P, c);
    if (st != SM_OK) return st;
    std::string err;
    if ((st = decode_shape_check(shape, P, err, false)) != SM_OK) return record_fail(seg, st, err);
    if (!b) return record_fail(seg, SM_E_ARGUMENT, std::string(P) + " buffers are null");
    SharedRes sr{};
    CombineRes cr{};
    uint64_t p_b, w_b, o_b;
    if (!mul_ok({shape->rows, shape->top_k, shape->hidden, 4}, p_b) || !mul_ok({shape->rows, shape->top_k, 4}, w_b) ||
        !mul_ok({shape->rows, shape->hidden, 4}, o_b))
        return record_fail(seg, SM_E_SHAPE, std::string(P) + " buffer size overflows");
    // The combine reads the shared output and gate logit this call writes (registered once, as
    // the shared stage's outputs).
    if (!check_shared_decode(c, *shape, fmt, b->shared, sr) ||
        !c.view(b->routed_parts, p_b, 16, "routed parts", false, cr.parts) ||
        !c.view(b->route_weights, w_b, 4, "route weights", false, cr.weights) ||
        !c.view(b->output, o_b, 16, "output", true, cr.out) || !c.aliases())
        return finish(seg, c);
    cr.shared = sr.out;
    cr.gate = sr.gl;
    encode_shared_decode_launch(seg, *shape, fmt, sr);
    encode_combine_decode_launch(seg, *shape, cr);
    return SM_OK;
}

sm_status sm_submit_moe_decode_layer(sm_context* ctx, void* stream, const sm_moe_shape* shape,
                                     const sm_layer_formats* formats, const sm_decode_layer_buffers* b, char* err,
                                     size_t cap) {
    SM_SUBMIT_BODY(sm_encode_moe_decode_layer(seg, shape, formats, b))
}

}  // extern "C"
