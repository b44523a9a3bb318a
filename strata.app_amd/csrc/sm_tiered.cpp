// Tiered expert residency: the expert store (cold tier -> device slots), slot leases and the
// per-layer handshake, host side.
//
// Follows the reference's ExpertStore / ExpertLeaseSet contract (include/strata/metal/
// experts.hpp:18-90) and the layer handshake of docs/mac/06-engine-host-port.md section 9.3:
// the GPU grouping marks each group resident or not (PfPlan grp_res, n_miss, skip); the host
// reads the plan, looks each missing (layer, expert) up in the slot cache of half layer % 2,
// reads a miss's gate, up and down slabs from the cold tier into a free or least recently used
// unpinned slot, publishes the slot addresses in the layer's address-table row and pins them in
// the lease set. Here the cold tier is the model's GGUF file (the page cache being the RAM tier)
// and the handshake runs between two committed segments on one stream instead of through
// GPU-side event waits. Misses are read by up to kFetchWorkers host threads at once (the
// reference's kExpertFetchWorkers, experts.hpp:14) into a ring of pinned staging slots, and
// each staged expert is copied to its device slot asynchronously on the caller's stream, so
// the expert stages committed after the resolve on that stream see it. prefetch warms chosen
// experts of a layer into unpinned slots ahead of its plan (prefetch_layer /
// prefetch_experts, experts.hpp:90-94).
#include <hip/hip_runtime_api.h>

#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "../../include/strata_moe.h"
#include "sm_internal.h"

namespace {
constexpr uint64_t kSlabAlign = 256;
constexpr uint32_t kPlanExperts = 512;
constexpr uint32_t kFetchWorkers = 8;            // host threads reading cold experts at once
constexpr uint32_t kMaxStaging = 16;             // pinned staging slots (two per worker) ...
constexpr uint64_t kStagingBudget = 256ull << 20;  // ... within this many bytes (at least two)

// PfPlan (prefill_moe.metal:23-40), as the grouping writes it.
struct PlanHost {
    uint32_t n_groups, n_entries, n_miss, skip, n_tiles, bad, pad[2];
    int32_t grp_e[kPlanExperts];
    int32_t grp_res[kPlanExperts];
    int32_t grp_start[kPlanExperts + 1];
};
static_assert(sizeof(PlanHost) == 6180, "PfPlan layout");

uint64_t up256(uint64_t v) { return (v + kSlabAlign - 1) & ~(kSlabAlign - 1); }

sm_status fail(char* err, size_t cap, sm_status st, const std::string& msg) {
    if (err && cap) std::snprintf(err, cap, "%s", msg.c_str());
    return st;
}
}  // namespace

struct sm_expert_store {
    sm_context* ctx = nullptr;
    sm_gguf* gguf = nullptr;
    sm_expert_layout layout{};
    uintptr_t arena = 0;
    uint64_t slot_bytes = 0, slab[3] = {0, 0, 0}, role_off[3] = {0, 0, 0};
    uint32_t per_half = 0;
    struct Slot {
        int32_t layer = -1, expert = -1;
        uint64_t last_use = 0;
        uint32_t pins = 0;
    };
    std::vector<Slot> slots[2];
    std::map<std::pair<uint32_t, uint32_t>, uint32_t> where[2];  // (layer, expert) -> slot
    uint64_t clock = 0;
    // Pinned staging ring (n_staging slots), made on the first cold read; staged[i] is the event
    // recorded after the copy out of slot i, which must complete before the slot is refilled.
    uint8_t* staging = nullptr;
    uint32_t n_staging = 0;
    std::vector<hipEvent_t> staged;
    std::vector<bool> staged_pending;
    std::mutex mu;
};

struct sm_lease_set {
    sm_expert_store* store = nullptr;
    struct Pin {
        uint32_t layer, half, slot;
        uint64_t address, bytes;
    };
    std::vector<Pin> pins;
};

namespace {
void unpin_where(sm_lease_set* set, bool (*match)(const sm_lease_set::Pin&, uint32_t), uint32_t arg) {
    sm_expert_store* st = set->store;
    std::lock_guard<std::mutex> lk(st->mu);
    std::vector<sm_lease_set::Pin> keep;
    for (const auto& p : set->pins) {
        if (match(p, arg)) {
            auto& slot = st->slots[p.half][p.slot];
            if (slot.pins > 0) --slot.pins;
        } else {
            keep.push_back(p);
        }
    }
    set->pins.swap(keep);
}
}  // namespace

namespace {
// A cold expert to bring into a slot of the current half.
struct Job {
    uint32_t slot;
    int32_t expert;
};

uintptr_t slot_base(const sm_expert_store* s, uint32_t half, uint32_t slot) {
    return s->arena + (uint64_t(half) * s->per_half + slot) * s->slot_bytes;
}

// The slot of half `half` holding (layer, expert), or -1 (the store's lock is held).
int64_t lookup(sm_expert_store* s, uint32_t half, uint32_t layer, int32_t e) {
    auto it = s->where[half].find(std::make_pair(layer, uint32_t(e)));
    return it == s->where[half].end() ? -1 : int64_t(it->second);
}

// A free slot, else the least recently used one that no live lease pins (and, with `skip`, that
// the caller has not marked), assigned to (layer, expert); -1 if there is none.
int64_t claim_slot(sm_expert_store* s, uint32_t half, uint32_t layer, int32_t e, const std::vector<bool>* skip) {
    int64_t pick = -1;
    for (uint32_t i = 0; i < s->per_half; ++i) {
        const auto& sl = s->slots[half][i];
        if (sl.pins != 0 || (skip && (*skip)[i])) continue;
        if (sl.layer < 0) { pick = i; break; }
        if (pick < 0 || sl.last_use < s->slots[half][uint32_t(pick)].last_use) pick = i;
    }
    if (pick < 0) return -1;
    auto& sl = s->slots[half][uint32_t(pick)];
    if (sl.layer >= 0) s->where[half].erase(std::make_pair(uint32_t(sl.layer), uint32_t(sl.expert)));
    sl.layer = int32_t(layer);
    sl.expert = e;
    s->where[half][std::make_pair(layer, uint32_t(e))] = uint32_t(pick);
    return pick;
}

// Undoes a failed resolve or prefetch: its pins are dropped and the slots it was filling are
// emptied (their copies, if any were queued, complete harmlessly).
void abandon(sm_expert_store* s, uint32_t half, const std::vector<Job>& jobs,
             const std::vector<sm_lease_set::Pin>& pins) {
    for (const auto& np : pins)
        if (s->slots[np.half][np.slot].pins > 0) --s->slots[np.half][np.slot].pins;
    for (const auto& j : jobs) {
        auto& sl = s->slots[half][j.slot];
        if (sl.layer >= 0) s->where[half].erase(std::make_pair(uint32_t(sl.layer), uint32_t(sl.expert)));
        sl.layer = -1;
        sl.expert = -1;
    }
}

// Reads each job's gate, up and down slabs from the cold tier and queues their copies into the
// job's slot on `hs`. Jobs go through the pinned staging ring in rounds of n_staging: up to
// kFetchWorkers threads read a round's experts at once, then each staged expert is copied with
// one asynchronous copy and an event that guards its staging slot. Nothing here waits for the
// copies; work committed on `hs` afterwards runs after them.
sm_status fetch(sm_expert_store* s, hipStream_t hs, uint32_t layer, uint32_t half, const std::vector<Job>& jobs,
                std::string* why) {
    if (jobs.empty()) return SM_OK;
    const uint64_t E = s->layout.n_experts;
    sm_gguf_tensor t[3];
    const char* roles[3] = {"gate", "up", "down"};
    for (int r = 0; r < 3; ++r) {
        const std::string name = "blk." + std::to_string(layer) + ".ffn_" + roles[r] + "_exps.weight";
        if (sm_gguf_find(s->gguf, name.c_str(), &t[r]) != SM_OK || t[r].bytes / E != s->slab[r]) {
            *why = "cold tier has no usable " + name;
            return SM_E_FILE;
        }
    }
    if (!s->staging) {
        const uint64_t fit = kStagingBudget / s->slot_bytes;
        const uint32_t n = uint32_t(std::max<uint64_t>(2, std::min<uint64_t>(kMaxStaging, fit)));
        if (hipHostMalloc(reinterpret_cast<void**>(&s->staging), n * s->slot_bytes, hipHostMallocDefault) != hipSuccess) {
            s->staging = nullptr;
            *why = "pinned staging ring cannot be allocated";
            return SM_E_DEVICE;
        }
        s->staged.assign(n, nullptr);
        s->staged_pending.assign(n, false);
        for (uint32_t i = 0; i < n; ++i)
            if (hipEventCreateWithFlags(&s->staged[i], hipEventDisableTiming) != hipSuccess) {
                for (uint32_t k = 0; k < i; ++k) (void)hipEventDestroy(s->staged[k]);
                (void)hipHostFree(s->staging);
                s->staging = nullptr;
                s->staged.clear();
                s->staged_pending.clear();
                *why = "staging events cannot be created";
                return SM_E_DEVICE;
            }
        s->n_staging = n;
    }
    const uint32_t R = s->n_staging;
    for (size_t b0 = 0; b0 < jobs.size(); b0 += R) {
        const uint32_t nb = uint32_t(std::min<size_t>(R, jobs.size() - b0));
        for (uint32_t i = 0; i < nb; ++i)
            if (s->staged_pending[i]) {
                if (hipEventSynchronize(s->staged[i]) != hipSuccess) {
                    *why = "waiting for a staging slot failed";
                    return SM_E_DEVICE;
                }
                s->staged_pending[i] = false;
            }
        std::atomic<uint32_t> next{0};
        std::atomic<bool> bad{false};
        auto worker = [&]() {
            for (uint32_t i = next++; i < nb && !bad; i = next++) {
                const int32_t e = jobs[b0 + i].expert;
                uint8_t* dst = s->staging + uint64_t(i) * s->slot_bytes;
                for (int r = 0; r < 3; ++r)
                    if (sm_internal_gguf_read(s->gguf, t[r].offset + uint64_t(e) * s->slab[r], s->slab[r],
                                              dst + s->role_off[r]) != SM_OK)
                        bad = true;
            }
        };
        const uint32_t nw = std::min(kFetchWorkers, nb);
        std::vector<std::thread> pool;
        for (uint32_t w = 1; w < nw; ++w) pool.emplace_back(worker);
        worker();
        for (auto& th : pool) th.join();
        if (bad) {
            *why = "cold tier read of layer " + std::to_string(layer) + " failed";
            return SM_E_FILE;
        }
        for (uint32_t i = 0; i < nb; ++i) {
            const uintptr_t dst = slot_base(s, half, jobs[b0 + i].slot);
            if (hipMemcpyAsync(reinterpret_cast<void*>(dst), s->staging + uint64_t(i) * s->slot_bytes, s->slot_bytes,
                               hipMemcpyHostToDevice, hs) != hipSuccess ||
                hipEventRecord(s->staged[i], hs) != hipSuccess) {
                *why = "slot upload failed";
                return SM_E_DEVICE;
            }
            s->staged_pending[i] = true;
        }
    }
    return SM_OK;
}
}  // namespace

extern "C" {

uint64_t sm_expert_slot_bytes(const sm_expert_layout* L) {
    if (!L) return 0;
    const uint64_t gu = sm_format_row_bytes(L->gate_up, L->hidden) * L->expert_ff;
    const uint64_t dn = sm_format_row_bytes(L->down, L->expert_ff) * L->hidden;
    return 2 * up256(gu) + up256(dn);
}

sm_status sm_expert_store_create(sm_context* ctx, sm_gguf* gguf, const sm_expert_layout* L, sm_view arena,
                                 uint32_t per_half, sm_expert_store** out, char* err, size_t cap) {
    if (!ctx || !gguf || !L || !out) return fail(err, cap, SM_E_ARGUMENT, "expert store arguments are null");
    if (per_half == 0) return fail(err, cap, SM_E_SHAPE, "expert store needs at least one slot per half");
    const uint64_t sb = sm_expert_slot_bytes(L);
    if (sb == 0) return fail(err, cap, SM_E_SHAPE, "expert layout has no slab size");
    uintptr_t base = 0;
    const sm_status vs = sm_internal_resolve_view(ctx, arena, 2ull * per_half * sb, kSlabAlign, &base);
    if (vs != SM_OK)
        return fail(err, cap, vs, vs == SM_E_OWNERSHIP ? "slot arena view is not owned by this context"
                                                       : "slot arena view is undersized or misaligned");
    auto* s = new (std::nothrow) sm_expert_store();
    if (!s) return fail(err, cap, SM_E_DEVICE, "out of host memory");
    s->ctx = ctx;
    s->gguf = gguf;
    s->layout = *L;
    s->arena = base;
    s->slot_bytes = sb;
    s->slab[0] = s->slab[1] = sm_format_row_bytes(L->gate_up, L->hidden) * L->expert_ff;
    s->slab[2] = sm_format_row_bytes(L->down, L->expert_ff) * L->hidden;
    s->role_off[0] = 0;
    s->role_off[1] = up256(s->slab[0]);
    s->role_off[2] = 2 * up256(s->slab[0]);
    s->per_half = per_half;
    s->slots[0].resize(per_half);
    s->slots[1].resize(per_half);
    *out = s;
    if (err && cap) err[0] = 0;
    return SM_OK;
}

void sm_expert_store_destroy(sm_expert_store* s) {
    if (!s) return;
    // Teardown is best effort: the staging ring is freed once its last copies have run.
    for (size_t i = 0; i < s->staged.size(); ++i) {
        if (s->staged_pending[i]) (void)hipEventSynchronize(s->staged[i]);
        (void)hipEventDestroy(s->staged[i]);
    }
    if (s->staging) (void)hipHostFree(s->staging);
    delete s;
}

sm_status sm_lease_set_create(sm_expert_store* store, sm_lease_set** out) {
    if (!store || !out) return SM_E_ARGUMENT;
    auto* l = new (std::nothrow) sm_lease_set();
    if (!l) return SM_E_DEVICE;
    l->store = store;
    *out = l;
    return SM_OK;
}

void sm_lease_set_destroy(sm_lease_set* l) {
    if (!l) return;
    unpin_where(l, [](const sm_lease_set::Pin&, uint32_t) { return true; }, 0);
    delete l;
}

void sm_lease_set_retire_layer(sm_lease_set* l, uint32_t layer) {
    if (!l) return;
    unpin_where(l, [](const sm_lease_set::Pin& p, uint32_t a) { return p.layer == a; }, layer);
}

int sm_lease_set_pins(const sm_lease_set* l, uint32_t layer, uint64_t address, uint64_t bytes) {
    if (!l) return 0;
    std::lock_guard<std::mutex> lk(l->store->mu);
    for (const auto& p : l->pins)
        if (p.layer == layer && address >= p.address && address - p.address <= p.bytes &&
            bytes <= p.bytes - (address - p.address))
            return 1;
    return 0;
}

sm_status sm_expert_store_resolve_layer(sm_expert_store* s, void* stream, uint32_t layer, sm_view plan_view,
                                        sm_lease_set* leases, uint64_t* table, uint64_t n_table,
                                        sm_store_stats* stats, char* err, size_t cap) {
    if (!s || !leases || !table || leases->store != s) return fail(err, cap, SM_E_ARGUMENT, "resolve arguments are null or mismatched");
    const sm_expert_layout& L = s->layout;
    const uint64_t E = L.n_experts;
    if (layer >= L.n_layers) return fail(err, cap, SM_E_ARGUMENT, "layer is outside the expert layout");
    if (n_table < (uint64_t(layer) + 1) * E * 3) return fail(err, cap, SM_E_ARGUMENT, "address table is too short for the layer");
    uintptr_t pdev = 0;
    sm_status st = sm_internal_resolve_view(s->ctx, plan_view, sizeof(PlanHost), 4, &pdev);
    if (st != SM_OK) return fail(err, cap, st, "PfPlan slot view is undersized, misaligned or not owned by this context");
    if (sm_internal_make_current(s->ctx) != SM_OK) return fail(err, cap, SM_E_DEVICE, "the context's device cannot be made current");
    const hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
    // The plan is ready once the stream's earlier work (the grouping) has completed; that also
    // proves every earlier layer's expert reads on this stream are done, so their pins retire.
    if (hipStreamSynchronize(hs) != hipSuccess) return fail(err, cap, SM_E_DEVICE, "waiting for the plan failed");
    unpin_where(leases, [](const sm_lease_set::Pin& p, uint32_t a) { return p.layer < a; }, layer);
    PlanHost p{};
    if (hipMemcpy(&p, reinterpret_cast<const void*>(pdev), 16, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(err, cap, SM_E_DEVICE, "reading the plan header failed");
    sm_store_stats local{};
    if (p.skip != 0) {
        if (p.n_miss != 0) return fail(err, cap, SM_E_ARGUMENT, "skipped plan reports misses");
        if (stats) *stats = local;
        return SM_OK;
    }
    if (hipMemcpy(&p, reinterpret_cast<const void*>(pdev), sizeof p, hipMemcpyDeviceToHost) != hipSuccess)
        return fail(err, cap, SM_E_DEVICE, "reading the plan failed");
    if (p.n_groups > kPlanExperts || p.n_groups > E) return fail(err, cap, SM_E_ARGUMENT, "plan group count is out of range");
    uint32_t misses = 0;
    for (uint32_t g = 0; g < p.n_groups; ++g) misses += p.grp_res[g] == 0 ? 1u : 0u;
    if (misses != p.n_miss) return fail(err, cap, SM_E_ARGUMENT, "plan miss count disagrees with its groups");
    for (uint32_t g = 0; g < p.n_groups; ++g)
        if (p.grp_res[g] == 0 && (p.grp_e[g] < 0 || uint64_t(p.grp_e[g]) >= E))
            return fail(err, cap, SM_E_ARGUMENT, "plan names an expert outside the layer");

    const uint32_t half = layer & 1u;
    std::lock_guard<std::mutex> lk(s->mu);
    std::vector<Job> jobs;
    std::vector<sm_lease_set::Pin> new_pins;
    for (uint32_t g = 0; g < p.n_groups; ++g) {
        if (p.grp_res[g] != 0) continue;
        const int32_t e = p.grp_e[g];
        ++local.lookups;
        int64_t slot = lookup(s, half, layer, e);
        if (slot >= 0) {
            ++local.hits;
        } else {
            // Every slot this resolve takes is pinned at once, so it is not taken twice.
            slot = claim_slot(s, half, layer, e, nullptr);
            if (slot < 0) {
                abandon(s, half, jobs, new_pins);
                return fail(err, cap, SM_E_SHAPE, "every slot of half " + std::to_string(half) + " is pinned");
            }
            jobs.push_back({uint32_t(slot), e});
        }
        auto& sl = s->slots[half][uint32_t(slot)];
        sl.last_use = ++s->clock;
        const uintptr_t base = slot_base(s, half, uint32_t(slot));
        for (int r = 0; r < 3; ++r) {  // one pin per slab; the slot counts every pin it holds
            table[(uint64_t(layer) * E + uint64_t(e)) * 3 + uint64_t(r)] = base + s->role_off[r];
            new_pins.push_back({layer, half, uint32_t(slot), base + s->role_off[r], s->slab[r]});
            ++sl.pins;
        }
    }
    std::string why;
    st = fetch(s, hs, layer, half, jobs, &why);
    if (st != SM_OK) {
        abandon(s, half, jobs, new_pins);
        return fail(err, cap, st, why);
    }
    local.file_reads = jobs.size();
    local.file_bytes = uint64_t(jobs.size()) * (s->slab[0] + s->slab[1] + s->slab[2]);
    for (const auto& np : new_pins) leases->pins.push_back(np);
    if (stats) *stats = local;
    if (err && cap) err[0] = 0;
    return SM_OK;
}

sm_status sm_expert_store_prefetch(sm_expert_store* s, void* stream, uint32_t layer, const int32_t* experts,
                                   uint32_t n_experts, sm_store_stats* stats, char* err, size_t cap) {
    if (!s) return fail(err, cap, SM_E_ARGUMENT, "prefetch store is null");
    const sm_expert_layout& L = s->layout;
    if (layer >= L.n_layers) return fail(err, cap, SM_E_ARGUMENT, "layer is outside the expert layout");
    const uint32_t n = experts ? n_experts : L.n_experts;
    for (uint32_t i = 0; experts && i < n; ++i)
        if (experts[i] < 0 || uint32_t(experts[i]) >= L.n_experts)
            return fail(err, cap, SM_E_ARGUMENT, "prefetch names an expert outside the layer");
    if (sm_internal_make_current(s->ctx) != SM_OK) return fail(err, cap, SM_E_DEVICE, "the context's device cannot be made current");
    const uint32_t half = layer & 1u;
    sm_store_stats local{};
    std::lock_guard<std::mutex> lk(s->mu);
    std::vector<Job> jobs;
    std::vector<bool> taken(s->per_half, false);  // slots this prefetch filled: never evicted by it
    for (uint32_t i = 0; i < n; ++i) {
        const int32_t e = experts ? experts[i] : int32_t(i);
        ++local.lookups;
        int64_t slot = lookup(s, half, layer, e);
        if (slot >= 0) {
            ++local.hits;
        } else {
            slot = claim_slot(s, half, layer, e, &taken);
            if (slot < 0) break;  // the half is full of pinned or just-prefetched slots
            jobs.push_back({uint32_t(slot), e});
        }
        taken[uint32_t(slot)] = true;
        s->slots[half][uint32_t(slot)].last_use = ++s->clock;
    }
    std::string why;
    const sm_status st = fetch(s, reinterpret_cast<hipStream_t>(stream), layer, half, jobs, &why);
    if (st != SM_OK) {
        std::vector<sm_lease_set::Pin> none;
        abandon(s, half, jobs, none);
        return fail(err, cap, st, why);
    }
    local.file_reads = jobs.size();
    local.file_bytes = uint64_t(jobs.size()) * (s->slab[0] + s->slab[1] + s->slab[2]);
    if (stats) *stats = local;
    if (err && cap) err[0] = 0;
    return SM_OK;
}

}  // extern "C"
