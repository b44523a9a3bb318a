"""Tiered expert residency: the grouping's residency marks, the expert store's slots, the lease
set and the per-layer handshake (the reference's ExpertStore / ExpertLeaseSet,
include/strata/metal/experts.hpp:18-90; handshake docs/mac/06-engine-host-port.md section 9.3;
status bit 2, prefill_moe_expert_dispatch.hpp:46-50).

CPU: slot-arena addresses count as declared storage; store creation checks its arena; a new
lease set pins nothing. GPU: a layer whose odd experts are not resident, resolved from the GGUF
file into slots between the routing segment and the expert segment, matches the CPU oracle stage
by stage at every grouped entry and token, and gives the full-residency output bit for bit; a second resolve of the layer hits the slot cache; expert stages on slot
addresses no lease pins report status bit 2 and zero those experts' rows; a half with too few
slots for the misses is refused.
"""
import ctypes as C

import numpy as np
import pytest

import gguf_util as gg
from test_abi_host import Fake


def _model(tmp_path, moe, E=16):
    tensors, experts = gg.expert_model(moe, n_layers=2, E=E, d=256, I=128)
    p = tmp_path / "tiered.gguf"
    gg.write_gguf(p, tensors, gg.KV)
    f = moe.GgufFile(p)
    assert f, f.error
    L, err = f.expert_layout(2)
    assert L is not None, err
    return f, L, experts


def test_slot_bytes_and_store_checks(tmp_path, moe):
    f, L, _ = _model(tmp_path, moe)
    sb = moe.library().sm_expert_slot_bytes(C.byref(L))
    assert sb == 2 * (128 * 144) + 256 * 136  # gate + up (Q4_K rows of 256) + down (Q8_0 rows of 128)
    fake = Fake(moe)
    small = fake.buf(2 * 4 * sb - 256)
    st = moe.ExpertStore(fake.ctx, f, L, small.view(), 4)
    assert st.handle is None and st.status == 3 and "undersized" in st.error
    st = moe.ExpertStore(fake.ctx, f, L, moe.View(0, 0, 1 << 20), 4)
    assert st.handle is None and st.status == 4
    arena = fake.buf(2 * 4 * sb)
    st = moe.ExpertStore(fake.ctx, f, L, arena.view(), 4)
    assert st.handle is not None, st.error
    leases = moe.LeaseSet(st)
    assert not leases.pins(0, arena.ptr, 16)
    leases.close()
    st.close()


def test_slot_arena_counts_as_storage(moe):
    fake = Fake(moe)
    arena = fake.buf(1 << 20)
    addr = list(fake.addr)
    addr[3 * 4 + 0] = arena.ptr                      # gate of expert 4 in the arena
    addr[3 * 4 + 1] = arena.ptr + fake.gu_bytes      # its up
    lb = fake.layer(addr=addr)
    t = moe.ExpertTable(addr, fake.snap_gu.view(), [fake.w_gate.view(), fake.w_up.view()], slot_arena=arena.view())
    lb.gate_up.weights = t.struct
    seg = fake.ctx.segment()
    ok, err = seg.encode_prefill_moe_gu(fake.shape, moe.Q4_K, lb.gate_up)
    seg.abort()
    assert ok, err
    t = moe.ExpertTable(addr, fake.snap_gu.view(), [fake.w_gate.view(), fake.w_up.view()])
    lb.gate_up.weights = t.struct
    seg = fake.ctx.segment()
    ok, err = seg.encode_prefill_moe_gu(fake.shape, moe.Q4_K, lb.gate_up)
    seg.abort()
    assert not ok and "expert 4 gate address is outside declared storage" in err


def _tiered_setup(tmp_path, moe, layer, gpu_ctx, stream, slots_per_half=8, E=16, cold=lambda e: e % 2 == 1):
    import torch
    f, L, experts = _model(tmp_path, moe, E)
    cfg = layer.LayerConfig("tiered", 128, 256, E, 4, 128, 0, moe.Q4_K, moe.Q8_0, moe.F16, seed=5)
    inp = layer.make_inputs(cfg)
    inp.w_gate, inp.w_up, inp.w_down = experts[1]
    ws = layer.LayerWorkspace(gpu_ctx, cfg, inp)
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    ref = {n: getattr(ws, n).tensor.cpu().numpy().copy() for n in ("out", "hidden")}
    storage = gpu_ctx.register(torch.empty(L.total_bytes, dtype=torch.uint8, device="cuda"))
    full = f.load_experts(gpu_ctx, stream, L, storage.view())
    resident = np.zeros((2, E), np.int32)
    for e in range(E):
        if cold(e):
            resident[:, e] = -1                      # these experts live only in the cold tier
    res_dev = gpu_ctx.register(torch.from_numpy(resident.ravel().copy()).cuda())
    tiered = list(full)
    for l in range(2):
        for e in range(E):
            if cold(e):
                for r in range(3):
                    tiered[(l * E + e) * 3 + r] = 0
    sb = moe.library().sm_expert_slot_bytes(C.byref(L))
    arena = gpu_ctx.register(torch.empty(2 * slots_per_half * sb, dtype=torch.uint8, device="cuda"))
    store = moe.ExpertStore(gpu_ctx, f, L, arena.view(), slots_per_half)
    assert store.handle is not None, store.error
    return dict(f=f, L=L, ws=ws, ref=ref, storage=storage, full=full, res_dev=res_dev, tiered=tiered, arena=arena,
                store=store, cfg=cfg, inp=inp)


def _route(gpu_ctx, stream, ws, res_dev, lay):
    import torch
    rg = ws.route_gather_buffers()
    rg.resident = res_dev.view()
    rg.layer = lay
    seg = gpu_ctx.segment()
    ok, err = seg.encode_prefill_moe_full_mode_route_gather(ws.shape, rg)
    assert ok, err
    seg.commit(stream)
    torch.cuda.synchronize()


def _experts(moe, gpu_ctx, stream, ws, table, t, leases):
    import torch
    for n in ("out", "hidden", "parts"):
        getattr(ws, n).tensor.view(torch.uint8).fill_(0x5A)
    ws.gu_table = moe.ExpertTable(list(table), ws.snap_gu.view(), [t["storage"].view()], n_layers=2, layer=1,
                                  slot_arena=t["arena"].view(), leases=leases)
    ws.dn_table = moe.ExpertTable(list(table), ws.snap_dn.view(), [t["storage"].view()], n_layers=2, layer=1,
                                  slot_arena=t["arena"].view(), leases=leases)
    seg = gpu_ctx.segment()
    for enc in (lambda s: s.encode_prefill_moe_gu(ws.shape, moe.Q4_K, ws.gate_up_buffers()),
                lambda s: s.encode_prefill_moe_down(ws.shape, moe.Q8_0, ws.down_buffers()),
                lambda s: s.encode_prefill_moe_combine(ws.shape, ws.combine_buffers())):
        ok, err = enc(seg)
        assert ok, err
    seg.commit(stream)
    torch.cuda.synchronize()
    return ws.read_status(stream)


@pytest.mark.gpu
def test_tiered_layer_matches_full_residency(tmp_path, moe, layer, orc, gpu_ctx, stream):
    print("case tiered layer", flush=True)
    t = _tiered_setup(tmp_path, moe, layer, gpu_ctx, stream)
    ws = t["ws"]
    for n in ("out", "hidden", "parts"):
        getattr(ws, n).tensor.view(__import__("torch").uint8).fill_(0x5A)
    _route(gpu_ctx, stream, ws, t["res_dev"], 1)
    pf = orc.plan_fields(ws.plan.tensor.cpu().numpy().view(np.uint8))
    used = pf["grp_e"][: pf["n_groups"]]
    assert list(pf["grp_res"][: pf["n_groups"]]) == [1 if e % 2 == 0 else 0 for e in used]
    n_odd = int((used % 2 == 1).sum())
    assert pf["n_miss"] == n_odd > 0 and pf["skip"] == 0
    leases = moe.LeaseSet(t["store"])
    table = (C.c_uint64 * len(t["tiered"]))(*t["tiered"])
    ok, stats = t["store"].resolve_layer(stream, 1, ws.plan.view(), leases, table)
    assert ok, stats
    assert stats["lookups"] == n_odd and stats["file_reads"] == n_odd and stats["hits"] == 0
    for e in used:
        assert (table[(16 + e) * 3] != 0) and (e % 2 == 0 or leases.pins(1, table[(16 + e) * 3], 16))
    assert _experts(moe, gpu_ctx, stream, ws, table, t, leases) == (0, 0, 0)
    # the tiered layer against the CPU oracle: routing, grouping (residency marks aside), gathered
    # rows, gate/up and down at every grouped entry, combine and the layer on every token
    from test_gpu_layer import _check_stages
    _check_stages(moe, layer, orc, ws, t["inp"], t["cfg"], n_sample_tokens=None, every_entry=True,
                  residency_marks=True)
    assert np.array_equal(ws.out.tensor.cpu().numpy().view(np.uint32), t["ref"]["out"].view(np.uint32))
    assert np.array_equal(ws.hidden.tensor.cpu().numpy().view(np.uint16), t["ref"]["hidden"].view(np.uint16))
    leases.close()
    # a second resolve of the layer finds every miss in the slot cache
    leases2 = moe.LeaseSet(t["store"])
    table2 = (C.c_uint64 * len(t["tiered"]))(*t["tiered"])
    ok, stats = t["store"].resolve_layer(stream, 1, ws.plan.view(), leases2, table2)
    assert ok and stats["hits"] == n_odd and stats["file_reads"] == 0, stats
    assert list(table2) == list(table)
    leases2.close()
    # expert stages on slot addresses no lease pins: status bit 2, those experts' rows zeroed
    st = _experts(moe, gpu_ctx, stream, ws, table, t, None)
    assert st[0] == 0 and st[1] & 4 and st[2] & 4, st
    hid = ws.hidden.tensor.cpu().numpy().view(np.uint16).reshape(-1, 128)
    for gi, e in enumerate(used):
        rows = hid[pf["grp_start"][gi]:pf["grp_start"][gi + 1]]
        assert (rows == 0).all() == (e % 2 == 1)
    t["store"].close()


@pytest.mark.gpu
def test_tiered_half_without_enough_slots(tmp_path, moe, layer, gpu_ctx, stream):
    print("case tiered slots exhausted", flush=True)
    t = _tiered_setup(tmp_path, moe, layer, gpu_ctx, stream, slots_per_half=3)
    ws = t["ws"]
    _route(gpu_ctx, stream, ws, t["res_dev"], 1)
    leases = moe.LeaseSet(t["store"])
    table = (C.c_uint64 * len(t["tiered"]))(*t["tiered"])
    ok, msg = t["store"].resolve_layer(stream, 1, ws.plan.view(), leases, table)
    assert not ok and "every slot of half 1 is pinned" in msg
    assert not leases.pins(1, t["arena"].ptr, 16)   # a failed resolve pins nothing
    leases.close()
    t["store"].close()


def _check_tiered_layer(moe, layer, orc, ws, t):
    from test_gpu_layer import _check_stages
    _check_stages(moe, layer, orc, ws, t["inp"], t["cfg"], n_sample_tokens=None, every_entry=True,
                  residency_marks=True)
    assert np.array_equal(ws.out.tensor.cpu().numpy().view(np.uint32), t["ref"]["out"].view(np.uint32))


@pytest.mark.gpu
def test_tiered_prefetch_then_resolve_hits(tmp_path, moe, layer, orc, gpu_ctx, stream):
    """prefetch_experts warms the odd (cold) experts of layer 1 into its half's slots; the resolve
    after the plan then finds every miss cached (no file read), and the layer on those slots
    matches the oracle and the full-residency output. prefetch_layer over a fresh store fills
    the half's slots and stops at the first expert it has no slot for; repeated, it hits the
    experts it placed."""
    print("case tiered prefetch", flush=True)
    t = _tiered_setup(tmp_path, moe, layer, gpu_ctx, stream)
    ws, store = t["ws"], t["store"]
    odd = list(range(1, 16, 2))
    ok, stats = store.prefetch(stream, 1, odd)
    assert ok and stats == dict(hits=0, lookups=8, file_reads=8, file_bytes=8 * (2 * 128 * 144 + 256 * 136)), stats
    _route(gpu_ctx, stream, ws, t["res_dev"], 1)
    pf = orc.plan_fields(ws.plan.tensor.cpu().numpy().view(np.uint8))
    used = pf["grp_e"][: pf["n_groups"]]
    n_odd = int((used % 2 == 1).sum())
    leases = moe.LeaseSet(store)
    table = (C.c_uint64 * len(t["tiered"]))(*t["tiered"])
    ok, stats = store.resolve_layer(stream, 1, ws.plan.view(), leases, table)
    assert ok and stats["hits"] == n_odd == stats["lookups"] and stats["file_reads"] == 0, stats
    assert _experts(moe, gpu_ctx, stream, ws, table, t, leases) == (0, 0, 0)
    _check_tiered_layer(moe, layer, orc, ws, t)
    leases.close()
    store.close()
    fresh = moe.ExpertStore(gpu_ctx, t["f"], t["L"], t["arena"].view(), 8)
    assert fresh.handle is not None, fresh.error
    ok, stats = fresh.prefetch(stream, 1)
    assert ok and (stats["lookups"], stats["hits"], stats["file_reads"]) == (9, 0, 8), stats
    ok, stats = fresh.prefetch(stream, 1)
    assert ok and (stats["lookups"], stats["hits"], stats["file_reads"]) == (9, 8, 0), stats
    ok, msg = fresh.prefetch(stream, 1, [3, 16])
    assert not ok and "outside the layer" in msg
    fresh.close()


@pytest.mark.gpu
def test_tiered_many_misses_through_the_staging_ring(tmp_path, moe, layer, orc, gpu_ctx, stream):
    """Every expert of a 48-expert layer is cold: the resolve reads more misses than the pinned
    staging ring holds (16), so the ring is reused across rounds, each slot refilled only after
    its previous copy has run; the layer matches the oracle and the full-residency output."""
    print("case tiered 48 cold experts", flush=True)
    t = _tiered_setup(tmp_path, moe, layer, gpu_ctx, stream, slots_per_half=48, E=48, cold=lambda e: True)
    ws, store = t["ws"], t["store"]
    _route(gpu_ctx, stream, ws, t["res_dev"], 1)
    pf = orc.plan_fields(ws.plan.tensor.cpu().numpy().view(np.uint8))
    assert pf["n_miss"] == pf["n_groups"] > 32, pf["n_groups"]
    leases = moe.LeaseSet(store)
    table = (C.c_uint64 * len(t["tiered"]))(*t["tiered"])
    ok, stats = store.resolve_layer(stream, 1, ws.plan.view(), leases, table)
    assert ok and stats["file_reads"] == pf["n_miss"] and stats["hits"] == 0, stats
    assert _experts(moe, gpu_ctx, stream, ws, table, t, leases) == (0, 0, 0)
    _check_tiered_layer(moe, layer, orc, ws, t)
    leases.close()
    store.close()
