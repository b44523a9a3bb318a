"""CPU: the C ABI's exports and the coordinators' host-side preflight.

No GPU is needed: views point at registered fake device ranges, and every case stops at
validation (nothing is committed). The rejection classes and message substrings restate
the reference's negative tests (tests/metal/metal_prefill_moe_grouping_test.mm:801-928,
metal_prefill_moe_full_pipeline_test.mm:987-1104): foreign and short views, misalignment,
aliasing outside the listed producer->consumer edges, bad shapes and formats, expert
addresses outside declared storage, and transactional poisoning of the segment.
"""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def test_library_exports_every_declared_symbol(moe):
    lib = moe.library()
    header = (ROOT / "include" / "strata_moe.h").read_text()
    declared = set(re.findall(r"^\s*(?:[\w\s\*]+?)\b(sm_\w+)\s*\(", header, re.M))
    declared = {d for d in declared if not d.startswith("sm_view") and d != "sm_status"}
    assert len(declared) >= 35
    missing = [d for d in sorted(declared) if not hasattr(lib, d)]
    assert not missing, missing
    assert set(moe.EXPORTS) <= declared
    assert lib.sm_abi_version() == 2


def test_scratch_size_helpers(moe):
    s = moe.Shape(2048, 2048, 512, 10, 512, 512)
    assert moe.histogram_bytes(s) == (20480 // 256 + 1) * 512 * 4
    assert moe.tiles_bytes(s) == (20480 // 64 + 512) * 8


class Fake:
    """A host-only context with fake, non-overlapping device ranges for one small layer."""
    BASE = 0x7F0000000000
    STRIDE = 1 << 32

    def __init__(self, moe, T=7, d=256, E=16, K=4, I=128, Is=256, fmt_gu=2, fmt_dn=1, fmt_sh=4):
        self.moe = moe
        self.ctx = moe.Context(0)
        self.n = 0
        self.shape = moe.Shape(T, d, E, K, I, Is)
        N = T * K
        self.fmts = moe.LayerFormats(fmt_gu, fmt_dn, fmt_sh)
        b = self.buf
        self.x, self.w_router, self.logits = b(T * d * 2), b(E * d * 4), b(T * E * 4)
        self.ids, self.rw = b(N * 4), b(N * 4)
        self.hist, self.plan, self.tiles = b(moe.histogram_bytes(self.shape)), b(6400), b(moe.tiles_bytes(self.shape))
        self.src, self.dst, self.xs = b(N * 4), b(N * 4), b(N * d * 2)
        self.gu_bytes = I * moe.row_bytes(fmt_gu, d)
        self.dn_bytes = d * moe.row_bytes(fmt_dn, I)
        self.w_gate, self.w_up, self.w_down = b(E * self.gu_bytes), b(E * self.gu_bytes), b(E * self.dn_bytes)
        self.snap_gu, self.snap_dn = b(E * 24), b(E * 24)
        self.hidden, self.parts, self.status = b(N * I * 2 + 64), b(N * d * 4), b(8)
        self.sh_g, self.sh_u, self.sh_d, self.sh_v = b(Is * d * 2), b(Is * d * 2), b(d * Is * 2), b(d * 2)
        self.sh_h, self.sh_o, self.sh_gl = b(T * Is * 2), b(T * d * 4), b(T * 4)
        self.out = b(T * d * 4)
        self.addr = []
        for e in range(E):
            self.addr += [self.w_gate.ptr + e * self.gu_bytes, self.w_up.ptr + e * self.gu_bytes,
                          self.w_down.ptr + e * self.dn_bytes]

    def buf(self, nbytes):
        ptr = self.BASE + self.n * self.STRIDE
        self.n += 1
        return self.ctx.register_ptr(ptr, nbytes)

    def layer(self, **over):
        m = self.moe
        v = {k: getattr(self, k).view() for k in ("x", "w_router", "logits", "ids", "rw", "hist", "plan", "tiles",
                                                   "src", "dst", "xs", "hidden", "parts", "sh_g", "sh_u", "sh_d",
                                                   "sh_v", "sh_h", "sh_o", "sh_gl", "out", "snap_gu", "snap_dn")}
        v["st_gu"], v["st_dn"] = self.status.view(0, 4), self.status.view(4, 4)
        v.update(over.pop("views", {}))
        addr = over.pop("addr", self.addr)
        self.gu_table = m.ExpertTable(addr, v["snap_gu"], [self.w_gate.view(), self.w_up.view()])
        self.dn_table = m.ExpertTable(addr, v["snap_dn"], [self.w_down.view()])
        rg = m.RouteGatherBuffers(v["x"], v["w_router"], v["logits"], v["ids"], v["rw"], v["hist"], v["plan"],
                                  v["tiles"], v["src"], v["dst"], v["xs"], m.NULL_VIEW)
        sh = m.SharedBuffers(v["x"], v["sh_g"], v["sh_u"], v["sh_d"], v["sh_v"], v["sh_h"], v["sh_o"], v["sh_gl"])
        gu = m.GateUpBuffers(self.gu_table.struct, over.pop("gu_xs", v["xs"]), v["plan"], v["tiles"], v["hidden"],
                             v["st_gu"])
        dn = m.DownBuffers(self.dn_table.struct, over.pop("dn_hidden", v["hidden"]), v["plan"], v["tiles"], v["dst"],
                           v["parts"], v["st_dn"])
        co = m.CombineBuffers(v["parts"], v["rw"], v["sh_o"], v["sh_gl"], over.pop("co_out", v["out"]))
        self._lb = m.LayerBuffers(rg, sh, gu, dn, co)
        return self._lb

    def encode(self, shape=None, fmts=None, **over):
        seg = self.ctx.segment()
        ok, err = seg.encode_prefill_moe_full_mode_layer(shape or self.shape, fmts or self.fmts, self.layer(**over))
        n = seg.launches
        seg.abort()
        return ok, err, n


@pytest.fixture
def fake(moe):
    return Fake(moe)


def test_valid_layer_encodes(fake):
    ok, err, n = fake.encode()
    assert ok, err
    # router, top-k, grouping, gather with the expert checks, shared x3, gate/up, down, combine
    assert n == 10


def test_commit_without_device_reports_device_error(moe, fake):
    import torch
    if torch.cuda.is_available():
        pytest.skip("host-only case")
    seg = fake.ctx.segment()
    ok, _ = seg.encode_prefill_moe_full_mode_layer(fake.shape, fake.fmts, fake.layer())
    assert ok
    with pytest.raises(RuntimeError, match="SM_E_DEVICE"):
        seg.commit(0)


def test_foreign_and_unregistered_views(moe, fake):
    other = Fake(moe)
    ok, err, _ = fake.encode(views={"xs": other.xs.view()})
    assert not ok and "not owned by this context" in err
    ok, err, _ = fake.encode(views={"plan": moe.View(0, 0, 6400)})
    assert not ok and "not owned by this context" in err
    h = fake.tiles.handle
    assert fake.ctx.unregister(h) == 0
    ok, err, _ = fake.encode()
    assert not ok and "tile list view is not owned" in err


def test_undersized_misaligned_and_out_of_range_views(fake):
    ok, err, _ = fake.encode(views={"hist": fake.hist.view(0, 16)})
    assert not ok and "histogram view is undersized or misaligned" in err
    ok, err, _ = fake.encode(views={"x": fake.x.view(2, fake.x.nbytes - 2)})
    assert not ok and "undersized or misaligned" in err
    ok, err, _ = fake.encode(views={"plan": fake.plan.view(16, 6400)})  # runs past the buffer
    assert not ok and "PfPlan slot view is undersized or misaligned" in err


def test_alias_rules(moe, fake):
    # Outputs of one stage overlapping each other, and an output overlapping an input.
    ok, err, _ = fake.encode(views={"src": fake.ids.view()})
    assert not ok and "overlaps active" in err and "source rows" in err
    ok, err, _ = fake.encode(views={"logits": fake.w_router.view(0, fake.logits.nbytes)})
    assert not ok and "logits overlaps active router weights" in err
    # Listed producer->consumer edges may alias at the same start (the default layout does).
    assert fake.encode()[0]
    # ... but not when the consumer starts elsewhere inside the producer's range.
    ok, err, _ = fake.encode(dn_hidden=fake.hidden.view(16, fake.hidden.nbytes - 16))
    assert not ok and "gate_up.hidden overlaps active down.hidden" in err
    # An unlisted cross-stage overlap: combine output on top of gate/up hidden.
    ok, err, _ = fake.encode(co_out=fake.hidden.view())
    assert not ok and "overlaps active" in err


@pytest.mark.parametrize("field,value,msg", [
    ("rows", 0, "row count"), ("rows", 500000, "row count"), ("n_experts", 0, "experts"),
    ("n_experts", 513, "experts"), ("top_k", 0, "top-k"), ("top_k", 33, "top-k"), ("hidden", 200, "hidden"),
    ("expert_ff", 96, "expert width"),
])
def test_shape_rejections(moe, fake, field, value, msg):
    s = moe.Shape(fake.shape.rows, fake.shape.hidden, fake.shape.n_experts, fake.shape.top_k,
                  fake.shape.expert_ff, fake.shape.shared_ff)
    setattr(s, field, value)
    ok, err, _ = fake.encode(shape=s)
    assert not ok and msg in err


def test_format_rejections(moe, fake):
    ok, err, _ = fake.encode(fmts=moe.LayerFormats(moe.F16, moe.Q8_0, moe.F16))
    assert not ok and "block format" in err
    ok, err, _ = fake.encode(fmts=moe.LayerFormats(moe.Q4_K, moe.Q8_0, moe.Q4_K))
    assert not ok and "F16 or BF16" in err


def test_expert_address_checks(fake):
    addr = list(fake.addr)
    addr[3 * 5 + 1] = fake.w_up.ptr + fake.w_up.nbytes - 16   # up of expert 5 runs past storage
    ok, err, _ = fake.encode(addr=addr)
    assert not ok and "expert 5 up address is outside declared storage" in err
    addr = list(fake.addr)
    addr[3 * 2 + 0] += 2                                     # misaligned gate of expert 2
    ok, err, _ = fake.encode(addr=addr)
    assert not ok and "expert 2 gate address" in err
    addr = list(fake.addr)
    addr[3 * 7 + 2] = fake.w_gate.ptr                        # down of expert 7 in gate storage
    ok, err, _ = fake.encode(addr=addr)
    assert not ok and "expert 7 down address" in err
    addr = list(fake.addr)
    addr[3 * 9 + 0] = 0                                      # null: reported on the GPU (status bit 0)
    assert fake.encode(addr=addr)[0]


def test_failed_encode_poisons_segment(moe, fake):
    seg = fake.ctx.segment()
    bad = fake.layer(views={"hist": fake.hist.view(0, 4)})
    ok, err = seg.encode_prefill_moe_full_mode_layer(fake.shape, fake.fmts, bad)
    assert not ok and seg.launches == 0
    good = fake.layer()
    ok2, err2 = seg.encode_prefill_moe_full_mode_layer(fake.shape, fake.fmts, good)
    assert not ok2 and "undersized" in err2          # the first failure is kept
    with pytest.raises(RuntimeError, match="SM_E_SEGMENT"):
        seg.commit(0)


def test_partial_prefix_then_failure_discards_all(moe, fake):
    """A caller-owned segment that encoded a prefix and then failed is discarded whole."""
    seg = fake.ctx.segment()
    lb = fake.layer()
    ok, _ = seg.encode_prefill_moe_full_mode_route_gather(fake.shape, lb.route_gather)
    assert ok and seg.launches > 0
    bad = moe.CombineBuffers(lb.combine.parts, lb.combine.weights, lb.combine.shared, lb.combine.gate,
                             moe.View(lb.combine.output.buffer, 0, 8))
    ok, err = seg.encode_prefill_moe_combine(fake.shape, bad)
    assert not ok and "output view is undersized" in err
    with pytest.raises(RuntimeError, match="SM_E_SEGMENT"):
        seg.commit(0)


def test_standalone_submit_reports_message(moe, fake):
    lib = moe.library()
    bad = fake.layer(views={"tiles": fake.tiles.view(0, 8)})
    err = C.create_string_buffer(256)
    st = lib.sm_submit_full_layer(fake.ctx.handle, None, C.byref(fake.shape), C.byref(fake.fmts), C.byref(bad),
                                  err, 256)
    assert st == 3 and b"tile list view is undersized or misaligned" in err.value


def test_stage_coordinators_validate_independently(moe, fake):
    lb = fake.layer()
    for name, call in [
        ("route", lambda s: s.encode_moe_route(fake.shape, True, moe.RouteBuffers(
            lb.route_gather.logits, lb.route_gather.route_ids, lb.route_gather.route_weights))),
        ("grouping", lambda s: s.encode_prefill_moe_grouping(fake.shape, moe.GroupingBuffers(
            lb.route_gather.route_ids, lb.route_gather.mixed_h, lb.route_gather.histogram, lb.route_gather.plan,
            lb.route_gather.tiles, lb.route_gather.source_rows, lb.route_gather.destination_rows,
            lb.route_gather.gathered_rows))),
        ("shared", lambda s: s.encode_prefill_moe_shared_ffn(fake.shape, moe.F16, lb.shared)),
        ("gate_up", lambda s: s.encode_prefill_moe_gu(fake.shape, moe.Q4_K, lb.gate_up)),
        ("down", lambda s: s.encode_prefill_moe_down(fake.shape, moe.Q8_0, lb.down)),
        ("combine", lambda s: s.encode_prefill_moe_combine(fake.shape, lb.combine)),
        ("swiglu", lambda s: s.encode_prefill_moe_swiglu(fake.shape.rows, 256, moe.SwiGLUBuffers(
            fake.sh_o.view(), fake.parts.view(), fake.sh_h.view()))),
    ]:
        seg = fake.ctx.segment()
        ok, err = call(seg)
        seg.abort()
        assert ok, (name, err)
    # The route stage alone rejects logits aliasing its outputs.
    seg = fake.ctx.segment()
    ok, err = seg.encode_moe_route(fake.shape, True, moe.RouteBuffers(fake.logits.view(), fake.logits.view(0, 112),
                                                                      fake.rw.view()))
    seg.abort()
    assert not ok and "route IDs overlaps active logits" in err


def test_expert_stage_plan_counters_are_written(moe, fake):
    """The expert stages write their work counters in the plan slot's padding, so a plan view
    whose padding overlaps another view of the stage is rejected (a read-only registration would
    have let it through and the counters would overwrite the tile list)."""
    lb = fake.layer()
    # One allocation holding the plan slot and, from byte 6208 on, the tile list: the PfPlan
    # fields (bytes 0..6207) stay clear of the tile list, the counter words do not.
    nt = moe.tiles_bytes(fake.shape)
    both = fake.buf(6400 + nt)
    plan_over_tiles = both.view(0, 6400)
    gu = moe.GateUpBuffers(lb.gate_up.weights, lb.gate_up.gathered_rows, plan_over_tiles, both.view(6208, nt),
                           lb.gate_up.hidden, lb.gate_up.status)
    seg = fake.ctx.segment()
    ok, err = seg.encode_prefill_moe_gu(fake.shape, moe.Q4_K, gu)
    seg.abort()
    assert not ok and "work counters overlaps active tile list" in err
    dn = moe.DownBuffers(lb.down.weights, lb.down.hidden, plan_over_tiles, both.view(6240, nt), lb.down.destinations,
                         lb.down.parts, lb.down.status)
    seg = fake.ctx.segment()
    ok, err = seg.encode_prefill_moe_down(fake.shape, moe.Q8_0, dn)
    seg.abort()
    assert not ok and "work counters overlaps active tile list" in err
    # The full layer accepts the grouping's own plan slot feeding both stages' counters.
    assert fake.encode()[0]


def test_route_gather_accepts_rows_times_hidden_past_2_32(moe):
    """Activation offsets are 64-bit in every kernel of the route/gather stage, so a chunk whose
    rows x hidden exceeds 2^32 elements is accepted (262,208 rows x 16,384)."""
    f = Fake.__new__(Fake)
    f.moe, f.ctx, f.n = moe, moe.Context(0), 0
    f.STRIDE = 1 << 36
    T, d, E, K = 262208, 16384, 16, 1
    s = moe.Shape(T, d, E, K, 128, 0)
    b = f.buf
    x, w, lg, ids, rw = b(T * d * 2), b(E * d * 4), b(T * E * 4), b(T * K * 4), b(T * K * 4)
    hist, plan, tiles = b(moe.histogram_bytes(s)), b(6400), b(moe.tiles_bytes(s))
    src, dst, xs = b(T * K * 4), b(T * K * 4), b(T * K * d * 2)
    rg = moe.RouteGatherBuffers(x.view(), w.view(), lg.view(), ids.view(), rw.view(), hist.view(), plan.view(),
                                tiles.view(), src.view(), dst.view(), xs.view(), moe.NULL_VIEW)
    seg = f.ctx.segment()
    ok, err = seg.encode_prefill_moe_full_mode_route_gather(s, rg)
    seg.abort()
    assert ok, err
