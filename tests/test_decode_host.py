"""CPU: host-side preflight of the decode-side coordinators (the Window MoE, T <= 8 rows).

Views point at registered fake device ranges and nothing is committed. The cases restate
the decode dispatch's contract (moe_dispatch.hpp:13-372): T = 1..8 rows and at most 80
routed entries, expert widths in whole 256-value super-blocks, Q8_1 activation and scratch
sizes, block formats only, the plan table indexed by layer, and aliasing between outputs
and inputs.
"""
import pytest


class FakeDecode:
    BASE = 0x7E0000000000
    STRIDE = 1 << 32

    def __init__(self, moe, T=4, d=512, E=32, K=10, I=256, Is=256, fmt_gu=2, fmt_dn=1, layers=2, layer=1):
        self.moe = moe
        self.ctx = moe.Context(0)
        self.n = 0
        self.shape = moe.Shape(T, d, E, K, I, Is)
        self.fmts = moe.LayerFormats(fmt_gu, fmt_dn, moe.F16)
        self.layer = layer
        N = T * K
        b = self.buf
        self.x, self.w_router, self.logits = b(T * d * 2), b(E * d * 4), b(T * E * 4)
        self.ids, self.rw = b(N * 4), b(N * 4)
        self.plans = b(layers * moe.MOE_PLAN_BYTES)
        self.resident, self.usage = b(layers * E * 4), b(layers * E * 4)
        self.xq = b(moe.q8_1_bytes(T, d))
        self.gate, self.up, self.hidden = b(N * I * 4), b(N * I * 4), b(N * I * 4)
        self.hq, self.parts, self.status = b(moe.q8_1_bytes(N, I)), b(N * d * 4), b(4)
        self.sh_g, self.sh_u, self.sh_d, self.sh_v = b(Is * d * 2), b(Is * d * 2), b(d * Is * 2), b(d * 2)
        self.sh_h, self.sh_o, self.sh_gl = b(T * Is * 4), b(T * d * 4), b(T * 4)  # decode hidden is F32
        self.out = b(T * d * 4)
        self.gu_bytes = I * moe.row_bytes(fmt_gu, d)
        self.dn_bytes = d * moe.row_bytes(fmt_dn, I)
        self.w_gate, self.w_up, self.w_down = b(E * self.gu_bytes), b(E * self.gu_bytes), b(E * self.dn_bytes)
        self.snap_gu, self.snap_dn = b(layers * E * 24), b(layers * E * 24)
        self.addr = []
        for _ in range(layers):
            for e in range(E):
                self.addr += [self.w_gate.ptr + e * self.gu_bytes, self.w_up.ptr + e * self.gu_bytes,
                              self.w_down.ptr + e * self.dn_bytes]
        self.layers = layers
        self.gu_table = moe.ExpertTable(self.addr, self.snap_gu.view(), [self.w_gate.view(), self.w_up.view()],
                                        layers, layer)
        self.dn_table = moe.ExpertTable(self.addr, self.snap_dn.view(), [self.w_down.view()], layers, layer)

    def buf(self, nbytes):
        ptr = self.BASE + self.n * self.STRIDE
        self.n += 1
        return self.ctx.register_ptr(ptr, nbytes)

    def routed(self, **over):
        m = self.moe
        v = dict(xq=self.xq.view(), plans=self.plans.view(), gate=self.gate.view(), up=self.up.view(),
                 hidden=self.hidden.view(), hq=self.hq.view(), parts=self.parts.view(), status=self.status.view())
        v.update(over)
        return m.MoeRoutedFFNBuffers(self.gu_table.struct, self.dn_table.struct, v["xq"], v["plans"], v["gate"],
                                     v["up"], v["hidden"], v["hq"], v["parts"], v["status"])

    def layer_buffers(self, routed=None, **over):
        m = self.moe
        v = dict(x=self.x.view(), w_router=self.w_router.view(), logits=self.logits.view(), ids=self.ids.view(),
                 rw=self.rw.view(), resident=m.NULL_VIEW, usage=m.NULL_VIEW, plans=self.plans.view(),
                 xq=self.xq.view(), out=self.out.view())
        v.update(over)
        sh = m.SharedBuffers(v["x"], self.sh_g.view(), self.sh_u.view(), self.sh_d.view(), self.sh_v.view(),
                             self.sh_h.view(), self.sh_o.view(), self.sh_gl.view())
        return m.DecodeLayerBuffers(v["x"], v["w_router"], m.NULL_VIEW, v["logits"], v["ids"], v["rw"],
                                    v["resident"], v["usage"], v["plans"], self.layer, v["xq"],
                                    routed or self.routed(), sh, v["out"])

    def run(self, fn):
        seg = self.ctx.segment()
        ok, err = fn(seg)
        n = seg.launches
        seg.abort()
        return ok, err, n


@pytest.fixture
def fd(moe):
    return FakeDecode(moe)


def shape_with(moe, s, **kw):
    v = dict(rows=s.rows, hidden=s.hidden, n_experts=s.n_experts, top_k=s.top_k, expert_ff=s.expert_ff,
             shared_ff=s.shared_ff)
    v.update(kw)
    return moe.Shape(v["rows"], v["hidden"], v["n_experts"], v["top_k"], v["expert_ff"], v["shared_ff"])


def test_decode_coordinators_encode(moe, fd):
    pb = moe.MoePlanBuffers(fd.ids.view(), fd.resident.view(), fd.usage.view(), fd.plans.view(), fd.status.view(),
                            fd.layer)
    assert fd.run(lambda s: s.encode_moe_plan(fd.shape, pb))[::2] == (True, 1)
    assert fd.run(lambda s: s.encode_quantize_q8_1(fd.shape.rows, fd.shape.hidden, False, fd.x.view(),
                                                   fd.xq.view()))[::2] == (True, 1)
    eb = moe.MoeExpertBuffers(fd.gu_table.struct, fd.xq.view(), fd.plans.view(), fd.gate.view(), fd.up.view(),
                              fd.status.view())
    assert fd.run(lambda s: s.encode_moe_experts(fd.shape, moe.Q4_K, eb))[::2] == (True, 2)  # snapshot + mat-vec
    db = moe.MoeDownBuffers(fd.dn_table.struct, fd.hq.view(), fd.plans.view(), fd.parts.view(), fd.status.view())
    assert fd.run(lambda s: s.encode_moe_down(fd.shape, moe.Q8_0, db))[::2] == (True, 2)
    sb = moe.SwiGLUBuffers(fd.gate.view(), fd.up.view(), fd.hidden.view())
    assert fd.run(lambda s: s.encode_moe_swiglu(40, 256, sb))[::2] == (True, 1)
    # snapshot, gate/up, SwiGLU + Q8_1, snapshot, down
    assert fd.run(lambda s: s.encode_moe_routed_ffn(fd.shape, moe.Q4_K, moe.Q8_0, fd.routed()))[::2] == (True, 5)
    cb = moe.CombineBuffers(fd.parts.view(), fd.rw.view(), fd.sh_o.view(), fd.sh_gl.view(), fd.out.view())
    assert fd.run(lambda s: s.encode_moe_combine(fd.shape, cb))[::2] == (True, 1)
    # shared gate/up + SwiGLU (+ the gate logit), down, combine
    sfb = moe.MoeSharedFFNBuffers(fd.layer_buffers().shared, fd.parts.view(), fd.rw.view(), fd.out.view())
    assert fd.run(lambda s: s.encode_moe_shared_ffn(fd.shape, moe.F16, sfb))[::2] == (True, 3)
    sfb.shared.hidden = fd.sh_h.view(0, fd.shape.rows * fd.shape.shared_ff * 2)  # an F16-sized hidden
    ok, err, _ = fd.run(lambda s: s.encode_moe_shared_ffn(fd.shape, moe.F16, sfb))
    assert not ok and "shared hidden view is undersized" in err
    # router + shared gate/up, top-k + plan + Q8_1 input + shared down, gate/up, SwiGLU + Q8_1, down, combine
    ok, err, n = fd.run(lambda s: s.encode_moe_decode_layer(fd.shape, fd.fmts, fd.layer_buffers()))
    assert ok, err
    assert n == 6
    ns = shape_with(moe, fd.shape, shared_ff=0)  # the same launches without the shared expert's parts
    ok, err, n = fd.run(lambda s: s.encode_moe_decode_layer(ns, fd.fmts, fd.layer_buffers()))
    assert ok and n == 6, err


@pytest.mark.parametrize("kw,msg", [
    (dict(rows=9), "T=1..8 rows"), (dict(rows=8, top_k=11), "at most 80 routed entries"),
    (dict(expert_ff=96), "multiple of 64"), (dict(hidden=200), "hidden"), (dict(n_experts=513), "experts"),
])
def test_decode_shape_rejections(moe, fd, kw, msg):
    s = shape_with(moe, fd.shape, **kw)
    ok, err, n = fd.run(lambda seg: seg.encode_moe_decode_layer(s, fd.fmts, fd.layer_buffers()))
    assert not ok and msg in err and n == 0
    ok, err, _ = fd.run(lambda seg: seg.encode_moe_routed_ffn(s, moe.Q4_K, moe.Q8_0, fd.routed()))
    assert not ok and msg in err


def test_decode_formats_and_layers(moe, fd):
    ok, err, _ = fd.run(lambda s: s.encode_moe_decode_layer(fd.shape, moe.LayerFormats(moe.F16, moe.Q8_0, moe.F16),
                                                             fd.layer_buffers()))
    assert not ok and "block format" in err
    # the plan table must hold the selected layer
    ok, err, _ = fd.run(lambda s: s.encode_moe_decode_layer(fd.shape, fd.fmts,
                                                             fd.layer_buffers(plans=fd.plans.view(0, 1620))))
    assert not ok and "MoePlan view is undersized" in err
    # expert tables selecting another layer than the plan
    other = moe.ExpertTable(fd.addr, fd.snap_gu.view(), [fd.w_gate.view(), fd.w_up.view()], fd.layers, 0)
    r = fd.routed()
    r.gate_up_weights = other.struct
    ok, err, _ = fd.run(lambda s: s.encode_moe_decode_layer(fd.shape, fd.fmts, fd.layer_buffers(routed=r)))
    assert not ok and "different layer" in err


def test_decode_views_sizes_and_aliases(moe, fd):
    ok, err, _ = fd.run(lambda s: s.encode_quantize_q8_1(4, 512, False, fd.x.view(), fd.xq.view(0, 36 * 60)))
    assert not ok and "Q8_1 output view is undersized" in err
    ok, err, _ = fd.run(lambda s: s.encode_quantize_q8_1(4, 500, False, fd.x.view(), fd.xq.view()))
    assert not ok and "multiple of 32" in err
    # the Q8_1 hidden scratch sized for T rows instead of T*k
    ok, err, _ = fd.run(lambda s: s.encode_moe_routed_ffn(fd.shape, moe.Q4_K, moe.Q8_0,
                                                          fd.routed(hq=fd.hq.view(0, moe.q8_1_bytes(4, 256)))))
    assert not ok and "Q8_1 hidden view is undersized" in err
    # gate written over the input activations
    ok, err, _ = fd.run(lambda s: s.encode_moe_routed_ffn(fd.shape, moe.Q4_K, moe.Q8_0,
                                                          fd.routed(gate=fd.parts.view(0, fd.gate.nbytes))))
    assert not ok and "overlaps active" in err
    # the layer output on top of the router weights
    ok, err, _ = fd.run(lambda s: s.encode_moe_decode_layer(fd.shape, fd.fmts,
                                                             fd.layer_buffers(out=fd.w_router.view(0, fd.out.nbytes))))
    assert not ok and "output overlaps active router weights" in err


def test_decode_submit_reports_message(moe, fd):
    import ctypes as C
    lib = moe.library()
    err = C.create_string_buffer(256)
    s = shape_with(moe, fd.shape, rows=9)
    b = fd.layer_buffers()
    st = lib.sm_submit_moe_decode_layer(fd.ctx.handle, None, C.byref(s), C.byref(fd.fmts), C.byref(b), err, 256)
    assert st != 0 and b"T=1..8 rows" in err.value


def test_decode_reference_model_widths(moe):
    """The reference model's decode widths (d = 2560, expert and shared width 640: twenty 32-value
    blocks, not whole 256-value super-blocks) encode with Q8_0 down weights; K-quant down weights
    of that width are rejected."""
    fd = FakeDecode(moe, T=8, d=2560, E=64, K=10, I=640, Is=640, fmt_gu=2, fmt_dn=1)
    ok, err, n = fd.run(lambda s: s.encode_moe_decode_layer(fd.shape, fd.fmts, fd.layer_buffers()))
    assert ok and n == 6, err
    ok, err, _ = fd.run(lambda s: s.encode_moe_routed_ffn(fd.shape, moe.Q4_K, moe.Q4_K, fd.routed()))
    assert not ok and "expert weight extent is invalid" in err
