"""GPU: reported failures and the standalone post-op kernels.

Failure conditions are forced from the host (every kernel still exits normally), as the
reference's negative tests do (prefill_moe_expert_dispatch.hpp:46-50 status bits,
prefill_moe.metal:556-601 zero paths, metal_prefill_moe_grouping_test.mm:478-659 invalid ids,
metal_prefill_moe_full_pipeline_test.mm:1081-1104 permutation faults).
"""
import numpy as np
import pytest

import gpu_util as gu
import ref_patterns as rp

pytestmark = pytest.mark.gpu


def _small_layer(moe, layer, ctx):
    cfg = layer.LayerConfig("fail", 32, 256, 16, 4, 128, 0, moe.Q4_K, moe.Q8_0, moe.F16, seed=91)
    inp = layer.make_inputs(cfg)
    return cfg, inp, layer.LayerWorkspace(ctx, cfg, inp)


def test_invalid_ids_report_bad_and_zero_outputs(moe, layer, orc, gpu_ctx, stream):
    print("case failure invalid ids", flush=True)
    cfg, inp, ws = _small_layer(moe, layer, gpu_ctx)
    T, K, E = cfg.rows, cfg.top_k, cfg.n_experts
    ids = rp.grouping_ids(T, E, "invalid_ids", K)
    ws.ids.tensor.copy_(gu.dev(ids).reshape(-1))
    ws.hidden.tensor.fill_(0x7C01)
    ws.parts.tensor.fill_(7.0)
    gb, gub, dnb = ws.grouping_buffers(), ws.gate_up_buffers(), ws.down_buffers()
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_grouping(cfg.shape(), gb))
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_gu(cfg.shape(), cfg.gate_up_fmt, gub))
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_down(cfg.shape(), cfg.down_fmt, dnb))
    bad, st_gu, st_dn = ws.read_status(stream)
    flat = ids.reshape(-1)
    assert bad == int(((flat < 0) | (flat >= E)).sum()) > 0
    assert st_gu & 2 and st_dn & 2
    assert (gu.host(ws.hidden, np.uint16) == 0).all()
    assert (gu.host(ws.parts, np.float32) == 0).all()


def test_null_expert_address_sets_status_bit0(moe, layer, orc, gpu_ctx, stream):
    print("case failure null expert address", flush=True)
    cfg, inp, ws = _small_layer(moe, layer, gpu_ctx)
    T, K, E, I = cfg.rows, cfg.top_k, cfg.n_experts, cfg.expert_ff
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    ids = gu.host(ws.ids, np.int32)
    victim = int(np.bincount(ids, minlength=E).argmax())
    addr = list(ws.addresses)
    addr[3 * victim + 1] = 0                       # up weights of an active expert missing
    table = moe.ExpertTable(addr, ws.snap_gu.view(), [ws.w_gate.view(), ws.w_up.view()])
    gub = moe.GateUpBuffers(table.struct, ws.xs.view(), ws.plan.view(), ws.tiles.view(), ws.hidden.view(),
                            ws.status.view(0, 4))
    ws.hidden.tensor.fill_(0x7C01)
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_gu(cfg.shape(), cfg.gate_up_fmt, gub))
    _, st_gu, _ = ws.read_status(stream)
    assert st_gu == 1
    g = orc.grouping(ids.reshape(T, K), E)
    pf = orc.plan_fields(g["plan"])
    gi = list(pf["grp_e"][: pf["n_groups"]]).index(victim)
    a0, a1 = pf["grp_start"][gi], pf["grp_start"][gi + 1]
    eh = gu.host(ws.hidden, np.uint16).reshape(T * K, I)
    assert (eh[a0:a1] == 0).all()
    assert (eh[:a0] != 0x7C01).all() and (eh[a1:] != 0x7C01).all()


def test_broken_destination_permutation_sets_status_bit1(moe, layer, orc, gpu_ctx, stream):
    print("case failure duplicate destination", flush=True)
    cfg, inp, ws = _small_layer(moe, layer, gpu_ctx)
    ws.run_layer(stream)
    dst = gu.host(ws.dst, np.int32).copy()
    dst[5] = dst[6]                                 # a duplicated route index
    ws.dst.tensor.copy_(gu.dev(dst))
    dnb = ws.down_buffers()
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_down(cfg.shape(), cfg.down_fmt, dnb))
    _, _, st_dn = ws.read_status(stream)
    assert st_dn & 2
    assert (gu.host(ws.parts, np.float32) == 0).all()


def test_swiglu_and_combine_bit_exact(moe, orc, gpu_ctx, stream):
    print("case swiglu/combine standalone", flush=True)
    rng = np.random.default_rng(4)
    rows, width = 37, 640
    g = (rng.standard_normal(rows * width) * 4).astype(np.float32)
    u = (rng.standard_normal(rows * width) * 4).astype(np.float32)
    g[:6] = [np.nan, np.inf, -np.inf, 1e-40, -1e-40, 60.0]
    u[:6] = [1.0, 1.0, 1.0, 1.0, 1.0, 5000.0]
    bg, bu = gpu_ctx.register(gu.dev(g)), gpu_ctx.register(gu.dev(u))
    out = gpu_ctx.register(gu.poison(rows * width * 2))
    b = moe.SwiGLUBuffers(bg.view(), bu.view(), out.view())
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_swiglu(rows, width, b))
    assert np.array_equal(gu.host(out, np.uint16), orc.swiglu(g, u))
    T, K, d = 19, 6, 512
    parts = rng.standard_normal((T * K, d)).astype(np.float32)
    w = rng.random((T, K)).astype(np.float32)
    sh = rng.standard_normal((T, d)).astype(np.float32)
    gl = (rng.standard_normal(T) * 3).astype(np.float32)
    bp, bw, bs, bg2 = (gpu_ctx.register(gu.dev(a)) for a in (parts, w, sh, gl))
    bo = gpu_ctx.register(gu.poison(T * d * 4))
    shape = moe.Shape(T, d, 64, K, 64, 256)
    cb = moe.CombineBuffers(bp.view(), bw.view(), bs.view(), bg2.view(), bo.view())
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_combine(shape, cb))
    ref = orc.combine(parts, w, sh, gl, T, K, d)
    assert np.array_equal(gu.host(bo, np.float32).reshape(T, d).view(np.uint32), ref.view(np.uint32))
    shape0 = moe.Shape(T, d, 64, K, 64, 0)
    cb0 = moe.CombineBuffers(bp.view(), bw.view(), moe.NULL_VIEW, moe.NULL_VIEW, bo.view())
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_combine(shape0, cb0))
    ref0 = orc.combine(parts, w, None, None, T, K, d)
    assert np.array_equal(gu.host(bo, np.float32).reshape(T, d).view(np.uint32), ref0.view(np.uint32))


def test_full_layer_clears_both_status_words_and_reports_null_address(moe, layer, orc, gpu_ctx, stream):
    """The full layer checks its plan once for both expert stages: both status words start
    cleared, and a missing weight address is still reported by the gate/up tiles."""
    print("case failure full layer status words", flush=True)
    cfg, inp, ws = _small_layer(moe, layer, gpu_ctx)
    ws.status.tensor.fill_(-1)                       # stale bits from an earlier failure
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    E = cfg.n_experts
    ids = gu.host(ws.ids, np.int32)
    victim = int(np.bincount(ids, minlength=E).argmax())
    addr = list(ws.addresses)
    addr[3 * victim + 1] = 0
    table = moe.ExpertTable(addr, ws.snap_gu.view(), [ws.w_gate.view(), ws.w_up.view()])
    lb = ws.layer_buffers()
    lb.gate_up = moe.GateUpBuffers(table.struct, ws.xs.view(), ws.plan.view(), ws.tiles.view(), ws.hidden.view(),
                                   ws.status.view(0, 4))
    ws.status.tensor.fill_(-1)
    seg = gpu_ctx.segment()
    ok, err = seg.encode_prefill_moe_full_mode_layer(ws.shape, ws.formats, lb, keep=table)
    assert ok, err
    seg.commit(stream)
    bad, st_gu, st_dn = ws.read_status(stream)
    assert (bad, st_gu, st_dn) == (0, 1, 0)


def _foreign(gpu_ctx, tensor, dtype, edit):
    host = gu.host(tensor, dtype).copy()
    edit(host)
    return gpu_ctx.register(gu.dev(host))


@pytest.mark.parametrize("fault", ["repeat", "out_of_range"])
def test_full_layer_checks_destinations_in_the_gather(moe, layer, orc, gpu_ctx, stream, fault):
    """A full layer whose down stage reads a destination map other than the grouping's: the
    gather launch marks it in the bitset, a repeated or out-of-range entry sets bit 1 of the
    down status only, and the down tiles write zeros (metal_prefill_moe_full_pipeline_test.mm:
    1081-1104 permutation faults)."""
    print(f"case failure full layer destination {fault}", flush=True)
    cfg, inp, ws = _small_layer(moe, layer, gpu_ctx)
    ws.run_layer(stream)
    N = cfg.rows * cfg.top_k

    def edit(d):
        if fault == "repeat":
            d[5] = d[6]
        else:
            d[N - 1] = N

    bad_dst = _foreign(gpu_ctx, ws.dst, np.int32, edit)
    lb = ws.layer_buffers()
    lb.down = moe.DownBuffers(ws.dn_table.struct, ws.hidden.view(), ws.plan.view(), ws.tiles.view(),
                              bad_dst.view(), ws.parts.view(), ws.status.view(4, 4))
    ws.status.tensor.fill_(-1)
    ws.parts.tensor.fill_(7.0)
    seg = gpu_ctx.segment()
    ok, err = seg.encode_prefill_moe_full_mode_layer(ws.shape, ws.formats, lb, keep=(ws, bad_dst))
    assert ok, err
    seg.commit(stream)
    bad, st_gu, st_dn = ws.read_status(stream)
    assert (bad, st_gu, st_dn) == (0, 0, 2)
    assert (gu.host(ws.parts, np.float32) == 0).all()
    # The same layer on the grouping's own map is clean again (the bitset is cleared per call).
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)


def test_full_layer_checks_a_foreign_plan_in_the_gather(moe, layer, orc, gpu_ctx, stream):
    """Both expert stages bound to one plan and tile list other than the grouping's, with a
    broken tile chain: the plan check in the gather launch sets bit 1 of both status words and
    both stages write zeros (prefill_moe.metal:603-733)."""
    print("case failure full layer foreign plan", flush=True)
    cfg, inp, ws = _small_layer(moe, layer, gpu_ctx)
    ws.run_layer(stream)
    plan2 = _foreign(gpu_ctx, ws.plan, np.uint8, lambda p: None)

    def edit(t):
        t[3] += 1                                    # second tile's first entry off the 64 grid
    tiles2 = _foreign(gpu_ctx, ws.tiles, np.uint32, edit)
    lb = ws.layer_buffers()
    lb.gate_up = moe.GateUpBuffers(ws.gu_table.struct, ws.xs.view(), plan2.view(), tiles2.view(),
                                   ws.hidden.view(), ws.status.view(0, 4))
    lb.down = moe.DownBuffers(ws.dn_table.struct, ws.hidden.view(), plan2.view(), tiles2.view(),
                              ws.dst.view(), ws.parts.view(), ws.status.view(4, 4))
    ws.status.tensor.fill_(-1)
    ws.hidden.tensor.fill_(0x7C01)
    ws.parts.tensor.fill_(7.0)
    seg = gpu_ctx.segment()
    ok, err = seg.encode_prefill_moe_full_mode_layer(ws.shape, ws.formats, lb, keep=(ws, plan2, tiles2))
    assert ok, err
    seg.commit(stream)
    bad, st_gu, st_dn = ws.read_status(stream)
    assert (bad, st_gu, st_dn) == (0, 2, 2)
    assert (gu.host(ws.hidden, np.uint16) == 0).all()
    assert (gu.host(ws.parts, np.float32) == 0).all()
