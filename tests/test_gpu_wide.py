"""GPU: the wide routed kernel (256-row units for groups of >= 128 entries).

Groups of at least 128 entries run on the wide kernel, smaller ones on the 64-row tile
kernels (gate/up: both in one launch, the tiles drawn after the wide units), so a skewed
routing exercises both in one stage. Each case checks the expert
stages and the full layer against the CPU oracle with the same bars as the benchmark
configurations (gate/up within 1 F16 ulp, down parts within 2e-5 + 2e-5 |x|, layer max-abs 2e-2 and
rel-L2 5e-3), over every weight format on both stages, with partial last units; and the
failure paths of the wide kernel (a missing expert address zeroes that group's rows and sets
status bit 0; a broken destination permutation zeroes the parts), as the reference's
negative tests do (prefill_moe_expert_dispatch.hpp:46-50, prefill_moe.metal:556-601).
"""
import numpy as np
import pytest

import gpu_util as gu
from test_gpu_layer import _check_layer

pytestmark = pytest.mark.gpu


def _skewed(layer, moe, gu_fmt, dn_fmt, seed=202):
    # 32 experts, top-4 over 512 tokens with a Zipf(0.8) bias: groups of 509, 450, 346, 236,
    # 162 (wide: two full + partial units, single partial units) and many below 128.
    return layer.LayerConfig("wide_mixed", 512, 512, 32, 4, 256, 0, gu_fmt, dn_fmt, moe.F16,
                             zipf_s=0.8, seed=seed)


@pytest.mark.parametrize("formats", [("Q4_K", "Q8_0"), ("Q8_0", "Q2_K"), ("Q2_K", "Q4_K")])
def test_wide_and_tile_kernels_mixed(moe, layer, orc, gpu_ctx, stream, formats):
    gu_fmt, dn_fmt = (getattr(moe, f) for f in formats)
    print(f"case wide mixed gate/up {formats[0]} down {formats[1]}", flush=True)
    cfg = _skewed(layer, moe, gu_fmt, dn_fmt)
    ws = _check_layer(moe, layer, orc, gpu_ctx, stream, cfg)
    counts = np.bincount(gu.host(ws.ids, np.int32), minlength=cfg.n_experts)
    assert (counts >= 256).sum() >= 2 and ((counts > 0) & (counts < 128)).sum() >= 4


def test_wide_only_partial_units(moe, layer, orc, gpu_ctx, stream):
    # 8 experts, top-2 over 640 tokens: every group has 148-177 entries, one partial unit each.
    print("case wide only partial units", flush=True)
    cfg = layer.LayerConfig("wide_only", 640, 512, 8, 2, 256, 0, moe.Q4_K, moe.Q8_0, moe.F16, seed=204)
    ws = _check_layer(moe, layer, orc, gpu_ctx, stream, cfg)
    counts = np.bincount(gu.host(ws.ids, np.int32), minlength=cfg.n_experts)
    assert counts.min() >= 128


def _victim_rows(orc, ws, cfg, victim):
    ids = gu.host(ws.ids, np.int32)
    g = orc.grouping(ids.reshape(cfg.rows, cfg.top_k), cfg.n_experts)
    pf = orc.plan_fields(g["plan"])
    gi = list(pf["grp_e"][: pf["n_groups"]]).index(victim)
    return int(pf["grp_start"][gi]), int(pf["grp_start"][gi + 1])


def test_wide_null_address_zeroes_group(moe, layer, orc, gpu_ctx, stream):
    print("case wide null expert address", flush=True)
    cfg = _skewed(layer, moe, moe.Q4_K, moe.Q8_0)
    inp = layer.make_inputs(cfg)
    ws = layer.LayerWorkspace(gpu_ctx, cfg, inp)
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    E, I, d, N = cfg.n_experts, cfg.expert_ff, cfg.hidden, cfg.entries
    victim = int(np.bincount(gu.host(ws.ids, np.int32), minlength=E).argmax())
    a0, a1 = _victim_rows(orc, ws, cfg, victim)
    assert a1 - a0 >= 256
    # gate/up: the victim's up weights missing
    addr = list(ws.addresses)
    addr[3 * victim + 1] = 0
    table = moe.ExpertTable(addr, ws.snap_gu.view(), [ws.w_gate.view(), ws.w_up.view()])
    gub = moe.GateUpBuffers(table.struct, ws.xs.view(), ws.plan.view(), ws.tiles.view(), ws.hidden.view(),
                            ws.status.view(0, 4))
    ws.hidden.tensor.fill_(0x7C01)
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_gu(cfg.shape(), cfg.gate_up_fmt, gub))
    _, st_gu, _ = ws.read_status(stream)
    assert st_gu == 1
    eh = gu.host(ws.hidden, np.uint16).reshape(N, I)
    assert (eh[a0:a1] == 0).all()
    assert (eh[:a0] != 0x7C01).all() and (eh[a1:] != 0x7C01).all()
    # down: the victim's down weights missing; its entries' parts rows are zero
    ws.run_layer(stream)
    addr = list(ws.addresses)
    addr[3 * victim + 2] = 0
    table = moe.ExpertTable(addr, ws.snap_dn.view(), [ws.w_down.view()])
    dnb = moe.DownBuffers(table.struct, ws.hidden.view(), ws.plan.view(), ws.tiles.view(), ws.dst.view(),
                          ws.parts.view(), ws.status.view(4, 4))
    ws.parts.tensor.fill_(float("nan"))
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_down(cfg.shape(), cfg.down_fmt, dnb))
    _, _, st_dn = ws.read_status(stream)
    assert st_dn == 1
    parts = gu.host(ws.parts, np.float32).reshape(N, d)
    dst = gu.host(ws.dst, np.int32)
    mine = np.zeros(N, bool)
    mine[dst[a0:a1]] = True
    assert (parts[mine] == 0).all()
    assert np.isfinite(parts[~mine]).all()


def test_small_group_null_address_beside_wide_units(moe, layer, orc, gpu_ctx, stream):
    # gate/up runs wide units and small-group tiles in one launch; a small group without up
    # weights zeroes its rows and sets status bit 0 while every other row is computed.
    print("case null address of a small group beside wide units", flush=True)
    cfg = _skewed(layer, moe, moe.Q4_K, moe.Q8_0)
    inp = layer.make_inputs(cfg)
    ws = layer.LayerWorkspace(gpu_ctx, cfg, inp)
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    E, I, N = cfg.n_experts, cfg.expert_ff, cfg.entries
    ref = gu.host(ws.hidden, np.uint16).reshape(N, I).copy()
    counts = np.bincount(gu.host(ws.ids, np.int32), minlength=E)
    assert counts.max() >= 256
    small = np.flatnonzero((counts > 0) & (counts < 128))
    victim = int(small[np.argmax(counts[small])])
    a0, a1 = _victim_rows(orc, ws, cfg, victim)
    addr = list(ws.addresses)
    addr[3 * victim + 1] = 0
    table = moe.ExpertTable(addr, ws.snap_gu.view(), [ws.w_gate.view(), ws.w_up.view()])
    gub = moe.GateUpBuffers(table.struct, ws.xs.view(), ws.plan.view(), ws.tiles.view(), ws.hidden.view(),
                            ws.status.view(0, 4))
    ws.hidden.tensor.fill_(0x7C01)
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_gu(cfg.shape(), cfg.gate_up_fmt, gub))
    _, st_gu, _ = ws.read_status(stream)
    assert st_gu == 1
    eh = gu.host(ws.hidden, np.uint16).reshape(N, I)
    assert (eh[a0:a1] == 0).all()
    assert np.array_equal(eh[:a0], ref[:a0]) and np.array_equal(eh[a1:], ref[a1:])


def test_wide_broken_destination_zeroes_parts(moe, layer, orc, gpu_ctx, stream):
    print("case wide duplicate destination", flush=True)
    cfg = _skewed(layer, moe, moe.Q4_K, moe.Q8_0)
    ws = layer.LayerWorkspace(gpu_ctx, cfg, layer.make_inputs(cfg))
    ws.run_layer(stream)
    dst = gu.host(ws.dst, np.int32).copy()
    dst[5] = dst[6]
    ws.dst.tensor.copy_(gu.dev(dst))
    dnb = ws.down_buffers()
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_down(cfg.shape(), cfg.down_fmt, dnb))
    _, _, st_dn = ws.read_status(stream)
    assert st_dn & 2
    assert (gu.host(ws.parts, np.float32) == 0).all()
