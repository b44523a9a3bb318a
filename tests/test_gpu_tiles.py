"""GPU: the 64-row tile kernels on layers whose groups are all below 128 entries.

Every group here is below 128 entries, so both expert stages run on the tile kernels; the
shapes cover Q4_K, Q2_K and Q8_0 weights on both stages, reductions of one to five
256-value slabs (activation slabs resident or streamed), one to eight column tiles per work
item, a down reduction of 384 values, which runs on the plain tile kernel, and more gate/up
items than workgroups (items run back to back). Each case checks every token of both stages and
the layer against the CPU oracle with the benchmark configurations' bars (gate/up within
1 F16 ulp, down parts within 2e-5 + 2e-5 |x|, layer max-abs 2e-2 and rel-L2 5e-3), and the failure
paths (a missing expert address zeroes that group's rows, leaves every other row as the clean
run wrote it, and sets status bit 0; a broken
destination permutation zeroes the parts and sets bit 1), as the reference's negative tests
do (prefill_moe_expert_dispatch.hpp:46-50, prefill_moe.metal:556-601).
"""
import numpy as np
import pytest

import gpu_util as gu
from test_gpu_layer import _check_layer

pytestmark = pytest.mark.gpu


def _cases(layer, moe):
    C = layer.LayerConfig
    return {
        # gate/up Q4_K: 5 slabs; down Q4_K: 2 slabs (resident), 5 column tiles of 256
        "q4k_5slab": C("tiles_q4k", 256, 1280, 24, 3, 512, 0, moe.Q4_K, moe.Q4_K, moe.F16, seed=301),
        # gate/up Q2_K: 4 slabs; down Q8_0: 4 slabs (streamed), 4 column tiles of 256
        "q2k_q80": C("tiles_q80", 256, 1024, 16, 4, 1024, 0, moe.Q2_K, moe.Q8_0, moe.F16, seed=302),
        # gate/up Q4_K: 1 slab, 4 column tiles of 128; down Q8_0: 2 slabs, 1 column tile
        "q80_2slab": C("tiles_q80b", 128, 256, 8, 2, 512, 0, moe.Q4_K, moe.Q8_0, moe.F16, seed=303),
        # gate/up Q4_K: 3 column tiles; down K = 384 on the plain tile kernel
        "odd_tiles": C("tiles_odd", 192, 512, 12, 2, 384, 0, moe.Q4_K, moe.Q8_0, moe.F16, seed=304),
        # 512 gate/up items (128 groups x 4 column tiles) on at most 256 workgroups: each
        # workgroup runs items back to back, the next one's copies issued by the current one
        "many_items": C("tiles_many", 1024, 1280, 128, 8, 512, 0, moe.Q4_K, moe.Q8_0, moe.F16, seed=305),
    }


@pytest.mark.parametrize("case", ["q4k_5slab", "q2k_q80", "q80_2slab", "odd_tiles"])
def test_tile_kernels_layer(moe, layer, orc, gpu_ctx, stream, case):
    cfg = _cases(layer, moe)[case]
    print(f"case tiles {case}: T {cfg.rows} d {cfg.hidden} E {cfg.n_experts} top-{cfg.top_k} "
          f"I {cfg.expert_ff}", flush=True)
    ws = _check_layer(moe, layer, orc, gpu_ctx, stream, cfg)
    counts = np.bincount(gu.host(ws.ids, np.int32), minlength=cfg.n_experts)
    assert counts.max() < 128


def _victim_rows(orc, ws, cfg, victim):
    ids = gu.host(ws.ids, np.int32)
    g = orc.grouping(ids.reshape(cfg.rows, cfg.top_k), cfg.n_experts)
    pf = orc.plan_fields(g["plan"])
    gi = list(pf["grp_e"][: pf["n_groups"]]).index(victim)
    return int(pf["grp_start"][gi]), int(pf["grp_start"][gi + 1])


@pytest.mark.parametrize("case", ["q4k_5slab", "q2k_q80", "many_items"])
def test_tile_null_address_zeroes_group(moe, layer, orc, gpu_ctx, stream, case):
    print(f"case tiles null expert address {case}", flush=True)
    cfg = _cases(layer, moe)[case]
    ws = layer.LayerWorkspace(gpu_ctx, cfg, layer.make_inputs(cfg))
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    E, I, d, N = cfg.n_experts, cfg.expert_ff, cfg.hidden, cfg.entries
    # The clean run's results: every other group must come out bit-identical without the
    # victim (same kernels, same item order; the victim's items are skipped, not reordered).
    eh_clean = gu.host(ws.hidden, np.uint16).reshape(N, I).copy()
    parts_clean = gu.host(ws.parts, np.float32).reshape(N, d).copy()
    victim = int(np.bincount(gu.host(ws.ids, np.int32), minlength=E).argmax())
    a0, a1 = _victim_rows(orc, ws, cfg, victim)
    assert 0 < a1 - a0 < 128
    # gate/up: the victim's gate weights missing
    addr = list(ws.addresses)
    addr[3 * victim] = 0
    table = moe.ExpertTable(addr, ws.snap_gu.view(), [ws.w_gate.view(), ws.w_up.view()])
    gub = moe.GateUpBuffers(table.struct, ws.xs.view(), ws.plan.view(), ws.tiles.view(), ws.hidden.view(),
                            ws.status.view(0, 4))
    ws.hidden.tensor.fill_(0x7C01)
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_gu(cfg.shape(), cfg.gate_up_fmt, gub))
    _, st_gu, _ = ws.read_status(stream)
    assert st_gu == 1
    eh = gu.host(ws.hidden, np.uint16).reshape(N, I)
    assert (eh[a0:a1] == 0).all()
    assert (eh[:a0] == eh_clean[:a0]).all() and (eh[a1:] == eh_clean[a1:]).all()
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
    assert np.array_equal(parts[~mine], parts_clean[~mine])


def test_tile_broken_destination_zeroes_parts(moe, layer, orc, gpu_ctx, stream):
    print("case tiles duplicate destination", flush=True)
    cfg = _cases(layer, moe)["q2k_q80"]
    ws = layer.LayerWorkspace(gpu_ctx, cfg, layer.make_inputs(cfg))
    ws.run_layer(stream)
    dst = gu.host(ws.dst, np.int32).copy()
    dst[3] = dst[4]
    ws.dst.tensor.copy_(gu.dev(dst))
    dnb = ws.down_buffers()
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_down(cfg.shape(), cfg.down_fmt, dnb))
    _, _, st_dn = ws.read_status(stream)
    assert st_dn & 2
    assert (gu.host(ws.parts, np.float32) == 0).all()
