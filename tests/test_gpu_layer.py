"""GPU parity of the expert stages and the full layer against the CPU oracle.

Each stage is checked on the GPU's own upstream outputs (stage isolation, as the reference's
staged tests do). The expert products are compared at the grouped entries that bound every
unit of work: the first and last entry of every plan group, of every 64-row tile of a small
group, and of every 256-row unit of a group the wide kernel takes (>= 128 entries). Bounds:
- gate/up SwiGLU outputs within 1 F16 ulp + 1e-4 of the FP64 product;
- down parts within 2e-5 + 2e-5 |x| of the FP64 product (the reference's down-tile bound,
  tests/metal/metal_prefill_moe_down_test.mm:591);
- routing, grouping and combine bit-exact on every token;
- the layer output within max-abs 2e-2 and rel-L2 5e-3 in F16.
"""
import numpy as np
import pytest

import gpu_util as gu

pytestmark = pytest.mark.gpu

WIDE_MIN = 128  # groups with at least this many entries run as wide units


def unit_rows(size: int) -> int:
    """Rows per wide unit of a group: ceil(size / 256) units, as even as 32-row blocks allow."""
    nu = -(-size // 256)
    return 32 * -(-size // (32 * nu))


def boundary_entries(plan_fields) -> np.ndarray:
    """Grouped entries at both ends of every group, 64-row tile and wide unit, and of every
    32-row block of a wide unit (the blocks a wave multiplies)."""
    n = plan_fields["n_groups"]
    starts = plan_fields["grp_start"][: n + 1].astype(np.int64)
    sel = []
    for gi in range(n):
        f, e = int(starts[gi]), int(starts[gi + 1])
        step = unit_rows(e - f) if e - f >= WIDE_MIN else 64
        for u0 in range(f, e, step):
            sel += [u0, min(u0 + step, e) - 1]
            if step != 64:
                sel += [b for b0 in range(u0 + 32, min(u0 + step, e), 32) for b in (b0 - 1, b0)]
    return np.unique(np.asarray(sel, np.int64))


def _check_stages(moe, layer, orc, ws, inp, cfg, chunk=0, n_sample_tokens=48, every_entry=False,
                  residency_marks=False):
    """Checks one layer call's outputs (already computed in `ws`): the expert products at the
    boundary entries (or at every entry), combine on every token, the layer on sampled tokens
    (n_sample_tokens None: every token). residency_marks: the plan was built with residency
    marks (tiered experts), so its n_miss, skip and grp_res fields are left out of the plan
    comparison. Returns the grouped entries checked."""
    T, d, E, K, I, Is = cfg.rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff, cfg.shared_ff
    N = T * K
    x = inp.x[chunk * T:(chunk + 1) * T]
    logits = gu.host(ws.logits, np.float32).reshape(T, E)
    ids = gu.host(ws.ids, np.int32).reshape(T, K)
    w = gu.host(ws.route_w, np.float32).reshape(T, K)
    ids_ref, w_ref = orc.route(logits, K, True)
    assert np.array_equal(ids, ids_ref) and np.array_equal(w.view(np.uint32), w_ref.view(np.uint32))
    g = orc.grouping(ids, E)
    assert np.array_equal(gu.host(ws.src, np.int32), g["src"])
    assert np.array_equal(gu.host(ws.dst, np.int32), g["dst"])
    plan = g["plan"]
    got_plan = gu.host(ws.plan, np.uint8)[:6180].copy()
    if residency_marks:
        # n_miss counts the groups marked non-resident and skip is set when there is none; the
        # rest of the plan must equal the full-residency plan
        words, ref_words = got_plan.view(np.int32), plan[:6180].view(np.int32)
        marks = words[520:520 + words[0]]
        assert words[2] == int((marks == 0).sum()) and words[3] == int(words[2] == 0)
        words[2:4] = ref_words[2:4]                  # n_miss, skip
        words[520:1032] = ref_words[520:1032]        # grp_res
    assert np.array_equal(got_plan, plan[:6180])
    pf = orc.plan_fields(plan)
    pos = np.arange(int(pf["grp_start"][pf["n_groups"]])) if every_entry else boundary_entries(pf)
    # gathered rows: bit-exact on every entry
    xs = gu.host(ws.xs, np.uint16).reshape(N, d)
    assert np.array_equal(xs, x[g["src"]]), "gathered rows differ"
    # gate/up on the GPU's gathered rows
    _, _, eh_ref = orc.gate_up_ref(cfg.gate_up_fmt, xs, d, I, plan, inp.w_gate, inp.w_up, inp.gu_stride, pos)
    eh = gu.host(ws.hidden, np.uint16).reshape(N, I)
    gu.assert_f16_close(eh[pos], eh_ref, ulps=1.0, atol=1e-4, what="gate/up SwiGLU")
    # down on the GPU's hidden rows, stored in route order
    parts_ref = orc.down_ref(cfg.down_fmt, eh, d, I, plan, inp.w_down, inp.dn_stride, pos)
    parts = gu.host(ws.parts, np.float32).reshape(N, d)
    got = parts[g["dst"][pos]]
    excess = np.abs(got - parts_ref) - (2e-5 + 2e-5 * np.abs(parts_ref))
    assert (excess <= 0).all(), f"down parts off by up to {float(np.abs(got - parts_ref).max()):.3e}"
    rng = np.random.default_rng(cfg.seed + chunk)
    tokens = np.arange(T) if n_sample_tokens is None else np.sort(rng.choice(T, n_sample_tokens, replace=False))
    # shared expert: every token holding a checked entry, plus the sampled ones
    sh = gl = None
    if Is:
        sh_tokens = np.unique(np.concatenate([g["src"][pos], tokens]))
        hid_ref, _, gl_ref = orc.shared_ref(cfg.shared_fmt, x, d, Is, inp.sh_gate, inp.sh_up, inp.sh_down,
                                            inp.sh_gvec, sh_tokens)
        hid = gu.host(ws.sh_hidden, np.uint16).reshape(T, Is)
        gu.assert_f16_close(hid[sh_tokens], hid_ref, ulps=1.0, atol=1e-4, what="shared SwiGLU")
        sh = gu.host(ws.sh_out, np.float32).reshape(T, d)
        gl = gu.host(ws.sh_gl, np.float32)
        assert np.allclose(gl[sh_tokens], gl_ref, atol=1e-4, rtol=1e-4)
        # shared down on the GPU's hidden rows
        wd = orc.dequant(cfg.shared_fmt, inp.sh_down, d * Is).view(np.float16).astype(np.float64).reshape(d, Is)
        sh_ref = gu.f16(hid[sh_tokens]) @ wd.T
        excess = np.abs(sh[sh_tokens] - sh_ref) - (2e-5 + 2e-5 * np.abs(sh_ref))
        assert (excess <= 0).all(), float(np.abs(sh[sh_tokens] - sh_ref).max())
    # combine: bit-exact against the ordered-FMA restatement on the GPU's inputs, every token
    out = gu.host(ws.out, np.float32).reshape(T, d)
    comb = orc.combine(parts, w, sh, gl, T, K, d)
    assert np.array_equal(out.view(np.uint32), comb.view(np.uint32)), "combine not bit-exact"
    # end to end on the sampled tokens, from the GPU's routing
    out_ref, _ = orc.layer_ref(cfg, inp, ids, w, tokens, chunk=chunk)
    err, rel = gu.layer_tolerance(out[tokens], out_ref)
    print(f"{cfg.name} chunk {chunk}: {len(pos)} boundary entries of {orc.plan_fields(plan)['n_groups']} groups; "
          f"layer max-abs {err:.3e} rel-L2 {rel:.3e} over {len(tokens)} tokens", flush=True)
    assert err <= 2e-2 and rel <= 5e-3
    return pos


def _run_and_check(moe, layer, orc, ctx, stream, cfg, n_sample_tokens=48, chunk=0, inp=None, every_entry=False):
    inp = inp if inp is not None else layer.make_inputs(cfg)
    ws = layer.LayerWorkspace(ctx, cfg, inp, chunk=chunk)
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    _check_stages(moe, layer, orc, ws, inp, cfg, chunk, n_sample_tokens, every_entry)
    return ws


def _check_layer(moe, layer, orc, ctx, stream, cfg):
    """A small layer: every grouped entry of both expert stages and every token."""
    return _run_and_check(moe, layer, orc, ctx, stream, cfg, n_sample_tokens=None, every_entry=True)


def test_layer_config0_full(moe, layer, orc, gpu_ctx, stream):
    print("case layer config 0", flush=True)
    _check_layer(moe, layer, orc, gpu_ctx, stream, layer.CONFIGS[0])


def test_layer_config2_every_group(moe, layer, orc, gpu_ctx, stream):
    print("case layer config 2 (every group)", flush=True)
    _run_and_check(moe, layer, orc, gpu_ctx, stream, layer.CONFIGS[2])


def test_layer_config3_zipf_every_unit(moe, layer, orc, gpu_ctx, stream):
    """Configuration 3 (Zipf-skewed): every group and every wide unit; the layer committed with
    the shared expert on the second stream (forked after top-k at this size) equals, bit for
    bit, the same layer with every launch on one stream."""
    print("case layer config 3 (every group and wide unit)", flush=True)
    import torch
    cfg = layer.CONFIGS[3]
    ws = _run_and_check(moe, layer, orc, gpu_ctx, stream, cfg)
    counts = np.bincount(gu.host(ws.ids, np.int32), minlength=cfg.n_experts)
    print(f"zipf rows per expert: max {counts.max()} median {int(np.median(counts))} "
          f"experts with <=5 rows {(counts <= 5).sum()}", flush=True)
    assert counts.max() > 1000
    two = {n: gu.host(getattr(ws, n), np.uint32).copy() for n in ("out", "sh_out", "sh_gl", "hidden", "parts")}
    for n in two:
        getattr(ws, n).tensor.fill_(0x7F)
    seg = gpu_ctx.segment()
    ok, err = ws.encode_layer(seg)
    assert ok, err
    seg.commit_timed(stream)
    torch.cuda.synchronize()
    for n, ref in two.items():
        assert np.array_equal(gu.host(getattr(ws, n), np.uint32), ref), f"{n} differs between the two commits"


def test_layer_config4_chunk_driver(moe, layer, orc, gpu_ctx, stream):
    """Configuration 4: the 16,384-token prompt through the chunk driver (four 4096-token
    chunks in one segment, one set of chunk scratch). Each chunk's output rows equal, bit for
    bit, the same chunk run as a layer of its own, whose stages are checked against the oracle
    at every group, tile and unit boundary."""
    cfg = layer.CONFIGS[4]
    inp = layer.make_inputs(cfg)
    print("case layer config 4 chunk driver", flush=True)
    pw = layer.PromptWorkspace(gpu_ctx, cfg, inp)
    pw.out_all.tensor.fill_(float("nan"))
    pw.run(stream)
    assert pw.read_status(stream) == (0, 0, 0)
    out_all = gu.host(pw.out_all, np.uint32).reshape(cfg.rows * cfg.chunks, cfg.hidden)
    for c in range(cfg.chunks):
        print(f"case layer config 4 chunk {c}", flush=True)
        ws = _run_and_check(moe, layer, orc, gpu_ctx, stream, cfg, n_sample_tokens=16, chunk=c, inp=inp)
        got = out_all[c * cfg.rows:(c + 1) * cfg.rows]
        assert np.array_equal(got, gu.host(ws.out, np.uint32).reshape(cfg.rows, cfg.hidden)), f"chunk {c} differs"


def test_two_layers_select_plan_slots_and_table_rows(moe, layer, gpu_ctx, stream):
    """Two layers in one segment, as a model's per-layer MoE runs: the plan slots are the two
    6,400-byte slots of one plans buffer and the expert tables the two rows of one
    [layer][E][3] table (the reference's `layer` argument); each layer's outputs equal those
    of the layer committed on its own."""
    import torch
    print("case two layers in one segment", flush=True)
    cfgs = [layer.LayerConfig(f"layer{i}", 256, 512, 32, 4, 256, 256, moe.Q4_K, moe.Q8_0, moe.F16, seed=71 + i)
            for i in range(2)]
    wss = [layer.LayerWorkspace(gpu_ctx, c, layer.make_inputs(c)) for c in cfgs]
    refs = []
    for ws in wss:
        ws.run_layer(stream)
        assert ws.read_status(stream) == (0, 0, 0)
        refs.append(gu.host(ws.out, np.uint32).copy())
        ws.out.tensor.fill_(float("nan"))
    plans = gpu_ctx.register(torch.zeros(2 * 6400, dtype=torch.uint8, device="cuda"))
    table = wss[0].addresses + wss[1].addresses
    storage_gu = [v for ws in wss for v in (ws.w_gate.view(), ws.w_up.view())]
    storage_dn = [ws.w_down.view() for ws in wss]
    seg = gpu_ctx.segment()
    keep = []
    for i, ws in enumerate(wss):
        lb = ws.layer_buffers()
        slot = plans.view(6400 * i, 6400)
        lb.route_gather.plan = lb.gate_up.plan = lb.down.plan = slot
        tg = moe.ExpertTable(table, ws.snap_gu.view(), storage_gu, n_layers=2, layer=i)
        td = moe.ExpertTable(table, ws.snap_dn.view(), storage_dn, n_layers=2, layer=i)
        lb.gate_up.weights, lb.down.weights = tg.struct, td.struct
        keep += [lb, tg, td]
        ok, err = seg.encode_prefill_moe_full_mode_layer(ws.shape, ws.formats, lb, keep=(tg, td))
        assert ok, err
    seg.commit(stream)
    torch.cuda.synchronize()
    for i, ws in enumerate(wss):
        st = gpu_ctx.read_layer_status(stream, plans.view(6400 * i, 6400), ws.status.view(0, 4), ws.status.view(4, 4))
        assert st == (0, 0, 0)
        assert np.array_equal(gu.host(ws.out, np.uint32), refs[i]), f"layer {i} differs"


def test_commit_timed_matches_commit(moe, layer, orc, gpu_ctx, stream):
    """The measurement commit runs the same launches (same outputs) and reports each one."""
    print("case timed commit", flush=True)
    cfg = layer.CONFIGS[0]
    ws = layer.LayerWorkspace(gpu_ctx, cfg, layer.make_inputs(cfg))
    ws.run_layer(stream)
    gub = ws.gate_up_buffers()
    ref = gu.host(ws.hidden, np.uint16).copy()
    ws.hidden.tensor.fill_(0x7C01)
    seg = gpu_ctx.segment()
    ok, err = seg.encode_prefill_moe_gu(cfg.shape(), cfg.gate_up_fmt, gub)
    assert ok, err
    got = seg.commit_timed(stream)
    assert [label for label, _ in got] == ["gate/up plan validate", "gate/up tiles"]
    assert all(ms > 0 for _, ms in got)
    assert np.array_equal(gu.host(ws.hidden, np.uint16), ref)


def test_layer_after_a_producer_in_one_segment(moe, layer, gpu_ctx, stream):
    """A segment holding a launch that writes the activations and then the full layer: the
    layer's shared expert (which runs on the context's second stream) sees the written values,
    so the outputs equal those of the layer committed on its own."""
    print("case layer behind a producer in one segment", flush=True)
    cfg = layer.LayerConfig("seg_order", 256, 256, 16, 4, 128, 256, moe.Q4_K, moe.Q8_0, moe.F16, seed=61)
    ws = layer.LayerWorkspace(gpu_ctx, cfg, layer.make_inputs(cfg))
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    out_ref = gu.host(ws.out, np.float32).copy()
    sh_ref = gu.host(ws.sh_out, np.float32).copy()
    T, d = cfg.rows, cfg.hidden
    x = gu.host(ws.x, np.uint16).reshape(T, d)
    # F16 "weights" [d rows][T values] whose K-major dequant [T][d] is x itself
    src = gpu_ctx.register(gu.dev(np.ascontiguousarray(x.T)))
    ws.x.tensor.fill_(0x7C01)  # poison: only the dequant in the same segment restores x
    ws.out.tensor.fill_(float("nan"))
    ws.sh_out.tensor.fill_(float("nan"))
    seg = gpu_ctx.segment()
    ok, err = seg.encode_prefill_dequant(moe.F16, d, T, src.view(), ws.x.view())
    assert ok, err
    ok, err = seg.encode_prefill_moe_full_mode_layer(ws.shape, ws.formats, ws.layer_buffers())
    assert ok, err
    seg.commit(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    assert np.array_equal(gu.host(ws.sh_out, np.float32).view(np.uint32), sh_ref.view(np.uint32))
    assert np.array_equal(gu.host(ws.out, np.float32).view(np.uint32), out_ref.view(np.uint32))

