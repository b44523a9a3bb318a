"""GPU: the decode-side MoE (the Window MoE over T <= 8 rows) against the oracle.

Integer work is bit-exact: the MoePlan and its usage counts, the Q8_1 quantizer (F16 and F32
inputs), route ids from the GPU's own logits. The F32 post-ops (SwiGLU, the decode combine)
are bit-exact against the oracle's restatement. The mat-vecs are checked against FP64 dots of
the same Q8_1 codes and weight blocks, within 32 F32 roundings of the block terms' magnitudes
(a lane sums at most a few blocks, then a butterfly of at most six steps). The layer output is
checked against a composed oracle within the layer bound (max-abs 2e-2, rel-L2 5e-3 in F16).
Failure paths are forced from the host (a null expert address, out-of-range ids, a damaged
plan header, route destinations that name no row): every kernel still exits normally.
"""
import numpy as np
import pytest

import gpu_util as gu

pytestmark = pytest.mark.gpu

F32_EPS = 2.0 ** -24
_INPUTS = {}


def _inputs(layer, cfg):
    key = (cfg.seed, cfg.hidden, cfg.n_experts, cfg.expert_ff, cfg.shared_ff, cfg.gate_up_fmt, cfg.down_fmt,
           cfg.shared_fmt)
    if key not in _INPUTS:
        big = layer.LayerConfig(cfg.name, 8, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff, cfg.shared_ff,
                                cfg.gate_up_fmt, cfg.down_fmt, cfg.shared_fmt, seed=cfg.seed)
        _INPUTS.clear()
        _INPUTS[key] = layer.make_inputs(big)
    return _INPUTS[key]


def _small(layer, moe, T=8):
    """The reference model's widths (d 2560, expert/shared 640) over 64 experts."""
    return layer.LayerConfig("dec_small", T, 2560, 64, 10, 640, 640, moe.Q4_K, moe.Q8_0, moe.F16, seed=0x5EED0D01)


def _ids(rng, T, K, E, collide=True):
    """Distinct experts per token; with `collide`, tokens share experts (larger groups)."""
    pool = E if not collide else max(K + 2, E // 8)
    return np.stack([rng.choice(pool, K, replace=False) for _ in range(T)]).astype(np.int32)


def _plan_fields(orc, plan):
    return plan.view(orc.PLAN_DTYPE)[0]


def _within(got, ref, mag, what, k=32):
    tol = k * F32_EPS * mag + 1e-30
    bad = np.abs(got.astype(np.float64) - ref) > tol
    assert not bad.any(), (f"{what}: {bad.sum()} of {bad.size} off; worst "
                           f"{float((np.abs(got - ref) / np.maximum(mag, 1e-30)).max()):.3e} of the magnitude")


def routed_ref(orc, cfg, inp, plan, xq, hq=None):
    """FP64 gate/up [N][I] (grouped entry order) from Q8_1 token rows xq, and, given the Q8_1
    hidden rows hq (grouped order), FP64 parts [N][d] in route order."""
    p = _plan_fields(orc, plan)
    T, d, K, I = cfg.rows, cfg.hidden, cfg.top_k, cfg.expert_ff
    N = T * K
    g = np.zeros((N, I)); u = np.zeros((N, I)); gm = np.zeros((N, I)); um = np.zeros((N, I))
    parts = np.zeros((N, d)); pm = np.zeros((N, d))
    for gi in range(int(p["n_groups"])):
        e = int(p["grp_e"][gi])
        a0, a1 = int(p["grp_start"][gi]), int(p["grp_start"][gi + 1])
        act = np.ascontiguousarray(xq.reshape(T, -1)[p["ent_tok"][a0:a1]])
        s = inp.gu_stride
        g[a0:a1], gm[a0:a1] = orc.q81_matvec(cfg.gate_up_fmt, inp.w_gate[e * s:(e + 1) * s], I, d, act)
        u[a0:a1], um[a0:a1] = orc.q81_matvec(cfg.gate_up_fmt, inp.w_up[e * s:(e + 1) * s], I, d, act)
        if hq is not None:
            s = inp.dn_stride
            hact = np.ascontiguousarray(hq.reshape(N, -1)[a0:a1])
            v, m = orc.q81_matvec(cfg.down_fmt, inp.w_down[e * s:(e + 1) * s], d, I, hact)
            parts[p["ent_dst"][a0:a1]] = v
            pm[p["ent_dst"][a0:a1]] = m
    return g, u, gm, um, parts, pm


def _dense(fmt, bits, shape):
    b = np.asarray(bits).view(np.uint16).reshape(shape)
    if fmt == 5:  # BF16
        return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    return b.view(np.float16).astype(np.float64)


# ---- plan ------------------------------------------------------------------------------------
@pytest.mark.parametrize("T,E", [(1, 512), (8, 512), (8, 64), (5, 16)])
def test_plan_bit_exact(moe, orc, gpu_ctx, stream, T, E):
    print(f"case decode plan T={T} E={E}", flush=True)
    rng = np.random.default_rng(T * 100 + E)
    K = 10
    shape = moe.Shape(T, 256, E, K, 64, 0)
    ids = _ids(rng, T, K, E, collide=E > 64)
    resident = np.where(rng.random((2, E)) < 0.6, 1, -1).astype(np.int32)
    usage0 = rng.integers(0, 50, (2, E)).astype(np.float32)
    b_ids, b_res, b_use = gpu_ctx.register(gu.dev(ids)), gpu_ctx.register(gu.dev(resident)), gpu_ctx.register(gu.dev(usage0))
    b_plan = gpu_ctx.register(gu.poison(2 * 1620))
    b_st = gpu_ctx.register(gu.dev(np.full(1, 0x55, np.uint32)))
    pb = moe.MoePlanBuffers(b_ids.view(), b_res.view(), b_use.view(), b_plan.view(), b_st.view(), 1)
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_plan(shape, pb))
    usage = usage0[1].copy()
    want, rc = orc.moe_plan(ids, E, resident[1], usage)
    got = gu.host(b_plan, np.uint8)
    assert rc == 0 and np.array_equal(got[1620:], want)
    assert (got[:1620] == 0xA5).all()  # layer 0's plan untouched
    assert np.array_equal(gu.host(b_use, np.float32).reshape(2, E)[1], usage)
    assert np.array_equal(gu.host(b_use, np.float32).reshape(2, E)[0], usage0[0])
    assert gu.host(b_st, np.uint32)[0] == 0
    # full mode (no residency, no usage): every group resident
    pb = moe.MoePlanBuffers(b_ids.view(), moe.NULL_VIEW, moe.NULL_VIEW, b_plan.view(), b_st.view(), 0)
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_plan(shape, pb))
    want, _ = orc.moe_plan(ids, E)
    assert np.array_equal(gu.host(b_plan, np.uint8)[:1620], want)


def test_plan_invalid_ids_empty_and_status(moe, orc, gpu_ctx, stream):
    print("case decode plan invalid ids", flush=True)
    T, K, E = 3, 10, 64
    ids = np.stack([np.arange(K) + 3 * t for t in range(T)]).astype(np.int32)
    ids[1, 4] = E  # out of range
    ids[2, 0] = -7
    shape = moe.Shape(T, 256, E, K, 64, 0)
    b_ids, b_plan = gpu_ctx.register(gu.dev(ids)), gpu_ctx.register(gu.poison(1620))
    b_st = gpu_ctx.register(gu.dev(np.zeros(1, np.uint32)))
    pb = moe.MoePlanBuffers(b_ids.view(), moe.NULL_VIEW, moe.NULL_VIEW, b_plan.view(), b_st.view(), 0)
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_plan(shape, pb))
    want, rc = orc.moe_plan(ids, E)
    assert rc == 1 and np.array_equal(gu.host(b_plan, np.uint8), want)
    assert gu.host(b_st, np.uint32)[0] == 2


# ---- Q8_1 ------------------------------------------------------------------------------------
def test_q8_1_bit_exact(moe, orc, gpu_ctx, stream):
    import test_oracle_decode as tod
    print("case decode Q8_1 f32 + f16", flush=True)
    rng = np.random.default_rng(17)
    x = tod.q81_cases(rng)
    rows, n = x.shape
    bx, by = gpu_ctx.register(gu.dev(x)), gpu_ctx.register(gu.poison(rows * n // 32 * 36))
    gu.run(gpu_ctx, stream, lambda s: s.encode_quantize_q8_1(rows, n, True, bx.view(), by.view()))
    assert np.array_equal(gu.host(by, np.uint8).reshape(rows, -1), orc.quantize_q8_1(x))
    h = (rng.standard_normal((8, 2560)) * np.float32(3)).astype(np.float16)
    h[0, :32] = 0
    h[1, 40:72] = np.float16(6e-8)  # F16 subnormals
    h[2, 100] = np.float16(65504)
    bh, bq = gpu_ctx.register(gu.dev(h.view(np.uint16))), gpu_ctx.register(gu.poison(8 * 80 * 36))
    gu.run(gpu_ctx, stream, lambda s: s.encode_quantize_q8_1(8, 2560, False, bh.view(), bq.view()))
    assert np.array_equal(gu.host(bq, np.uint8).reshape(8, -1), orc.quantize_q8_1(h.astype(np.float32)))


# ---- grouped mat-vecs ------------------------------------------------------------------------
@pytest.mark.parametrize("gu_fmt,dn_fmt,d,I", [(2, 1, 2560, 640), (1, 2, 2048, 512), (3, 2, 1024, 768)])
def test_expert_stages_against_fp64(moe, layer, orc, gpu_ctx, stream, gu_fmt, dn_fmt, d, I):
    print(f"case decode experts gu={gu_fmt} dn={dn_fmt} d={d} I={I}", flush=True)
    T, K, E = 8, 10, 40
    cfg = layer.LayerConfig("dec_stage", T, d, E, K, I, 0, gu_fmt, dn_fmt, moe.F16, seed=0x5EED0D02 + gu_fmt)
    inp = layer.make_inputs(cfg)
    rng = np.random.default_rng(d + I)
    ids = _ids(rng, T, K, E)
    plan, _ = orc.moe_plan(ids, E)
    x = inp.x[:T].view(np.float16).astype(np.float32)
    xq = orc.quantize_q8_1(x)
    N = T * K
    hid = (rng.standard_normal((N, I)) * 0.05).astype(np.float32)
    hq = orc.quantize_q8_1(hid)
    g, u, gm, um, parts, pm = routed_ref(orc, cfg, inp, plan, xq, hq)
    ws_addr = []
    bw_g, bw_u, bw_d = (gpu_ctx.register(gu.dev(a)) for a in (inp.w_gate, inp.w_up, inp.w_down))
    for e in range(E):
        ws_addr += [bw_g.ptr + e * inp.gu_stride, bw_u.ptr + e * inp.gu_stride, bw_d.ptr + e * inp.dn_stride]
    snap_g, snap_d = gpu_ctx.register(gu.poison(E * 24)), gpu_ctx.register(gu.poison(E * 24))
    tg = moe.ExpertTable(ws_addr, snap_g.view(), [bw_g.view(), bw_u.view()])
    td = moe.ExpertTable(ws_addr, snap_d.view(), [bw_d.view()])
    b_xq, b_plan, b_hq = gpu_ctx.register(gu.dev(xq)), gpu_ctx.register(gu.dev(plan)), gpu_ctx.register(gu.dev(hq))
    b_g, b_u = gpu_ctx.register(gu.poison(N * I * 4)), gpu_ctx.register(gu.poison(N * I * 4))
    b_p, b_st = gpu_ctx.register(gu.poison(N * d * 4)), gpu_ctx.register(gu.dev(np.full(1, 9, np.uint32)))
    shape = cfg.shape()
    eb = moe.MoeExpertBuffers(tg.struct, b_xq.view(), b_plan.view(), b_g.view(), b_u.view(), b_st.view())
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_experts(shape, gu_fmt, eb, keep=tg))
    assert gu.host(b_st, np.uint32)[0] == 0
    _within(gu.host(b_g, np.float32).reshape(N, I), g, gm, "gate")
    _within(gu.host(b_u, np.float32).reshape(N, I), u, um, "up")
    db = moe.MoeDownBuffers(td.struct, b_hq.view(), b_plan.view(), b_p.view(), b_st.view())
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_down(shape, dn_fmt, db, keep=td))
    assert gu.host(b_st, np.uint32)[0] == 0
    _within(gu.host(b_p, np.float32).reshape(N, d), parts, pm, "down parts")


def test_null_expert_and_damaged_plan(moe, layer, orc, gpu_ctx, stream):
    print("case decode failure paths", flush=True)
    cfg = _small(layer, moe)
    T, d, E, K, I = cfg.rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff
    N = T * K
    inp = layer.make_inputs(cfg)
    rng = np.random.default_rng(5)
    ids = _ids(rng, T, K, E)
    plan, _ = orc.moe_plan(ids, E)
    pf = _plan_fields(orc, plan)
    xq = orc.quantize_q8_1(inp.x[:T].view(np.float16).astype(np.float32))
    g, _, gm, _, _, _ = routed_ref(orc, cfg, inp, plan, xq)
    bw_g, bw_u = gpu_ctx.register(gu.dev(inp.w_gate)), gpu_ctx.register(gu.dev(inp.w_up))
    victim = int(pf["grp_e"][1])
    addr = []
    for e in range(E):
        addr += [bw_g.ptr + e * inp.gu_stride, 0 if e == victim else bw_u.ptr + e * inp.gu_stride, 0]
    snap = gpu_ctx.register(gu.poison(E * 24))
    tg = moe.ExpertTable(addr, snap.view(), [bw_g.view(), bw_u.view()])
    b_xq, b_plan = gpu_ctx.register(gu.dev(xq)), gpu_ctx.register(gu.dev(plan))
    b_g, b_u = gpu_ctx.register(gu.poison(N * I * 4)), gpu_ctx.register(gu.poison(N * I * 4))
    b_st = gpu_ctx.register(gu.dev(np.zeros(1, np.uint32)))
    eb = moe.MoeExpertBuffers(tg.struct, b_xq.view(), b_plan.view(), b_g.view(), b_u.view(), b_st.view())
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_experts(cfg.shape(), cfg.gate_up_fmt, eb, keep=tg))
    assert gu.host(b_st, np.uint32)[0] == 1
    a0, a1 = int(pf["grp_start"][1]), int(pf["grp_start"][2])
    got = gu.host(b_g, np.float32).reshape(N, I)
    assert (got[a0:a1] == 0).all() and (gu.host(b_u, np.float32).reshape(N, I)[a0:a1] == 0).all()
    keep = np.r_[0:a0, a1:N]
    _within(got[keep], g[keep], gm[keep], "gate beside the faulting group")
    # a plan whose entry count disagrees with the shape: status bit 1, every output row zero
    bad = plan.copy()
    bad[4:8] = np.frombuffer(np.uint32(N - 1).tobytes(), np.uint8)
    b_plan.tensor.copy_(gu.dev(bad))
    b_g.tensor.fill_(0x7F)
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_experts(cfg.shape(), cfg.gate_up_fmt, eb, keep=tg))
    assert gu.host(b_st, np.uint32)[0] == 2
    assert (gu.host(b_g, np.float32) == 0).all() and (gu.host(b_u, np.float32) == 0).all()
    # more groups than entries (each group holds at least one): the same
    bad = plan.copy()
    bad[0:4] = np.frombuffer(np.uint32(N + 1).tobytes(), np.uint8)
    b_plan.tensor.copy_(gu.dev(bad))
    b_g.tensor.fill_(0x7F)
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_experts(cfg.shape(), cfg.gate_up_fmt, eb, keep=tg))
    assert gu.host(b_st, np.uint32)[0] == 2
    assert (gu.host(b_g, np.float32) == 0).all() and (gu.host(b_u, np.float32) == 0).all()


def test_down_damaged_destinations(moe, layer, orc, gpu_ctx, stream):
    """A plan whose route destinations (ent_dst) name no row: the down stage reports status bit 1,
    zeroes the named rows of the groups holding such an entry, and writes nothing for the entry
    that names none (its real destination row keeps its old bytes); every other group's rows are
    the FP64 products."""
    print("case decode down with damaged destinations", flush=True)
    T, K, E, d, I = 8, 10, 40, 1024, 512
    cfg = layer.LayerConfig("dec_dst", T, d, E, K, I, 0, moe.Q4_K, moe.Q8_0, moe.F16, seed=0x5EED0D0D)
    inp = layer.make_inputs(cfg)
    rng = np.random.default_rng(77)
    ids = _ids(rng, T, K, E)
    plan, _ = orc.moe_plan(ids, E)
    xq = orc.quantize_q8_1(inp.x[:T].view(np.float16).astype(np.float32))
    N = T * K
    hq = orc.quantize_q8_1((rng.standard_normal((N, I)) * 0.05).astype(np.float32))
    _, _, _, _, parts, pm = routed_ref(orc, cfg, inp, plan, xq, hq)
    pf = _plan_fields(orc, plan)
    bad = plan.copy()
    bf = bad.view(orc.PLAN_DTYPE)[0]
    g1, g2 = 1, 2
    e1, e2 = int(pf["grp_start"][g1]), int(pf["grp_start"][g2])  # first entry of each group
    lost = [int(pf["ent_dst"][e1]), int(pf["ent_dst"][e2])]
    bf["ent_dst"][e1] = -1
    bf["ent_dst"][e2] = N + 7
    bw_d = gpu_ctx.register(gu.dev(inp.w_down))
    addr = []
    for e in range(E):
        addr += [0, 0, bw_d.ptr + e * inp.dn_stride]
    snap = gpu_ctx.register(gu.poison(E * 24))
    td = moe.ExpertTable(addr, snap.view(), [bw_d.view()])
    b_hq, b_plan = gpu_ctx.register(gu.dev(hq)), gpu_ctx.register(gu.dev(bad))
    b_p, b_st = gpu_ctx.register(gu.poison(N * d * 4)), gpu_ctx.register(gu.dev(np.zeros(1, np.uint32)))
    db = moe.MoeDownBuffers(td.struct, b_hq.view(), b_plan.view(), b_p.view(), b_st.view())
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_down(cfg.shape(), moe.Q8_0, db, keep=td))
    assert gu.host(b_st, np.uint32)[0] == 2
    got = gu.host(b_p, np.uint32).reshape(N, d)
    poison = np.full(d, 0xA5A5A5A5, np.uint32)  # gu.poison's fill byte
    damaged = set()
    for g in (g1, g2):
        for a in range(int(pf["grp_start"][g]), int(pf["grp_start"][g + 1])):
            dst = int(bf["ent_dst"][a])
            if 0 <= dst < N:
                damaged.add(dst)
                assert (got[dst] == 0).all(), f"row {dst} of a damaged group not zeroed"
    for row in lost:
        assert np.array_equal(got[row], poison), f"row {row} written although no entry names it"
    keep = np.array([r for r in range(N) if r not in damaged and r not in lost])
    _within(got.view(np.float32)[keep], parts[keep], pm[keep], "down parts beside the damaged groups")


# ---- post-ops and the shared expert ----------------------------------------------------------
def test_swiglu_combine_bit_exact(moe, orc, gpu_ctx, stream):
    print("case decode swiglu/combine", flush=True)
    rng = np.random.default_rng(23)
    rows, width = 80, 640
    g = (rng.standard_normal(rows * width) * 4).astype(np.float32)
    u = (rng.standard_normal(rows * width) * 4).astype(np.float32)
    g[:5] = [0.0, -0.0, 90.0, -90.0, 1e-40]
    bg, bu, bo = gpu_ctx.register(gu.dev(g)), gpu_ctx.register(gu.dev(u)), gpu_ctx.register(gu.poison(rows * width * 4))
    b = moe.SwiGLUBuffers(bg.view(), bu.view(), bo.view())
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_swiglu(rows, width, b))
    assert np.array_equal(gu.host(bo, np.float32).view(np.uint32), orc.swiglu_f32(g, u).view(np.uint32))
    for T, K, d, shared in [(8, 10, 2560, True), (1, 10, 2560, True), (5, 8, 1024, False)]:
        parts = rng.standard_normal((T * K, d)).astype(np.float32)
        w = rng.random((T, K)).astype(np.float32)
        sh = rng.standard_normal((T, d)).astype(np.float32) if shared else None
        gl = (rng.standard_normal(T) * 3).astype(np.float32) if shared else None
        bp, bw = gpu_ctx.register(gu.dev(parts)), gpu_ctx.register(gu.dev(w))
        bs = gpu_ctx.register(gu.dev(sh)) if shared else None
        bl = gpu_ctx.register(gu.dev(gl)) if shared else None
        bo = gpu_ctx.register(gu.poison(T * d * 4))
        cb = moe.CombineBuffers(bp.view(), bw.view(), bs.view() if shared else moe.NULL_VIEW,
                                bl.view() if shared else moe.NULL_VIEW, bo.view())
        shape = moe.Shape(T, d, 64, K, 64, 640 if shared else 0)
        gu.run(gpu_ctx, stream, lambda s: s.encode_moe_combine(shape, cb))
        want = orc.combine_decode(parts, w, sh, gl, T, K, d)
        assert np.array_equal(gu.host(bo, np.float32).reshape(T, d).view(np.uint32), want.view(np.uint32))


# (4, 8, 4096, 4096): the widest rows, whose staged activations need more than 64 KB of LDS
# (the shared down's F32 hidden rows, 8 x 4096 x 4 bytes).
@pytest.mark.parametrize("fmt,T,d,Is", [(4, 8, 2560, 640), (5, 3, 4096, 1536), (4, 1, 2048, 512), (4, 8, 4096, 4096)])
def test_shared_ffn_against_fp64(moe, orc, gpu_ctx, stream, fmt, T, d, Is):
    print(f"case decode shared fmt={fmt} T={T} d={d} Is={Is}", flush=True)
    gen = moe.synth_normal_bf16 if fmt == moe.BF16 else moe.synth_normal_f16
    wg, wu, wd, gv = (gen(0x5EED, 50 + i, 0.02, n) for i, n in enumerate((Is * d, Is * d, d * Is, d)))
    x = moe.synth_normal_f16(0x5EED, 60, 1.0, T * d).reshape(T, d)
    K = 10
    rng = np.random.default_rng(Is)
    parts = rng.standard_normal((T * K, d)).astype(np.float32) * np.float32(0.01)
    w = rng.random((T, K)).astype(np.float32)
    reg = lambda a: gpu_ctx.register(gu.dev(a))  # noqa: E731
    bx, bg, bu, bd, bv, bp, bw = (reg(a) for a in (x, wg, wu, wd, gv, parts, w))
    bh, bso, bgl = gpu_ctx.register(gu.poison(T * Is * 4)), gpu_ctx.register(gu.poison(T * d * 4)), gpu_ctx.register(gu.poison(T * 4))
    bo = gpu_ctx.register(gu.poison(T * d * 4))
    sb = moe.SharedBuffers(bx.view(), bg.view(), bu.view(), bd.view(), bv.view(), bh.view(), bso.view(), bgl.view())
    fb = moe.MoeSharedFFNBuffers(sb, bp.view(), bw.view(), bo.view())
    shape = moe.Shape(T, d, 64, K, 64, Is)
    gu.run(gpu_ctx, stream, lambda s: s.encode_moe_shared_ffn(shape, fmt, fb))
    x64 = x.view(np.float16).astype(np.float64)
    Wg, Wu, Wd = _dense(fmt, wg, (Is, d)), _dense(fmt, wu, (Is, d)), _dense(fmt, wd, (d, Is))
    g, u = x64 @ Wg.T, x64 @ Wu.T
    gmag, umag = np.abs(x64) @ np.abs(Wg).T, np.abs(x64) @ np.abs(Wu).T
    hid = gu.host(bh, np.float32).reshape(T, Is)
    # hidden = silu(g) * u with g, u accumulated in F32: compare against the F32 SwiGLU of the
    # FP64 dots, allowing the dots' F32 rounding through the SwiGLU's slope.
    ref_h = orc.swiglu_f32(g.astype(np.float32), u.astype(np.float32)).astype(np.float64)
    slope = np.abs(u) * 1.2 * gmag + np.abs(g) * umag + np.abs(ref_h)
    _within(hid, ref_h, slope, "shared hidden", k=64)
    out = gu.host(bso, np.float32).reshape(T, d)
    h64 = hid.astype(np.float64)
    _within(out, h64 @ Wd.T, np.abs(h64) @ np.abs(Wd).T, "shared down")
    gl = gu.host(bgl, np.float32)
    gvv = _dense(fmt, gv, (d,))
    _within(gl, x64 @ gvv, np.abs(x64) @ np.abs(gvv), "shared gate logit")
    want = orc.combine_decode(parts, w, out, gl, T, K, d)
    assert np.array_equal(gu.host(bo, np.float32).reshape(T, d).view(np.uint32), want.view(np.uint32))


# ---- the whole decode layer ------------------------------------------------------------------
def layer_ref(orc, cfg, inp, ws_ids, ws_logits):
    """Composed oracle of one decode layer given the GPU's route ids (checked bit-exact against
    the oracle's top-k of the GPU's logits first)."""
    T, d, E, K, I, Is = cfg.rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff, cfg.shared_ff
    ids, w = orc.route(ws_logits, K, False)
    assert np.array_equal(ids, ws_ids)
    plan, _ = orc.moe_plan(ids, E)
    x = inp.x[:T].view(np.float16).astype(np.float32)
    xq = orc.quantize_q8_1(x)
    g, u, *_ = routed_ref(orc, cfg, inp, plan, xq)
    hid = orc.swiglu_f32(g.astype(np.float32), u.astype(np.float32))
    hq = orc.quantize_q8_1(hid)
    *_, parts, _ = routed_ref(orc, cfg, inp, plan, xq, hq)
    sh = gl = None
    if Is:
        x64 = x.astype(np.float64)
        f = cfg.shared_fmt
        Wg, Wu, Wd = _dense(f, inp.sh_gate, (Is, d)), _dense(f, inp.sh_up, (Is, d)), _dense(f, inp.sh_down, (d, Is))
        h = orc.swiglu_f32((x64 @ Wg.T).astype(np.float32), (x64 @ Wu.T).astype(np.float32)).astype(np.float64)
        sh = (h @ Wd.T).astype(np.float32)
        gl = (x64 @ _dense(f, inp.sh_gvec, (d,))).astype(np.float32)
    return orc.combine_decode(parts.astype(np.float32), w, sh, gl, T, K, d), plan, xq


def _extra_decode(layer, moe, name):
    """Small layers for the two top-k layouts of the front launch (one token per wave up to 4
    rows, two per wave above) at expert counts that leave most slots as padding, one without
    a shared expert."""
    return {"small_t3": layer.LayerConfig("small_t3", 3, 512, 40, 5, 256, 256, moe.Q4_K, moe.Q8_0, moe.F16,
                                          seed=0x5EED0D02),
            "small_t6": layer.LayerConfig("small_t6", 6, 512, 100, 7, 256, 0, moe.Q8_0, moe.Q8_0, moe.F16,
                                          seed=0x5EED0D03),
            "small_t2": layer.LayerConfig("small_t2", 2, 512, 64, 8, 256, 256, moe.Q4_K, moe.Q8_0, moe.F16,
                                          seed=0x5EED0D04),
            "small_t1": layer.LayerConfig("small_t1", 1, 512, 40, 5, 256, 0, moe.Q4_K, moe.Q8_0, moe.F16,
                                          seed=0x5EED0D05)}[name]


@pytest.mark.parametrize("name", ["window_t1", "window_t8", "full_layer_t8", "low_bit_t4", "small_t3", "small_t6",
                                  "small_t2", "small_t1"])
def test_decode_layer(moe, layer, orc, gpu_ctx, stream, name):
    print(f"case decode layer {name}", flush=True)
    cfg = layer.DECODE_CONFIGS[name] if name in layer.DECODE_CONFIGS else _extra_decode(layer, moe, name)
    inp = _inputs(layer, cfg)
    ws = layer.DecodeWorkspace(gpu_ctx, cfg, inp)
    ws.out.tensor.fill_(float("nan"))
    ws.run(stream)
    import torch
    torch.cuda.synchronize()
    assert ws.read_status() == 0
    T, d, K = cfg.rows, cfg.hidden, cfg.top_k
    logits = gu.host(ws.logits, np.float32).reshape(T, cfg.n_experts)
    ref_logits = orc.router_ref(inp.x[:T], inp.w_router)
    # Each logit is a chain of fma over the 4-value F32 chunks a lane of its row holds (lpr lanes
    # per row, chosen as the launch does), then a log2(lpr)-level xor tree: n roundings on the
    # longest path, so the deterministic bound is |err| <= gamma_n * sum_k |x_k w_k| with
    # gamma_n = n u / (1 - n u), u = 2^-24 (n = 46, about 2^-18.5, at d = 2560).
    nch, lpr = d // 4, 8
    while lpr < 64 and -(-nch // lpr) > 4:
        lpr *= 2
    n_round = 4 * -(-nch // lpr) + lpr.bit_length() - 1
    gamma = n_round * 2.0 ** -24 / (1 - n_round * 2.0 ** -24)
    mag = np.abs(inp.x[:T].view(np.float16).astype(np.float64)) @ np.abs(inp.w_router.astype(np.float64)).T
    assert (np.abs(logits - ref_logits) <= gamma * mag + 1e-9).all(), "decode router logits"
    ids = gu.host(ws.ids, np.int32).reshape(T, K)
    want, plan, xq = layer_ref(orc, cfg, inp, ids, logits)
    assert np.array_equal(gu.host(ws.plans, np.uint8), plan)
    assert np.array_equal(gu.host(ws.xq, np.uint8).reshape(T, -1), xq)
    # The SwiGLU rows and their Q8_1 blocks follow from the GPU's own gate/up rows bit for bit.
    N, I = T * K, cfg.expert_ff
    g_rows, u_rows = gu.host(ws.gate, np.float32).reshape(N, I), gu.host(ws.up, np.float32).reshape(N, I)
    hid = gu.host(ws.hidden, np.float32).reshape(N, I)
    assert np.array_equal(hid.view(np.uint32), orc.swiglu_f32(g_rows, u_rows).view(np.uint32)), "decode SwiGLU rows"
    assert np.array_equal(gu.host(ws.hq, np.uint8).reshape(N, -1), orc.quantize_q8_1(hid)), "decode Q8_1 hidden"
    out = gu.host(ws.out, np.float32).reshape(T, d)
    assert np.isfinite(out).all()
    err, rel = gu.layer_tolerance(out, want)
    print(f"  {name}: max-abs {err:.3e} rel-L2 {rel:.3e}", flush=True)
    assert err <= 2e-2 and rel <= 5e-3
    # a second call on the same workspace gives the same bits (no state carried between calls)
    first = out.copy()
    ws.run(stream)
    torch.cuda.synchronize()
    assert np.array_equal(gu.host(ws.out, np.float32).reshape(T, d).view(np.uint32), first.view(np.uint32))


@pytest.mark.parametrize("name", ["window_t1", "window_t8"])
def test_decode_layer_null_expert_address(moe, layer, orc, gpu_ctx, stream, name):
    """A routed expert without an up matrix: status bit 0, its group's gate/up rows, SwiGLU rows
    and parts zero, the other groups unchanged."""
    print(f"case decode layer null expert {name}", flush=True)
    import torch
    cfg = layer.DECODE_CONFIGS[name]
    inp = _inputs(layer, cfg)
    ws = layer.DecodeWorkspace(gpu_ctx, cfg, inp)
    ws.run(stream)
    torch.cuda.synchronize()
    assert ws.read_status() == 0
    T, d, K, I = cfg.rows, cfg.hidden, cfg.top_k, cfg.expert_ff
    N = T * K
    good_gate = gu.host(ws.gate, np.float32).reshape(N, I).copy()
    good_out = gu.host(ws.out, np.float32).reshape(T, d).copy()
    victim = int(gu.host(ws.ids, np.int32)[0])
    addr = list(ws.addresses)
    addr[3 * victim + 1] = 0
    ws.gu_table = moe.ExpertTable(addr, ws.snap_gu.view(), [ws.w_gate.view(), ws.w_up.view()])
    ws.run(stream)
    torch.cuda.synchronize()
    assert ws.read_status() == 1
    pf = _plan_fields(orc, gu.host(ws.plans, np.uint8))
    gi = list(pf["grp_e"][: int(pf["n_groups"])]).index(victim)
    a0, a1 = int(pf["grp_start"][gi]), int(pf["grp_start"][gi + 1])
    gate = gu.host(ws.gate, np.float32).reshape(N, I)
    assert (gate[a0:a1] == 0).all() and (gu.host(ws.hidden, np.float32).reshape(N, I)[a0:a1] == 0).all()
    keep = np.r_[0:a0, a1:N]
    assert np.array_equal(gate[keep].view(np.uint32), good_gate[keep].view(np.uint32))
    parts = gu.host(ws.parts, np.float32).reshape(N, d)
    dst = pf["ent_dst"][a0:a1]
    assert (parts[dst] == 0).all()
    out = gu.host(ws.out, np.float32).reshape(T, d)
    assert np.isfinite(out).all() and not np.array_equal(out, good_out)
