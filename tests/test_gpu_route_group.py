"""GPU parity: router GEMM, softmax top-k, grouping and gather against the CPU oracle.

Integer stages (ids, histogram, PfPlan bytes, tile list, src/dst, gathered rows) and the
route weights must be bit-exact; the F32 router logits are checked against FP64 within
a magnitude-scaled bound, and top-k is then checked bit-exact on the GPU's own logits.
"""
import numpy as np
import pytest

import gpu_util as gu
import ref_patterns as rp

pytestmark = pytest.mark.gpu


def _route_case(moe, orc, ctx, stream, logits, K, divide):
    import torch
    T, E = logits.shape
    shape = moe.Shape(T, 256, E, K, 64, 0)
    L = ctx.register(gu.dev(logits))
    ids = ctx.register(torch.full((T * K,), -7, dtype=torch.int32, device="cuda"))
    w = ctx.register(torch.zeros(T * K, dtype=torch.float32, device="cuda"))
    b = moe.RouteBuffers(L.view(), ids.view(), w.view())
    gu.run(ctx, stream, lambda s: s.encode_moe_route(shape, divide, b))
    return gu.host(ids, np.int32).reshape(T, K), gu.host(w, np.float32).reshape(T, K)


# Up to 1024 tokens the kernel takes one token per wave, above that two per wave: both layouts
# meet every slot count (E up to 64 / 128 / 256 / 512 per wave, 32 / 64 / 128 / 256 / 512 per
# half-wave) and the reference's golden rows (K = 10, E = 512 in each layout).
@pytest.mark.parametrize("T,E,K", [(64, 16, 4), (4096, 512, 10), (1000, 256, 8), (37, 40, 5), (9, 512, 32),
                                   (8, 512, 10), (300, 100, 6), (1025, 100, 6), (2000, 40, 10), (1500, 200, 10)])
@pytest.mark.parametrize("divide", [True, False])
def test_route_topk_bit_exact(moe, orc, gpu_ctx, stream, T, E, K, divide):
    print(f"case route T={T} E={E} K={K} divide={divide}", flush=True)
    rng = np.random.default_rng(1000 * T + E + K)
    logits = (rng.standard_normal((T, E)) * 1.5).astype(np.float32)
    if E >= 20 and T >= 8:
        logits[:4] = rp.special_logits(E)
        logits[4:8] = rp.shuffled_rank_logits(4, E, T)
    if T > 12:  # NaN / inf rows exercise the -FLT_MAX replacement
        logits[9, 3] = np.nan
        logits[10, 1] = np.inf
        logits[11, :] = -np.inf
        logits[12, :] = 0.0
    ids, w = _route_case(moe, orc, gpu_ctx, stream, logits, K, divide)
    ids_ref, w_ref = orc.route(logits, K, divide)
    assert np.array_equal(ids, ids_ref)
    assert np.array_equal(w.view(np.uint32), w_ref.view(np.uint32))
    if E in (256, 512) and K == 10 and T >= 8:  # the expert counts the golden rows hold for
        assert np.array_equal(ids[:4], rp.special_ids(E))
        gold = rp.NONUNIFORM_DIVIDE_BITS if divide else rp.NONUNIFORM_MULTIPLY_BITS
        assert list(w[2].view(np.uint32)) == gold
        assert list(w[0].view(np.uint32)) == rp.EQUAL_WEIGHT_BITS


@pytest.mark.parametrize("E", [256, 512])
@pytest.mark.parametrize("T", [1, 7, 25, 26, 64, 300, 4096])
@pytest.mark.parametrize("pattern", rp.PATTERNS)
def test_grouping_gather_bit_exact(moe, orc, gpu_ctx, stream, pattern, T, E):
    _check_grouping_gather(moe, orc, gpu_ctx, stream, pattern, T, E)


# The scan keeps up to 16 of its 256-entry tiles per thread in registers (512 tiles: N = 131072
# entries); longer columns take its re-reading loop. 13107 tokens x 10 is 512 tiles, 16384 x 10
# is 640.
@pytest.mark.parametrize("T", [13107, 16384])
@pytest.mark.parametrize("pattern", ["mixed", "invalid_ids"])
def test_grouping_gather_long_columns(moe, orc, gpu_ctx, stream, pattern, T):
    _check_grouping_gather(moe, orc, gpu_ctx, stream, pattern, T, 512)


def _check_grouping_gather(moe, orc, gpu_ctx, stream, pattern, T, E):
    import torch
    print(f"case grouping pattern={pattern} T={T} E={E}", flush=True)
    K, d = 10, 256
    shape = moe.Shape(T, d, E, K, 64, 0)
    N = T * K
    ids = rp.grouping_ids(T, E, pattern, K)
    x = moe.synth_normal_f16(7, T, 1.0, T * d).reshape(T, d)
    ctx = gpu_ctx
    reg = ctx.register
    b_ids, b_x = reg(gu.dev(ids)), reg(gu.dev(x))
    hist = reg(gu.poison(moe.histogram_bytes(shape)))
    plan = reg(gu.poison(moe.PLAN_SLOT_BYTES))
    tiles = reg(gu.poison(moe.tiles_bytes(shape)))
    src, dst = reg(gu.poison(N * 4)), reg(gu.poison(N * 4))
    xs = reg(gu.poison(N * d * 2))
    b = moe.GroupingBuffers(b_ids.view(), b_x.view(), hist.view(), plan.view(), tiles.view(), src.view(),
                            dst.view(), xs.view())
    gu.run(ctx, stream, lambda s: s.encode_prefill_moe_grouping(shape, b))
    ref = orc.grouping(ids, E)
    pf = orc.plan_fields(ref["plan"])
    n_valid = N - pf["bad"]
    n_count = (N + 255) // 256
    assert np.array_equal(gu.host(plan, np.uint8), ref["plan"]), "PfPlan slot bytes"
    assert np.array_equal(gu.host(hist, np.uint32).reshape(-1, E)[:n_count], ref["hist"]), "histogram"
    tl = gu.host(tiles, np.uint32).reshape(-1, 2)
    assert np.array_equal(tl[: ref["n_tiles"]], ref["tiles"]), "tile list"
    g_src, g_dst = gu.host(src, np.int32), gu.host(dst, np.int32)
    assert np.array_equal(g_src[:n_valid], ref["src"][:n_valid]), "source rows"
    assert np.array_equal(g_dst[:n_valid], ref["dst"][:n_valid]), "destination rows"
    poison32 = np.frombuffer(b"\xa5" * 4, np.int32)[0]
    assert (g_src[n_valid:] == poison32).all() and (g_dst[n_valid:] == poison32).all(), "tails written"
    g_xs = gu.host(xs, np.uint16).reshape(N, d)
    assert np.array_equal(g_xs[:n_valid], orc.gather(x, ref["src"], n_valid)), "gathered rows"
    assert (g_xs[n_valid:] == 0xA5A5).all(), "gather tail written"
    torch.cuda.synchronize()


@pytest.mark.parametrize("cfg_index", [0, 1])
def test_route_gather_composition(moe, layer, orc, gpu_ctx, stream, cfg_index):
    """Steps 1-6 as one segment at configuration 0 and 1 (T=4096, E=512, k=10)."""
    print(f"case route_gather config={cfg_index}", flush=True)
    cfg = layer.CONFIGS[cfg_index]
    inp = layer.make_inputs(cfg, with_experts=False)
    ws = layer.LayerWorkspace(gpu_ctx, cfg, inp)
    rg = ws.route_gather_buffers()
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_moe_full_mode_route_gather(cfg.shape(), rg))
    T, E, K, d = cfg.rows, cfg.n_experts, cfg.top_k, cfg.hidden
    logits = gu.host(ws.logits, np.float32).reshape(T, E)
    ref64 = orc.router_ref(inp.x[:T], inp.w_router)
    # F32-class bound on the logits: |err| <= 2^-20 * sum_k |x_k w_k| (plus a floor).
    mag = np.abs(inp.x[:T].view(np.float16).astype(np.float64)) @ np.abs(inp.w_router.astype(np.float64)).T
    assert (np.abs(logits - ref64) <= 2.0 ** -20 * mag + 1e-7).all(), "router logits"
    ids = gu.host(ws.ids, np.int32).reshape(T, K)
    w = gu.host(ws.route_w, np.float32).reshape(T, K)
    ids_ref, w_ref = orc.route(logits, K, True)
    assert np.array_equal(ids, ids_ref) and np.array_equal(w.view(np.uint32), w_ref.view(np.uint32))
    # How many tokens would flip between the GPU logits and FP64 logits (reported, not failed).
    ids64, _ = orc.route(ref64.astype(np.float32), K, True)
    flips = int((ids64 != ids).any(axis=1).sum())
    print(f"route_gather config={cfg_index}: tokens whose top-{K} differs under FP64 logits: {flips}/{T}")
    g = orc.grouping(ids_ref, E)
    n_valid = T * K - orc.plan_fields(g["plan"])["bad"]
    # In this composition top-k counts the entries into the histogram (the router clears it)
    # and the count kernel does not run: the per-tile counts must still be the count kernel's.
    n_count = (T * K + 255) // 256
    assert np.array_equal(gu.host(ws.hist, np.uint32).reshape(-1, E)[:n_count], g["hist"]), "histogram"
    assert np.array_equal(gu.host(ws.plan, np.uint8), g["plan"])
    assert np.array_equal(gu.host(ws.src, np.int32)[:n_valid], g["src"][:n_valid])
    assert np.array_equal(gu.host(ws.dst, np.int32)[:n_valid], g["dst"][:n_valid])
    xs = gu.host(ws.xs, np.uint16).reshape(T * K, d)
    assert np.array_equal(xs[:n_valid], orc.gather(inp.x[:T], g["src"], n_valid))
