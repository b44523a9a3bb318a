"""CPU: expert products, shared expert, SwiGLU and combine of the oracle.

GEMM references are checked against numpy float64 matmuls over the dequantized weights (the
products' operands); combine and SwiGLU against the reference's own CPU twins
(tests/metal/oracles/moe_combine.cpp, moe_swiglu.cpp built into oracle/_ref) within the
reference's tolerances, and against closed forms.
"""
import numpy as np
import pytest


def _deq(orc, fmt, blob, rows, k):
    return orc.dequant(fmt, blob, rows * k).view(np.float16).astype(np.float64).reshape(rows, k)


@pytest.mark.parametrize("fmt_gu,fmt_dn", [(1, 1), (2, 1), (3, 2)])
def test_expert_products_against_numpy(moe, layer, orc, fmt_gu, fmt_dn):
    cfg = layer.LayerConfig("t", 48, 256, 8, 3, 256, 0, fmt_gu, fmt_dn, moe.F16, seed=77)
    inp = layer.make_inputs(cfg)
    T, d, E, K, I = cfg.rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff
    rng = np.random.default_rng(5)
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.int32)
    g = orc.grouping(ids, E)
    N = T * K
    xs = orc.gather(inp.x, g["src"], N)
    entries = np.arange(N)
    gg, uu, eh = orc.gate_up_ref(fmt_gu, xs, d, I, g["plan"], inp.w_gate, inp.w_up, inp.gu_stride, entries)
    pf = orc.plan_fields(g["plan"])
    xs64 = xs.view(np.float16).astype(np.float64)
    for gi in range(pf["n_groups"]):
        e = pf["grp_e"][gi]
        a0, a1 = pf["grp_start"][gi], pf["grp_start"][gi + 1]
        wg = _deq(orc, fmt_gu, inp.w_gate[e * inp.gu_stride:(e + 1) * inp.gu_stride], I, d)
        wu = _deq(orc, fmt_gu, inp.w_up[e * inp.gu_stride:(e + 1) * inp.gu_stride], I, d)
        assert np.allclose(gg[a0:a1], xs64[a0:a1] @ wg.T, rtol=1e-12, atol=1e-12)
        assert np.allclose(uu[a0:a1], xs64[a0:a1] @ wu.T, rtol=1e-12, atol=1e-12)
    g32, u32 = gg.astype(np.float32), uu.astype(np.float32)
    assert np.array_equal(eh, orc.swiglu(g32, u32))  # eh = half_sat(silu(g) * u)
    out = orc.down_ref(fmt_dn, eh, d, I, g["plan"], inp.w_down, inp.dn_stride, entries)
    eh64 = eh.view(np.float16).astype(np.float64)
    for gi in range(pf["n_groups"]):
        e = pf["grp_e"][gi]
        a0, a1 = pf["grp_start"][gi], pf["grp_start"][gi + 1]
        wd = _deq(orc, fmt_dn, inp.w_down[e * inp.dn_stride:(e + 1) * inp.dn_stride], d, I)
        assert np.allclose(out[a0:a1], eh64[a0:a1] @ wd.T, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("fmt", [4, 5])
def test_shared_expert_against_numpy(moe, layer, orc, fmt):
    cfg = layer.LayerConfig("t", 16, 256, 8, 2, 256, 256, 1, 1, fmt, seed=78)
    inp = layer.make_inputs(cfg, with_experts=False)
    T, d, Is = cfg.rows, cfg.hidden, cfg.shared_ff
    tokens = np.arange(T)
    hid, out, gl = orc.shared_ref(fmt, inp.x, d, Is, inp.sh_gate, inp.sh_up, inp.sh_down, inp.sh_gvec, tokens)
    x = inp.x.view(np.float16).astype(np.float64)
    wg = _deq(orc, fmt, inp.sh_gate.view(np.uint8), Is, d)
    wu = _deq(orc, fmt, inp.sh_up.view(np.uint8), Is, d)
    wd = _deq(orc, fmt, inp.sh_down.view(np.uint8), d, Is)
    gv = _deq(orc, fmt, inp.sh_gvec.view(np.uint8), 1, d)[0]
    assert np.allclose(gl, x @ gv, rtol=1e-12, atol=1e-12)
    g, u = (x @ wg.T).astype(np.float32), (x @ wu.T).astype(np.float32)
    assert np.array_equal(hid, orc.swiglu(g, u))
    assert np.allclose(out, hid.view(np.float16).astype(np.float64) @ wd.T, rtol=1e-12, atol=1e-12)


def test_combine_closed_forms(orc):
    rng = np.random.default_rng(3)
    T, K, d = 5, 4, 64
    parts = rng.standard_normal((T * K, d)).astype(np.float32)
    # Power-of-two weights and small-integer parts make every fma exact.
    w = np.float32([[0.5, 0.25, 0.125, 0.125]] * T)
    pint = np.round(parts * 8).astype(np.float32)
    out = orc.combine(pint, w, None, None, T, K, d)
    assert np.array_equal(out, (pint.reshape(T, K, d) * w[:, :, None]).sum(axis=1).astype(np.float32))
    one = orc.combine(parts[:T], np.ones((T, 1), np.float32), None, None, T, 1, d)
    assert np.array_equal(one, parts[:T])
    # sigmoid(0) = 0.5 exactly, so the gated term is fma(shared, 0.5, s) = one rounding of an
    # exact float64 sum.
    sh = rng.standard_normal((T, d)).astype(np.float32)
    gl = np.float32([0.0] * T)
    outs = orc.combine(pint, w, sh, gl, T, K, d)
    ref = (0.5 * sh.astype(np.float64) + out.astype(np.float64)).astype(np.float32)
    assert np.array_equal(outs, ref)


def test_combine_and_swiglu_against_reference_twins(orc):
    ref = orc.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    rng = np.random.default_rng(11)
    T, K, d = 7, 10, 2560
    parts = rng.standard_normal((T * K, d)).astype(np.float32)
    w = rng.random((T, K)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    sh = rng.standard_normal((T, d)).astype(np.float32)
    gl = rng.standard_normal(T).astype(np.float32)
    ours = orc.combine(parts, w, sh, gl, T, K, d)
    theirs = np.empty((T, d), np.float32)
    assert ref.ref_combine(parts.ctypes.data, w.ctypes.data, sh.ctypes.data, gl.ctypes.data, T,
                           theirs.ctypes.data) == 0
    assert (np.abs(ours - theirs) <= 2e-6 * np.maximum(1.0, np.abs(theirs))).all()
    n = 640 * 3
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = (rng.standard_normal(n) * 4).astype(np.float32)
    twin = np.empty(n, np.float32)
    assert ref.ref_swiglu(g.ctypes.data, u.ctypes.data, n, twin.ctypes.data) == 0
    h = orc.swiglu(g, u).view(np.float16).astype(np.float64)
    tw = twin.astype(np.float16).astype(np.float64)
    assert (np.abs(h - tw) <= np.maximum(np.abs(tw) * 2.0 ** -10, 2.0 ** -24)).all()  # <= 1 half-ULP


def test_router_ref_against_numpy(moe, layer, orc):
    """or_router_ref against numpy's float64 x @ W.T on a slice of configuration 1 (F16
    activations, F32 router weights [E, d])."""
    cfg = layer.CONFIGS[1]
    inp = layer.make_inputs(cfg, with_experts=False)
    x = inp.x[:48]
    w = inp.w_router
    got = orc.router_ref(x, w)
    ref = x.view(np.float16).astype(np.float64) @ w.astype(np.float64).T
    assert got.shape == (48, cfg.n_experts)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-15)
    # transposed roles (W rows against x columns) or a dropped last K term would not pass
    short = x.view(np.float16).astype(np.float64)[:, :-1] @ w.astype(np.float64)[:, :-1].T
    assert not np.allclose(got, short, rtol=1e-12, atol=1e-15)
