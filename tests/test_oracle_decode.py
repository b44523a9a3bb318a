"""CPU: the decode-side oracle (the Window MoE over T <= 8 rows).

The plan is checked against brute-force invariants and a hand-worked case; the Q8_1
quantizer bit for bit against the reference's own q8_1.cpp (built into oracle/_ref) over
random, zero, subnormal and overflowing blocks; the FP64 mat-vec exactly against FP64 dots of
the (separately pinned) dequantized weights on weights whose values are exact in F16, and
against the reference's q8_0_mv.cpp / q4_k_mv.cpp twins within their F32 rounding; SwiGLU and
combine against moe_swiglu.cpp / moe_combine.cpp.
"""
import numpy as np
import pytest

F32_EPS = 2.0 ** -24


def _ref(orc):
    r = orc.ref()
    if r is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    return r


# ---- plan ------------------------------------------------------------------------------------
def test_plan_hand_worked(orc):
    ids = np.array([[3, 1, 3], [1, 2, 0]], np.int32)  # rows 2, top_k 3
    plan, rc = orc.moe_plan(ids, 4)
    p = plan.view(orc.PLAN_DTYPE)[0]
    assert rc == 0 and p["n_groups"] == 4 and p["n_entries"] == 6 and p["n_miss"] == 0 and p["skip"] == 1
    assert list(p["grp_e"][:4]) == [3, 1, 2, 0]
    assert list(p["grp_start"][:5]) == [0, 2, 4, 5, 6]
    assert list(p["ent_dst"][:6]) == [0, 2, 1, 3, 4, 5]
    assert list(p["ent_tok"][:6]) == [0, 0, 0, 1, 1, 1]
    assert not p["grp_e"][4:].any() and not p["ent_dst"][6:].any() and not p["grp_start"][5:].any()


@pytest.mark.parametrize("rows,top_k,E", [(1, 10, 256), (4, 10, 256), (8, 10, 512), (8, 10, 16), (5, 7, 9)])
def test_plan_invariants(orc, rows, top_k, E):
    rng = np.random.default_rng(rows * 1000 + E)
    for trial in range(20):
        ids = np.stack([rng.choice(E, top_k, replace=False) for _ in range(rows)]).astype(np.int32)
        resident = np.where(rng.random(E) < 0.7, rng.integers(0, 99, E), -1).astype(np.int32)
        usage = np.zeros(E, np.float32)
        plan, rc = orc.moe_plan(ids, E, resident, usage)
        p = plan.view(orc.PLAN_DTYPE)[0]
        flat = ids.ravel()
        n = flat.size
        assert rc == 0 and p["n_entries"] == n
        uniq, first = np.unique(flat, return_index=True)
        order = uniq[np.argsort(first)]  # experts in first-appearance order
        G = len(order)
        assert p["n_groups"] == G and list(p["grp_e"][:G]) == list(order)
        starts = p["grp_start"][:G + 1]
        assert starts[0] == 0 and starts[G] == n and (np.diff(starts) > 0).all()
        dst = p["ent_dst"][:n]
        assert sorted(dst) == list(range(n))  # every route entry exactly once
        for g in range(G):
            members = dst[starts[g]:starts[g + 1]]
            assert (flat[members] == order[g]).all() and (np.diff(members) > 0).all()
            assert len(members) == (flat == order[g]).sum()
        assert (p["ent_tok"][:n] == dst // top_k).all()
        res = resident[order] >= 0
        assert list(p["grp_res"][:G]) == list(res.astype(int))
        assert p["n_miss"] == (~res).sum() and p["skip"] == int((~res).sum() == 0)
        assert np.array_equal(usage, np.bincount(flat, minlength=E).astype(np.float32))


def test_plan_bad_id_is_empty(orc):
    ids = np.array([[0, 5, 2]], np.int32)
    usage = np.zeros(4, np.float32)
    plan, rc = orc.moe_plan(ids, 4, None, usage)
    p = plan.view(orc.PLAN_DTYPE)[0]
    assert rc == 1 and p["n_groups"] == 0 and p["n_entries"] == 0 and p["skip"] == 1
    assert not plan[16:].any() and not usage.any()
    plan, rc = orc.moe_plan(np.array([[-1, 1]], np.int32), 4)
    assert rc == 1


# ---- Q8_1 ------------------------------------------------------------------------------------
def q81_cases(rng):
    """Rows of 256 F32 values exercising every path of the quantizer."""
    n = 256
    rows = []
    for scale in (1.0, 1e-3, 37.0, 1e4):
        rows.append((rng.standard_normal(n) * scale).astype(np.float32))
    r = rng.standard_normal(n).astype(np.float32)
    r[:32] = 0.0  # all-zero block
    r[32:64] = -0.0
    r[64:96] *= np.float32(2.0 ** -140)  # amax well inside the subnormal range of d
    r[96:128] = 0.0
    r[100] = np.float32(2.0 ** -140)
    rows.append(r)
    r = np.zeros(n, np.float32)
    tiny = (rng.integers(-70, 70, 32) * 2.0 ** -149).astype(np.float32)  # subnormal x, d rounds to 0
    r[:32] = tiny
    r[32:64] = (rng.integers(-2 ** 22, 2 ** 22, 32) * 2.0 ** -149).astype(np.float32)  # subnormal x and d
    r[64:96] = (rng.standard_normal(32) * 2.0 ** -120).astype(np.float32)  # normal x, subnormal d
    r[96:128] = (rng.standard_normal(32) * 2.0 ** -118).astype(np.float32)  # d near the normal edge
    r[128:160] = rng.standard_normal(32).astype(np.float32) * np.float32(3e4)  # sum overflows F16
    r[160:192] = np.float32(3.4e38) * np.sign(rng.standard_normal(32)).astype(np.float32)  # d overflows F16
    r[192:224] = (np.arange(32) - 15.5).astype(np.float32) * np.float32(0.5)  # .5 ties of x/d
    r[224:256] = np.float32([127.0, -63.5, 0.5, -0.5] * 8)  # d = 1: exact half-way codes
    rows.append(r)
    x = rng.standard_normal(n).astype(np.float32)
    x[::7] = np.float32(2.0 ** -130)  # subnormal inputs in normal blocks
    rows.append(x)
    return np.stack(rows)


def test_q8_1_against_reference_twin(orc):
    ref = _ref(orc)
    rng = np.random.default_rng(3)
    for trial in range(5):
        x = q81_cases(rng)
        ours = orc.quantize_q8_1(x)
        theirs = np.empty_like(ours)
        assert ref.ref_q8_1(x.ctypes.data, x.shape[1], x.shape[0], theirs.ctypes.data) == 0
        assert np.array_equal(ours, theirs), np.argwhere(ours != theirs)[:5]


def test_q8_1_closed_forms(orc):
    # d = 1 exactly: codes are the values, the sum is exact, ties round away from zero.
    x = np.zeros((1, 32), np.float32)
    x[0, :4] = [127.0, -2.5, 2.5, 0.5]
    q = orc.quantize_q8_1(x)[0]
    hd, hs = q[:4].view(np.float16)
    assert hd == 1.0 and hs == np.float16(127.5)
    assert list(q[4:8].view(np.int8)) == [127, -3, 3, 1]
    # an all-zero block has d = 0 and zero codes
    assert not orc.quantize_q8_1(np.zeros((2, 64), np.float32)).any()
    # codes bracket the values: |x - q d| <= d / 2 for normal blocks, and |q| <= 127
    rng = np.random.default_rng(8)
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    q = orc.quantize_q8_1(x).reshape(4, 32, 36)
    d = (np.abs(x.reshape(4, 32, 32)).max(axis=2) / np.float32(127)).astype(np.float32)
    codes = q[:, :, 4:].view(np.int8).astype(np.float64)
    err = np.abs(x.reshape(4, 32, 32) - codes * d[..., None])
    assert (err <= d[..., None] * (0.5 + 1e-6)).all()
    assert (np.abs(codes).max(axis=2) == 127).all()


# ---- mat-vec ---------------------------------------------------------------------------------
def _blocks_exact(rng, fmt, rows, k):
    """Weight rows whose dequantized values are exact small multiples of a power of two."""
    if fmt == 1:
        nb = rows * k // 32
        b = np.zeros((nb, 34), np.uint8)
        b[:, :2] = (2.0 ** -rng.integers(2, 9, nb)).astype(np.float16).view(np.uint8).reshape(nb, 2)
        b[:, 2:] = rng.integers(-128, 128, (nb, 32)).astype(np.int8).view(np.uint8)
    elif fmt == 2:
        nb = rows * k // 256
        b = rng.integers(0, 256, (nb, 144)).astype(np.uint8)
        dd = (2.0 ** -rng.integers(2, 9, nb)).astype(np.float16).view(np.uint8).reshape(nb, 2)
        b[:, 0:2] = dd
        b[:, 2:4] = dd
    else:
        nb = rows * k // 256
        b = rng.integers(0, 256, (nb, 84)).astype(np.uint8)
        dd = (2.0 ** -rng.integers(2, 9, nb)).astype(np.float16).view(np.uint8).reshape(nb, 2)
        b[:, 80:82] = dd
        b[:, 82:84] = dd
    return b.ravel()


def _act_exact(rng, nc, k):
    """Activations whose Q8_1 blocks have d = 2^-s exactly and codes equal to x / d."""
    q = rng.integers(-127, 128, (nc, k)).astype(np.float64)
    q.reshape(nc, k // 32, 32)[:, :, 0] = 127
    s = rng.integers(3, 7, (nc, k // 32, 1))
    return (q.reshape(nc, k // 32, 32) * 2.0 ** -s).reshape(nc, k).astype(np.float32)


@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_matvec_exact_against_dequant(orc, fmt):
    rng = np.random.default_rng(40 + fmt)
    rows, k, nc = 24, 512, 5
    w = _blocks_exact(rng, fmt, rows, k)
    deq = orc.dequant(fmt, w, rows * k).view(np.float16).astype(np.float64).reshape(rows, k)
    x = _act_exact(rng, nc, k)
    act = orc.quantize_q8_1(x)
    blk = act.reshape(nc, k // 32, 36)
    dx = blk[:, :, :2].copy().view(np.float16).astype(np.float64)  # [nc, nb, 1]
    qx = blk[:, :, 4:].view(np.int8).astype(np.float64)
    assert np.array_equal((qx * dx).reshape(nc, k), x.astype(np.float64))  # the activation is exact
    want = (qx * dx).reshape(nc, k) @ deq.T
    got, mag = orc.q81_matvec(fmt, w, rows, k, act)
    assert np.array_equal(got, want)
    assert (mag >= np.abs(got)).all()
    # a dropped last block or a transposed activation would not pass
    short = (qx * dx).reshape(nc, k)[:, :-32] @ deq[:, :-32].T
    assert not np.array_equal(got, short)


@pytest.mark.parametrize("fmt,k", [(1, 2560), (1, 640), (2, 2560), (2, 512)])
def test_matvec_against_reference_twins(orc, fmt, k):
    ref = _ref(orc)
    rng = np.random.default_rng(fmt * 7 + k)
    rows = 40
    rb = orc.lib().or_row_bytes(fmt, k)
    if fmt == 1:
        nb = rows * k // 32
        w = np.zeros((nb, 34), np.uint8)
        w[:, :2] = (rng.random(nb) * 0.02 + 1e-3).astype(np.float16).view(np.uint8).reshape(nb, 2)
        w[:, 2:] = rng.integers(-128, 128, (nb, 32)).astype(np.int8).view(np.uint8)
    else:
        nb = rows * k // 256
        w = rng.integers(0, 256, (nb, 144)).astype(np.uint8)
        w[:, 0:2] = (rng.random(nb) * 0.01 + 1e-4).astype(np.float16).view(np.uint8).reshape(nb, 2)
        w[:, 2:4] = (rng.random(nb) * 0.01 + 1e-4).astype(np.float16).view(np.uint8).reshape(nb, 2)
    w = w.ravel()
    assert w.size == rows * rb
    for nc in (1, 2, 4, 8):
        x = rng.standard_normal((nc, k)).astype(np.float32)
        act = orc.quantize_q8_1(x)
        got, mag = orc.q81_matvec(fmt, w, rows, k, act)
        twin = np.empty((nc, rows), np.float32)
        fn = ref.ref_q80_mv if fmt == 1 else ref.ref_q4k_mv
        assert fn(w.ctypes.data, act.ctypes.data, k, rows, nc, twin.ctypes.data) == 0
        # the twin's F32 accumulation stays within a few dozen roundings of each block term
        tol = 64 * F32_EPS * mag + 1e-30
        assert (np.abs(twin - got) <= tol).all(), float((np.abs(twin - got) / mag).max())


# ---- SwiGLU and combine ----------------------------------------------------------------------
def test_swiglu_f32(orc):
    rng = np.random.default_rng(21)
    n = 640 * 4
    g = (rng.standard_normal(n) * 4).astype(np.float32)
    u = (rng.standard_normal(n) * 4).astype(np.float32)
    g[:3] = [0.0, -0.0, 100.0]
    got = orc.swiglu_f32(g, u)
    assert got[0] == 0.0 and got[2] == np.float32(100.0) * u[2]
    g64 = g.astype(np.float64)
    exact = g64 / (1.0 + np.exp(-g64)) * u.astype(np.float64)
    assert (np.abs(got - exact) <= 4 * F32_EPS * np.abs(exact) + 1e-37).all()
    ref = orc.ref()
    if ref is not None:
        twin = np.empty(n, np.float32)
        assert ref.ref_swiglu(g.ctypes.data, u.ctypes.data, n, twin.ctypes.data) == 0
        assert (np.abs(got - twin) <= 4 * F32_EPS * np.abs(twin) + 1e-37).all()


def test_combine_decode(orc):
    rng = np.random.default_rng(31)
    T, K, d = 6, 10, 2560
    parts = rng.standard_normal((T * K, d)).astype(np.float32)
    w = rng.random((T, K)).astype(np.float32)
    w /= w.sum(axis=1, keepdims=True)
    sh = rng.standard_normal((T, d)).astype(np.float32)
    # without a shared expert: one product then rank-ordered fma (K = 1 is the plain product)
    one = orc.combine_decode(parts[:T], w[:, :1], None, None, T, 1, d)
    assert np.array_equal(one, parts[:T] * w[:, :1])
    ref = orc.ref()
    # sigmoid(0) = 0.5 exactly in both: the twin must agree bit for bit
    gl0 = np.zeros(T, np.float32)
    ours = orc.combine_decode(parts, w, sh, gl0, T, K, d)
    p3 = parts.reshape(T, K, d)
    s = p3[:, 0] * w[:, :1]
    for r in range(1, K):
        s = (p3[:, r].astype(np.float64) * w[:, r:r + 1] + s).astype(np.float32)  # fma: one rounding
    assert np.array_equal(ours, (s + sh * np.float32(0.5)).astype(np.float32))
    if ref is not None:
        theirs = np.empty((T, d), np.float32)
        assert ref.ref_combine(parts.ctypes.data, w.ctypes.data, sh.ctypes.data, gl0.ctypes.data, T,
                               theirs.ctypes.data) == 0
        assert np.array_equal(ours, theirs)
        gl = rng.standard_normal(T).astype(np.float32)
        ours = orc.combine_decode(parts, w, sh, gl, T, K, d)
        assert ref.ref_combine(parts.ctypes.data, w.ctypes.data, sh.ctypes.data, gl.ctypes.data, T,
                               theirs.ctypes.data) == 0
        assert (np.abs(ours - theirs) <= 4 * F32_EPS * np.maximum(1.0, np.abs(theirs))).all()
