"""CPU: the grouping oracle (counting sort, histogram cursors, PfPlan, tile list) pinned
against numpy's stable argsort and the layout facts the reference asserts
(tests/metal/metal_prefill_moe_grouping_test.mm:42-45), on the reference's id patterns
(tests/metal/pf_sort_eq_host_grouping.mm:126-178)."""
import numpy as np
import pytest

import ref_patterns as rp


def _expected(ids, E):
    flat = ids.reshape(-1).astype(np.int64)
    N = flat.size
    valid = (flat >= 0) & (flat < E)
    vidx = np.nonzero(valid)[0]
    order = vidx[np.argsort(flat[vidx], kind="stable")]
    counts = np.bincount(flat[vidx], minlength=E)
    first = np.concatenate([[0], np.cumsum(counts)[:-1]])
    n_count = (N + 255) // 256
    hist = np.empty((n_count, E), np.int64)
    for t in range(n_count):
        seen = flat[: t * 256]
        seen = seen[(seen >= 0) & (seen < E)]
        hist[t] = first + np.bincount(seen, minlength=E)
    return order, counts, first, hist, int((~valid).sum())


@pytest.mark.parametrize("E", [16, 256, 512])
@pytest.mark.parametrize("T", [1, 7, 25, 26, 64, 300, 4096])
@pytest.mark.parametrize("pattern", rp.PATTERNS)
def test_grouping_against_stable_sort(orc, pattern, T, E):
    ids = rp.grouping_ids(T, E, pattern)
    g = orc.grouping(ids, E)
    order, counts, first, hist, bad = _expected(ids, E)
    n_valid = order.size
    assert np.array_equal(g["dst"][:n_valid], order)
    assert np.array_equal(g["src"][:n_valid], order // ids.shape[1])
    assert (g["src"][n_valid:] == -1).all() and (g["dst"][n_valid:] == -1).all()
    assert np.array_equal(g["hist"], hist)
    pf = orc.plan_fields(g["plan"])
    used = np.nonzero(counts)[0]
    assert pf["n_groups"] == used.size and pf["bad"] == bad and pf["n_entries"] == ids.size
    assert pf["n_miss"] == 0 and pf["skip"] == 1
    assert np.array_equal(pf["grp_e"][: used.size], used) and (pf["grp_e"][used.size:] == -1).all()
    assert (pf["grp_res"][: used.size] == 1).all() and (pf["grp_res"][used.size:] == -1).all()
    assert np.array_equal(pf["grp_start"][: used.size], first[used])
    assert pf["grp_start"][used.size] == n_valid and (pf["grp_start"][used.size + 1:] == 0).all()
    assert (g["plan"][6180:] == 0).all() and (g["plan"][24:32] == 0).all()
    tiles = [(gi, first[e] + 64 * j) for gi, e in enumerate(used) for j in range(-(-counts[e] // 64))]
    assert g["n_tiles"] == pf["n_tiles"] == len(tiles)
    assert [tuple(t) for t in g["tiles"]] == tiles


def test_plan_layout_constants():
    # PfPlan field offsets and size asserted by the reference's grouping test.
    import ctypes as C

    class PfPlan(C.Structure):
        _fields_ = [("n_groups", C.c_uint32), ("n_entries", C.c_uint32), ("n_miss", C.c_uint32),
                    ("skip", C.c_uint32), ("n_tiles", C.c_uint32), ("bad", C.c_uint32),
                    ("pad", C.c_uint32 * 2), ("grp_e", C.c_int32 * 512), ("grp_res", C.c_int32 * 512),
                    ("grp_start", C.c_int32 * 513)]
    assert C.sizeof(PfPlan) == 6180
    assert PfPlan.grp_e.offset == 32 and PfPlan.grp_res.offset == 2080 and PfPlan.grp_start.offset == 4128


def test_invalid_ids_counted_and_dropped(orc):
    E = 256
    ids = rp.grouping_ids(300, E, "invalid_ids")
    g = orc.grouping(ids, E)
    flat = ids.reshape(-1)
    assert orc.plan_fields(g["plan"])["bad"] == int(((flat < 0) | (flat >= E)).sum()) > 0


@pytest.mark.parametrize("E", [16, 512])
@pytest.mark.parametrize("pattern", rp.PATTERNS)
def test_gather_is_row_indexing(orc, pattern, E):
    """or_gather against numpy fancy indexing x[src[:n_valid]], bit for bit, on the reference's id
    patterns (pf_sort_eq_host_grouping.mm:462-480 checks Xs[a] == mixed_h[src[a]])."""
    T, d = 300, 256
    rng = np.random.default_rng(E)
    x = rng.integers(0, 1 << 16, size=(T, d), dtype=np.uint16)
    ids = rp.grouping_ids(T, E, pattern)
    g = orc.grouping(ids, E)
    n_valid = ids.size - orc.plan_fields(g["plan"])["bad"]
    xs = orc.gather(x, g["src"], n_valid)
    assert xs.shape == (n_valid, d)
    assert np.array_equal(xs, x[g["src"][:n_valid]])
    # a planted off-by-one in the source rows is caught by the same comparison
    shifted = np.where(g["src"][:n_valid] + 1 < T, g["src"][:n_valid] + 1, 0).astype(np.int32)
    assert not np.array_equal(orc.gather(x, shifted, n_valid), x[g["src"][:n_valid]])
