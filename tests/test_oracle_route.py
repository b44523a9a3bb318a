"""CPU: the route oracle (softmax top-k, divide/multiply weights) pinned independently.

Pins: the reference's golden weight bits and tie patterns (tests/metal/metal_moe_test.mm:
124-141, 270-309, 605-652); the reference's own moe_route.cpp built into oracle/_ref (ids
exact, weights within the reference's U(16) tolerance); a brute-force order check (top-k ids
equal a stable sort of the logits when no two probabilities collide); the weight sum.
"""
import numpy as np
import pytest

import ref_patterns as rp


@pytest.mark.parametrize("E", [256, 512])
@pytest.mark.parametrize("divide", [True, False])
def test_golden_bits_and_ties(orc, E, divide):
    L = rp.special_logits(E)
    ids, w = orc.route(L, 10, divide)
    assert np.array_equal(ids, rp.special_ids(E))
    assert list(w[0].view(np.uint32)) == rp.EQUAL_WEIGHT_BITS
    gold = rp.NONUNIFORM_DIVIDE_BITS if divide else rp.NONUNIFORM_MULTIPLY_BITS
    assert list(w[2].view(np.uint32)) == gold


def test_weight_mode_probe_arithmetic():
    # metal_moe_test.mm:136-139: sel 0x3dcccccd, sum 0x3e99999a -> divide 0x3eaaaaaa,
    # multiply-by-reciprocal 0x3eaaaaab. The oracle's two weight formulas are these float ops.
    sel = np.uint32(0x3DCCCCCD).view(np.float32)
    ssum = np.uint32(0x3E99999A).view(np.float32)
    assert (sel / ssum).view(np.uint32) == 0x3EAAAAAA
    assert (sel * (np.float32(1.0) / ssum)).view(np.uint32) == 0x3EAAAAAB


def _ulp_dist(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


@pytest.mark.parametrize("E", [256, 512])
@pytest.mark.parametrize("divide", [True, False])
def test_against_reference_twin(orc, E, divide):
    ref = orc.ref()
    if ref is None:
        pytest.skip("oracle/_ref not built (needs the reference checkout)")
    rng = np.random.default_rng(E + divide)
    L = np.concatenate([rp.special_logits(E), rp.shuffled_rank_logits(6, E, 9),
                        (rng.standard_normal((200, E)) * 2).astype(np.float32)])
    ids, w = orc.route(L, 10, divide)
    rids = np.empty_like(ids)
    rw = np.empty_like(w)
    assert ref.ref_route(L.ctypes.data, L.shape[0], E, int(divide), rids.ctypes.data, rw.ctypes.data) == 0
    assert np.array_equal(ids, rids)
    assert _ulp_dist(w, rw).max() <= 16  # the reference's U(16) route-weight bound


@pytest.mark.parametrize("E,K", [(16, 4), (40, 5), (256, 8), (512, 10), (100, 32)])
def test_ids_are_stable_logit_order(orc, E, K):
    rng = np.random.default_rng(E * K)
    # Distinct logits spaced far enough apart that rounded probabilities cannot collide.
    L = np.stack([rng.permutation(E).astype(np.float32) * 0.05 for _ in range(64)])
    ids, w = orc.route(L, K, True)
    order = np.argsort(-L, axis=1, kind="stable")[:, :K]
    assert np.array_equal(ids, order)
    assert (np.abs(w.sum(axis=1) - 1.0) < 2e-5).all()
    # Weights against a float64 softmax renormalised over the selected ids.
    p = np.exp(L.astype(np.float64) - L.max(axis=1, keepdims=True))
    sel = np.take_along_axis(p, order, axis=1)
    assert np.allclose(w, sel / sel.sum(axis=1, keepdims=True), rtol=1e-5, atol=1e-7)


def test_equal_values_prefer_lower_ids(orc):
    E, K = 64, 6
    L = np.full((3, E), -5.0, np.float32)
    L[0, [60, 3, 40, 7, 22, 50, 9]] = 2.0        # 7-way tie for 6 slots
    L[1, :] = 1.0                                 # all equal
    L[2, [63, 62, 61]] = 3.0
    L[2, [10, 20]] = 3.0                          # 5-way tie, then the rest
    ids, _ = orc.route(L, K, True)
    assert list(ids[0]) == [3, 7, 9, 22, 40, 50]
    assert list(ids[1]) == [0, 1, 2, 3, 4, 5]
    assert list(ids[2][:5]) == [10, 20, 61, 62, 63] and ids[2][5] == 0


def test_nonfinite_rows(orc):
    E, K = 64, 4
    L = np.zeros((3, E), np.float32)
    L[0, 5] = np.nan        # NaN probability -> -FLT_MAX, never preferred over finite ones
    L[1, 7] = np.inf        # inf - inf: every probability NaN -> lowest ids win
    L[2, :] = -np.inf
    ids, w = orc.route(L, K, True)
    assert 5 not in ids[0] and list(ids[0]) == [0, 1, 2, 3]
    assert list(ids[1]) == [0, 1, 2, 3]
    assert list(ids[2]) == [0, 1, 2, 3]
