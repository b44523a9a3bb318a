"""Input patterns the reference's own tests use, restated as generators.

Route logits: tests/metal/metal_moe_test.mm:270-309 (make_logits). Grouping ids:
tests/metal/pf_sort_eq_host_grouping.mm:126-178 (make_ids). Golden route-weight bits:
tests/metal/metal_moe_test.mm:124-141.
"""
from __future__ import annotations

import numpy as np

EQUAL_WEIGHT_BITS = [0x3DCCCCCD] * 10
NONUNIFORM_DIVIDE_BITS = [0x3ECAD2AA, 0x3E760961, 0x3E153A90, 0x3DB5060D, 0x3D5B97C0,
                          0x3D053093, 0x3CA1913C, 0x3C43FDB7, 0x3BEDBFCB, 0x3B9033C2]
NONUNIFORM_MULTIPLY_BITS = [0x3ECAD2AB, 0x3E760962, 0x3E153A91, 0x3DB5060E, 0x3D5B97C0,
                            0x3D053094, 0x3CA1913C, 0x3C43FDB8, 0x3BEDBFCC, 0x3B9033C2]


def special_logits(E: int) -> np.ndarray:
    """Rows 0-3 of the reference's fixture set (E >= 20):
    0 all equal; 1 a 12-way tie at 8.0 on E-20..E-9 over -16; 2 the nonuniform row
    80 - 0.5 r on ids E-1, 0, E-2, 1, ... over -80; 3 alternating +100 / -100."""
    L = np.zeros((4, E), np.float32)
    L[1] = -16.0
    L[1, E - 20:E - 8] = 8.0
    L[2] = -80.0
    for r in range(11):
        e = E - 1 - r // 2 if r % 2 == 0 else r // 2
        L[2, e] = 80.0 - 0.5 * r
    L[3] = np.where(np.arange(E) % 2 == 0, 100.0, -100.0)
    return L


def special_ids(E: int, K: int = 10) -> np.ndarray:
    """Expected ids of special_logits rows (k = 10)."""
    return np.array([
        list(range(K)),
        [E - 20 + r for r in range(K)],
        [E - 1 - r // 2 if r % 2 == 0 else r // 2 for r in range(K)],
        [2 * r for r in range(K)],
    ], np.int32)


def shuffled_rank_logits(T: int, E: int, seed: int) -> np.ndarray:
    """The reference's "random" set: each row a shuffled ramp rank*0.125 - E*0.0625."""
    rng = np.random.default_rng(seed)
    out = np.empty((T, E), np.float32)
    for t in range(T):
        out[t] = rng.permutation(E).astype(np.float32) * 0.125 - E * 0.0625
    return out


PATTERNS = ("mixed", "one_expert", "all_experts", "tile_boundaries", "invalid_ids")


def grouping_ids(rows: int, E: int, pattern: str, K: int = 10) -> np.ndarray:
    """Route ids of the reference grouping patterns, token-major [rows, K]."""
    n = rows * K
    idx = np.arange(n, dtype=np.int64)
    mixed = ((idx * 73 + (idx // 11) * 29) % E).astype(np.int64)
    if pattern == "mixed":
        ids = mixed
    elif pattern == "one_expert":
        ids = np.zeros(n, np.int64)
    elif pattern == "all_experts":
        ids = idx % E
    elif pattern == "tile_boundaries":
        ends = [63, 127, 192, 319, 447, 576]
        ids = np.full(n, 6, np.int64)
        for b in reversed(range(len(ends))):
            ids[idx <= ends[b]] = b
        ids = ids % E
    elif pattern == "invalid_ids":
        ids = mixed.copy()
        sel = idx % 7 == 3
        kind = (idx // 7) % 4
        bad = np.where(kind == 0, -1, np.where(kind == 1, E, np.where(kind == 2, E + 1, -(2 ** 31))))
        ids[sel] = bad[sel]
    else:
        raise ValueError(pattern)
    return ids.astype(np.int32).reshape(rows, K)
