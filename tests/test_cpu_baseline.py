"""The timed CPU baseline (`or_cpu_layer`, oracle/cpu_baseline.cpp, built -ffast-math) against the
pinned FP64 restatement (`layer_ref`) on the same seeded inputs.

`or_cpu_layer` is what bench.py's `cpu_baseline` leg times. It routes from its own F32 logits;
the check routes the FP64 logits (`or_router_ref`, pinned against numpy) rounded to F32 with the
pinned `or_route`, and requires the baseline's output to agree with `layer_ref` on that routing
within the layer bound (max-abs 2e-2, rel-L2 5e-3 in F16). A routing difference on any token
would move that token's output by a whole expert's contribution and fail the bound.
"""
import numpy as np
import pytest

import gpu_util as gu


def _cfg_small_full(moe, layer):
    """Configuration 2's widths and formats (d 2048, k 10, I 512, Q4_K / Q8_0, F16 shared) at 48 tokens
    over 128 experts."""
    return layer.LayerConfig("full_layer_small", 48, 2048, 128, 10, 512, 512, moe.Q4_K, moe.Q8_0, moe.F16,
                             seed=layer.SEED_BASE + 2)


def _cfg_small_low_bit(moe, layer):
    """Configuration 4's formats (Q2_K / Q4_K, BF16 shared) at reduced widths."""
    return layer.LayerConfig("low_bit_small", 32, 1024, 64, 8, 512, 512, moe.Q2_K, moe.Q4_K, moe.BF16,
                             seed=layer.SEED_BASE + 4)


@pytest.mark.parametrize("which", ["config0", "full_small", "low_bit_small"])
def test_cpu_layer_matches_layer_ref(moe, layer, orc, which):
    cfg = {"config0": lambda: layer.CONFIGS[0], "full_small": lambda: _cfg_small_full(moe, layer),
           "low_bit_small": lambda: _cfg_small_low_bit(moe, layer)}[which]()
    inp = layer.make_inputs(cfg)
    out, stage_us, threads = orc.cpu_layer(cfg, inp, n_threads=4)
    assert threads == 4 and (stage_us >= 0).all()
    x = inp.x[: cfg.rows]
    logits = orc.router_ref(x, inp.w_router).astype(np.float32)
    ids, w = orc.route(logits, cfg.top_k, True)
    ref, _ = orc.layer_ref(cfg, inp, ids, w)
    err, rel = gu.layer_tolerance(out, ref)
    assert err <= 2e-2 and rel <= 5e-3, (err, rel)
    # The bound is not vacuous: the baseline is far tighter than it, and a planted mistake (the
    # shared expert's gate left out) fails it.
    assert rel < 1e-4, rel
    if cfg.shared_ff:
        _, sh, gl = orc.shared_ref(cfg.shared_fmt, x, cfg.hidden, cfg.shared_ff, inp.sh_gate, inp.sh_up, inp.sh_down,
                                   inp.sh_gvec, np.arange(cfg.rows))
        bad = ref - sh * orc.sigmoid64(gl)[:, None] + sh
        err_b, rel_b = gu.layer_tolerance(out, bad)
        assert not (err_b <= 2e-2 and rel_b <= 5e-3), (err_b, rel_b)
