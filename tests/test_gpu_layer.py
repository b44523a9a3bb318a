"""GPU parity of the expert stages and the full layer against the CPU oracle.

Each stage is checked on the GPU's own upstream outputs (stage isolation, as the reference's
staged tests do): gate/up SwiGLU outputs within 1 F16 ulp of the FP64 product; down parts
within 1e-4 abs + 1e-4 rel of the FP64 product; combine bit-exact against the ordered-FMA
restatement; the layer output within max-abs 2e-2 and rel-L2 5e-3 in F16.
"""
import numpy as np
import pytest

import gpu_util as gu

pytestmark = pytest.mark.gpu


def _check_layer(moe, layer, orc, ctx, stream, cfg, n_sample_tokens=None, chunk=0, inp=None):
    inp = inp if inp is not None else layer.make_inputs(cfg)
    ws = layer.LayerWorkspace(ctx, cfg, inp, chunk=chunk)
    ws.run_layer(stream)
    bad, st_gu, st_dn = ws.read_status(stream)
    assert (bad, st_gu, st_dn) == (0, 0, 0)
    T, d, E, K, I, Is = cfg.rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff, cfg.shared_ff
    N = T * K
    x = inp.x[chunk * T:(chunk + 1) * T]
    logits = gu.host(ws.logits, np.float32).reshape(T, E)
    ids = gu.host(ws.ids, np.int32).reshape(T, K)
    w = gu.host(ws.route_w, np.float32).reshape(T, K)
    ids_ref, w_ref = orc.route(logits, K, True)
    assert np.array_equal(ids, ids_ref) and np.array_equal(w.view(np.uint32), w_ref.view(np.uint32))
    rng = np.random.default_rng(cfg.seed)
    tokens = np.arange(T) if n_sample_tokens is None else np.sort(rng.choice(T, n_sample_tokens, replace=False))
    out_ref, g = orc.layer_ref(cfg, inp, ids, w, tokens, chunk=chunk)
    assert np.array_equal(gu.host(ws.src, np.int32), g["src"])
    assert np.array_equal(gu.host(ws.dst, np.int32), g["dst"])
    plan = g["plan"]
    # gate/up on the GPU's gathered rows
    xs = gu.host(ws.xs, np.uint16).reshape(N, d)
    inv = np.empty(N, np.int64)
    inv[g["dst"]] = np.arange(N)
    pos = inv[(tokens[:, None] * K + np.arange(K)).ravel()]
    gg, uu, eh_ref = orc.gate_up_ref(cfg.gate_up_fmt, xs, d, I, plan, inp.w_gate, inp.w_up, inp.gu_stride, pos)
    eh = gu.host(ws.hidden, np.uint16).reshape(N, I)
    gu.assert_f16_close(eh[pos], eh_ref, ulps=1.0, atol=1e-4, what="gate/up SwiGLU")
    # down on the GPU's hidden rows
    parts_ref = orc.down_ref(cfg.down_fmt, eh, d, I, plan, inp.w_down, inp.dn_stride, pos)
    parts = gu.host(ws.parts, np.float32).reshape(N, d)
    got = parts[g["dst"][pos]]
    assert np.allclose(got, parts_ref, atol=1e-4, rtol=1e-4), float(np.abs(got - parts_ref).max())
    # shared expert
    sh = gl = None
    if Is:
        hid_ref, sh_ref, gl_ref = orc.shared_ref(cfg.shared_fmt, x, d, Is, inp.sh_gate, inp.sh_up, inp.sh_down,
                                                 inp.sh_gvec, tokens)
        hid = gu.host(ws.sh_hidden, np.uint16).reshape(T, Is)
        gu.assert_f16_close(hid[tokens], hid_ref, ulps=1.0, atol=1e-4, what="shared SwiGLU")
        sh = gu.host(ws.sh_out, np.float32).reshape(T, d)
        gl = gu.host(ws.sh_gl, np.float32)
        assert np.allclose(gl[tokens], gl_ref, atol=1e-4, rtol=1e-4)
        # shared down on the GPU's hidden rows
        wd = orc.dequant(cfg.shared_fmt, inp.sh_down, d * Is).view(np.float16).astype(np.float64).reshape(d, Is)
        sh_ref = gu.f16(hid[tokens]) @ wd.T
        assert np.allclose(sh[tokens], sh_ref, atol=1e-4, rtol=1e-4), float(np.abs(sh[tokens] - sh_ref).max())
    # combine: bit-exact against the ordered-FMA restatement on the GPU's inputs
    out = gu.host(ws.out, np.float32).reshape(T, d)
    comb = orc.combine(parts, w, sh, gl, T, K, d)
    assert np.array_equal(out.view(np.uint32), comb.view(np.uint32)), "combine not bit-exact"
    err, rel = gu.layer_tolerance(out[tokens], out_ref)
    print(f"{cfg.name} chunk {chunk}: layer max-abs {err:.3e} rel-L2 {rel:.3e} over {len(tokens)} tokens", flush=True)
    assert err <= 2e-2 and rel <= 5e-3
    return ws


def test_layer_config0_full(moe, layer, orc, gpu_ctx, stream):
    print("case layer config 0", flush=True)
    _check_layer(moe, layer, orc, gpu_ctx, stream, layer.CONFIGS[0])


def test_layer_config2_sampled(moe, layer, orc, gpu_ctx, stream):
    print("case layer config 2 (sampled tokens)", flush=True)
    _check_layer(moe, layer, orc, gpu_ctx, stream, layer.CONFIGS[2], n_sample_tokens=48)


def test_layer_config3_zipf_sampled(moe, layer, orc, gpu_ctx, stream):
    print("case layer config 3 (sampled tokens)", flush=True)
    cfg = layer.CONFIGS[3]
    ws = _check_layer(moe, layer, orc, gpu_ctx, stream, cfg, n_sample_tokens=32)
    counts = np.bincount(gu.host(ws.ids, np.int32), minlength=cfg.n_experts)
    print(f"zipf rows per expert: max {counts.max()} median {int(np.median(counts))} "
          f"experts with <=5 rows {(counts <= 5).sum()}", flush=True)
    assert counts.max() > 1000


def test_layer_config4_chunk_sampled(moe, layer, orc, gpu_ctx, stream):
    print("case layer config 4 chunk 0 (sampled tokens)", flush=True)
    _check_layer(moe, layer, orc, gpu_ctx, stream, layer.CONFIGS[4], n_sample_tokens=24)


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

