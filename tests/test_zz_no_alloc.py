"""The allocation-free full layer (sm_submit_full_layer_fixed_scratch): its workspace (the
grouping histogram and both address snapshots) lives in the library's fixed per-GPU scratch.

CPU: the entry point's own preflight (null workspace views required, the histogram bound).
GPU: through the C ABI, two calls in a row, the second on a smaller layer, each equal bit for
bit to the same layer run by sm_submit_full_layer with caller workspace views; a call on a
capturing stream is refused before anything is encoded.
"""
import ctypes as C

import numpy as np
import pytest

from test_abi_host import Fake

SM_E_ARGUMENT, SM_E_SHAPE, SM_E_DEVICE = 1, 2, 9


def _fixed_views(moe, lb):
    """The layer buffers with the three workspace views the fixed scratch replaces set null."""
    lb.route_gather.histogram = moe.NULL_VIEW
    lb.gate_up.weights.address_snapshot = moe.NULL_VIEW
    lb.down.weights.address_snapshot = moe.NULL_VIEW
    return lb


def _submit_fixed(moe, ctx, stream, shape, formats, lb):
    err = C.create_string_buffer(512)
    st = moe.library().sm_submit_full_layer_fixed_scratch(ctx.handle, C.c_void_p(stream), C.byref(shape),
                                                          C.byref(formats), C.byref(lb), err, 512)
    return st, err.value.decode()


def test_fixed_scratch_preflight(moe):
    import torch
    fake = Fake(moe)
    lb = fake.layer()
    st, err = _submit_fixed(moe, fake.ctx, 0, fake.shape, fake.fmts, lb)
    assert st == SM_E_ARGUMENT and "histogram view must be null" in err
    lb = _fixed_views(moe, fake.layer())
    lb.gate_up.weights.address_snapshot = fake.snap_gu.view()
    st, err = _submit_fixed(moe, fake.ctx, 0, fake.shape, fake.fmts, lb)
    assert st == SM_E_ARGUMENT and "address snapshot view must be null" in err
    # 2^20 bytes hold (ceil(T*k/256) + 1) * E * 4 only up to 511 histogram rows at E = 512
    big = Fake(moe, T=13312, d=256, E=512, K=10, I=128, Is=256)
    st, err = _submit_fixed(moe, big.ctx, 0, big.shape, big.fmts, _fixed_views(moe, big.layer()))
    assert st == SM_E_SHAPE and "histogram needs 1048576 bytes" not in err and "more than the fixed scratch" in err
    if not torch.cuda.is_available():
        st, err = _submit_fixed(moe, fake.ctx, 0, fake.shape, fake.fmts, _fixed_views(moe, fake.layer()))
        assert st == SM_E_DEVICE and "fixed scratch is not available" in err


@pytest.mark.gpu
def test_fixed_scratch_layer_matches_caller_workspace(moe, layer, gpu_ctx, stream):
    import torch
    big = layer.CONFIGS[2]
    small = layer.LayerConfig("fixed_small", 192, 512, 32, 4, 256, 256, moe.Q4_K, moe.Q8_0, moe.F16, seed=91)
    for cfg in (big, small):  # the second call's layer is smaller than the first's
        print(f"case fixed scratch {cfg.name}: T {cfg.rows}", flush=True)
        ws = layer.LayerWorkspace(gpu_ctx, cfg, layer.make_inputs(cfg))
        lb = ws.layer_buffers()
        err = C.create_string_buffer(512)
        st = moe.library().sm_submit_full_layer(gpu_ctx.handle, C.c_void_p(stream), C.byref(ws.shape),
                                                C.byref(ws.formats), C.byref(lb), err, 512)
        assert st == 0, err.value
        assert ws.read_status(stream) == (0, 0, 0)
        names = ("out", "plan", "src", "dst", "xs", "hidden", "parts")
        ref = {n: getattr(ws, n).tensor.cpu().numpy().view(np.uint8).copy() for n in names}
        for n in names:
            getattr(ws, n).tensor.view(torch.uint8).fill_(0xA5)
        ws.status.tensor.fill_(-1)
        st, msg = _submit_fixed(moe, gpu_ctx, stream, ws.shape, ws.formats, _fixed_views(moe, ws.layer_buffers()))
        assert st == 0, msg
        assert ws.read_status(stream) == (0, 0, 0)
        for n in names:
            got = getattr(ws, n).tensor.cpu().numpy().view(np.uint8)
            assert np.array_equal(got, ref[n]), f"{cfg.name}: {n} differs from the caller-workspace layer"


@pytest.mark.gpu
def test_fixed_scratch_refuses_a_capturing_stream(moe, layer, gpu_ctx):
    """Under stream capture the entry point returns SM_E_ARGUMENT before encoding anything (its
    expert address tables would be replayed from a reusable host slot), so the capture holds
    no launch and the outputs stay as they were."""
    import torch
    print("case fixed scratch under capture", flush=True)
    cfg = layer.LayerConfig("fixed_capture", 64, 256, 16, 4, 128, 0, moe.Q8_0, moe.Q8_0, moe.F16, seed=93)
    ws = layer.LayerWorkspace(gpu_ctx, cfg, layer.make_inputs(cfg))
    lb = _fixed_views(moe, ws.layer_buffers())
    ws.out.tensor.view(torch.uint8).fill_(0xA5)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side, capture_error_mode="thread_local"):
        st, msg = _submit_fixed(moe, gpu_ctx, side.cuda_stream, ws.shape, ws.formats, lb)
    assert st == SM_E_ARGUMENT and "capturing stream" in msg, (st, msg)
    torch.cuda.synchronize()
    assert (ws.out.tensor.view(torch.uint8).cpu().numpy() == 0xA5).all()
