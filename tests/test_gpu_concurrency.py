"""GPU: layers committed on one context from two streams at once, back to back.

The reference runs its GPU tests under serial and concurrent dispatch (cmake/metal/tests.cmake:
330-339). Here two full prefill layers (with a shared expert, so the context's second stream is
used too) and two decode layers, each pair on different weights, are committed alternately on
two streams without a wait in between, often enough to cycle the context's 64-slot ring of
expert address tables several times. Every output must equal the same layer run alone, bit for
bit: a ring slot handed out while a launch could still read it, or a table copied for the wrong
layer, would put another layer's experts into the products.
"""
import numpy as np
import pytest

import gpu_util as gu

pytestmark = pytest.mark.gpu


def _prefill(layer, moe, seed):
    return layer.LayerConfig("concurrent", 256, 512, 64, 4, 256, 256, moe.Q4_K, moe.Q8_0, moe.F16, seed=seed)


def _decode(layer, moe, seed):
    return layer.LayerConfig("concurrent_decode", 2, 512, 64, 8, 256, 256, moe.Q4_K, moe.Q8_0, moe.F16, seed=seed)


def _out(ws):
    return gu.host(ws.out, np.float32).copy()


def test_two_streams_alternating_commits(moe, layer, gpu_ctx):
    import torch
    print("case concurrent commits on two streams", flush=True)
    pre = [layer.LayerWorkspace(gpu_ctx, c, layer.make_inputs(c)) for c in (_prefill(layer, moe, 0xC0C0A),
                                                                             _prefill(layer, moe, 0xC0C0B))]
    dec = [layer.DecodeWorkspace(gpu_ctx, c, layer.make_inputs(c)) for c in (_decode(layer, moe, 0xC0C0C),
                                                                             _decode(layer, moe, 0xC0C0D))]
    # Each layer alone first: the references.
    main = torch.cuda.current_stream().cuda_stream
    want_pre, want_dec = [], []
    for ws in pre:
        ws.run_layer(main)
        torch.cuda.synchronize()
        assert ws.read_status(main) == (0, 0, 0)
        want_pre.append(_out(ws))
    for ws in dec:
        ws.run(main)
        torch.cuda.synchronize()
        assert ws.read_status() == 0
        want_dec.append(_out(ws))
    assert not np.array_equal(want_pre[0], want_pre[1]) and not np.array_equal(want_dec[0], want_dec[1])
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]  # default priority
    for rnd in range(4):
        for _ in range(20):  # 20 x (2 prefill + 2 decode) commits of two ring slots each per round
            for i in (0, 1):
                pre[i].run_layer(streams[i].cuda_stream)
                dec[i].run(streams[i].cuda_stream)
        torch.cuda.synchronize()
        for i in (0, 1):
            assert pre[i].read_status(main) == (0, 0, 0)
            assert dec[i].read_status() == 0
            assert np.array_equal(_out(pre[i]).view(np.uint32), want_pre[i].view(np.uint32)), (rnd, "prefill", i)
            assert np.array_equal(_out(dec[i]).view(np.uint32), want_dec[i].view(np.uint32)), (rnd, "decode", i)
