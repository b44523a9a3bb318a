"""GPU parity of the in-register block decoders: every dequantized value bit-exact.

The products decode weights with per-lane fragment decoders; encode_prefill_dequant runs
the same decoders (the reference's decode probes, prefill_moe.metal:735-769, and its
dequant dispatch, prefill_dequant_dispatch.hpp). Blocks are both quantized N(0,0.02) data
and random bytes with finite random F16 scales, which reach every code and scale field.
"""
import numpy as np
import pytest

import gpu_util as gu

pytestmark = pytest.mark.gpu

BLOCK = {1: (32, 34, [0]), 2: (256, 144, [0, 2]), 3: (256, 84, [80, 82])}  # values, bytes, f16 offsets


def _random_blocks(fmt, rows, k, seed):
    vals, nbytes, f16_offs = BLOCK[fmt]
    rng = np.random.default_rng(seed)
    nb = rows * k // vals
    raw = rng.integers(0, 256, size=(nb, nbytes), dtype=np.uint8)
    for off in f16_offs:  # finite F16 scale fields: clear the top exponent bit pattern 31
        h = raw[:, off:off + 2].copy().view(np.uint16)
        h &= np.uint16(0xBFFF)
        raw[:, off:off + 2] = h.view(np.uint8)
    return raw.reshape(-1)


@pytest.mark.parametrize("fmt,rows,k", [(1, 48, 512), (1, 16, 128), (2, 40, 1024), (3, 32, 1024),
                                         (4, 16, 512), (5, 16, 512)])
@pytest.mark.parametrize("source", ["quantized", "random"])
def test_dequant_bit_exact(moe, orc, gpu_ctx, stream, fmt, rows, k, source):
    print(f"case dequant fmt={fmt} rows={rows} k={k} source={source}", flush=True)
    if fmt in (4, 5):
        gen = moe.synth_normal_bf16 if fmt == 5 else moe.synth_normal_f16
        w = gen(11, fmt, 0.02 if source == "quantized" else 3.0, rows * k).view(np.uint8)
    elif source == "quantized":
        w = moe.synth_quantized(fmt, 11, fmt, 0.02, rows, k)
    else:
        w = _random_blocks(fmt, rows, k, 1234 + fmt)
    bw = gpu_ctx.register(gu.dev(w))
    out = gpu_ctx.register(gu.poison(rows * k * 2))
    gu.run(gpu_ctx, stream, lambda s: s.encode_prefill_dequant(fmt, rows, k, bw.view(), out.view()))
    got = gu.host(out, np.uint16).reshape(k, rows).T
    rb = moe.row_bytes(fmt, k)
    ref = np.stack([orc.dequant(fmt, w[r * rb:(r + 1) * rb], k) for r in range(rows)])
    assert np.array_equal(got, ref), f"{(got != ref).sum()} values differ"
