"""Helpers shared by the GPU parity tests: device uploads, run-and-sync, tolerance checks."""
from __future__ import annotations

import numpy as np


def dev(a: np.ndarray):
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    elif a.dtype == np.uint32:
        a = a.view(np.int32)
    elif a.dtype == np.uint64:
        a = a.view(np.int64)
    return torch.from_numpy(a).cuda()


def poison(nbytes: int, byte: int = 0xA5):
    import torch
    return torch.full((nbytes,), byte, dtype=torch.uint8, device="cuda")


def host(buf, dtype) -> np.ndarray:
    """Device buffer (moe.Buffer) -> numpy array of `dtype`."""
    return buf.tensor.cpu().numpy().view(np.uint8).view(dtype)


def run(ctx, stream, encode):
    """Encodes into a fresh segment via encode(seg) -> (ok, err), commits, synchronises."""
    import torch
    seg = ctx.segment()
    ok, err = encode(seg)
    if not ok:
        seg.abort()
        raise AssertionError(err)
    seg.commit(stream)
    torch.cuda.synchronize()


def f16(bits: np.ndarray) -> np.ndarray:
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def assert_f16_close(gpu_bits, ref_bits, ulps: float = 1.0, atol: float = 1e-5, what: str = ""):
    g, r = f16(gpu_bits), f16(ref_bits)
    tol = ulps * np.maximum(np.abs(r) * 2.0 ** -10, 2.0 ** -24) + atol
    bad = np.abs(g - r) > tol
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} F16 values off; first at {np.argwhere(bad)[0]}: gpu {g[bad][0]} ref {r[bad][0]}"


def layer_tolerance(out: np.ndarray, ref: np.ndarray):
    """Layer-output bound: max-abs 2e-2 and rel-L2 5e-3 after rounding both to F16."""
    o = out.astype(np.float16).astype(np.float64)
    r = ref.astype(np.float16).astype(np.float64)
    err = float(np.abs(o - r).max())
    rel = float(np.linalg.norm(o - r) / max(np.linalg.norm(r), 1e-30))
    return err, rel
