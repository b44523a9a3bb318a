"""Writes small GGUF v3 files for the model-file tests (test infrastructure).

Layout per the published GGUF format: magic "GGUF", u32 version, u64 tensor count, u64
key/value count, the key/values, the tensor directory (name, u32 n_dims, u64 ne[n_dims],
u32 ggml type, u64 data offset relative to the data section), padding to general.alignment,
then the tensor data, each tensor aligned.
"""
from __future__ import annotations

import struct

import numpy as np

T_U32, T_I32, T_F32, T_STRING, T_ARRAY, T_U64 = 4, 5, 6, 8, 9, 10
GGML = {"F32": 0, "F16": 1, "Q8_0": 8, "Q2_K": 10, "Q4_K": 12, "Q6_K": 14, "BF16": 30}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(t: int, v) -> bytes:
    if t == T_U32:
        return struct.pack("<I", v)
    if t == T_I32:
        return struct.pack("<i", v)
    if t == T_F32:
        return struct.pack("<f", v)
    if t == T_U64:
        return struct.pack("<Q", v)
    if t == T_STRING:
        return _str(v)
    if t == T_ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    raise ValueError(t)


def write_gguf(path, tensors, kv=(), alignment: int = 32, version: int = 3, misalign: str = "",
               truncate: int = 0, magic: bytes = b"GGUF"):
    """tensors: [(name, ggml type id, ne tuple, data bytes)]; kv: [(key, type, value)].
    misalign: name of a tensor whose recorded offset is moved off the alignment;
    truncate: bytes cut from the end of the file."""
    kvs = list(kv)
    if alignment != 32:
        kvs.append(("general.alignment", T_U32, alignment))
    head = magic + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += _str(k) + struct.pack("<I", t) + _value(t, v)
    offsets, cur = [], 0
    for name, ty, ne, data in tensors:
        cur = -(-cur // alignment) * alignment
        offsets.append(cur)
        cur += len(data)
    for (name, ty, ne, data), off in zip(tensors, offsets):
        if name == misalign:
            off += 4
        head += _str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne) + struct.pack("<IQ", ty, off)
    pad = -len(head) % alignment
    blob = bytearray(head + b"\0" * pad)
    base = len(blob)
    for (name, ty, ne, data), off in zip(tensors, offsets):
        need = base + off - len(blob)
        blob += b"\0" * need + bytes(data)
    if truncate:
        blob = blob[:-truncate]
    with open(path, "wb") as f:
        f.write(bytes(blob))


def expert_model(moe, n_layers=2, E=16, d=256, I=128, gu="Q4_K", dn="Q8_0", seed=5):
    """Tensors of a small model: per layer the router (F32 [d, E]), the three expert tensors, plus
    an F16 token embedding and a Q6_K output tensor (a type the experts do not use). Returns
    (tensors, {layer: (gate, up, down) bytes})."""
    fmt = {"Q8_0": moe.Q8_0, "Q4_K": moe.Q4_K, "Q2_K": moe.Q2_K}
    tensors = [("token_embd.weight", GGML["F16"], (d, 64), np.zeros(d * 64, np.uint16).tobytes())]
    experts = {}
    for l in range(n_layers):
        g = moe.synth_quantized(fmt[gu], seed, 100 * l + 1, 0.02, E * I, d)
        u = moe.synth_quantized(fmt[gu], seed, 100 * l + 2, 0.02, E * I, d)
        w = moe.synth_quantized(fmt[dn], seed, 100 * l + 3, 0.02, E * d, I)
        r = moe.synth_normal_f32(seed, 100 * l + 4, 0.02, E * d)
        experts[l] = (g, u, w)
        tensors += [(f"blk.{l}.ffn_gate_inp.weight", GGML["F32"], (d, E), r.tobytes()),
                    (f"blk.{l}.ffn_gate_exps.weight", GGML[gu], (d, I, E), g.tobytes()),
                    (f"blk.{l}.ffn_up_exps.weight", GGML[gu], (d, I, E), u.tobytes()),
                    (f"blk.{l}.ffn_down_exps.weight", GGML[dn], (I, d, E), w.tobytes())]
    tensors.append(("output.weight", GGML["Q6_K"], (256, 4), np.zeros(4 * 210, np.uint8).tobytes()))
    return tensors, experts


KV = [("general.architecture", T_STRING, "strata-test"),
      ("tokenizer.ggml.tokens", T_ARRAY, (T_STRING, ["<s>", "</s>", "a", "bb"])),
      ("test.counts", T_ARRAY, (T_U32, [1, 2, 3])),
      ("test.scale", T_F32, 0.5)]
