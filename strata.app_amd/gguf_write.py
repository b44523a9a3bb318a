"""Writes GGUF v3 model files holding a layer stack's routed-expert tensors (synthetic model
files for the tiered-residency measurement and the model-file tests).

Layout per the published GGUF format: magic "GGUF", u32 version, u64 tensor count, u64
key/value count, the key/values, the tensor directory (name, u32 n_dims, u64 ne[n_dims],
u32 ggml type, u64 data offset relative to the data section), padding to general.alignment,
then the tensor data, each tensor aligned.
"""
from __future__ import annotations

import struct

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
    """tensors: [(name, ggml type id, ne tuple, data bytes-like)]; kv: [(key, type, value)].
    misalign: name of a tensor whose recorded offset is moved off the alignment;
    truncate: bytes cut from the end of the file. The data is streamed to the file."""
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
        cur += len(memoryview(data).cast("B"))
    for (name, ty, ne, data), off in zip(tensors, offsets):
        if name == misalign:
            off += 4
        head += _str(name) + struct.pack("<I", len(ne)) + struct.pack(f"<{len(ne)}Q", *ne) + struct.pack("<IQ", ty, off)
    head += b"\0" * (-len(head) % alignment)
    total = len(head) + cur
    with open(path, "wb") as f:
        f.write(head)
        pos = 0
        for (name, ty, ne, data), off in zip(tensors, offsets):
            f.write(b"\0" * (off - pos))
            mv = memoryview(data).cast("B")
            f.write(mv)
            pos = off + len(mv)
        if truncate:
            f.truncate(total - truncate)


def expert_tensors(layers, hidden: int, expert_ff: int, n_experts: int, gate_up: str, down: str):
    """The blk.<l>.ffn_{gate,up,down}_exps tensors of `layers` ([(gate, up, down) block bytes]):
    gate/up [hidden, expert_ff, n_experts], down [expert_ff, hidden, n_experts] (ggml order)."""
    out = []
    for l, (g, u, w) in enumerate(layers):
        out += [(f"blk.{l}.ffn_gate_exps.weight", GGML[gate_up], (hidden, expert_ff, n_experts), g),
                (f"blk.{l}.ffn_up_exps.weight", GGML[gate_up], (hidden, expert_ff, n_experts), u),
                (f"blk.{l}.ffn_down_exps.weight", GGML[down], (expert_ff, hidden, n_experts), w)]
    return out
