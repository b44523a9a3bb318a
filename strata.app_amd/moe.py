"""Python host mirror of the Prefill MoE coordinators over libstrata_moe.so.

Names, argument meaning and error behaviour follow the reference's C++ coordinators in
namespace strata::metal (include/strata/metal/prefill_moe_*.hpp): every ``encode_*`` call
returns ``(ok, error)`` like the reference's ``bool`` + ``std::string& error``; a failed
encode poisons the segment, which must then be aborted (the reference's "propagate false so
the whole segment is discarded"). Device memory is plain torch tensors registered with a
``Context``; the library itself never allocates on the layer path.

The HIP library is required: importing this module on a machine without the built
``libstrata_moe.so`` raises, and there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path
from typing import Optional, Sequence

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "libstrata_moe.so"

# ---- formats / status (include/strata_moe.h) -------------------------------------------
Q8_0, Q4_K, Q2_K, F16, BF16 = 1, 2, 3, 4, 5
FORMAT_NAMES = {Q8_0: "Q8_0", Q4_K: "Q4_K", Q2_K: "Q2_K", F16: "F16", BF16: "BF16"}
STATUS_NAMES = {
    0: "SM_OK", 1: "SM_E_ARGUMENT", 2: "SM_E_SHAPE", 3: "SM_E_VIEW", 4: "SM_E_OWNERSHIP",
    5: "SM_E_ALIAS", 6: "SM_E_SEGMENT", 7: "SM_E_FORMAT", 8: "SM_E_ADDRESS", 9: "SM_E_DEVICE", 10: "SM_E_FILE",
}
PLAN_BYTES = 6180
PLAN_SLOT_BYTES = 6400
COUNT_TILE = 256
EXPERT_TILE = 64

# The C ABI's exported symbols; tests check the library exports each one.
EXPORTS = (
    "sm_abi_version", "sm_histogram_bytes", "sm_tiles_bytes", "sm_format_row_bytes",
    "sm_context_create", "sm_context_destroy", "sm_buffer_register", "sm_buffer_unregister",
    "sm_segment_begin", "sm_segment_commit", "sm_segment_abort", "sm_segment_error",
    "sm_segment_launches", "sm_segment_commit_timed",
    "sm_encode_route", "sm_encode_grouping", "sm_encode_route_gather", "sm_encode_shared_ffn",
    "sm_encode_gate_up", "sm_encode_down", "sm_encode_swiglu", "sm_encode_combine",
    "sm_encode_full_layer", "sm_encode_dequant", "sm_submit_dequant",
    "sm_submit_route", "sm_submit_grouping", "sm_submit_route_gather", "sm_submit_shared_ffn",
    "sm_submit_gate_up", "sm_submit_down", "sm_submit_swiglu", "sm_submit_combine",
    "sm_submit_full_layer", "sm_read_layer_status",
    "sm_build_chunk_schedule", "sm_chunk_count", "sm_chunk_range_at", "sm_encode_prefill_moe_chunks",
    "sm_submit_prefill_moe_chunks", "sm_submit_full_layer_fixed_scratch",
    "sm_gguf_open", "sm_gguf_close", "sm_gguf_tensor_count", "sm_gguf_find", "sm_gguf_expert_layout",
    "sm_gguf_load_experts", "sm_expert_slot_bytes", "sm_expert_store_create", "sm_expert_store_destroy",
    "sm_lease_set_create", "sm_lease_set_destroy", "sm_lease_set_retire_layer", "sm_lease_set_pins",
    "sm_expert_store_resolve_layer", "sm_expert_store_prefetch",
    "sm_encode_moe_plan", "sm_encode_quantize_q8_1", "sm_encode_moe_experts", "sm_encode_moe_down",
    "sm_encode_moe_swiglu", "sm_encode_moe_routed_ffn", "sm_encode_moe_combine", "sm_encode_moe_shared_ffn",
    "sm_encode_moe_decode_layer",
    "sm_submit_moe_decode_layer",
    "sm_synth_normal_f32", "sm_synth_normal_f16", "sm_synth_normal_bf16", "sm_quantize",
    "sm_synth_quantized",
)


class View(C.Structure):
    _fields_ = [("buffer", C.c_uint64), ("offset", C.c_uint64), ("length", C.c_uint64)]


NULL_VIEW = View(0, 0, 0)


class Shape(C.Structure):
    _fields_ = [("rows", C.c_uint32), ("hidden", C.c_uint32), ("n_experts", C.c_uint32),
                ("top_k", C.c_uint32), ("expert_ff", C.c_uint32), ("shared_ff", C.c_uint32)]


class RouteBuffers(C.Structure):
    _fields_ = [("logits", View), ("ids", View), ("weights", View)]


class GroupingBuffers(C.Structure):
    _fields_ = [("ids", View), ("mixed_h", View), ("histogram", View), ("plan", View),
                ("tiles", View), ("source_rows", View), ("destination_rows", View),
                ("gathered_rows", View), ("resident", View), ("layer", C.c_uint32)]


class RouteGatherBuffers(C.Structure):
    _fields_ = [("mixed_h", View), ("router_weights", View), ("logits", View),
                ("route_ids", View), ("route_weights", View), ("histogram", View),
                ("plan", View), ("tiles", View), ("source_rows", View),
                ("destination_rows", View), ("gathered_rows", View), ("router_bias", View),
                ("resident", View), ("layer", C.c_uint32)]


class ExpertWeights(C.Structure):
    _fields_ = [("addresses", C.POINTER(C.c_uint64)), ("n_layers", C.c_uint32), ("layer", C.c_uint32),
                ("address_snapshot", View), ("storage", C.POINTER(View)), ("n_storage", C.c_uint32),
                ("slot_arena", View), ("leases", C.c_void_p)]


class GateUpBuffers(C.Structure):
    _fields_ = [("weights", ExpertWeights), ("gathered_rows", View), ("plan", View),
                ("tiles", View), ("hidden", View), ("status", View)]


class DownBuffers(C.Structure):
    _fields_ = [("weights", ExpertWeights), ("hidden", View), ("plan", View), ("tiles", View),
                ("destinations", View), ("parts", View), ("status", View)]


class SharedBuffers(C.Structure):
    _fields_ = [("mixed_h", View), ("gate_weights", View), ("up_weights", View),
                ("down_weights", View), ("gate_vector", View), ("hidden", View),
                ("output", View), ("gate_logit", View)]


class SwiGLUBuffers(C.Structure):
    _fields_ = [("gate", View), ("up", View), ("output", View)]


class CombineBuffers(C.Structure):
    _fields_ = [("parts", View), ("weights", View), ("shared", View), ("gate", View),
                ("output", View)]


class LayerFormats(C.Structure):
    _fields_ = [("gate_up", C.c_int), ("down", C.c_int), ("shared", C.c_int)]


class LayerBuffers(C.Structure):
    _fields_ = [("route_gather", RouteGatherBuffers), ("shared", SharedBuffers),
                ("gate_up", GateUpBuffers), ("down", DownBuffers),
                ("combine", CombineBuffers)]


# ---- decode-side MoE (the Window MoE over T <= 8 rows) ----------------------------------------
DECODE_MAX_ROWS = 8
MOE_PLAN_BYTES = 1620
MOE_PLAN_MAX_ENTRIES = 80
Q8_1_BLOCK_BYTES = 36


class MoePlanBuffers(C.Structure):
    _fields_ = [("ids", View), ("resident", View), ("usage", View), ("plans", View), ("status", View),
                ("layer", C.c_uint32)]


class MoeExpertBuffers(C.Structure):
    _fields_ = [("weights", ExpertWeights), ("activations", View), ("plans", View), ("gate", View),
                ("up", View), ("status", View)]


class MoeDownBuffers(C.Structure):
    _fields_ = [("weights", ExpertWeights), ("activations", View), ("plans", View), ("parts", View),
                ("status", View)]


class MoeRoutedFFNBuffers(C.Structure):
    _fields_ = [("gate_up_weights", ExpertWeights), ("down_weights", ExpertWeights),
                ("input_activations", View), ("plans", View), ("gate", View), ("up", View),
                ("hidden", View), ("down_activations", View), ("parts", View), ("status", View)]


class MoeSharedFFNBuffers(C.Structure):
    _fields_ = [("shared", SharedBuffers), ("routed_parts", View), ("route_weights", View), ("output", View)]


class DecodeLayerBuffers(C.Structure):
    _fields_ = [("mixed_h", View), ("router_weights", View), ("router_bias", View), ("logits", View),
                ("route_ids", View), ("route_weights", View), ("resident", View), ("usage", View),
                ("plans", View), ("layer", C.c_uint32), ("input_activations", View),
                ("routed", MoeRoutedFFNBuffers), ("shared", SharedBuffers), ("output", View)]


def q8_1_bytes(rows: int, n: int) -> int:
    return rows * (n // 32) * Q8_1_BLOCK_BYTES


class GgufTensor(C.Structure):
    _fields_ = [("ggml_type", C.c_uint32), ("n_dims", C.c_uint32), ("ne", C.c_uint64 * 4), ("offset", C.c_uint64),
                ("bytes", C.c_uint64)]


GGUF_MAX_LAYERS = 64


class ExpertLayout(C.Structure):
    _fields_ = [("n_layers", C.c_uint32), ("n_experts", C.c_uint32), ("hidden", C.c_uint32), ("expert_ff", C.c_uint32),
                ("gate_up", C.c_int), ("down", C.c_int), ("total_bytes", C.c_uint64),
                ("offsets", (C.c_uint64 * 3) * GGUF_MAX_LAYERS)]


class StoreStats(C.Structure):
    _fields_ = [("hits", C.c_uint64), ("lookups", C.c_uint64), ("file_reads", C.c_uint64), ("file_bytes", C.c_uint64)]


class ChunkSchedule(C.Structure):
    """PrefillChunkSchedule (include/strata/metal/prefill.hpp:47-72)."""
    _fields_ = [("pos0", C.c_uint32), ("chunk_rows", C.c_uint32), ("token_count", C.c_uint64)]


class ChunkRange(C.Structure):
    """PrefillChunkRange (prefill.hpp:40-45)."""
    _fields_ = [("token_offset", C.c_uint64), ("pos0", C.c_uint32), ("rows", C.c_uint32)]


_lib: Optional[C.CDLL] = None


def library() -> C.CDLL:
    """Loads libstrata_moe.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() first")
    # The library and PyTorch must share one HIP runtime. PyTorch carries its own
    # libamdhip64 under the same soname; loading it first makes this library bind to it,
    # whereas loading the system runtime first leaves PyTorch without a usable device.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = C.CDLL(str(LIB_PATH))
    P, U32, U64, I = C.c_void_p, C.c_uint32, C.c_uint64, C.c_int
    sig = {
        "sm_abi_version": (U32, []),
        "sm_histogram_bytes": (U64, [C.POINTER(Shape)]),
        "sm_tiles_bytes": (U64, [C.POINTER(Shape)]),
        "sm_format_row_bytes": (U64, [I, U64]),
        "sm_context_create": (I, [I, C.POINTER(P)]),
        "sm_context_destroy": (None, [P]),
        "sm_buffer_register": (I, [P, P, U64, C.POINTER(U64)]),
        "sm_buffer_unregister": (I, [P, U64]),
        "sm_segment_begin": (I, [P, C.POINTER(P)]),
        "sm_segment_commit": (I, [P, P]),
        "sm_segment_commit_timed": (I, [P, P, C.POINTER(C.c_float), C.POINTER(C.c_char_p), U32,
                                        C.POINTER(U32)]),
        "sm_segment_abort": (None, [P]),
        "sm_segment_error": (C.c_char_p, [P]),
        "sm_segment_launches": (U32, [P]),
        "sm_encode_route": (I, [P, C.POINTER(Shape), I, C.POINTER(RouteBuffers)]),
        "sm_encode_grouping": (I, [P, C.POINTER(Shape), C.POINTER(GroupingBuffers)]),
        "sm_encode_route_gather": (I, [P, C.POINTER(Shape), C.POINTER(RouteGatherBuffers)]),
        "sm_encode_shared_ffn": (I, [P, C.POINTER(Shape), I, C.POINTER(SharedBuffers)]),
        "sm_encode_gate_up": (I, [P, C.POINTER(Shape), I, C.POINTER(GateUpBuffers)]),
        "sm_encode_down": (I, [P, C.POINTER(Shape), I, C.POINTER(DownBuffers)]),
        "sm_encode_swiglu": (I, [P, U32, U32, C.POINTER(SwiGLUBuffers)]),
        "sm_encode_combine": (I, [P, C.POINTER(Shape), C.POINTER(CombineBuffers)]),
        "sm_encode_full_layer": (I, [P, C.POINTER(Shape), C.POINTER(LayerFormats),
                                     C.POINTER(LayerBuffers)]),
        "sm_encode_dequant": (I, [P, I, U32, U32, View, View]),
        "sm_submit_full_layer": (I, [P, P, C.POINTER(Shape), C.POINTER(LayerFormats),
                                     C.POINTER(LayerBuffers), C.c_char_p, C.c_size_t]),
        "sm_read_layer_status": (I, [P, P, View, View, View, C.POINTER(U32), C.POINTER(U32),
                                     C.POINTER(U32)]),
        "sm_gguf_open": (I, [C.c_char_p, C.POINTER(P), C.c_char_p, C.c_size_t]),
        "sm_gguf_close": (None, [P]),
        "sm_gguf_tensor_count": (U64, [P]),
        "sm_gguf_find": (I, [P, C.c_char_p, C.POINTER(GgufTensor)]),
        "sm_gguf_expert_layout": (I, [P, U32, C.POINTER(ExpertLayout), C.c_char_p, C.c_size_t]),
        "sm_gguf_load_experts": (I, [P, P, P, C.POINTER(ExpertLayout), View, C.POINTER(C.c_uint64), U64, C.c_char_p,
                                     C.c_size_t]),
        "sm_expert_slot_bytes": (U64, [C.POINTER(ExpertLayout)]),
        "sm_expert_store_create": (I, [P, P, C.POINTER(ExpertLayout), View, U32, C.POINTER(P), C.c_char_p,
                                       C.c_size_t]),
        "sm_expert_store_destroy": (None, [P]),
        "sm_lease_set_create": (I, [P, C.POINTER(P)]),
        "sm_lease_set_destroy": (None, [P]),
        "sm_lease_set_retire_layer": (None, [P, U32]),
        "sm_lease_set_pins": (I, [P, U32, U64, U64]),
        "sm_expert_store_resolve_layer": (I, [P, P, U32, View, P, C.POINTER(C.c_uint64), U64, C.POINTER(StoreStats),
                                              C.c_char_p, C.c_size_t]),
        "sm_expert_store_prefetch": (I, [P, P, U32, C.POINTER(C.c_int32), U32, C.POINTER(StoreStats), C.c_char_p,
                                         C.c_size_t]),
        "sm_build_chunk_schedule": (I, [U32, U64, U32, C.POINTER(ChunkSchedule), C.c_char_p, C.c_size_t]),
        "sm_chunk_count": (U64, [C.POINTER(ChunkSchedule)]),
        "sm_chunk_range_at": (I, [C.POINTER(ChunkSchedule), U64, C.POINTER(ChunkRange)]),
        "sm_encode_prefill_moe_chunks": (I, [P, C.POINTER(ChunkSchedule), C.POINTER(Shape), C.POINTER(LayerFormats),
                                             View, View, C.POINTER(LayerBuffers)]),
        "sm_submit_full_layer_fixed_scratch": (I, [P, P, C.POINTER(Shape), C.POINTER(LayerFormats),
                                                   C.POINTER(LayerBuffers), C.c_char_p, C.c_size_t]),
        "sm_submit_prefill_moe_chunks": (I, [P, P, C.POINTER(ChunkSchedule), C.POINTER(Shape),
                                             C.POINTER(LayerFormats), View, View, C.POINTER(LayerBuffers),
                                             C.c_char_p, C.c_size_t]),
        "sm_encode_moe_plan": (I, [P, C.POINTER(Shape), C.POINTER(MoePlanBuffers)]),
        "sm_encode_quantize_q8_1": (I, [P, U32, U32, I, View, View]),
        "sm_encode_moe_experts": (I, [P, C.POINTER(Shape), I, C.POINTER(MoeExpertBuffers)]),
        "sm_encode_moe_down": (I, [P, C.POINTER(Shape), I, C.POINTER(MoeDownBuffers)]),
        "sm_encode_moe_swiglu": (I, [P, U32, U32, C.POINTER(SwiGLUBuffers)]),
        "sm_encode_moe_routed_ffn": (I, [P, C.POINTER(Shape), I, I, C.POINTER(MoeRoutedFFNBuffers)]),
        "sm_encode_moe_combine": (I, [P, C.POINTER(Shape), C.POINTER(CombineBuffers)]),
        "sm_encode_moe_shared_ffn": (I, [P, C.POINTER(Shape), I, C.POINTER(MoeSharedFFNBuffers)]),
        "sm_encode_moe_decode_layer": (I, [P, C.POINTER(Shape), C.POINTER(LayerFormats),
                                           C.POINTER(DecodeLayerBuffers)]),
        "sm_submit_moe_decode_layer": (I, [P, P, C.POINTER(Shape), C.POINTER(LayerFormats),
                                           C.POINTER(DecodeLayerBuffers), C.c_char_p, C.c_size_t]),
        "sm_synth_normal_f32": (None, [U64, U64, C.c_float, P, U64]),
        "sm_synth_normal_f16": (None, [U64, U64, C.c_float, P, U64]),
        "sm_synth_normal_bf16": (None, [U64, U64, C.c_float, P, U64]),
        "sm_quantize": (I, [I, P, U64, U64, P]),
        "sm_synth_quantized": (I, [I, U64, U64, C.c_float, U64, U64, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def row_bytes(fmt: int, values: int) -> int:
    return int(library().sm_format_row_bytes(fmt, values))


def histogram_bytes(shape: Shape) -> int:
    return int(library().sm_histogram_bytes(C.byref(shape)))


def tiles_bytes(shape: Shape) -> int:
    return int(library().sm_tiles_bytes(C.byref(shape)))


class Buffer:
    """A device allocation registered with a Context (the reference's BufferRef owner)."""

    def __init__(self, ctx: "Context", tensor, handle: int):
        self.ctx, self.tensor, self.handle = ctx, tensor, handle
        self.nbytes = tensor.numel() * tensor.element_size()

    @property
    def ptr(self) -> int:
        return self.tensor.data_ptr()

    def view(self, offset: int = 0, length: Optional[int] = None) -> View:
        return View(self.handle, offset, self.nbytes - offset if length is None else length)


class RawBuffer:
    """A registered raw device address range."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int, handle: int):
        self.ctx, self.ptr, self.nbytes, self.handle = ctx, ptr, nbytes, handle

    def view(self, offset: int = 0, length: Optional[int] = None) -> View:
        return View(self.handle, offset, self.nbytes - offset if length is None else length)


class Context:
    """Owns the allocation registry that backs the 'owned by this context' checks."""

    def __init__(self, device: int = 0):
        self.lib = library()
        h = C.c_void_p()
        st = self.lib.sm_context_create(device, C.byref(h))
        if st != 0:
            raise RuntimeError(f"sm_context_create failed: {STATUS_NAMES.get(st, st)}")
        self.handle = h
        self._buffers: list[Buffer] = []

    def register(self, tensor) -> Buffer:
        if not tensor.is_cuda or not tensor.is_contiguous():
            raise ValueError("register() needs a contiguous device tensor")
        hd = C.c_uint64()
        st = self.lib.sm_buffer_register(self.handle, C.c_void_p(tensor.data_ptr()),
                                         tensor.numel() * tensor.element_size(), C.byref(hd))
        if st != 0:
            raise RuntimeError(f"sm_buffer_register failed: {STATUS_NAMES.get(st, st)}")
        b = Buffer(self, tensor, hd.value)
        self._buffers.append(b)
        return b

    def register_ptr(self, ptr: int, nbytes: int) -> "RawBuffer":
        """Registers a raw device address range (no tensor); used by callers that manage
        their own allocations and by host-only validation tests."""
        hd = C.c_uint64()
        st = self.lib.sm_buffer_register(self.handle, C.c_void_p(ptr), nbytes, C.byref(hd))
        if st != 0:
            raise RuntimeError(f"sm_buffer_register failed: {STATUS_NAMES.get(st, st)}")
        return RawBuffer(self, ptr, nbytes, hd.value)

    def unregister(self, handle: int) -> int:
        return int(self.lib.sm_buffer_unregister(self.handle, handle))

    def segment(self) -> "Segment":
        return Segment(self)

    def read_layer_status(self, stream, plan: View, gate_up_status: View = NULL_VIEW,
                          down_status: View = NULL_VIEW):
        bad, gu, dn = C.c_uint32(), C.c_uint32(), C.c_uint32()
        st = self.lib.sm_read_layer_status(self.handle, C.c_void_p(stream), plan, gate_up_status,
                                           down_status, C.byref(bad), C.byref(gu), C.byref(dn))
        if st != 0:
            raise RuntimeError(f"sm_read_layer_status failed: {STATUS_NAMES.get(st, st)}")
        return bad.value, gu.value, dn.value

    def close(self):
        if self.handle:
            self.lib.sm_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class ExpertTable:
    """Host copy of the [layer][E][3] (gate, up, down) expert address table plus its storage;
    `layer` selects the row the stage reads (the reference's `layer` argument). Tiered mode adds
    the expert store's slot arena and the lease set that must pin its slot addresses."""

    def __init__(self, addresses: Sequence[int], snapshot: View, storage: Sequence[View], n_layers: int = 1,
                 layer: int = 0, slot_arena: View = None, leases: "LeaseSet" = None):
        n = len(addresses)
        self._addr = (C.c_uint64 * n)(*addresses)
        self._storage = (View * max(1, len(storage)))(*storage)
        self._leases = leases
        self.struct = ExpertWeights(C.cast(self._addr, C.POINTER(C.c_uint64)), n_layers, layer, snapshot,
                                    C.cast(self._storage, C.POINTER(View)), len(storage),
                                    slot_arena if slot_arena is not None else NULL_VIEW,
                                    leases.handle if leases is not None else None)


class ExpertStore:
    """Tiered residency: a slot arena in two halves over the experts of a GGUF file (sm_expert_store_*)."""

    def __init__(self, ctx: "Context", gguf: "GgufFile", layout: "ExpertLayout", arena: View, slots_per_half: int):
        self.lib, self.ctx, self.gguf = library(), ctx, gguf
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        self.status = self.lib.sm_expert_store_create(ctx.handle, gguf.handle, C.byref(layout), arena, slots_per_half,
                                                      C.byref(h), err, 512)
        self.error = err.value.decode()
        self.handle = h if self.status == 0 else None

    def resolve_layer(self, stream, layer: int, plan: View, leases: "LeaseSet", table):
        """resolve_layer_after_plan: (True, stats) or (False, message); `table` is a ctypes u64 array."""
        stats = StoreStats()
        err = C.create_string_buffer(512)
        st = self.lib.sm_expert_store_resolve_layer(self.handle, C.c_void_p(stream), layer, plan, leases.handle,
                                                    table, len(table), C.byref(stats), err, 512)
        if st != 0:
            return False, f"{STATUS_NAMES.get(st, st)}: {err.value.decode()}"
        return True, dict(hits=stats.hits, lookups=stats.lookups, file_reads=stats.file_reads,
                          file_bytes=stats.file_bytes)

    def prefetch(self, stream, layer: int, experts=None):
        """prefetch_layer (experts None) / prefetch_experts: (True, stats) or (False, message)."""
        stats = StoreStats()
        err = C.create_string_buffer(512)
        ids = None if experts is None else (C.c_int32 * len(experts))(*experts)
        n = 0 if experts is None else len(experts)
        st = self.lib.sm_expert_store_prefetch(self.handle, C.c_void_p(stream), layer, ids, n, C.byref(stats), err, 512)
        if st != 0:
            return False, f"{STATUS_NAMES.get(st, st)}: {err.value.decode()}"
        return True, dict(hits=stats.hits, lookups=stats.lookups, file_reads=stats.file_reads,
                          file_bytes=stats.file_bytes)

    def close(self):
        if self.handle:
            self.lib.sm_expert_store_destroy(self.handle)
            self.handle = None


class LeaseSet:
    """Slot pins of one command sequence (sm_lease_set_*); destroy only after its GPU work completed."""

    def __init__(self, store: ExpertStore):
        self.lib = library()
        h = C.c_void_p()
        assert self.lib.sm_lease_set_create(store.handle, C.byref(h)) == 0
        self.handle = h

    def pins(self, layer: int, address: int, nbytes: int) -> bool:
        return bool(self.lib.sm_lease_set_pins(self.handle, layer, address, nbytes))

    def retire_layer(self, layer: int):
        self.lib.sm_lease_set_retire_layer(self.handle, layer)

    def close(self):
        if self.handle:
            self.lib.sm_lease_set_destroy(self.handle)
            self.handle = None


class GgufFile:
    """A GGUF model file: its tensor directory and the routed-expert layout (sm_gguf_*)."""

    def __init__(self, path):
        self.lib = library()
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        self.status = self.lib.sm_gguf_open(str(path).encode(), C.byref(h), err, 512)
        self.error = err.value.decode()
        self.handle = h if self.status == 0 else None

    def __bool__(self):
        return self.handle is not None

    def tensor_count(self) -> int:
        return int(self.lib.sm_gguf_tensor_count(self.handle))

    def find(self, name: str):
        t = GgufTensor()
        if self.lib.sm_gguf_find(self.handle, name.encode(), C.byref(t)) != 0:
            return None
        return dict(type=t.ggml_type, ne=tuple(t.ne[: t.n_dims]), offset=t.offset, bytes=t.bytes)

    def expert_layout(self, n_layers: int):
        """(ExpertLayout, "") or (None, message)."""
        out = ExpertLayout()
        err = C.create_string_buffer(512)
        st = self.lib.sm_gguf_expert_layout(self.handle, n_layers, C.byref(out), err, 512)
        return (out, "") if st == 0 else (None, f"{STATUS_NAMES.get(st, st)}: {err.value.decode()}")

    def load_experts(self, ctx: "Context", stream, layout: ExpertLayout, storage: View):
        """Copies the expert tensors into `storage`; returns the [n_layers * E * 3] address list."""
        n = layout.n_layers * layout.n_experts * 3
        table = (C.c_uint64 * n)()
        err = C.create_string_buffer(512)
        st = self.lib.sm_gguf_load_experts(self.handle, ctx.handle, C.c_void_p(stream), C.byref(layout), storage,
                                           table, n, err, 512)
        if st != 0:
            raise RuntimeError(f"sm_gguf_load_experts: {STATUS_NAMES.get(st, st)}: {err.value.decode()}")
        return list(table)

    def close(self):
        if self.handle:
            self.lib.sm_gguf_close(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def build_chunk_schedule(pos0: int, token_count: int, chunk_rows: int):
    """build_prefill_chunk_schedule: (ChunkSchedule, "") or (None, error message)."""
    out = ChunkSchedule()
    err = C.create_string_buffer(256)
    st = library().sm_build_chunk_schedule(pos0, token_count, chunk_rows, C.byref(out), err, 256)
    return (out, "") if st == 0 else (None, err.value.decode())


def chunk_ranges(schedule: ChunkSchedule):
    """Every PrefillChunkRange of a schedule, in order (range_at over chunk_count)."""
    lib = library()
    out = []
    for i in range(int(lib.sm_chunk_count(C.byref(schedule)))):
        r = ChunkRange()
        assert lib.sm_chunk_range_at(C.byref(schedule), i, C.byref(r)) == 1
        out.append((int(r.token_offset), int(r.pos0), int(r.rows)))
    return out


class Segment:
    """An ordered, validated list of launches: commit() runs it, abort() discards it."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.lib = ctx.lib
        h = C.c_void_p()
        st = self.lib.sm_segment_begin(ctx.handle, C.byref(h))
        if st != 0:
            raise RuntimeError("sm_segment_begin failed")
        self.handle = h
        self._keep: list = []

    def _ret(self, st: int):
        if st == 0:
            return True, ""
        return False, self.error() or STATUS_NAMES.get(st, str(st))

    def error(self) -> str:
        msg = self.lib.sm_segment_error(self.handle)
        return msg.decode() if msg else ""

    @property
    def launches(self) -> int:
        return int(self.lib.sm_segment_launches(self.handle))

    # Reference coordinator names (namespace strata::metal):
    def encode_moe_route(self, shape: Shape, divide_weights: bool, b: RouteBuffers):
        return self._ret(self.lib.sm_encode_route(self.handle, C.byref(shape), int(divide_weights), C.byref(b)))

    def encode_prefill_moe_grouping(self, shape: Shape, b: GroupingBuffers):
        return self._ret(self.lib.sm_encode_grouping(self.handle, C.byref(shape), C.byref(b)))

    def encode_prefill_moe_full_mode_route_gather(self, shape: Shape, b: RouteGatherBuffers):
        return self._ret(self.lib.sm_encode_route_gather(self.handle, C.byref(shape), C.byref(b)))

    def encode_prefill_moe_shared_ffn(self, shape: Shape, fmt: int, b: SharedBuffers):
        return self._ret(self.lib.sm_encode_shared_ffn(self.handle, C.byref(shape), fmt, C.byref(b)))

    def encode_prefill_moe_gu(self, shape: Shape, fmt: int, b: GateUpBuffers, keep=None):
        self._keep.append(keep)
        return self._ret(self.lib.sm_encode_gate_up(self.handle, C.byref(shape), fmt, C.byref(b)))

    def encode_prefill_moe_down(self, shape: Shape, fmt: int, b: DownBuffers, keep=None):
        self._keep.append(keep)
        return self._ret(self.lib.sm_encode_down(self.handle, C.byref(shape), fmt, C.byref(b)))

    def encode_prefill_moe_swiglu(self, rows: int, width: int, b: SwiGLUBuffers):
        return self._ret(self.lib.sm_encode_swiglu(self.handle, rows, width, C.byref(b)))

    def encode_prefill_moe_combine(self, shape: Shape, b: CombineBuffers):
        return self._ret(self.lib.sm_encode_combine(self.handle, C.byref(shape), C.byref(b)))

    def encode_prefill_moe_full_mode_layer(self, shape: Shape, formats: LayerFormats,
                                           b: LayerBuffers, keep=None):
        self._keep.append(keep)
        return self._ret(self.lib.sm_encode_full_layer(self.handle, C.byref(shape), C.byref(formats),
                                                       C.byref(b)))

    def encode_prefill_moe_chunks(self, schedule: ChunkSchedule, shape: Shape, formats: LayerFormats, input: View,
                                  output: View, b: LayerBuffers, keep=None):
        """The layer over every range of a chunk schedule (Prefill::run's per-chunk MoE)."""
        self._keep.append((schedule, keep))
        return self._ret(self.lib.sm_encode_prefill_moe_chunks(self.handle, C.byref(schedule), C.byref(shape),
                                                               C.byref(formats), input, output, C.byref(b)))

    # Decode side (namespace strata::metal, moe_dispatch.hpp):
    def encode_moe_plan(self, shape: Shape, b: MoePlanBuffers):
        return self._ret(self.lib.sm_encode_moe_plan(self.handle, C.byref(shape), C.byref(b)))

    def encode_quantize_q8_1(self, rows: int, n: int, f32_input: bool, input: View, output: View):
        return self._ret(self.lib.sm_encode_quantize_q8_1(self.handle, rows, n, int(f32_input), input, output))

    def encode_moe_experts(self, shape: Shape, fmt: int, b: MoeExpertBuffers, keep=None):
        self._keep.append(keep)
        return self._ret(self.lib.sm_encode_moe_experts(self.handle, C.byref(shape), fmt, C.byref(b)))

    def encode_moe_down(self, shape: Shape, fmt: int, b: MoeDownBuffers, keep=None):
        self._keep.append(keep)
        return self._ret(self.lib.sm_encode_moe_down(self.handle, C.byref(shape), fmt, C.byref(b)))

    def encode_moe_swiglu(self, rows: int, width: int, b: SwiGLUBuffers):
        return self._ret(self.lib.sm_encode_moe_swiglu(self.handle, rows, width, C.byref(b)))

    def encode_moe_routed_ffn(self, shape: Shape, gate_up_fmt: int, down_fmt: int, b: MoeRoutedFFNBuffers,
                              keep=None):
        self._keep.append(keep)
        return self._ret(self.lib.sm_encode_moe_routed_ffn(self.handle, C.byref(shape), gate_up_fmt, down_fmt,
                                                           C.byref(b)))

    def encode_moe_combine(self, shape: Shape, b: CombineBuffers):
        return self._ret(self.lib.sm_encode_moe_combine(self.handle, C.byref(shape), C.byref(b)))

    def encode_moe_shared_ffn(self, shape: Shape, fmt: int, b: MoeSharedFFNBuffers):
        return self._ret(self.lib.sm_encode_moe_shared_ffn(self.handle, C.byref(shape), fmt, C.byref(b)))

    def encode_moe_decode_layer(self, shape: Shape, formats: LayerFormats, b: DecodeLayerBuffers, keep=None):
        self._keep.append(keep)
        return self._ret(self.lib.sm_encode_moe_decode_layer(self.handle, C.byref(shape), C.byref(formats),
                                                             C.byref(b)))

    def encode_prefill_dequant(self, fmt: int, n_out: int, k: int, weights: View, k_major_f16: View):
        return self._ret(self.lib.sm_encode_dequant(self.handle, fmt, n_out, k, weights, k_major_f16))

    def commit(self, stream=0) -> None:
        st = self.lib.sm_segment_commit(self.handle, C.c_void_p(stream))
        self.handle = None
        if st != 0:
            raise RuntimeError(f"sm_segment_commit failed: {STATUS_NAMES.get(st, st)}")

    def commit_timed(self, stream=0):
        """Commits and returns [(label, milliseconds)] of every launch, in order (waits for
        the stream)."""
        n = int(self.lib.sm_segment_launches(self.handle))
        ms = (C.c_float * max(n, 1))()
        labels = (C.c_char_p * max(n, 1))()
        got = C.c_uint32(0)
        st = self.lib.sm_segment_commit_timed(self.handle, C.c_void_p(stream), ms, labels, max(n, 1), C.byref(got))
        self.handle = None
        if st != 0:
            raise RuntimeError(f"sm_segment_commit_timed failed: {STATUS_NAMES.get(st, st)}")
        return [(labels[i].decode(), float(ms[i])) for i in range(got.value)]

    def abort(self) -> None:
        if self.handle:
            self.lib.sm_segment_abort(self.handle)
            self.handle = None


# ---- synthetic inputs (host numpy arrays) ------------------------------------------------

def synth_normal_f32(seed: int, stream: int, sigma: float, n: int):
    import numpy as np
    out = np.empty(n, np.float32)
    library().sm_synth_normal_f32(seed, stream, sigma, out.ctypes.data, n)
    return out


def synth_normal_f16(seed: int, stream: int, sigma: float, n: int):
    import numpy as np
    out = np.empty(n, np.uint16)
    library().sm_synth_normal_f16(seed, stream, sigma, out.ctypes.data, n)
    return out


def synth_normal_bf16(seed: int, stream: int, sigma: float, n: int):
    import numpy as np
    out = np.empty(n, np.uint16)
    library().sm_synth_normal_bf16(seed, stream, sigma, out.ctypes.data, n)
    return out


def quantize(fmt: int, x, rows: int, k: int):
    import numpy as np
    out = np.empty(rows * row_bytes(fmt, k), np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    st = library().sm_quantize(fmt, x.ctypes.data, rows, k, out.ctypes.data)
    if st != 0:
        raise RuntimeError(f"sm_quantize failed: {STATUS_NAMES.get(st, st)}")
    return out


def synth_quantized(fmt: int, seed: int, stream: int, sigma: float, rows: int, k: int):
    import numpy as np
    out = np.empty(rows * row_bytes(fmt, k), np.uint8)
    st = library().sm_synth_quantized(fmt, seed, stream, sigma, rows, k, out.ctypes.data)
    if st != 0:
        raise RuntimeError(f"sm_synth_quantized failed: {STATUS_NAMES.get(st, st)}")
    return out
