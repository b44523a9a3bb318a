"""Layer configurations, synthetic inputs, and a device workspace for one Prefill MoE layer.

`LayerWorkspace` allocates every caller-owned view of the full-mode layer on the GPU
(torch tensors registered with a `Context`), fills the inputs, and wires the
`LayerBuffers` struct the C ABI takes. It is what tests, the smoke check and the benchmark
drive; the coordinators themselves live in libstrata_moe.so.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import numpy as np

from . import moe

SEED_BASE = 0x5EED0000


@dataclasses.dataclass(frozen=True)
class LayerConfig:
    name: str
    rows: int
    hidden: int
    n_experts: int
    top_k: int
    expert_ff: int
    shared_ff: int
    gate_up_fmt: int
    down_fmt: int
    shared_fmt: int
    zipf_s: float = 0.0          # > 0: Zipf(s) logit bias over a seeded expert permutation
    chunks: int = 1              # sequential layer calls of `rows` tokens each
    seed: int = SEED_BASE

    def shape(self) -> moe.Shape:
        return moe.Shape(self.rows, self.hidden, self.n_experts, self.top_k, self.expert_ff,
                         self.shared_ff)

    @property
    def entries(self) -> int:
        return self.rows * self.top_k


# The five configurations of the benchmark specification (0-based, in its order).
CONFIGS = {
    0: LayerConfig("tiny", 64, 256, 16, 4, 128, 0, moe.Q8_0, moe.Q8_0, moe.F16, seed=SEED_BASE + 0),
    1: LayerConfig("route_group", 4096, 2048, 512, 10, 512, 0, moe.Q4_K, moe.Q8_0, moe.F16,
                   seed=SEED_BASE + 1),
    2: LayerConfig("full_layer", 2048, 2048, 512, 10, 512, 512, moe.Q4_K, moe.Q8_0, moe.F16,
                   seed=SEED_BASE + 2),
    3: LayerConfig("zipf_stress", 8192, 2048, 512, 10, 512, 512, moe.Q4_K, moe.Q8_0, moe.F16,
                   zipf_s=1.1, seed=SEED_BASE + 3),
    4: LayerConfig("low_bit", 4096, 4096, 256, 8, 1536, 1536, moe.Q2_K, moe.Q4_K, moe.BF16,
                   chunks=4, seed=SEED_BASE + 4),
}

# Synthetic-input streams (one SplitMix64 stream per tensor).
S_X, S_ROUTER, S_GATE, S_UP, S_DOWN, S_SH_GATE, S_SH_UP, S_SH_DOWN, S_GVEC, S_PERM = range(1, 11)


def zipf_bias(cfg: LayerConfig) -> Optional[np.ndarray]:
    """b[pi(r)] = -s * ln(r + 1) for a seeded permutation pi of the experts."""
    if cfg.zipf_s <= 0:
        return None
    rng = np.random.Generator(np.random.PCG64(cfg.seed ^ S_PERM))
    perm = rng.permutation(cfg.n_experts)
    b = np.empty(cfg.n_experts, np.float32)
    b[perm] = (-cfg.zipf_s * np.log(np.arange(cfg.n_experts, dtype=np.float64) + 1.0)).astype(np.float32)
    return b


@dataclasses.dataclass
class HostInputs:
    x: np.ndarray          # F16 bits [chunks*T, d]
    w_router: np.ndarray   # F32 [E, d]
    w_gate: np.ndarray     # bytes, E experts x I rows x row_bytes(d)
    w_up: np.ndarray
    w_down: np.ndarray     # bytes, E experts x d rows x row_bytes(I)
    sh_gate: Optional[np.ndarray]
    sh_up: Optional[np.ndarray]
    sh_down: Optional[np.ndarray]
    sh_gvec: Optional[np.ndarray]
    bias: Optional[np.ndarray]
    gu_stride: int
    dn_stride: int


def make_inputs(cfg: LayerConfig, with_experts: bool = True) -> HostInputs:
    """Seeded inputs: activations N(0,1) in F16; all weights N(0, 0.02) before quantization."""
    T, d, E, I, Is = cfg.rows * cfg.chunks, cfg.hidden, cfg.n_experts, cfg.expert_ff, cfg.shared_ff
    s = cfg.seed
    x = moe.synth_normal_f16(s, S_X, 1.0, T * d).reshape(T, d)
    w_router = moe.synth_normal_f32(s, S_ROUTER, 0.02, E * d).reshape(E, d)
    gu_stride = I * moe.row_bytes(cfg.gate_up_fmt, d)
    dn_stride = d * moe.row_bytes(cfg.down_fmt, I)
    if with_experts:
        w_gate = moe.synth_quantized(cfg.gate_up_fmt, s, S_GATE, 0.02, E * I, d)
        w_up = moe.synth_quantized(cfg.gate_up_fmt, s, S_UP, 0.02, E * I, d)
        w_down = moe.synth_quantized(cfg.down_fmt, s, S_DOWN, 0.02, E * d, I)
    else:
        w_gate = w_up = w_down = np.zeros(0, np.uint8)
    sh = [None] * 4
    if Is:
        gen = moe.synth_normal_bf16 if cfg.shared_fmt == moe.BF16 else moe.synth_normal_f16
        sh = [gen(s, S_SH_GATE, 0.02, Is * d), gen(s, S_SH_UP, 0.02, Is * d),
              gen(s, S_SH_DOWN, 0.02, d * Is), gen(s, S_GVEC, 0.02, d)]
    return HostInputs(x, w_router, w_gate, w_up, w_down, *sh, zipf_bias(cfg), gu_stride, dn_stride)


def _dev(a: np.ndarray, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


GUARD_BYTES = 4096
GUARD_FILL = 0xA5


class _Guarded:
    """Allocates output buffers; with `on`, each is the interior of a larger allocation with
    GUARD_BYTES of GUARD_FILL on both sides (only the interior is registered), so a write past
    either end shows up in bad()."""

    def __init__(self, dev, on: bool):
        self.dev, self.on, self.wholes = dev, on, []

    def empty(self, nbytes: int, dtype):
        import torch
        if not self.on:
            return torch.empty(nbytes // torch.tensor([], dtype=dtype).element_size(), dtype=dtype, device=self.dev)
        whole = torch.full((nbytes + 2 * GUARD_BYTES,), GUARD_FILL, dtype=torch.uint8, device=self.dev)
        self.wholes.append(whole)
        return whole[GUARD_BYTES:GUARD_BYTES + nbytes].view(dtype)

    def bad(self) -> list:
        """Indices (allocation order) of the buffers whose guard bytes changed."""
        out = []
        for i, whole in enumerate(self.wholes):
            if not (bool((whole[:GUARD_BYTES] == GUARD_FILL).all()) and bool((whole[-GUARD_BYTES:] == GUARD_FILL).all())):
                out.append(i)
        return out


class LayerWorkspace:
    """Device buffers and C-ABI structs of one layer call (one chunk of `cfg.rows` tokens).

    guard: every buffer the layer writes is the interior of a larger allocation with
    GUARD_BYTES of GUARD_FILL on both sides (the registered buffer is the interior only), so a
    write past either end of an output shows up in check_guards()."""

    def __init__(self, ctx: moe.Context, cfg: LayerConfig, inputs: HostInputs, device="cuda:0",
                 chunk: int = 0, guard: bool = True):
        import torch
        self.ctx, self.cfg, self.inputs = ctx, cfg, inputs
        T, d, E, K, I, Is = cfg.rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff, cfg.shared_ff
        N = T * K
        shape = cfg.shape()
        self.shape = shape
        dev = torch.device(device)
        self._guards = _Guarded(dev, guard)

        def empty(nbytes, dtype=torch.uint8):
            return self._guards.empty(nbytes, dtype)

        reg = ctx.register
        self.x = reg(_dev(inputs.x[chunk * T:(chunk + 1) * T].view(np.uint16).view(np.int16), dev))
        self.w_router = reg(_dev(inputs.w_router, dev))
        self.bias = reg(_dev(inputs.bias, dev)) if inputs.bias is not None else None
        self.logits = reg(empty(T * E * 4, torch.float32))
        self.ids = reg(empty(N * 4, torch.int32))
        self.route_w = reg(empty(N * 4, torch.float32))
        self.hist = reg(empty(moe.histogram_bytes(shape), torch.int32))
        self.plan = reg(empty(moe.PLAN_SLOT_BYTES, torch.int32))
        self.tiles = reg(empty(moe.tiles_bytes(shape), torch.int32))
        self.src = reg(empty(N * 4, torch.int32))
        self.dst = reg(empty(N * 4, torch.int32))
        self.xs = reg(empty(N * d * 2, torch.int16))
        self.hidden = reg(empty(N * I * 2, torch.int16))
        self.parts = reg(empty(N * d * 4, torch.float32))
        self.status = reg(empty(16, torch.int32).zero_())   # [gate/up, down, -, -]
        self.snap_gu = reg(empty(E * 3 * 8, torch.int64))
        self.snap_dn = reg(empty(E * 3 * 8, torch.int64))
        self.out = reg(empty(T * d * 4, torch.float32))
        self.has_experts = inputs.w_gate.size > 0
        if self.has_experts:
            self.w_gate = reg(_dev(inputs.w_gate, dev))
            self.w_up = reg(_dev(inputs.w_up, dev))
            self.w_down = reg(_dev(inputs.w_down, dev))
            addr = []
            for e in range(E):
                addr += [self.w_gate.ptr + e * inputs.gu_stride, self.w_up.ptr + e * inputs.gu_stride,
                         self.w_down.ptr + e * inputs.dn_stride]
            self.addresses = addr
            self.gu_table = moe.ExpertTable(addr, self.snap_gu.view(), [self.w_gate.view(), self.w_up.view()])
            self.dn_table = moe.ExpertTable(addr, self.snap_dn.view(), [self.w_down.view()])
        if Is:
            self.sh_gate = reg(_dev(inputs.sh_gate, dev))
            self.sh_up = reg(_dev(inputs.sh_up, dev))
            self.sh_down = reg(_dev(inputs.sh_down, dev))
            self.sh_gvec = reg(_dev(inputs.sh_gvec, dev))
            self.sh_hidden = reg(empty(T * Is * 2, torch.int16))
            self.sh_out = reg(empty(T * d * 4, torch.float32))
            self.sh_gl = reg(empty(T * 4, torch.float32))
        self.formats = moe.LayerFormats(cfg.gate_up_fmt, cfg.down_fmt, cfg.shared_fmt)

    def check_guards(self) -> list:
        """Indices (allocation order) of the output buffers whose guards were written."""
        return self._guards.bad()

    # ---- per-stage buffer structs ----
    def route_gather_buffers(self) -> moe.RouteGatherBuffers:
        return moe.RouteGatherBuffers(
            self.x.view(), self.w_router.view(), self.logits.view(), self.ids.view(),
            self.route_w.view(), self.hist.view(), self.plan.view(), self.tiles.view(),
            self.src.view(), self.dst.view(), self.xs.view(),
            self.bias.view() if self.bias is not None else moe.NULL_VIEW)

    def route_buffers(self) -> moe.RouteBuffers:
        return moe.RouteBuffers(self.logits.view(), self.ids.view(), self.route_w.view())

    def grouping_buffers(self) -> moe.GroupingBuffers:
        return moe.GroupingBuffers(self.ids.view(), self.x.view(), self.hist.view(), self.plan.view(),
                                   self.tiles.view(), self.src.view(), self.dst.view(), self.xs.view())

    def gate_up_buffers(self) -> moe.GateUpBuffers:
        return moe.GateUpBuffers(self.gu_table.struct, self.xs.view(), self.plan.view(), self.tiles.view(),
                                 self.hidden.view(), self.status.view(0, 4))

    def down_buffers(self) -> moe.DownBuffers:
        return moe.DownBuffers(self.dn_table.struct, self.hidden.view(), self.plan.view(), self.tiles.view(),
                               self.dst.view(), self.parts.view(), self.status.view(4, 4))

    def shared_buffers(self) -> moe.SharedBuffers:
        if not self.cfg.shared_ff:
            return moe.SharedBuffers()
        return moe.SharedBuffers(self.x.view(), self.sh_gate.view(), self.sh_up.view(), self.sh_down.view(),
                                 self.sh_gvec.view(), self.sh_hidden.view(), self.sh_out.view(),
                                 self.sh_gl.view())

    def combine_buffers(self) -> moe.CombineBuffers:
        sh = self.sh_out.view() if self.cfg.shared_ff else moe.NULL_VIEW
        gl = self.sh_gl.view() if self.cfg.shared_ff else moe.NULL_VIEW
        return moe.CombineBuffers(self.parts.view(), self.route_w.view(), sh, gl, self.out.view())

    def layer_buffers(self) -> moe.LayerBuffers:
        return moe.LayerBuffers(self.route_gather_buffers(), self.shared_buffers(), self.gate_up_buffers(),
                                self.down_buffers(), self.combine_buffers())

    def encode_layer(self, seg: moe.Segment):
        self._lb = self.layer_buffers()
        return seg.encode_prefill_moe_full_mode_layer(self.shape, self.formats, self._lb, keep=self)

    def run_layer(self, stream=0) -> None:
        seg = self.ctx.segment()
        ok, err = self.encode_layer(seg)
        if not ok:
            seg.abort()
            raise RuntimeError(err)
        seg.commit(stream)

    def read_status(self, stream=0):
        return self.ctx.read_layer_status(stream, self.plan.view(), self.status.view(0, 4),
                                          self.status.view(4, 4))


class PromptWorkspace:
    """The chunk driver over a whole prompt: the prompt's input rows (F16 [chunks*T, d]) and output
    rows (F32), and one chunk's scratch (a LayerWorkspace of `cfg.rows` rows) that every chunk
    reuses. One segment runs every chunk (sm_encode_prefill_moe_chunks)."""

    def __init__(self, ctx: moe.Context, cfg: LayerConfig, inputs: HostInputs, device="cuda:0", guard: bool = True):
        import torch
        self.ctx, self.cfg = ctx, cfg
        self.chunk = LayerWorkspace(ctx, cfg, inputs, device, chunk=0, guard=guard)
        n = cfg.rows * cfg.chunks
        dev = torch.device(device)
        self._guards = _Guarded(dev, guard)
        self.x_all = ctx.register(_dev(inputs.x.view(np.uint16).view(np.int16), dev))
        self.out_all = ctx.register(self._guards.empty(n * cfg.hidden * 4, torch.float32))
        sched, err = moe.build_chunk_schedule(0, n, cfg.rows)
        if sched is None:
            raise ValueError(err)
        self.schedule = sched

    def encode(self, seg: moe.Segment):
        ws = self.chunk
        self._lb = ws.layer_buffers()
        return seg.encode_prefill_moe_chunks(self.schedule, ws.shape, ws.formats, self.x_all.view(),
                                             self.out_all.view(), self._lb, keep=self)

    def run(self, stream=0) -> None:
        seg = self.ctx.segment()
        ok, err = self.encode(seg)
        if not ok:
            seg.abort()
            raise RuntimeError(err)
        seg.commit(stream)

    def read_status(self, stream=0):
        return self.chunk.read_status(stream)

    def check_guards(self) -> list:
        """The chunk scratch's written guards, then "out_all" if the prompt output's were."""
        return self.chunk.check_guards() + (["out_all"] if self._guards.bad() else [])


# Decode-side layers (the Window MoE, T <= 8 rows). The first two are the reference model's own
# widths (d 2560, 512 experts top-10, expert and shared width 640) and share one seed, so their
# weights are the same and T=1's input is T=8's first row; the last two are the prefill
# configurations 2 and 4 at decode row counts (the step after prefill on the same layer).
DECODE_CONFIGS = {
    "window_t1": LayerConfig("window_t1", 1, 2560, 512, 10, 640, 640, moe.Q4_K, moe.Q8_0, moe.F16,
                             seed=SEED_BASE + 28),
    "window_t8": LayerConfig("window_t8", 8, 2560, 512, 10, 640, 640, moe.Q4_K, moe.Q8_0, moe.F16,
                             seed=SEED_BASE + 28),
    "full_layer_t8": LayerConfig("full_layer_t8", 8, 2048, 512, 10, 512, 512, moe.Q4_K, moe.Q8_0, moe.F16,
                                 seed=SEED_BASE + 32),
    "low_bit_t4": LayerConfig("low_bit_t4", 4, 4096, 256, 8, 1536, 1536, moe.Q2_K, moe.Q4_K, moe.BF16,
                              seed=SEED_BASE + 44),
}


class DecodeWorkspace:
    """Device buffers and C-ABI structs of one decode layer call (T <= 8 rows): the route, the
    MoePlan (one layer), the Q8_1 input, the routed FFN's scratch, the shared expert and the
    output (sm_encode_moe_decode_layer)."""

    def __init__(self, ctx: moe.Context, cfg: LayerConfig, inputs: HostInputs, device="cuda:0", guard: bool = True):
        import torch
        self.ctx, self.cfg, self.inputs = ctx, cfg, inputs
        T, d, E, K, I, Is = cfg.rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff, cfg.shared_ff
        N = T * K
        self.shape = cfg.shape()
        dev = torch.device(device)
        self._guards = _Guarded(dev, guard)

        def empty(nbytes, dtype=torch.uint8):
            return self._guards.empty(nbytes, dtype)

        reg = ctx.register
        self.x = reg(_dev(inputs.x[:T].view(np.uint16).view(np.int16), dev))
        self.w_router = reg(_dev(inputs.w_router, dev))
        self.bias = reg(_dev(inputs.bias, dev)) if inputs.bias is not None else None
        self.logits = reg(empty(T * E * 4, torch.float32))
        self.ids = reg(empty(N * 4, torch.int32))
        self.route_w = reg(empty(N * 4, torch.float32))
        self.plans = reg(empty(moe.MOE_PLAN_BYTES, torch.int32))
        self.xq = reg(empty(moe.q8_1_bytes(T, d), torch.int32))
        self.gate = reg(empty(N * I * 4, torch.float32))
        self.up = reg(empty(N * I * 4, torch.float32))
        self.hidden = reg(empty(N * I * 4, torch.float32))
        self.hq = reg(empty(moe.q8_1_bytes(N, I), torch.int32))
        self.parts = reg(empty(N * d * 4, torch.float32))
        self.status = reg(empty(4, torch.int32).zero_())
        self.snap_gu = reg(empty(E * 3 * 8, torch.int64))
        self.snap_dn = reg(empty(E * 3 * 8, torch.int64))
        self.out = reg(empty(T * d * 4, torch.float32))
        self.w_gate = reg(_dev(inputs.w_gate, dev))
        self.w_up = reg(_dev(inputs.w_up, dev))
        self.w_down = reg(_dev(inputs.w_down, dev))
        addr = []
        for e in range(E):
            addr += [self.w_gate.ptr + e * inputs.gu_stride, self.w_up.ptr + e * inputs.gu_stride,
                     self.w_down.ptr + e * inputs.dn_stride]
        self.addresses = addr
        self.gu_table = moe.ExpertTable(addr, self.snap_gu.view(), [self.w_gate.view(), self.w_up.view()])
        self.dn_table = moe.ExpertTable(addr, self.snap_dn.view(), [self.w_down.view()])
        if Is:
            self.sh_gate = reg(_dev(inputs.sh_gate, dev))
            self.sh_up = reg(_dev(inputs.sh_up, dev))
            self.sh_down = reg(_dev(inputs.sh_down, dev))
            self.sh_gvec = reg(_dev(inputs.sh_gvec, dev))
            self.sh_hidden = reg(empty(T * Is * 4, torch.float32))
            self.sh_out = reg(empty(T * d * 4, torch.float32))
            self.sh_gl = reg(empty(T * 4, torch.float32))
        self.formats = moe.LayerFormats(cfg.gate_up_fmt, cfg.down_fmt, cfg.shared_fmt)

    def routed_buffers(self) -> moe.MoeRoutedFFNBuffers:
        return moe.MoeRoutedFFNBuffers(self.gu_table.struct, self.dn_table.struct, self.xq.view(), self.plans.view(),
                                       self.gate.view(), self.up.view(), self.hidden.view(), self.hq.view(),
                                       self.parts.view(), self.status.view())

    def shared_buffers(self) -> moe.SharedBuffers:
        if not self.cfg.shared_ff:
            return moe.SharedBuffers()
        return moe.SharedBuffers(self.x.view(), self.sh_gate.view(), self.sh_up.view(), self.sh_down.view(),
                                 self.sh_gvec.view(), self.sh_hidden.view(), self.sh_out.view(), self.sh_gl.view())

    def layer_buffers(self, resident: moe.View = moe.NULL_VIEW, usage: moe.View = moe.NULL_VIEW):
        return moe.DecodeLayerBuffers(
            self.x.view(), self.w_router.view(), self.bias.view() if self.bias is not None else moe.NULL_VIEW,
            self.logits.view(), self.ids.view(), self.route_w.view(), resident, usage, self.plans.view(), 0,
            self.xq.view(), self.routed_buffers(), self.shared_buffers(), self.out.view())

    def encode(self, seg: moe.Segment, **kw):
        self._lb = self.layer_buffers(**kw)
        return seg.encode_moe_decode_layer(self.shape, self.formats, self._lb, keep=self)

    def run(self, stream=0, **kw) -> None:
        seg = self.ctx.segment()
        ok, err = self.encode(seg, **kw)
        if not ok:
            seg.abort()
            raise RuntimeError(err)
        seg.commit(stream)

    def read_status(self) -> int:
        return int(self.status.tensor.cpu().item())

    def check_guards(self) -> list:
        """Indices (allocation order) of the output buffers whose guards were written."""
        return self._guards.bad()


def decode_weight_bytes(cfg: LayerConfig, n_active: int) -> int:
    """Weight bytes a decode layer streams: the active experts' gate, up and down matrices, the
    shared expert, and the router."""
    d, I, Is, E = cfg.hidden, cfg.expert_ff, cfg.shared_ff, cfg.n_experts
    routed = n_active * (2 * I * moe.row_bytes(cfg.gate_up_fmt, d) + d * moe.row_bytes(cfg.down_fmt, I))
    shared = 3 * Is * d * 2 + d * 2 if Is else 0
    return routed + shared + E * d * 4


def layer_flops(cfg: LayerConfig) -> float:
    """Algorithmic FLOPs of one layer call (router, gate/up, down, shared)."""
    T, d, E, K, I, Is = cfg.rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff, cfg.shared_ff
    N = T * K
    return 2.0 * T * E * d + 2.0 * N * 2 * I * d + 2.0 * N * d * I + (2.0 * T * 3 * Is * d + 2.0 * T * d if Is else 0.0)


def ceil_div(a: int, b: int) -> int:
    return -(-a // b)


__all__ = ["LayerConfig", "CONFIGS", "DECODE_CONFIGS", "HostInputs", "make_inputs", "LayerWorkspace",
           "PromptWorkspace", "DecodeWorkspace", "decode_weight_bytes", "layer_flops", "zipf_bias"]
