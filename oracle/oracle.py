"""ctypes wrapper of the CPU oracle (liboracle_moe.so) and the reference twins (_ref/).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, never by the product package.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle_moe.so"
NATIVE_LIB = HERE / "_native" / "liboracle_moe.so"
REF_LIB = HERE / "_ref" / "libref_twins.so"
_lib = None
_native = None
_ref = None
P = C.c_void_p


def build(reference_root: str = "/root/reference") -> None:
    """Builds liboracle_moe.so, and oracle/_ref when the reference checkout is present."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    if Path(reference_root, "tests/metal/oracles").is_dir():
        subprocess.run([str(HERE / "build_ref.sh"), reference_root], check=True)


def build_native() -> bool:
    """Builds oracle/_native/liboracle_moe.so for this host's instruction set (-march=native),
    where the CPU baseline is timed; False if the build fails (the portable library is used)."""
    res = subprocess.run(["make", "-s", "-C", str(HERE), "native"], capture_output=True, text=True)
    return res.returncode == 0 and NATIVE_LIB.exists()


def lib(native: bool = False) -> C.CDLL:
    global _lib, _native
    if native:
        if _native is None:
            _native = _bind(C.CDLL(str(NATIVE_LIB)))
        return _native
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = _bind(C.CDLL(str(LIB)))
    return _lib


def _bind(L: C.CDLL) -> C.CDLL:
    """Declares the oracle library's signatures."""
    U32, U64, I, F = C.c_uint32, C.c_uint64, C.c_int, C.c_float
    sig = {
        "or_exp": (F, [F]), "or_f32_to_f16": (C.c_uint16, [F]), "or_f16_to_f32": (F, [C.c_uint16]),
        "or_half_sat": (C.c_uint16, [F]), "or_silu": (F, [F]), "or_sigmoid": (F, [F]),
        "or_row_bytes": (U64, [I, U64]), "or_dequant": (I, [I, P, U64, P]),
        "or_route": (I, [P, U32, U32, U32, I, P, P]),
        "or_grouping": (I, [P, U32, U32, U32, P, P, P, P, P, P]),
        "or_gather": (I, [P, U32, U32, P, U32, P]),
        "or_router_ref": (I, [P, P, U32, U32, U32, P]),
        "or_gate_up_ref": (I, [I, P, U32, U32, P, P, P, U64, P, U32, P, P, P]),
        "or_down_ref": (I, [I, P, U32, U32, P, P, U64, P, U32, P]),
        "or_shared_ref": (I, [I, P, U32, U32, P, P, P, P, P, U32, P, P, P]),
        "or_swiglu": (I, [P, P, U64, P]),
        "or_combine": (I, [P, P, P, P, U32, U32, U32, P]),
        "or_moe_plan": (I, [P, U32, U32, U32, P, P, P]),
        "or_quantize_q8_1": (I, [P, U32, U32, P]),
        "or_q81_matvec": (I, [I, P, U32, U32, P, U32, P, P]),
        "or_swiglu_f32": (I, [P, P, U64, P]),
        "or_combine_decode": (I, [P, P, P, P, U32, U32, U32, P]),
        "or_cpu_layer": (I, [U32, U32, U32, U32, U32, U32, I, I, I, P, P, P, P, U64, P, U64,
                             P, P, P, P, I, P, P]),
    }
    for n, (r, a) in sig.items():
        f = getattr(L, n)
        f.restype, f.argtypes = r, a
    return L


def ref() -> C.CDLL | None:
    """The reference's own CPU twins, if oracle/_ref was built (None otherwise)."""
    global _ref
    if _ref is None and REF_LIB.exists():
        R = C.CDLL(str(REF_LIB))
        R.ref_route.argtypes = [P, C.c_uint32, C.c_uint32, C.c_int, P, P]
        R.ref_combine.argtypes = [P, P, P, P, C.c_uint32, P]
        R.ref_swiglu.argtypes = [P, P, C.c_uint64, P]
        R.ref_q8_1.argtypes = [P, C.c_uint32, C.c_uint32, P]
        R.ref_q80_mv.argtypes = [P, P, C.c_uint32, C.c_uint32, C.c_uint32, P]
        R.ref_q4k_mv.argtypes = [P, P, C.c_uint32, C.c_uint32, C.c_uint32, P]
        _ref = R
    return _ref


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


def route(logits: np.ndarray, top_k: int, divide: bool = True):
    T, E = logits.shape
    logits = np.ascontiguousarray(logits, np.float32)
    ids = np.empty((T, top_k), np.int32)
    w = np.empty((T, top_k), np.float32)
    assert lib().or_route(_p(logits), T, E, top_k, int(divide), _p(ids), _p(w)) == 0
    return ids, w


def grouping(ids: np.ndarray, n_experts: int):
    T, K = ids.shape
    N = T * K
    ids = np.ascontiguousarray(ids, np.int32)
    hist = np.zeros(((N + 255) // 256) * n_experts, np.uint32)
    plan = np.zeros(6400, np.uint8)
    tiles = np.zeros(2 * ((N + 63) // 64 + n_experts), np.uint32)
    nt = C.c_uint32()
    src = np.empty(N, np.int32)
    dst = np.empty(N, np.int32)
    assert lib().or_grouping(_p(ids), T, K, n_experts, _p(hist), _p(plan), _p(tiles), C.byref(nt),
                             _p(src), _p(dst)) == 0
    return dict(hist=hist.reshape(-1, n_experts), plan=plan, tiles=tiles.reshape(-1, 2)[: nt.value],
                n_tiles=nt.value, src=src, dst=dst)


def plan_fields(plan: np.ndarray) -> dict:
    w = plan[:6180].view(np.int32)
    return dict(n_groups=int(w[0]), n_entries=int(w[1]), n_miss=int(w[2]), skip=int(w[3]),
                n_tiles=int(w[4]), bad=int(w[5]), grp_e=w[8:520], grp_res=w[520:1032],
                grp_start=w[1032:1545])


def gather(x: np.ndarray, src: np.ndarray, n_valid: int):
    T, d = x.shape
    x = np.ascontiguousarray(x, np.uint16)
    xs = np.zeros((n_valid, d), np.uint16)
    assert lib().or_gather(_p(x), T, d, _p(np.ascontiguousarray(src, np.int32)), n_valid, _p(xs)) == 0
    return xs


def dequant(fmt: int, blocks: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, np.uint16)
    raw = np.ascontiguousarray(blocks).view(np.uint8)
    assert raw.size >= lib().or_row_bytes(fmt, n), "block buffer too small"
    assert lib().or_dequant(fmt, _p(raw), n, _p(out)) == 0
    return out


def router_ref(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    T, d = x.shape
    E = w.shape[0]
    out = np.empty((T, E), np.float64)
    assert lib().or_router_ref(_p(np.ascontiguousarray(x, np.uint16)), _p(np.ascontiguousarray(w, np.float32)),
                               T, d, E, _p(out)) == 0
    return out


def gate_up_ref(fmt, xs, d, I, plan, w_gate, w_up, stride, entries):
    entries = np.ascontiguousarray(entries, np.uint32)
    n = entries.size
    g = np.empty((n, I), np.float64)
    u = np.empty((n, I), np.float64)
    eh = np.empty((n, I), np.uint16)
    r = lib().or_gate_up_ref(fmt, _p(np.ascontiguousarray(xs, np.uint16)), d, I, _p(plan), _p(w_gate), _p(w_up),
                             stride, _p(entries), n, _p(g), _p(u), _p(eh))
    assert r == 0, r
    return g, u, eh


def down_ref(fmt, eh, d, I, plan, w_down, stride, entries):
    entries = np.ascontiguousarray(entries, np.uint32)
    n = entries.size
    out = np.empty((n, d), np.float64)
    r = lib().or_down_ref(fmt, _p(np.ascontiguousarray(eh, np.uint16)), d, I, _p(plan), _p(w_down), stride,
                          _p(entries), n, _p(out))
    assert r == 0, r
    return out


def shared_ref(fmt, x, d, Is, wg, wu, wd, gv, tokens):
    tokens = np.ascontiguousarray(tokens, np.uint32)
    n = tokens.size
    hidden = np.empty((n, Is), np.uint16)
    out = np.empty((n, d), np.float64)
    gl = np.empty(n, np.float64)
    r = lib().or_shared_ref(fmt, _p(np.ascontiguousarray(x, np.uint16)), d, Is, _p(wg), _p(wu), _p(wd), _p(gv),
                            _p(tokens), n, _p(hidden), _p(out), _p(gl))
    assert r == 0, r
    return hidden, out, gl


def swiglu(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate = np.ascontiguousarray(gate, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    out = np.empty(gate.shape, np.uint16)
    assert lib().or_swiglu(_p(gate), _p(up), gate.size, _p(out)) == 0
    return out


def combine(parts, weights, shared, gl, rows, top_k, d):
    out = np.empty((rows, d), np.float32)
    assert lib().or_combine(_p(np.ascontiguousarray(parts, np.float32)), _p(np.ascontiguousarray(weights, np.float32)),
                            _p(None if shared is None else np.ascontiguousarray(shared, np.float32)),
                            _p(None if gl is None else np.ascontiguousarray(gl, np.float32)),
                            rows, top_k, d, _p(out)) == 0
    return out


# ---- decode-side MoE ----------------------------------------------------------------------
PLAN_DTYPE = np.dtype([("n_groups", "<u4"), ("n_entries", "<u4"), ("n_miss", "<u4"), ("skip", "<u4"),
                       ("grp_e", "<i4", 80), ("grp_res", "<i4", 80), ("grp_start", "<i4", 81),
                       ("ent_tok", "<i4", 80), ("ent_dst", "<i4", 80)])
assert PLAN_DTYPE.itemsize == 1620


def moe_plan(ids: np.ndarray, n_experts: int, resident: np.ndarray | None = None,
             usage: np.ndarray | None = None):
    """MoePlan bytes (1620) and the return code (0, or 1 for an out-of-range id)."""
    rows, top_k = ids.shape
    ids = np.ascontiguousarray(ids, np.int32)
    res = None if resident is None else np.ascontiguousarray(resident, np.int32)
    plan = np.zeros(1620, np.uint8)
    rc = lib().or_moe_plan(_p(ids), rows, top_k, n_experts, _p(res), _p(usage), _p(plan))
    assert rc in (0, 1)
    return plan, rc


def quantize_q8_1(x: np.ndarray) -> np.ndarray:
    """[rows, n] F32 values (F16 inputs are widened first) -> [rows, n/32 * 36] Q8_1 bytes."""
    x = np.ascontiguousarray(np.asarray(x).astype(np.float32))
    rows, n = x.shape
    out = np.empty((rows, n // 32 * 36), np.uint8)
    assert lib().or_quantize_q8_1(_p(x), rows, n, _p(out)) == 0
    return out


def q81_matvec(fmt: int, w: np.ndarray, n_out: int, k: int, act: np.ndarray):
    """FP64 [nc, n_out] values and magnitudes of n_out weight rows against nc Q8_1 rows."""
    w = np.ascontiguousarray(w, np.uint8)
    act = np.ascontiguousarray(act, np.uint8)
    nc = act.size // (k // 32 * 36)
    out = np.empty((nc, n_out), np.float64)
    mag = np.empty((nc, n_out), np.float64)
    assert lib().or_q81_matvec(fmt, _p(w), n_out, k, _p(act), nc, _p(out), _p(mag)) == 0
    return out, mag


def swiglu_f32(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    gate = np.ascontiguousarray(gate, np.float32)
    up = np.ascontiguousarray(up, np.float32)
    out = np.empty(gate.shape, np.float32)
    assert lib().or_swiglu_f32(_p(gate), _p(up), gate.size, _p(out)) == 0
    return out


def combine_decode(parts, weights, shared, gl, rows, top_k, d):
    out = np.empty((rows, d), np.float32)
    assert lib().or_combine_decode(
        _p(np.ascontiguousarray(parts, np.float32)), _p(np.ascontiguousarray(weights, np.float32)),
        _p(None if shared is None else np.ascontiguousarray(shared, np.float32)),
        _p(None if gl is None else np.ascontiguousarray(gl, np.float32)), rows, top_k, d, _p(out)) == 0
    return out


def cpu_layer(cfg, inputs, n_threads: int = 0, chunk: int = 0, native: bool = False):
    """Times the CPU restatement of one layer call; returns (out, stage_us, threads)."""
    T, d = cfg.rows, cfg.hidden
    x = np.ascontiguousarray(inputs.x[chunk * T:(chunk + 1) * T])
    out = np.empty((T, d), np.float32)
    st = np.zeros(7, np.float64)
    Is = cfg.shared_ff
    th = lib(native).or_cpu_layer(T, d, cfg.n_experts, cfg.top_k, cfg.expert_ff, Is, cfg.gate_up_fmt, cfg.down_fmt,
                            cfg.shared_fmt, _p(x), _p(inputs.w_router), _p(inputs.w_gate), _p(inputs.w_up),
                            inputs.gu_stride, _p(inputs.w_down), inputs.dn_stride,
                            _p(inputs.sh_gate) if Is else None, _p(inputs.sh_up) if Is else None,
                            _p(inputs.sh_down) if Is else None, _p(inputs.sh_gvec) if Is else None,
                            n_threads, _p(out), _p(st))
    assert th > 0, th
    return out, st, th


def sigmoid64(x):
    return 1.0 / (1.0 + np.exp(-np.asarray(x, np.float64)))


def layer_ref(cfg, inp, ids, weights, tokens=None, chunk: int = 0):
    """FP64 restatement of steps 3-13 of one layer call from given routing (ids, weights).

    Expert products are FP64 sums over the F16-rounded dequantized weights; the SwiGLU
    outputs are rounded to F16 (half_sat) as the layer stores them. Returns (out [n, d]
    float64 for `tokens`, grouping dict)."""
    T, d, E, K, I, Is = cfg.rows, cfg.hidden, cfg.n_experts, cfg.top_k, cfg.expert_ff, cfg.shared_ff
    N = T * K
    x = np.ascontiguousarray(inp.x[chunk * T:(chunk + 1) * T])
    g = grouping(ids, E)
    plan = g["plan"]
    pf = plan_fields(plan)
    n_valid = N - pf["bad"]
    xs = gather(x, g["src"], n_valid)
    if tokens is None:
        tokens = np.arange(T)
    tokens = np.asarray(tokens, np.int64)
    inv = np.full(N, -1, np.int64)
    inv[g["dst"][:n_valid]] = np.arange(n_valid)
    routes = (tokens[:, None] * K + np.arange(K)[None, :]).ravel()
    pos = inv[routes]
    assert (pos >= 0).all()
    xs_full = np.zeros((N, d), np.uint16)
    xs_full[:n_valid] = xs
    _, _, eh = gate_up_ref(cfg.gate_up_fmt, xs_full, d, I, plan, inp.w_gate, inp.w_up, inp.gu_stride, pos)
    eh_full = np.zeros((N, I), np.uint16)
    eh_full[pos] = eh
    parts = down_ref(cfg.down_fmt, eh_full, d, I, plan, inp.w_down, inp.dn_stride, pos).reshape(len(tokens), K, d)
    w = np.asarray(weights, np.float64).reshape(T, K)[tokens]
    out = np.einsum("tk,tkd->td", w, parts)
    if Is:
        _, sh, gl = shared_ref(cfg.shared_fmt, x, d, Is, inp.sh_gate, inp.sh_up, inp.sh_down, inp.sh_gvec, tokens)
        out = out + sh * sigmoid64(gl)[:, None]
    return out, g
