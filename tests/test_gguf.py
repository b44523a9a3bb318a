"""Model files: GGUF expert tensors into device storage and the [layer][E][3] address table.

CPU: the GGUF directory parse and the expert layout against what the writer recorded, and the
rejections (bad magic and version, truncated file, data outside the file or off the alignment,
duplicate tensors, a missing or misshapen expert tensor, gate/up of different types, a
non-block expert type), following the reference's layout checks (src/metal/engine/window.cpp:
34-56,128-270). GPU: the experts loaded from a file drive a full layer whose output equals, bit
for bit, the same layer on weights uploaded directly.
"""
import numpy as np
import pytest

import gguf_util as gg


def _write(tmp_path, moe, name="m.gguf", **kw):
    over = {k: kw.pop(k) for k in list(kw) if k in ("tensors_fn",)}
    tensors, experts = gg.expert_model(moe, **{k: v for k, v in kw.items() if k in ("n_layers", "E", "d", "I", "gu", "dn")})
    if "tensors_fn" in over:
        tensors = over["tensors_fn"](tensors)
    write_kw = {k: v for k, v in kw.items() if k in ("alignment", "version", "misalign", "truncate", "magic")}
    p = tmp_path / name
    gg.write_gguf(p, tensors, gg.KV, **write_kw)
    return p, tensors, experts


def test_directory_and_layout(tmp_path, moe):
    p, tensors, _ = _write(tmp_path, moe, alignment=64)
    f = moe.GgufFile(p)
    assert f, f.error
    assert f.tensor_count() == len(tensors)
    t = f.find("blk.1.ffn_down_exps.weight")
    assert t["type"] == 8 and t["ne"] == (128, 256, 16) and t["bytes"] == 16 * 256 * 4 * 34
    assert t["offset"] % 64 == 0
    with open(p, "rb") as fh:
        fh.seek(t["offset"])
        assert fh.read(t["bytes"]) == dict((n, d) for n, _, _, d in tensors)["blk.1.ffn_down_exps.weight"]
    assert f.find("no.such.tensor") is None
    assert f.find("output.weight")["bytes"] == 4 * 210  # Q6_K: 210 bytes per 256 values
    L, err = f.expert_layout(2)
    assert L is not None, err
    assert (L.n_layers, L.n_experts, L.hidden, L.expert_ff, L.gate_up, L.down) == (2, 16, 256, 128, moe.Q4_K, moe.Q8_0)
    offs = [L.offsets[l][r] for l in range(2) for r in range(3)]
    assert offs[0] == 0 and all(o % 256 == 0 for o in offs) and offs == sorted(offs)
    sizes = [16 * 128 * 144, 16 * 128 * 144, 16 * 256 * 136]
    assert L.total_bytes == offs[-1] + -(-sizes[2] // 256) * 256
    L1, err = f.expert_layout(3)
    assert L1 is None and "blk.2.ffn_gate_exps.weight" in err


@pytest.mark.parametrize("case,msg", [
    ({"magic": b"GGUX"}, "magic"),
    ({"version": 1}, "version"),
    ({"truncate": 100}, "outside the file"),
    ({"misalign": "blk.0.ffn_up_exps.weight"}, "misaligned"),
])
def test_bad_files(tmp_path, moe, case, msg):
    p, _, _ = _write(tmp_path, moe, **case)
    f = moe.GgufFile(p)
    assert not f and f.status == 10 and msg in f.error


def test_truncated_directory(tmp_path, moe):
    p, _, _ = _write(tmp_path, moe)
    data = p.read_bytes()
    (tmp_path / "cut.gguf").write_bytes(data[:300])
    f = moe.GgufFile(tmp_path / "cut.gguf")
    assert not f and f.status == 10
    f = moe.GgufFile(tmp_path / "missing.gguf")
    assert not f and f.status == 10 and "cannot be opened" in f.error


def _edit(name, fn):
    def apply(tensors):
        return [fn(t) if t[0] == name else t for t in tensors]
    return apply


@pytest.mark.parametrize("fn,msg", [
    (lambda ts: ts + [ts[1]], "appears twice"),
    (lambda ts: [t for t in ts if t[0] != "blk.1.ffn_down_exps.weight"], "no tensor blk.1.ffn_down_exps.weight"),
    (_edit("blk.0.ffn_down_exps.weight", lambda t: (t[0], t[1], (256, 128, 16), t[3])), "disagree in shape"),
    (_edit("blk.1.ffn_up_exps.weight", lambda t: (t[0], gg.GGML["Q2_K"], t[2], t[3][: 16 * 128 * 84])), "differ in type"),
    (_edit("blk.0.ffn_gate_exps.weight", lambda t: (t[0], gg.GGML["F16"], t[2], bytes(256 * 128 * 16 * 2))),
     "not Q8_0, Q4_K or Q2_K"),
    (_edit("blk.1.ffn_gate_exps.weight", lambda t: (t[0], t[1], (256, 128, 16, 1)[:2], t[3])), "3-D"),
])
def test_layout_rejections(tmp_path, moe, fn, msg):
    p, _, _ = _write(tmp_path, moe, tensors_fn=fn)
    f = moe.GgufFile(p)
    if not f:
        assert msg in f.error
        return
    L, err = f.expert_layout(2)
    assert L is None and msg in err, err


@pytest.mark.gpu
def test_layer_on_experts_loaded_from_file(tmp_path, moe, layer, gpu_ctx, stream):
    """Layer 1's experts loaded from a GGUF file into one device allocation, selected through the
    [layer][E][3] table, give the same layer output as the same bytes uploaded directly."""
    import torch
    print("case layer on GGUF experts", flush=True)
    p, _, experts = _write(tmp_path, moe, n_layers=2, E=16, d=256, I=128)
    f = moe.GgufFile(p)
    assert f, f.error
    L, err = f.expert_layout(2)
    assert L is not None, err
    storage = gpu_ctx.register(torch.empty(L.total_bytes, dtype=torch.uint8, device="cuda"))
    table = f.load_experts(gpu_ctx, stream, L, storage.view())
    cfg = layer.LayerConfig("gguf", 128, 256, 16, 4, 128, 0, moe.Q4_K, moe.Q8_0, moe.F16, seed=5)
    inp = layer.make_inputs(cfg)
    inp.w_gate, inp.w_up, inp.w_down = experts[1]
    ws = layer.LayerWorkspace(gpu_ctx, cfg, inp)
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    ref = ws.out.tensor.cpu().numpy().copy()
    assert table[(1 * 16 + 3) * 3 + 2] == storage.ptr + L.offsets[1][2] + 3 * 256 * 4 * 34
    ws.gu_table = moe.ExpertTable(table, ws.snap_gu.view(), [storage.view()], n_layers=2, layer=1)
    ws.dn_table = moe.ExpertTable(table, ws.snap_dn.view(), [storage.view()], n_layers=2, layer=1)
    ws.out.tensor.fill_(float("nan"))
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    assert np.array_equal(ws.out.tensor.cpu().numpy().view(np.uint32), ref.view(np.uint32))
