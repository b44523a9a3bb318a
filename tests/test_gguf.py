"""Model files: GGUF expert tensors into device storage and the [layer][E][3] address table.

CPU: the GGUF directory parse and the expert layout against what the writer recorded, and the
rejections (bad magic and version, truncated file, data outside the file or off the alignment,
duplicate tensors, a missing or misshapen expert tensor, gate/up of different types, a
non-block expert type), following the reference's layout checks (src/metal/engine/window.cpp:
34-56,128-270). GPU: the device storage equals the file's tensor bytes and the table points at
every expert; the experts loaded from a file drive a full layer checked stage by stage against
the CPU oracle on the file's bytes, and equal, bit for bit, the same layer on the same bytes
uploaded directly.
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


def test_load_rejects_a_layout_the_file_does_not_give(tmp_path, moe):
    """The layout the caller passes must be the one this file gives for its layer count: an
    edited offset or size, a layer count past the file or the bound, or a layout from another
    file is refused before anything is read or copied (SM_E_ARGUMENT)."""
    from test_abi_host import Fake
    p, _, _ = _write(tmp_path, moe, n_layers=2, E=16, d=256, I=128)
    f = moe.GgufFile(p)
    L, err = f.expert_layout(2)
    assert L is not None, err
    p2, _, _ = _write(tmp_path, moe, name="other.gguf", n_layers=2, E=8, d=256, I=128)
    L_other, err = moe.GgufFile(p2).expert_layout(2)
    assert L_other is not None, err
    fake = Fake(moe)
    storage = fake.buf(L.total_bytes + (1 << 20))

    def edited(fn):
        c = moe.ExpertLayout.from_buffer_copy(L)
        fn(c)
        return c

    def more_layers(c):
        c.n_layers = 3

    def too_many(c):
        c.n_layers = 65

    def offset(c):
        c.offsets[1][2] += 256

    def total(c):
        c.total_bytes -= 256

    def fmt(c):
        c.down = moe.Q4_K

    cases = [(edited(more_layers), "does not fit this GGUF file"), (edited(too_many), "1..SM_GGUF_MAX_LAYERS"),
             (edited(offset), "does not match"), (edited(total), "does not match"), (edited(fmt), "does not match"),
             (L_other, "does not match")]
    for bad, msg in cases:
        with pytest.raises(RuntimeError, match="SM_E_ARGUMENT") as ex:
            f.load_experts(fake.ctx, 0, bad, storage.view())
        assert msg in str(ex.value), str(ex.value)


@pytest.mark.gpu
def test_layer_on_experts_loaded_from_file(tmp_path, moe, layer, orc, gpu_ctx, stream):
    """Every expert tensor of both layers lands in device storage byte for byte as the file holds
    it, and the [layer][E][3] table points at each expert's slab. Layer 1's experts, selected
    through the table, drive a full layer whose stages match the CPU oracle run on the file's
    own bytes at every grouped entry and token, and whose output equals, bit for bit, the same
    layer on the same bytes uploaded directly."""
    import torch
    from test_gpu_layer import _check_stages
    print("case layer on GGUF experts", flush=True)
    E, n_layers = 16, 2
    p, _, experts = _write(tmp_path, moe, n_layers=n_layers, E=E, d=256, I=128)
    f = moe.GgufFile(p)
    assert f, f.error
    L, err = f.expert_layout(n_layers)
    assert L is not None, err
    storage = gpu_ctx.register(torch.empty(L.total_bytes, dtype=torch.uint8, device="cuda"))
    storage.tensor.fill_(0x5A)
    table = f.load_experts(gpu_ctx, stream, L, storage.view())
    torch.cuda.synchronize()
    dev = storage.tensor.cpu().numpy()
    raw = p.read_bytes()
    file_w = {}
    for l in range(n_layers):
        for r, nm in enumerate(("gate", "up", "down")):
            t = f.find(f"blk.{l}.ffn_{nm}_exps.weight")
            want = np.frombuffer(raw, np.uint8, count=t["bytes"], offset=t["offset"])
            assert want.tobytes() == experts[l][r].tobytes(), f"file bytes of layer {l} {nm}"
            got = dev[L.offsets[l][r]:L.offsets[l][r] + t["bytes"]]
            assert np.array_equal(got, want), f"device storage of layer {l} {nm} differs from the file"
            slab = t["bytes"] // E
            for e in range(E):
                assert table[(l * E + e) * 3 + r] == storage.ptr + L.offsets[l][r] + e * slab
            file_w[l, r] = want.copy()
    cfg = layer.LayerConfig("gguf", 128, 256, E, 4, 128, 0, moe.Q4_K, moe.Q8_0, moe.F16, seed=5)
    inp = layer.make_inputs(cfg)
    inp.w_gate, inp.w_up, inp.w_down = file_w[1, 0], file_w[1, 1], file_w[1, 2]
    ws = layer.LayerWorkspace(gpu_ctx, cfg, inp)
    ws.gu_table = moe.ExpertTable(table, ws.snap_gu.view(), [storage.view()], n_layers=n_layers, layer=1)
    ws.dn_table = moe.ExpertTable(table, ws.snap_dn.view(), [storage.view()], n_layers=n_layers, layer=1)
    for n in ("hidden", "parts", "out"):
        getattr(ws, n).tensor.view(torch.uint8).fill_(0x7F)
    ws.run_layer(stream)
    assert ws.read_status(stream) == (0, 0, 0)
    _check_stages(moe, layer, orc, ws, inp, cfg, n_sample_tokens=None, every_entry=True)
    loaded = ws.out.tensor.cpu().numpy().copy()
    direct = layer.LayerWorkspace(gpu_ctx, cfg, inp)
    direct.run_layer(stream)
    assert direct.read_status(stream) == (0, 0, 0)
    assert np.array_equal(direct.out.tensor.cpu().numpy().view(np.uint32), loaded.view(np.uint32))
