"""Small GGUF v3 model files for the model-file tests (test infrastructure), written with the
package's GGUF writer (strata.app_amd/gguf_write.py).
"""
from __future__ import annotations

import numpy as np

import __graft_entry__ as ge

_gw = ge.load_package().gguf_write
T_U32, T_I32, T_F32, T_STRING, T_ARRAY, T_U64 = _gw.T_U32, _gw.T_I32, _gw.T_F32, _gw.T_STRING, _gw.T_ARRAY, _gw.T_U64
GGML = _gw.GGML
write_gguf = _gw.write_gguf


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
