"""Write the small golden fixtures under tests/golden/ (run from the repo root).

Every expected value comes from transformers 5.15.0 (the third-party library
whose Qwen3.5-MoE helpers the reference calls, see
v2/src/router_ia/qwen36_linear_attention_hf.py:81-100) or from the float64
closed form, never from this repository's code under test.  Inputs are seeded.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

from pathlib import Path

import torch
import torch.nn.functional as F
from safetensors.torch import save_file

OUT = Path(__file__).resolve().parent


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def main() -> None:
    import transformers
    from transformers.models.qwen3_5_moe import modeling_qwen3_5_moe as hf
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig

    meta = {"source": f"transformers {transformers.__version__}"}

    # Gated delta rule, recurrent (64 tokens, 4 heads, initial state) and chunked (130 tokens).
    for name, length, fn in (("delta_recurrent_L64_H4", 64, "recurrent"), ("delta_chunk_L130_H4", 130, "chunk")):
        g = _gen(100 + length)
        q = torch.randn((1, length, 4, 128), generator=g)
        k = torch.randn((1, length, 4, 128), generator=g)
        v = torch.randn((1, length, 4, 128), generator=g)
        gl = -F.softplus(torch.randn((1, length, 4), generator=g)) * torch.exp(torch.rand((1, length, 4), generator=g) * 4 - 4)
        beta = torch.sigmoid(torch.randn((1, length, 4), generator=g))
        s0 = torch.randn((1, 4, 128, 128), generator=g) * 0.02
        if fn == "recurrent":
            o, s = hf.torch_recurrent_gated_delta_rule(q, k, v, gl, beta, initial_state=s0, output_final_state=True,
                                                      use_qk_l2norm_in_kernel=True)
        else:
            o, s = hf.torch_chunk_gated_delta_rule(q, k, v, gl, beta, initial_state=s0, output_final_state=True,
                                                  use_qk_l2norm_in_kernel=True)
        save_file({"q": q[0], "k": k[0], "v": v[0], "g": gl[0], "beta": beta[0], "state0": s0[0],
                   "out": o[0].contiguous(), "state": s[0].contiguous()}, str(OUT / f"{name}.safetensors"), meta)

    # Depthwise conv update (bf16, 512 channels, 5 tokens from a random window).
    g = _gen(7)
    w = (torch.randn((512, 4), generator=g) * 0.5).to(torch.bfloat16)
    state = torch.randn((1, 512, 4), generator=g).to(torch.bfloat16)
    xs = torch.randn((5, 512), generator=g).to(torch.bfloat16)
    st = state.clone()
    outs = [hf.causal_conv1d_update(xs[t].reshape(1, 512, 1), st, w, activation="silu")[0, :, 0] for t in range(5)]
    save_file({"weight": w, "state0": state, "x": xs, "out": torch.stack(outs), "state": st},
              str(OUT / "conv_update_C512_T5.safetensors"), meta)

    # RoPE tables of the Qwen3.5/3.6 text rotary embedding (theta 1e7, 64 of 256 dims).
    cfg = Qwen3_5MoeTextConfig(rope_parameters={"rope_theta": 10_000_000.0, "partial_rotary_factor": 0.25,
                                                 "rope_type": "default"})
    rot = hf.Qwen3_5MoeTextRotaryEmbedding(cfg)
    pos = torch.tensor([[0, 17, 4096, 4351, 32767]])
    cos, sin = rot(torch.zeros(1, 5, 256), pos)
    save_file({"positions": pos[0].to(torch.int64), "cos": cos[0].contiguous(), "sin": sin[0].contiguous()},
              str(OUT / "rope_tables.safetensors"), meta)

    # Decode attention reference: softmax attention in float64 (closed form), GQA 8:1, gate per (head, dim).
    g = _gen(9)
    T = 33
    qr = torch.randn((16, 256), generator=g, dtype=torch.float64)
    K = torch.randn((2, T, 256), generator=g, dtype=torch.float64)
    V = torch.randn((2, T, 256), generator=g, dtype=torch.float64)
    gate = torch.randn((16, 256), generator=g, dtype=torch.float64)
    probs = torch.softmax((qr[:, None, :] * K.repeat_interleave(8, 0)).sum(-1) / 16.0, dim=-1)
    out = (probs[..., None] * V.repeat_interleave(8, 0)).sum(1) * torch.sigmoid(gate)
    save_file({"q_rot": qr.float(), "k": K.float(), "v": V.float(), "gate": gate.float(), "out": out.float()},
              str(OUT / "decode_attention_T33.safetensors"), {"source": "float64 closed form"})
    print("wrote", sorted(p.name for p in OUT.glob("*.safetensors")))


if __name__ == "__main__":
    main()
