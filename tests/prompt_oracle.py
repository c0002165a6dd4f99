"""Token-by-token oracle chains for the prefill and module-boundary GPU tests
(imported, not collected).

A prompt's context encoding must leave the caches and hidden states that the
same tokens decoded one at a time would (the reference's CTE layer path,
megakernels/qwen3_moe/qwen_with_megakernel.py:496-526, produces the context the
TKG path then reads).  These helpers run that decode chain on the CPU oracle,
each token through every layer, routed to the experts the GPU's routing log
recorded for that token and layer (the routing itself is checked separately
against the oracle router on the GPU's own residual).
"""
import torch

from oracle import ref


def qwen_ref_layers(hfs):
    """QwenLayer per layer with fp32 weights (converted once, not per token)."""
    out = []
    for hf in hfs:
        f = {k: v.float() for k, v in hf.items()}
        out.append(ref.QwenLayer(wq=f["q_proj"], wk=f["k_proj"], wv=f["v_proj"], wo=f["o_proj"],
                                 q_norm=f["q_norm"], k_norm=f["k_norm"], ln_in=f["input_layernorm"],
                                 ln_post=f["post_attention_layernorm"], router=f["gate"],
                                 gate_up=f["gate_up_proj"], down=f["down_proj"]))
    return out


def qwen_prompt_chain(x_rows, lws, k_caches, v_caches, p0, shape, logs=None, emulate_bf16=True,
                      theta=1e6, mx_experts=False):
    """Decode tokens p0 .. p0 + T - 1 of one sequence through every layer.

    x_rows [T, H] (bf16 values): each token's input to layer 0; k_caches /
    v_caches per layer [1, nkv, S, d], updated in place (row p0 + t of token t);
    logs: the GPU routing log per layer (idx [T, K]) or None for the oracle's own
    top-k.  Returns (out [T, H] fp32 holding bf16 values, aux per layer per token)."""
    T = x_rows.shape[0]
    outs, auxes = [], [[] for _ in lws]
    for t in range(T):
        pos = torch.tensor([p0 + t])
        cos, sin = ref.rope_cos_sin(pos, shape.d, theta)
        x = x_rows[t:t + 1].float()
        for l, lw in enumerate(lws):
            force = logs[l]["idx"][t:t + 1].long() if logs is not None else None
            x, aux = ref.qwen_decoder_layer(x, lw, k_caches[l], v_caches[l], cos, sin, pos, shape,
                                            emulate_bf16=emulate_bf16, mx_experts=mx_experts,
                                            force_idx=force)
            auxes[l].append(aux)
        outs.append(x)
    return torch.cat(outs, 0), auxes
