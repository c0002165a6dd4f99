"""Exact router ties at the top-k boundary through the decode paths that form
the top-k inside other kernels: the gate/up GEMM whose blocks select the
experts themselves (bs = 1) and the persistent layer kernel.  The lowest expert
index wins, as in the reference's top-k (max8 + nc_find_index8, router_topk.py:
626-646) and the oracle's stable sort.  Experts 20 and 30 get bit-identical
router rows whose logits tie for the 8th place (with the sign of the shared
direction positive; the negated case routes elsewhere and is a plain check);
picking 30 instead of 20 would change an eighth of the MoE output."""
import dataclasses

import pytest
import torch

from conftest import max_abs_rel
from oracle import ref

pytestmark = pytest.mark.gpu
TOL = 2e-2


@pytest.mark.parametrize("path", ["multi_kernel", "persistent"])
def test_router_boundary_tie_lowest_index_wins(mk, dev, path):
    # one of the two signs of the shared direction puts the tie at the boundary
    involved = [_tie_case(dev, path, sign) for sign in (1.0, -1.0)]
    assert any(involved)


def _tie_case(dev, path, sign):
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    print(f"router tie: path={path} sign={sign}", flush=True)
    B, S = 1, 512
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=1, max_batch=B, max_seq=S)
    hf = Q.random_layer_hf(cfg, 0, 77, "cpu")
    g = torch.Generator().manual_seed(77)
    u = torch.randn(cfg.hidden_size, generator=g) * 0.02 * sign
    alpha = 0.5 * torch.rand(cfg.num_experts, generator=g)
    for i in range(7):
        alpha[i] = 1.0 + 0.01 * i
    alpha[20] = alpha[30] = 0.99
    hf["gate"] = (alpha[:, None] * u[None, :]).to(torch.bfloat16)
    assert torch.equal(hf["gate"][20], hf["gate"][30])
    pos = torch.tensor([300], dtype=torch.int32)
    # a small residual stream, so that the MoE output is a large part of y
    x = (0.05 * torch.randn(B, cfg.hidden_size, generator=g)).to(torch.bfloat16)
    kc = torch.randn(B, 4, S, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, 4, S, 128, generator=g).to(torch.bfloat16)
    model = Q.Qwen3MoeMegakernelModel(cfg, [Q.pack_layer({k: v.to(dev) for k, v in hf.items()})], B, dev)
    Q.set_decode_path(path)
    try:
        if path == "persistent":
            assert model.layer_kernel_status(B)[0]
        model.kv_mgr.k(0).copy_(kc.to(dev))
        model.kv_mgr.v(0).copy_(vc.to(dev))
        y = x.to(dev).contiguous()
        model.decode_layers(y, pos.to(dev))
        torch.cuda.synchronize()
        if path == "persistent":
            assert not model.layer_kernel_status(B)[1]
    finally:
        Q.set_decode_path("multi_kernel")
    lw = ref.QwenLayer(wq=hf["q_proj"], wk=hf["k_proj"], wv=hf["v_proj"], wo=hf["o_proj"],
                       q_norm=hf["q_norm"], k_norm=hf["k_norm"], ln_in=hf["input_layernorm"],
                       ln_post=hf["post_attention_layernorm"], router=hf["gate"],
                       gate_up=hf["gate_up_proj"], down=hf["down_proj"])
    cos, sin = ref.rope_cos_sin(pos, 128, cfg.rope_theta)
    y_ref, _ = ref.qwen_decoder_layer(x, lw, kc.clone(), vc.clone(), cos, sin, pos, ref.QwenShape())
    err = max_abs_rel(y.cpu(), y_ref)
    assert err < TOL, err
    # the oracle with expert 30's FFN in expert 20's place is what a wrong
    # tie-break computes: it must differ clearly when the tie is routed
    gu, dn = hf["gate_up_proj"].clone(), hf["down_proj"].clone()
    gu[20], dn[20] = hf["gate_up_proj"][30], hf["down_proj"][30]
    lw_swap = dataclasses.replace(lw, gate_up=gu, down=dn)
    y_swap, _ = ref.qwen_decoder_layer(x, lw_swap, kc.clone(), vc.clone(), cos, sin, pos, ref.QwenShape())
    if torch.equal(y_swap, y_ref):
        return False                                      # experts 20 / 30 not routed
    assert max_abs_rel(y_swap, y_ref) > 5 * TOL           # the tie decides the output
    return True
