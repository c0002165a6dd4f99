"""GPU parity at the BASELINE configurations' own shapes (one decoder layer,
teacher-forced: the same input to the GPU and to the CPU oracle), plus the
48-layer, V = 151936 decode step of configs[1] checked by its properties and by
teacher-forcing its first and last layers.

Per layer the routing log (what the decode path's own router produced: expert
indices, weights, logits and the residual the router read) is checked:
  * the selection is the stable top-k of the GPU's own logits, bit-exact;
  * the oracle router on the GPU's residual gives the same logits (fp32) and the
    same indices, except fp32 near-ties (gap < 1e-4) -- the reference contract;
  * the weights follow the reference's formula on those logits.
Hidden states are held to 2e-2 (5e-2 with MX experts) against the
bf16-emulating oracle and against its fp32 flow (emulate_bf16=False), both
routed to the experts the GPU's router chose (`force_idx`): the residual the
router reads differs from the oracle's by bf16 rounding, so a near-tie between
the 8th and 9th expert can go either way, and one flipped expert moves a
token's output by far more than the tolerance.  Where the oracle's own routing
differs, the test asserts the flip is such a near-tie: the oracle's logit gap
is within the measured logit difference of the two residuals.  The KV rows are
written exactly at each sequence's position and nowhere else.

Oracle flows: oracle/ref.py qwen_decoder_layer (megakernels/qwen3_moe/
attn_fused_nki.py:50-973, moe_fused_nki.py:70-762), gpt_oss_decoder_layer
(megakernels/gpt_oss/transformer_gpt_oss.py:239-522).
"""
import math

import pytest
import torch

from conftest import max_abs_rel
from oracle import ref
from routing_checks import (check_oracle_flips, check_qwen_routing, check_selection,
                            check_against_oracle_logits)

pytestmark = pytest.mark.gpu

TOL = 2e-2
TOL_MX = 5e-2
TIE = 1e-4


def bf(t):
    return t.to(torch.bfloat16)


def _ref_layer(hf):
    return ref.QwenLayer(wq=hf["q_proj"], wk=hf["k_proj"], wv=hf["v_proj"], wo=hf["o_proj"],
                         q_norm=hf["q_norm"], k_norm=hf["k_norm"], ln_in=hf["input_layernorm"],
                         ln_post=hf["post_attention_layernorm"], router=hf["gate"],
                         gate_up=hf["gate_up_proj"], down=hf["down_proj"])


def qwen_parity(y_gpu, rec, x, lw, kc, vc, cos, sin, pos, mx=False, K=8):
    """Routing contract, then hidden-state parity against both oracle flows routed
    like the GPU; returns the oracle's caches after the layer (new rows written)."""
    tol = TOL_MX if mx else TOL
    check_qwen_routing(rec, lw, 1e-6, K)
    gidx = rec["idx"].long()
    kr, vr = kc.clone(), vc.clone()
    y_bf, aux = ref.qwen_decoder_layer(x, lw, kr, vr, cos, sin, pos, ref.QwenShape(), mx_experts=mx,
                                       force_idx=gidx)
    y_32, _ = ref.qwen_decoder_layer(x, lw, kc.clone(), vc.clone(), cos, sin, pos, ref.QwenShape(),
                                     emulate_bf16=False, mx_experts=mx, force_idx=gidx)
    e_bf, e_32, e_ref = max_abs_rel(y_gpu, y_bf), max_abs_rel(y_gpu, y_32), max_abs_rel(y_bf, y_32)
    e_r = max_abs_rel(rec["r"], aux["r"])
    flips, dl = check_oracle_flips(rec["idx"], rec["logits"], aux["logits"], K)
    print(f"  hidden vs oracle {e_bf:.2e}, vs fp32 flow {e_32:.2e} (oracle bf16 vs fp32 {e_ref:.2e}); "
          f"router input {e_r:.2e}; oracle's own top-k differs in {flips}/{x.shape[0]} tokens "
          f"(near-ties within the logit difference {dl:.1e})", flush=True)
    assert e_bf < tol and e_r < TOL
    assert e_32 < tol, (e_32, e_ref)
    return kr, vr


def _fill_kv(model, kc, vc, layer=0):
    """Copy flat [B, nkv, S, d] caches into the model's layer caches (flat or paged)."""
    kv = model.kv_mgr
    dev = model.device
    if kv.block_table is None:
        kv.k(layer)[:, :, : kc.shape[2]].copy_(kc.to(dev))
        kv.v(layer)[:, :, : vc.shape[2]].copy_(vc.to(dev))
        return
    B, nkv, S, d = kc.shape
    blk = kv.block_len
    nb = S // blk
    table = kv.block_table[:, :nb].reshape(-1).long()
    for src, dst in ((kc, kv.k(layer)), (vc, kv.v(layer))):
        blocks = src.to(dev).reshape(B, nkv, nb, blk, d).permute(0, 2, 3, 1, 4).reshape(B * nb, blk, nkv, d)
        dst[table] = blocks


def _read_kv(model, B, S, layer=0):
    """The layer caches as flat [B, nkv, S, d] CPU tensors."""
    kv = model.kv_mgr
    if kv.block_table is None:
        return kv.k(layer)[:, :, :S].cpu(), kv.v(layer)[:, :, :S].cpu()
    blk = kv.block_len
    nb = S // blk
    table = kv.block_table[:, :nb].reshape(-1).long()
    out = []
    for t in (kv.k(layer), kv.v(layer)):
        g = t[table].reshape(B, nb, blk, t.shape[2], t.shape[3]).permute(0, 3, 1, 2, 4)
        out.append(g.reshape(B, t.shape[2], S, t.shape[3]).cpu())
    return out


def _check_kv_rows(new, old, pos, k_ref):
    """Only row pos[b] of sequence b changed, and it holds the oracle's new row."""
    for b in range(new.shape[0]):
        p = int(pos[b])
        changed = (new[b] != old[b]).any(-1).any(0).nonzero().flatten().tolist()
        assert changed == [p], (b, p, changed[:8])
        assert max_abs_rel(new[b, :, p], k_ref[b, :, p]) < TOL


@pytest.fixture
def decode_path():
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    yield Q.set_decode_path
    Q.set_decode_path("multi_kernel")


# (batch, paged block length (0 = flat), KV lengths: "fixed" or "ragged" U[512, 8192], path)
QWEN_CASES = [
    (1, 0, "fixed", "multi_kernel"),       # configs[0]/[1] shape: select-fused gate/up
    (4, 0, "fixed", "persistent"),         # the persistent layer kernel's select stage
    (16, 64, "ragged", "multi_kernel"),    # configs[2], paged
    (64, 64, "ragged", "multi_kernel"),    # configs[2], paged
    (64, 0, "ragged", "multi_kernel"),     # configs[2], flat
]


@pytest.mark.parametrize("B,blk,lens,path", QWEN_CASES)
def test_qwen_layer_baseline_shape(mk, dev, decode_path, B, blk, lens, path):
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    print(f"qwen layer B={B} blk={blk} lens={lens} path={path}", flush=True)
    decode_path(path)
    g = torch.Generator().manual_seed(1000 + B + blk)
    if lens == "ragged":
        pos = torch.randint(512, 8192 + 1, (B,), generator=g, dtype=torch.int32)
    else:
        pos = torch.full((B,), 2048, dtype=torch.int32)
    S = (int(pos.max()) + 1 + 127) // 128 * 128
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=1, max_batch=B, max_seq=S, kv_block_len=blk)
    hf = Q.random_layer_hf(cfg, 0, 500 + B, "cpu")
    x = bf(torch.randn(B, cfg.hidden_size, generator=g))
    kc = bf(torch.randn(B, 4, S, 128, generator=g))
    vc = bf(torch.randn(B, 4, S, 128, generator=g))
    layers = [Q.pack_layer({k: v.to(dev) for k, v in hf.items()})]
    model = Q.Qwen3MoeMegakernelModel(cfg, layers, B, dev)
    model.enable_route_log(B)
    if path == "persistent":
        assert model.layer_kernel_status(B)[0]
    _fill_kv(model, kc, vc)
    y = x.to(dev).contiguous()
    model.decode_layers(y, pos.to(dev))
    torch.cuda.synchronize()
    if path == "persistent":
        assert not model.layer_kernel_status(B)[1]
    rec = model.route_log(B)[0]
    knew, vnew = _read_kv(model, B, S)
    lw = _ref_layer(hf)
    cos, sin = ref.rope_cos_sin(pos, 128, cfg.rope_theta)
    kr, vr = qwen_parity(y, rec, x, lw, kc, vc, cos, sin, pos)
    _check_kv_rows(knew, kc, pos, kr)
    _check_kv_rows(vnew, vc, pos, vr)


def test_qwen_layer_mxfp8_batch32(mk, dev):
    """MXFP8 experts (E4M3 + E8M0 per 32 along K), activations
    dynamically MXFP8, attention and norms bf16, batch 32, KV lengths
    U[512, 8192] (configs[2]'s distribution; configs[3] names none); against the
    oracle on the dequantised weights at 5e-2."""
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    from oracle import mx as omx
    B = 32
    g = torch.Generator().manual_seed(3232)
    pos = torch.randint(512, 8192 + 1, (B,), generator=g, dtype=torch.int32)
    S = (int(pos.max()) + 1 + 127) // 128 * 128
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=1, max_batch=B, max_seq=S, expert_format="mxfp8")
    hf = Q.random_layer_hf(cfg, 0, 33, "cpu")
    x = bf(torch.randn(B, cfg.hidden_size, generator=g))
    kc = bf(torch.randn(B, 4, S, 128, generator=g))
    vc = bf(torch.randn(B, 4, S, 128, generator=g))
    model = Q.Qwen3MoeMegakernelModel(cfg, [Q.pack_layer({k: v.to(dev) for k, v in hf.items()}, "mxfp8")],
                                      B, dev)
    model.enable_route_log(B)
    _fill_kv(model, kc, vc)
    y = x.to(dev).contiguous()
    model.decode_layers(y, pos.to(dev))
    torch.cuda.synchronize()
    rec = model.route_log(B)[0]
    lw = _ref_layer(hf)
    lw.gate_up = torch.from_numpy(omx.dequantize_mx(*omx.quantize_mx(hf["gate_up_proj"].float().numpy(), "e4m3"), "e4m3"))
    lw.down = torch.from_numpy(omx.dequantize_mx(*omx.quantize_mx(hf["down_proj"].float().numpy(), "e4m3"), "e4m3"))
    cos, sin = ref.rope_cos_sin(pos, 128, cfg.rope_theta)
    print("mxfp8 B=32", flush=True)
    kr, _ = qwen_parity(y, rec, x, lw, kc, vc, cos, sin, pos, mx=True)
    knew, _ = _read_kv(model, B, S)
    _check_kv_rows(knew, kc, pos, kr)
    _check_mx_input_fusion(model, x, pos, dev, lambda: _fill_kv(model, kc, vc), y)


def _check_mx_input_fusion(model, x_in, pos, dev, reload, y_fused):
    """The experts' MXFP8 input written by the post-attention norm itself equals
    the separate quantisation launch (set_decode_path("separate_launches") keeps
    it): the layer's output bit for bit."""
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    Q.set_decode_path("separate_launches")
    try:
        reload()
        y2 = x_in.to(dev).contiguous()
        model.decode_layers(y2, pos.to(dev))
        torch.cuda.synchronize()
    finally:
        Q.set_decode_path("multi_kernel")
    assert torch.equal(y_fused.cpu(), y2.cpu())


def _dequant_mx_torch(codes, scales, fmt, k):
    """Independent dequantiser: element value table x 2^(scale - 127)."""
    import numpy as np
    from oracle import mx as omx
    if fmt == "e2m1":
        tab = torch.from_numpy(omx.decode_elements(np.arange(16, dtype=np.uint8), "e2m1")).float()
        c = codes.long()
        vals = torch.stack([tab[c & 15], tab[c >> 4]], -1).reshape(*codes.shape[:-1], -1)
    else:
        tab = torch.from_numpy(np.nan_to_num(omx.decode_elements(np.arange(256, dtype=np.uint8), "e4m3"))).float()
        vals = tab[codes.long()]
    vals = vals[..., :k]
    sc = torch.exp2(scales[..., : k // 32].float() - 127).repeat_interleave(32, -1)
    return vals * sc


@pytest.mark.parametrize("sliding", [True, False])
def test_gpt_oss_layer_baseline_shape(mk, dev, sliding):
    """GPT-OSS-20B layer at its full expert shape (E = 32, top-4,
    I = 2880, MXFP4 experts), batch 32, KV lengths U[1024, 4096]; a sliding-window
    (128-row ring) and a full-attention layer."""
    from nki_moe_megakernel_amd import gpt_oss_with_megakernel as G
    from nki_moe_megakernel_amd import mx
    B = 32
    print(f"gpt-oss layer B={B} sliding={sliding}", flush=True)
    g = torch.Generator().manual_seed(4000 + int(sliding))
    pos = torch.randint(1024, 4096 + 1, (B,), generator=g, dtype=torch.int32)
    S = (int(pos.max()) + 1 + 127) // 128 * 128
    cfg = G.GptOssMKConfig(num_hidden_layers=1, max_batch=B, max_seq=S, expert_format="mxfp4",
                           first_sliding=sliding)
    hf = G.random_layer_hf(cfg, 0, 44, "cpu")
    rows = 128 if sliding else S
    x = bf(torch.randn(B, cfg.hidden_size, generator=g))
    kc = bf(torch.randn(B, 8, rows, 64, generator=g))
    vc = bf(torch.randn(B, 8, rows, 64, generator=g))
    model = G.GptOssMegakernelModel(cfg, [G.pack_layer({k: v.to(dev) for k, v in hf.items()}, cfg)], B, dev)
    model.enable_route_log(B)
    model.kv_mgr.k(0).copy_(kc.to(dev))
    model.kv_mgr.v(0).copy_(vc.to(dev))
    xp = torch.zeros(B, cfg.hidden_pad, dtype=torch.bfloat16)
    xp[:, : cfg.hidden_size] = x
    y = xp.to(dev).contiguous()
    model.decode_layers(y, pos.to(dev))
    torch.cuda.synchronize()
    yc = y.cpu()
    assert torch.equal(yc[:, cfg.hidden_size:], torch.zeros(B, cfg.hidden_pad - cfg.hidden_size, dtype=torch.bfloat16))

    def reload():
        model.kv_mgr.k(0).copy_(kc.to(dev))
        model.kv_mgr.v(0).copy_(vc.to(dev))
    _check_mx_input_fusion(model, xp, pos, dev, reload, y)
    rec = model.route_log(B)[0]
    lw = ref.GptOssLayer(
        wq=hf["q_proj.weight"], bq=hf["q_proj.bias"], wk=hf["k_proj.weight"], bk=hf["k_proj.bias"],
        wv=hf["v_proj.weight"], bv=hf["v_proj.bias"], wo=hf["o_proj.weight"], bo=hf["o_proj.bias"],
        sinks=hf["sinks"], ln_in=hf["input_layernorm"], ln_post=hf["post_attention_layernorm"],
        router_w=hf["router.weight"], router_b=hf["router.bias"], gate_up=hf["experts.gate_up_proj"],
        gate_up_b=hf["experts.gate_up_proj_bias"], down=hf["experts.down_proj"],
        down_b=hf["experts.down_proj_bias"])
    c = G.convert_layer({k: v.to(dev) for k, v in hf.items()}, cfg)
    E, N2, Hp = c["gate_up"].shape
    I = N2 // 2
    gc, gs = mx.quantize_mx(c["gate_up"].reshape(E * N2, Hp), 2, Hp)
    rows_deq = _dequant_mx_torch(gc.cpu(), gs.cpu(), "e2m1", Hp).reshape(E, N2, Hp)[:, :, : cfg.hidden_size]
    gu = torch.empty(E, cfg.hidden_size, N2)
    gu[:, :, 0::2] = rows_deq[:, :I].transpose(1, 2)
    gu[:, :, 1::2] = rows_deq[:, I:].transpose(1, 2)
    lw.gate_up = gu
    dc, ds = mx.quantize_mx(c["down"].reshape(E * Hp, I), 2, (I + 127) // 128 * 128)
    dn = _dequant_mx_torch(dc.cpu(), ds.cpu(), "e2m1", I).reshape(E, Hp, I)[:, : cfg.hidden_size]
    lw.down = dn.transpose(1, 2).contiguous()
    del c, gc, gs, dc, ds
    cos, sin = model.rope_cos_sin(pos.to(dev))
    cos, sin = cos[:, :32].cpu(), sin[:, :32].cpu()
    shape = ref.GptOssShape()
    # routing: top-4 of the biased logits on the bf16 norm of the logged residual,
    # softmax over the top-4 (router_topk.py:868-887)
    check_selection(rec, 4)
    r = rec["r"][:, : cfg.hidden_size].float()
    assert torch.equal(rec["r"][:, cfg.hidden_size:], torch.zeros(B, cfg.hidden_pad - cfg.hidden_size,
                                                                  dtype=torch.bfloat16))
    n = bf(ref.rmsnorm_tkg(r, lw.ln_post, shape.eps)).float()
    lg_o = n @ lw.router_w.float().t() + lw.router_b.float()
    assert (rec["logits"] - lg_o).abs().max().item() < 5e-5
    check_against_oracle_logits(rec["idx"], lg_o, 4)
    top = torch.gather(rec["logits"], 1, rec["idx"].long())
    assert torch.allclose(rec["w"], torch.softmax(top, -1), rtol=1e-5, atol=1e-6)
    gidx = rec["idx"].long()
    win = 128 if sliding else 0
    kr = kc.clone()
    y_ref, aux = ref.gpt_oss_decoder_layer(x, lw, kr, vc.clone(), cos, sin, pos, win, shape,
                                           mx_experts=True, force_idx=gidx)
    y32, _ = ref.gpt_oss_decoder_layer(x, lw, kc.clone(), vc.clone(), cos, sin, pos, win, shape,
                                       mx_experts=True, emulate_bf16=False, force_idx=gidx)
    e_bf = max_abs_rel(yc[:, : cfg.hidden_size], y_ref)
    e_32 = max_abs_rel(yc[:, : cfg.hidden_size], y32)
    e_ref = max_abs_rel(y_ref, y32)
    flips, dl = check_oracle_flips(rec["idx"], rec["logits"], aux["logits"], 4)
    print(f"  hidden vs oracle {e_bf:.2e}, vs fp32 flow {e_32:.2e} (oracle bf16 vs fp32 {e_ref:.2e}); "
          f"oracle's own top-k differs in {flips}/{B} tokens (logit difference {dl:.1e})", flush=True)
    assert e_bf < TOL_MX and e_32 < TOL_MX
    # KV: the ring row pos % 127 (sliding) or row pos (full), nowhere else
    kn = model.kv_mgr.k(0).cpu()
    for b in range(B):
        row = int(pos[b]) % 127 if sliding else int(pos[b])
        changed = (kn[b] != kc[b]).any(-1).any(0).nonzero().flatten().tolist()
        assert changed == [row], (b, row, changed[:8])
        assert max_abs_rel(kn[b, :, row], kr[b, :, row]) < TOL


# ---------------------------------------------------------------- the whole step
def test_configs1_decode_step_48_layers(mk, dev):
    """the bench's model (48 layers, V = 151936, bs = 1, KV context
    2048 of seeded N(0,1)).  Properties of the whole step: logits finite, next
    token == arg-max of the logits, every layer's K/V cache changed only at the
    position, a HIP-graph replay bit-identical to the eager step.  Teacher-forced
    parity of layers 0 and 47 and of the lm_head against the oracle."""
    import bench
    import __graft_entry__ as ge
    ge.load_package()
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    B, ctx, seed = 1, 2048, 1234
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=48, max_batch=B, max_seq=ctx + 128)
    model = bench.build_model(Q, cfg, B, dev, seed)
    bench.prefill_kv(model, cfg, ctx, seed, dev)
    model.enable_route_log(B)
    Ln = cfg.num_hidden_layers
    k0 = [model.kv_mgr.k(l).clone() for l in range(Ln)]
    v0 = [model.kv_mgr.v(l).clone() for l in range(Ln)]
    ids = torch.tensor([77777], dtype=torch.int32, device=dev)
    pos = torch.tensor([ctx], dtype=torch.int32, device=dev)
    hidden = torch.empty(B, cfg.hidden_size, dtype=torch.bfloat16, device=dev)
    logits = torch.empty(B, cfg.vocab_size, dtype=torch.float32, device=dev)
    nxt = torch.empty(B, dtype=torch.int32, device=dev)
    print("configs[1] eager step", flush=True)
    model.step(ids, pos, hidden, logits, nxt)
    torch.cuda.synchronize()
    lg_e, nx_e, h_e = logits.clone(), nxt.clone(), hidden.clone()
    k_e = [model.kv_mgr.k(l).clone() for l in range(Ln)]
    assert torch.isfinite(lg_e).all()
    m = lg_e.max(-1)
    assert int(nx_e[0]) == int((lg_e[0] == m.values[0]).nonzero()[0, 0])
    for l in range(Ln):
        for new, old in ((model.kv_mgr.k(l), k0[l]), (model.kv_mgr.v(l), v0[l])):
            changed = (new[0] != old[0]).any(-1).any(0).nonzero().flatten().tolist()
            assert changed == [ctx], (l, changed[:8])
    logs = model.route_log(B)
    assert len(logs) == Ln
    for rec in logs:
        check_selection(rec, 8)
    # graph replay from the same state: bit-identical
    print("configs[1] graph replay", flush=True)
    for l in range(Ln):
        model.kv_mgr.k(l).copy_(k0[l])
        model.kv_mgr.v(l).copy_(v0[l])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        model.step(ids, pos, hidden, logits, nxt)
    for rep in range(3):
        for l in range(Ln):
            model.kv_mgr.k(l).copy_(k0[l])
            model.kv_mgr.v(l).copy_(v0[l])
        logits.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(logits, lg_e), rep
        assert torch.equal(nxt, nx_e) and torch.equal(hidden, h_e)
        assert all(torch.equal(model.kv_mgr.k(l), k_e[l]) for l in range(Ln))
    del graph
    # teacher-forced layers 0 and 47, then the lm_head on the final hidden state
    from nki_moe_megakernel_amd import _lib as L
    print("configs[1] teacher-forced layers", flush=True)
    x = torch.empty(B, cfg.hidden_size, dtype=torch.bfloat16, device=dev)
    L.check(L.load().mkd_embed(ids.data_ptr(), model.embed_tokens.data_ptr(), x.data_ptr(), B,
                               cfg.hidden_size, cfg.vocab_size, L.stream_ptr(dev)), "embed")
    cos, sin = ref.rope_cos_sin(pos.cpu(), 128, cfg.rope_theta)
    for l, (lo, hi) in ((0, (0, 1)), (47, (47, 48))):
        for j in range(Ln):
            model.kv_mgr.k(j).copy_(k0[j])
            model.kv_mgr.v(j).copy_(v0[j])
        xin = x.clone()
        if lo > 0:
            model.decode_layers(xin, pos, layers=(0, lo))
        x_in_cpu = xin.cpu()
        y = xin.clone()
        model.decode_layers(y, pos, layers=(lo, hi))
        torch.cuda.synchronize()
        rec = model.route_log(B)[lo]
        hf = {k: v.cpu() for k, v in Q.random_layer_hf(cfg, l, seed, dev).items()}
        lw = _ref_layer(hf)
        kc, vc = k0[l].cpu()[:, :, :ctx + 1], v0[l].cpu()[:, :, :ctx + 1]
        print(f"  layer {l}", flush=True)
        kr, _ = qwen_parity(y, rec, x_in_cpu, lw, kc, vc, cos, sin, pos.cpu())
        assert max_abs_rel(model.kv_mgr.k(l).cpu()[0, :, ctx], kr[0, :, ctx]) < TOL
        del hf, lw
    # lm_head + greedy on the eager step's final hidden state
    gl = torch.Generator(device=dev)
    gl.manual_seed(seed + 1)
    torch.randn(cfg.vocab_size, cfg.hidden_size, generator=gl, device=dev)          # embedding draw
    lm = (0.02 * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=gl, device=dev)).to(torch.bfloat16)
    lnf = (1 + 0.02 * torch.randn(cfg.hidden_size, generator=gl, device=dev)).to(torch.bfloat16)
    lg_ref, nx_ref = ref.final_norm_lm_head(h_e.cpu(), lnf.cpu(), lm.cpu(), cfg.rms_norm_eps)
    assert max_abs_rel(lg_e, lg_ref) < TOL
    top2 = torch.topk(lg_ref[0], 2).values
    if (top2[0] - top2[1]).item() > 1e-2 * lg_ref.abs().max().item():
        assert int(nx_e[0]) == int(nx_ref[0])


class _RoutedExperts:
    """The routed experts of one layer (expert id -> weights [2I, H] or [H, I])
    standing in for the [E, ...] expert tensor the oracle indexes by expert id."""

    def __init__(self, full_shape, rows):
        self.shape = full_shape
        self.rows = rows

    def __getitem__(self, e):
        return self.rows[int(e)]


def test_configs1_full_depth_parity(mk, dev):
    """configs[1] through its whole depth, like the reference's whole-model logit
    validation (main.py:559-640): one decode step of the bench's model (48
    layers, V = 151936, bs = 1, KV context 2048) against the CPU oracle on the
    same seeded weights (drawn on the GPU exactly as the bench draws them, then
    copied to the host one layer at a time).

    * Every one of the 48 layers teacher-forced: the GPU layer run alone on its
      own chain's input, against both oracle flows on that input, routed like
      the GPU, within 2e-2 -- with the routing contract on the GPU's residual
      (check_qwen_routing) and every flip of the oracle's own top-k a near-tie.
      The layer-by-layer GPU chain is bit-identical to the one-call step.
    * The whole chain: the oracle's bf16-emulating and fp32 flows chained through
      all 48 layers (routed like the GPU's routing log) against the step's final
      hidden state and its V = 151936 logits.  With random-init weights a
      rounding difference early in the chain grows layer by layer, and the
      oracle's own two flows end ~9e-2 apart, so the bar here is relative: the
      GPU may be no further from either flow than the flows are from each other
      (x 1.5, + 5e-3).  The per-layer drift curve is printed."""
    import bench
    import __graft_entry__ as ge
    ge.load_package()
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    B, ctx, seed, tok = 1, 2048, 1234, 77777
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=48, max_batch=B, max_seq=ctx + 128)
    model = bench.build_model(Q, cfg, B, dev, seed)
    bench.prefill_kv(model, cfg, ctx, seed, dev)
    model.enable_route_log(B)
    Ln = cfg.num_hidden_layers
    k0 = [model.kv_mgr.k(l).clone() for l in range(Ln)]
    v0 = [model.kv_mgr.v(l).clone() for l in range(Ln)]
    ids = torch.tensor([tok], dtype=torch.int32, device=dev)
    pos = torch.tensor([ctx], dtype=torch.int32, device=dev)
    hidden = torch.empty(B, cfg.hidden_size, dtype=torch.bfloat16, device=dev)
    logits = torch.empty(B, cfg.vocab_size, dtype=torch.float32, device=dev)
    nxt = torch.empty(B, dtype=torch.int32, device=dev)
    print("configs[1] full-depth step on the GPU", flush=True)
    model.step(ids, pos, hidden, logits, nxt)
    torch.cuda.synchronize()
    assert not model.layer_kernel_status()[1]      # no in-launch wait timed out
    lg_gpu, h_gpu = logits.cpu(), hidden.cpu()
    logs = model.route_log(B)
    assert len(logs) == Ln
    for l in range(Ln):
        model.kv_mgr.k(l).copy_(k0[l])
        model.kv_mgr.v(l).copy_(v0[l])
    x = model.embed_tokens[tok:tok + 1].clone()
    x_bf = x.cpu()
    x_32 = x_bf.float()
    cos, sin = ref.rope_cos_sin(pos.cpu(), cfg.head_dim, cfg.rope_theta)
    pc = pos.cpu()
    shape = ref.QwenShape()
    curve, tf = [], []
    for l in range(Ln):
        x_in = x.cpu()
        model.decode_layers(x, pos, layers=(l, l + 1))
        torch.cuda.synchronize()
        rec = model.route_log(B)[l]
        assert torch.equal(rec["idx"], logs[l]["idx"]) and torch.equal(rec["r"], logs[l]["r"])
        hf = Q.random_layer_hf(cfg, l, seed, dev)
        sel = sorted(set(rec["idx"][0].tolist()))
        gu = _RoutedExperts(tuple(hf["gate_up_proj"].shape), {e: hf["gate_up_proj"][e].cpu() for e in sel})
        dn = _RoutedExperts(tuple(hf["down_proj"].shape), {e: hf["down_proj"][e].cpu() for e in sel})
        lw = ref.QwenLayer(wq=hf["q_proj"].cpu(), wk=hf["k_proj"].cpu(), wv=hf["v_proj"].cpu(),
                           wo=hf["o_proj"].cpu(), q_norm=hf["q_norm"].cpu(), k_norm=hf["k_norm"].cpu(),
                           ln_in=hf["input_layernorm"].cpu(), ln_post=hf["post_attention_layernorm"].cpu(),
                           router=hf["gate"].cpu(), gate_up=gu, down=dn)
        del hf
        kc, vc = k0[l][:, :, :ctx + 1].cpu(), v0[l][:, :, :ctx + 1].cpu()
        # teacher-forced: this layer on the GPU chain's own input (qwen_parity asserts 2e-2)
        kr, _ = qwen_parity(x.cpu(), rec, x_in, lw, kc, vc, cos, sin, pc)
        assert max_abs_rel(model.kv_mgr.k(l)[:, :, ctx].cpu(), kr[:, :, ctx]) < TOL
        tf.append(max_abs_rel(x.cpu(), ref.qwen_decoder_layer(x_in, lw, kc.clone(), vc.clone(), cos, sin, pc,
                                                              shape, force_idx=rec["idx"].long())[0]))
        # the chains
        force = logs[l]["idx"].long()
        x_bf, aux = ref.qwen_decoder_layer(x_bf, lw, kc.clone(), vc.clone(), cos, sin, pc, shape,
                                           force_idx=force)
        x_32, aux32 = ref.qwen_decoder_layer(x_32, lw, kc.clone(), vc.clone(), cos, sin, pc, shape,
                                             emulate_bf16=False, force_idx=force)
        flips, dl = check_oracle_flips(logs[l]["idx"], logs[l]["logits"], aux["logits"], 8)
        curve.append((max_abs_rel(logs[l]["r"], aux["r"]), max_abs_rel(logs[l]["r"], aux32["r"]),
                      max_abs_rel(aux["r"], aux32["r"]), flips))
        if l % 8 == 7:
            print("  layers %2d-%2d teacher-forced: %s" % (l - 7, l, " ".join("%.1e" % e for e in tf[-8:])),
                  flush=True)
            print("                chained router input vs bf16 flow / fp32 flow / flows apart: %s" % (
                "  ".join("%.1e/%.1e/%.1e%s" % (a, b, c, "*" if f else "") for a, b, c, f in curve[-8:])),
                flush=True)
    assert torch.equal(x.cpu(), h_gpu)             # layer by layer == the one-call step
    e_bf, e_32, e_flows = max_abs_rel(h_gpu, x_bf), max_abs_rel(h_gpu, x_32), max_abs_rel(x_bf, x_32)
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 1)
    torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g, device=dev)           # embedding draw
    lm = (0.02 * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g, device=dev)).to(torch.bfloat16).cpu()
    lnf = (1 + 0.02 * torch.randn(cfg.hidden_size, generator=g, device=dev)).to(torch.bfloat16).cpu()
    lg_bf, nx_bf = ref.final_norm_lm_head(x_bf, lnf, lm, cfg.rms_norm_eps)
    lg_32, nx_32 = ref.final_norm_lm_head(x_32, lnf, lm, cfg.rms_norm_eps, emulate_bf16=False)
    l_bf, l_32, l_flows = max_abs_rel(lg_gpu, lg_bf), max_abs_rel(lg_gpu, lg_32), max_abs_rel(lg_bf, lg_32)
    print(f"  after 48 layers: hidden vs bf16 flow {e_bf:.2e}, vs fp32 flow {e_32:.2e} (flows apart "
          f"{e_flows:.2e}); logits vs bf16 flow {l_bf:.2e}, vs fp32 flow {l_32:.2e} (flows apart "
          f"{l_flows:.2e}); greedy token gpu {int(nxt[0])}, oracle bf16 flow {int(nx_bf[0])}, "
          f"fp32 flow {int(nx_32[0])}; teacher-forced layers max {max(tf):.2e}", flush=True)
    assert max(tf) < TOL
    for e in (e_bf, e_32):
        assert e <= 1.5 * e_flows + 5e-3, (e, e_flows)
    for e in (l_bf, l_32):
        assert e <= 1.5 * l_flows + 5e-3, (e, l_flows)
    # the step's own lm_head on its final hidden state (teacher-forced)
    lg_tf, nx_tf = ref.final_norm_lm_head(h_gpu, lnf, lm, cfg.rms_norm_eps)
    assert max_abs_rel(lg_gpu, lg_tf) < TOL
    top2 = torch.topk(lg_tf[0], 2).values
    if (top2[0] - top2[1]).item() > 1e-2 * lg_tf.abs().max().item():
        assert int(nxt[0]) == int(nx_tf[0])
    del model
    torch.cuda.empty_cache()
