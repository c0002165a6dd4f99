"""The persistent decoder-layer kernel (one launch per layer, stages separated by
grid barriers) against the fp32 oracle (qwen_decoder_layer, the reference
layer flow qwen_with_megakernel.py:414-531) and against the multi-kernel layer
path on the same inputs.  Hidden states within 2e-2 (max-abs error relative to
the reference's max-abs), bit-identical from run to run, KV rows written only at
each sequence's position, no grid-barrier timeout."""
import pytest
import torch

from conftest import max_abs_rel
from oracle import ref

pytestmark = pytest.mark.gpu
TOL = 2e-2


def bf(t):
    return t.to(torch.bfloat16)


def _ref_layer(hf):
    return ref.QwenLayer(wq=hf["q_proj"], wk=hf["k_proj"], wv=hf["v_proj"], wo=hf["o_proj"],
                         q_norm=hf["q_norm"], k_norm=hf["k_norm"], ln_in=hf["input_layernorm"],
                         ln_post=hf["post_attention_layernorm"], router=hf["gate"],
                         gate_up=hf["gate_up_proj"], down=hf["down_proj"])


@pytest.fixture
def persistent():
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    Q.set_decode_path("persistent")
    yield
    Q.set_decode_path("multi_kernel")


def _setup(dev, B, S, seed, kv_block=0):
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=1, max_batch=B, max_seq=S, kv_block_len=kv_block)
    hf = Q.random_layer_hf(cfg, 0, seed, "cpu")
    g = torch.Generator().manual_seed(seed)
    pos = torch.randint(S // 2, S - 1, (B,), generator=g, dtype=torch.int32)
    x = bf(torch.randn(B, cfg.hidden_size, generator=g))
    kc = bf(torch.randn(B, 4, S, 128, generator=g))
    vc = bf(torch.randn(B, 4, S, 128, generator=g))
    layers = [Q.pack_layer({k: v.to(dev) for k, v in hf.items()}, cfg.expert_format)]
    model = Q.Qwen3MoeMegakernelModel(cfg, layers, B, dev)
    return Q, cfg, hf, pos, x, kc, vc, model


def _run(model, x, kc, vc, pos, dev):
    model.kv_mgr.k(0).copy_(kc.to(dev))
    model.kv_mgr.v(0).copy_(vc.to(dev))
    y = x.to(dev).contiguous()
    model.decode_layers(y, pos.to(dev))
    torch.cuda.synchronize()
    return y.cpu(), model.kv_mgr.k(0).cpu(), model.kv_mgr.v(0).cpu()


@pytest.mark.parametrize("B,S", [(1, 1024), (2, 1024), (4, 1024), (2, 4096)])
def test_layer_kernel_vs_oracle_and_multi_kernel(mk, dev, persistent, B, S):
    print(f"layer kernel B={B} S={S}", flush=True)
    Q, cfg, hf, pos, x, kc, vc, model = _setup(dev, B, S, seed=31 + B + S)
    assert model.layer_kernel_status(B)[0], "persistent kernel not planned for this shape"
    y1, k1, v1 = _run(model, x, kc, vc, pos, dev)
    used, timeout = model.layer_kernel_status(B)
    assert used and not timeout
    y1b, _, _ = _run(model, x, kc, vc, pos, dev)
    assert torch.equal(y1, y1b)
    Q.set_decode_path("multi_kernel")
    try:
        assert not model.layer_kernel_status(B)[0]
        y2, k2, v2 = _run(model, x, kc, vc, pos, dev)
    finally:
        Q.set_decode_path("persistent")
    cos, sin = ref.rope_cos_sin(pos, 128, cfg.rope_theta)
    y_ref, _ = ref.qwen_decoder_layer(x, _ref_layer(hf), kc.clone(), vc.clone(), cos, sin, pos,
                                      ref.QwenShape())
    assert max_abs_rel(y1, y_ref) < TOL
    assert max_abs_rel(y1, y2) < TOL
    for b in range(B):
        p = int(pos[b])
        for new, old, other in ((k1, kc, k2), (v1, vc, v2)):
            changed = (new[b] != old[b]).any(-1).any(0).nonzero().flatten().tolist()
            assert changed == [p], (b, p, changed[:8])
            assert max_abs_rel(new[b, :, p], other[b, :, p]) < TOL


def test_layer_kernel_three_layers_one_launch(mk, dev, persistent):
    """Three full-shape layers in one persistent launch (the rows stay in LDS
    between layers) vs the oracle applied layer by layer and the multi-kernel path.

    Each path's routing log is checked layer by layer (selection exact on its own
    logits; oracle router on its own residual, near-ties < 1e-4 excepted) and the
    oracle chain is routed to the experts that path chose: over chained layers
    the residuals of the GPU and of the oracle differ by bf16 rounding (~5e-3),
    and a near-tie at the 8th expert then picks a different expert, which moves
    that token by ~2-3e-2 -- measured, a discrete flip rather than accumulated
    rounding (the oracle's own bf16 and fp32 flows stay within 7e-3 over these
    three layers)."""
    from routing_checks import check_oracle_flips, check_qwen_routing
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    B, S, Ln = 2, 512, 3
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=Ln, max_batch=B, max_seq=S)
    hf = [Q.random_layer_hf(cfg, l, 71, "cpu") for l in range(Ln)]
    g = torch.Generator().manual_seed(71)
    pos = torch.tensor([300, 17], dtype=torch.int32)
    x = bf(torch.randn(B, cfg.hidden_size, generator=g))
    kc = [bf(torch.randn(B, 4, S, 128, generator=g)) for _ in range(Ln)]
    vc = [bf(torch.randn(B, 4, S, 128, generator=g)) for _ in range(Ln)]
    layers = [Q.pack_layer({k: v.to(dev) for k, v in h.items()}, cfg.expert_format) for h in hf]
    model = Q.Qwen3MoeMegakernelModel(cfg, layers, B, dev)
    model.enable_route_log(B)
    assert model.layer_kernel_status(B)[0]

    def run():
        for l in range(Ln):
            model.kv_mgr.k(l).copy_(kc[l].to(dev))
            model.kv_mgr.v(l).copy_(vc[l].to(dev))
        y = x.to(dev).contiguous()
        model.decode_layers(y, pos.to(dev))
        torch.cuda.synchronize()
        return y.cpu(), [model.kv_mgr.k(l).cpu() for l in range(Ln)], model.route_log(B)

    y1, k1, log1 = run()
    assert not model.layer_kernel_status(B)[1]
    Q.set_decode_path("multi_kernel")
    try:
        y2, k2, log2 = run()
    finally:
        Q.set_decode_path("persistent")
    cos, sin = ref.rope_cos_sin(pos, 128, cfg.rope_theta)

    def oracle_chain(logs):
        y, own = x.float(), 0
        for l in range(Ln):
            lw = _ref_layer(hf[l])
            check_qwen_routing(logs[l], lw, 1e-6, 8)
            y_in = y
            y, aux = ref.qwen_decoder_layer(y_in, lw, kc[l].clone(), vc[l].clone(), cos, sin, pos,
                                            ref.QwenShape(), force_idx=logs[l]["idx"].long())
            own += check_oracle_flips(logs[l]["idx"], logs[l]["logits"], aux["logits"], 8)[0]
        return y, own

    y_ref1, f1 = oracle_chain(log1)
    y_ref2, f2 = oracle_chain(log2)
    e1, e2, e12 = max_abs_rel(y1, y_ref1), max_abs_rel(y2, y_ref2), max_abs_rel(y1, y2)
    print(f"persistent vs oracle {e1:.4f}, multi-kernel vs oracle {e2:.4f}, between {e12:.4f}; "
          f"near-tie flips against the oracle's own routing: {f1}, {f2}", flush=True)
    assert e1 < TOL and e2 < TOL
    if all(torch.equal(a["idx"], b["idx"]) for a, b in zip(log1, log2)):
        assert e12 < TOL
    for l in range(Ln):
        for b in range(B):
            p = int(pos[b])
            assert max_abs_rel(k1[l][b, :, p], k2[l][b, :, p]) < TOL


def test_layer_kernel_paged_kv_matches_flat(mk, dev, persistent):
    """Block (paged) KV pool through the persistent kernel: bit-identical hidden
    states to the flat cache holding the same rows; new rows at the table slot."""
    B, S, blk = 3, 1024, 64
    Q, cfg, hf, pos, x, kc, vc, mf = _setup(dev, B, S, seed=5)
    _, _, _, _, _, _, _, mp = _setup(dev, B, S, seed=5, kv_block=blk)
    assert mf.layer_kernel_status(B)[0] and mp.layer_kernel_status(B)[0]
    pos = torch.tensor([1000, 63, 640], dtype=torch.int32)
    table = mp.kv_mgr.block_table.cpu().long()
    kp = torch.zeros(mp.kv_mgr.num_blocks, blk, 4, 128, dtype=torch.bfloat16)
    vp = torch.zeros_like(kp)
    for b in range(B):
        for j in range(S // blk):
            kp[table[b, j]] = kc[b, :, j * blk:(j + 1) * blk].permute(1, 0, 2)
            vp[table[b, j]] = vc[b, :, j * blk:(j + 1) * blk].permute(1, 0, 2)
    yf, kf, _ = _run(mf, x, kc, vc, pos, dev)
    mp.kv_mgr.k(0).copy_(kp.to(dev))
    mp.kv_mgr.v(0).copy_(vp.to(dev))
    yp = x.to(dev).contiguous()
    mp.decode_layers(yp, pos.to(dev))
    torch.cuda.synchronize()
    assert torch.equal(yf, yp.cpu())
    kp_new = mp.kv_mgr.k(0).cpu()
    changed = (kp_new != kp).any(-1).any(-1).nonzero().tolist()
    want = sorted([int(table[b, int(pos[b]) // blk]), int(pos[b]) % blk] for b in range(B))
    assert sorted(changed) == want
    for b in range(B):
        p = int(pos[b])
        assert torch.equal(kp_new[table[b, p // blk], p % blk], kf[b, :, p])
    assert not mp.layer_kernel_status(B)[1]


def test_layer_kernel_not_planned_for_large_batch(mk, dev, persistent):
    """Batches above the persistent kernel's limit run the multi-kernel layers."""
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=1, max_batch=8, max_seq=256)
    hf = Q.random_layer_hf(cfg, 0, 3, "cpu")
    layers = [Q.pack_layer({k: v.to(dev) for k, v in hf.items()}, cfg.expert_format)]
    model = Q.Qwen3MoeMegakernelModel(cfg, layers, 8, dev)
    assert not model.layer_kernel_status(8)[0]
    assert model.layer_kernel_status(4)[0]
