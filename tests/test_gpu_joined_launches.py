"""The joined launches of the few-token decode step: attention, chunk combine,
output projection and router GEMM in one kernel (the combine blocks wait inside
the launch for their kv group's chunk blocks, the projection blocks for every
combine block, the router blocks -- residual add, post-attention norm, router
logits -- for every projection block), and the expert launch (router top-k, gate/up and down in one kernel
whose down blocks wait for their expert's gate/up blocks) with the one-token
router selection inside it.

Checked, at full Qwen3-30B-A3B layer shapes (H 2048, 32 / 4 heads, 128 experts
top-8, I 768), 3 layers chained:
* against the same layers with every stage a launch of its own
  (set_decode_path("separate_launches")): identical routing in layer 0,
  hidden states and written K rows within 1e-2 (only fp32 summation orders
  differ) unless a later layer's top-k differs at a near-tie of the two paths'
  logits (asserted to be one);
* against the fp32 oracle, teacher-forced on the decode path's own routing log
  (router rows checked against the oracle router, near-tie flips against the
  oracle's logit gap), within 2e-2;
* bit-identical from call to call and across graph replays (the flag words are
  cleared, and at one token the data-polled exchange buffers filled with their
  empty marker, at the start of every call, including inside a captured graph);
* at one token up to 8192 positions: the merge + projection blocks read a head's
  chunk partials in several batches;
* no in-launch wait timed out;
* a call at a short position between two at a long one (the exchange words are
  reset only up to the position) changes nothing for the later call."""
import pytest
import torch

from conftest import max_abs_rel
from oracle import ref
from routing_checks import check_oracle_flips, check_qwen_routing

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _ref_layer(hf):
    return ref.QwenLayer(wq=hf["q_proj"], wk=hf["k_proj"], wv=hf["v_proj"], wo=hf["o_proj"],
                         q_norm=hf["q_norm"], k_norm=hf["k_norm"], ln_in=hf["input_layernorm"],
                         ln_post=hf["post_attention_layernorm"], router=hf["gate"],
                         gate_up=hf["gate_up_proj"], down=hf["down_proj"])


@pytest.fixture
def restore_path():
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    yield Q
    Q.set_decode_path("multi_kernel")


def _setup(dev, layers, B, S, seed):
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=layers, max_batch=B, max_seq=S)
    hfs = [Q.random_layer_hf(cfg, l, seed, "cpu") for l in range(layers)]
    g = torch.Generator().manual_seed(seed)
    pos = torch.randint(S // 2, S - 1, (B,), generator=g, dtype=torch.int32)
    x = torch.randn(B, cfg.hidden_size, generator=g).to(torch.bfloat16)
    kcs = [torch.randn(B, 4, S, 128, generator=g).to(torch.bfloat16) for _ in range(layers)]
    vcs = [torch.randn(B, 4, S, 128, generator=g).to(torch.bfloat16) for _ in range(layers)]
    packed = [Q.pack_layer({k: v.to(dev) for k, v in h.items()}, cfg.expert_format) for h in hfs]
    model = Q.Qwen3MoeMegakernelModel(cfg, packed, B, dev)
    model.enable_route_log(B)
    return cfg, hfs, pos, x, kcs, vcs, model


def _load_caches(model, kcs, vcs, dev):
    for l in range(len(kcs)):
        model.kv_mgr.k(l).copy_(kcs[l].to(dev))
        model.kv_mgr.v(l).copy_(vcs[l].to(dev))


def _run(model, x, kcs, vcs, pos, dev):
    _load_caches(model, kcs, vcs, dev)
    y = x.to(dev).contiguous()
    model.decode_layers(y, pos.to(dev))
    torch.cuda.synchronize()
    used, timeout = model.layer_kernel_status(x.shape[0])
    assert not used and not timeout
    return y.cpu(), [model.kv_mgr.k(l).cpu() for l in range(len(kcs))], model.route_log(x.shape[0])


@pytest.mark.parametrize("B,S", [(1, 1024), (1, 4096), (1, 8192), (4, 2048)])
def test_joined_launches_vs_separate_and_oracle(mk, dev, restore_path, B, S):
    Q = restore_path
    print(f"joined launches: B={B} S={S}", flush=True)
    cfg, hfs, pos, x, kcs, vcs, model = _setup(dev, 3, B, S, 17 + B)
    assert model.joined_attention(B) and model.router_in_attention(B)
    y_f, k_f, log_f = _run(model, x, kcs, vcs, pos, dev)
    y_f2, _, _ = _run(model, x, kcs, vcs, pos, dev)
    assert torch.equal(y_f, y_f2)                     # deterministic call to call
    Q.set_decode_path("separate_launches")
    assert not model.router_in_attention(B)
    y_s, k_s, log_s = _run(model, x, kcs, vcs, pos, dev)
    e = max_abs_rel(y_f, y_s)
    # the two paths add in different orders (one token: the attention's chunks
    # span 8 waves of 16 positions, the router's K in slices), so a later
    # layer's top-k may differ at a near-tie; then each expert the joined path
    # chose beyond the other's top-k must sit within twice the two paths' logit
    # difference of its K-th logit, and the hidden states are not compared
    flipped = [l for l in range(3) if not torch.equal(log_f[l]["idx"], log_s[l]["idx"])]
    print(f"joined vs separate launches, 3 layers: {e:.2e} (routing differs in layers {flipped})", flush=True)
    for l in flipped:
        check_oracle_flips(log_f[l]["idx"], log_f[l]["logits"], log_s[l]["logits"], 8)
    if not flipped:
        assert e < 1e-2
    # layer 0 sees identical inputs on both paths: identical routing, and its
    # post-attention residual within 1e-2
    assert 0 not in flipped
    assert max_abs_rel(log_f[0]["r"], log_s[0]["r"]) < 1e-2
    for l in range(3):
        for b in range(B):
            p = int(pos[b])
            changed = (k_f[l][b] != kcs[l][b]).any(-1).any(0).nonzero().flatten().tolist()
            assert changed == [p], (l, b, p, changed[:8])
            if not any(f < l for f in flipped):
                assert max_abs_rel(k_f[l][b, :, p], k_s[l][b, :, p]) < 1e-2
    # the joined path's layers against the oracle, teacher-forced on its routing log
    lws = [_ref_layer(h) for h in hfs]
    cos, sin = ref.rope_cos_sin(pos, 128, cfg.rope_theta)
    shape = ref.QwenShape()
    for l in range(3):
        check_qwen_routing(log_f[l], lws[l], 1e-6, 8)
    y = x.float()
    for l in range(3):
        y, aux = ref.qwen_decoder_layer(y, lws[l], kcs[l].clone(), vcs[l].clone(), cos, sin, pos, shape,
                                        force_idx=log_f[l]["idx"].long())
        check_oracle_flips(log_f[l]["idx"], log_f[l]["logits"], aux["logits"], 8)
    e = max_abs_rel(y_f, y)
    print(f"joined launches, 3 layers vs the oracle (teacher-forced routing): {e:.2e}", flush=True)
    assert e < TOL


def test_joined_launches_graph_replays(mk, dev):
    """Captured step replayed several times with eager work between the replays:
    every replay bit-identical to the eager call (the flag words start cleared)."""
    cfg, hfs, pos, x, kcs, vcs, model = _setup(dev, 2, 1, 512, 23)
    y_eager, k_eager, _ = _run(model, x, kcs, vcs, pos, dev)
    y = x.to(dev).contiguous()
    p = pos.to(dev)
    _load_caches(model, kcs, vcs, dev)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        model.decode_layers(y, p)          # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        model.decode_layers(y, p)
    for rep in range(3):
        _load_caches(model, kcs, vcs, dev)
        y.copy_(x.to(dev))
        junk = torch.randn(1 << 20, device=dev).sum()      # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(y.cpu(), y_eager), rep
        assert torch.equal(model.kv_mgr.k(1).cpu(), k_eager[1]), rep
        assert model.layer_kernel_status(1) == (False, False)


def test_one_token_positions_long_short_long(mk, dev, restore_path):
    """The one-token exchange buffers are reset only up to the call's position:
    a call at a long position, then a short one, then the long one again -- the
    third call equals the first bit for bit, and the short call matches the
    separate-launch path (which uses no exchange buffers)."""
    Q = restore_path
    cfg, hfs, pos, x, kcs, vcs, model = _setup(dev, 2, 1, 4096, 29)
    p_long = torch.tensor([3900], dtype=torch.int32)
    p_short = torch.tensor([100], dtype=torch.int32)
    print("exchange reset: positions 3900, 100, 3900", flush=True)
    y1, k1, log1 = _run(model, x, kcs, vcs, p_long, dev)
    y2, k2, log2 = _run(model, x, kcs, vcs, p_short, dev)
    y3, k3, _ = _run(model, x, kcs, vcs, p_long, dev)
    assert torch.equal(y1, y3)
    assert all(torch.equal(a, b) for a, b in zip(k1, k3))
    Q.set_decode_path("separate_launches")
    y2s, _, log2s = _run(model, x, kcs, vcs, p_short, dev)
    flipped = [l for l in range(2) if not torch.equal(log2[l]["idx"], log2s[l]["idx"])]
    for l in flipped:
        check_oracle_flips(log2[l]["idx"], log2[l]["logits"], log2s[l]["logits"], 8)
    assert 0 not in flipped
    if not flipped:
        assert max_abs_rel(y2, y2s) < 1e-2
