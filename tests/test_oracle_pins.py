"""Pins of the CPU oracle (oracle/ref.py) against independent sources.

Each check is chosen so that a plausible mistake in the oracle (a dropped term,
a wrong sign or index, a transposed operand) fails it:
  * HF transformers modules (fp32) for RMSNorm, RoPE, router, experts, and the
    whole decoder layer (committed golden fixture, tests/golden/);
  * closed forms and special cases (zero rows, padding law, S=1 attention,
    uniform scores, one-hot routing == dense MLP, position 0 RoPE);
  * brute force on tiny inputs (top-k).
"""
import math
import os

import pytest
import torch

from oracle import ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "qwen3moe_layer_fp32.safetensors")


def _hf():
    from transformers.models.qwen3_moe import modeling_qwen3_moe as M
    from transformers.models.qwen3_moe.configuration_qwen3_moe import Qwen3MoeConfig
    return M, Qwen3MoeConfig


# ------------------------------------------------------------------ rmsnorm
def test_rmsnorm_matches_hf_fp32():
    M, _ = _hf()
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 256, generator=g)
    w = 1 + 0.1 * torch.randn(256, generator=g)
    m = M.Qwen3MoeRMSNorm(256, eps=1e-6)
    with torch.no_grad():
        m.weight.copy_(w)
        y_hf = m(x)
    y = ref.rmsnorm_tkg(x, w, 1e-6)
    assert torch.allclose(y, y_hf, rtol=1e-6, atol=1e-6)


def test_rmsnorm_closed_forms():
    # constant row c: y = gamma * c / sqrt(c^2 + eps)
    x = torch.full((1, 128), 3.0)
    w = torch.linspace(0.5, 1.5, 128)
    y = ref.rmsnorm_tkg(x, w, 1e-6)
    assert torch.allclose(y, w * 3.0 / math.sqrt(9.0 + 1e-6), rtol=1e-6)
    # zero row -> zero
    assert torch.all(ref.rmsnorm_tkg(torch.zeros(2, 128), w, 1e-6) == 0)


def test_rmsnorm_padding_law():
    # zero-padding H with hidden_actual = true width leaves the real part unchanged
    g = torch.Generator().manual_seed(1)
    x = torch.randn(3, 2880, generator=g)
    w = torch.randn(2880, generator=g)
    xp = torch.cat([x, torch.zeros(3, 192)], 1)
    wp = torch.cat([w, torch.ones(192)])
    y = ref.rmsnorm_tkg(x, w, 1e-5)
    yp = ref.rmsnorm_tkg(xp, wp, 1e-5, hidden_actual=2880)
    assert torch.allclose(yp[:, :2880], y, rtol=1e-6, atol=1e-7)
    assert torch.all(yp[:, 2880:] == 0)


# ------------------------------------------------------------------ top-k / router
def test_stable_topk_brute_force():
    g = torch.Generator().manual_seed(2)
    for _ in range(50):
        x = torch.randint(0, 5, (6,), generator=g).float()   # many exact ties
        v, i = ref.stable_topk(x, 3)
        order = sorted(range(6), key=lambda j: (-x[j].item(), j))[:3]
        assert i.tolist() == order
        assert v.tolist() == [x[j].item() for j in order]


def test_router_matches_hf_qwen_fp32():
    M, C = _hf()
    cfg = C(hidden_size=128, num_experts=16, num_experts_per_tok=4, norm_topk_prob=True)
    r = M.Qwen3MoeTopKRouter(cfg)
    g = torch.Generator().manual_seed(3)
    with torch.no_grad():
        r.weight.copy_(0.1 * torch.randn(16, 128, generator=g))
    x = torch.randn(7, 128, generator=g)
    with torch.no_grad():
        logits_hf, w_hf, idx_hf = r(x)
    logits, idx, aff, vals = ref.router_topk(x, r.weight.detach().t(), None, "softmax", 4,
                                             router_pre_norm=True, norm_topk_prob=True)
    assert torch.allclose(logits, logits_hf, rtol=1e-6, atol=1e-6)
    assert torch.equal(idx, idx_hf)
    assert torch.allclose(vals, w_hf, rtol=1e-6, atol=1e-7)
    # scattered affinities: K non-zeros per row summing to 1
    assert torch.all((aff > 0).sum(1) == 4)
    assert torch.allclose(aff.sum(1), torch.ones(7), atol=1e-6)
    # Qwen fused flow without bf16 emulation is the same math
    lq, iq, wq = ref.qwen_router(x, r.weight.detach().t(), 4, emulate_bf16=False)
    assert torch.equal(iq, idx_hf)
    assert torch.allclose(wq, w_hf, rtol=1e-6, atol=1e-7)


def test_router_act2_is_softmax_of_topk():
    # ACT2 pipeline (GPT-OSS): softmax over the top-k logits only (HF modeling_gpt_oss.py:126-130)
    g = torch.Generator().manual_seed(4)
    x = torch.randn(5, 64, generator=g)
    w = torch.randn(64, 32, generator=g) * 0.2
    b = torch.randn(32, generator=g) * 0.1
    logits, idx, aff, vals = ref.router_topk(x, w, b, "softmax", 4, router_pre_norm=False)
    full = x @ w + b
    tv, ti = torch.topk(full, 4, dim=-1)
    assert torch.equal(idx, ti)
    assert torch.allclose(vals, torch.softmax(tv, -1), atol=1e-6)
    assert torch.allclose(aff.sum(1), torch.ones(5), atol=1e-6)


def test_router_act1_without_norm_keeps_full_activation():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 64, generator=g)
    w = torch.randn(64, 16, generator=g) * 0.2
    logits, idx, aff, vals = ref.router_topk(x, w, None, "softmax", 2, router_pre_norm=True)
    assert torch.allclose(aff, torch.softmax(x @ w, -1), atol=1e-6)


# ------------------------------------------------------------------ experts
def _hf_experts(E=8, H=64, I=32, seed=6):
    M, C = _hf()
    cfg = C(hidden_size=H, num_experts=E, num_experts_per_tok=2, moe_intermediate_size=I)
    cfg._experts_implementation = "eager"
    ex = M.Qwen3MoeExperts(cfg)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        ex.gate_up_proj.copy_(0.1 * torch.randn(E, 2 * I, H, generator=g))
        ex.down_proj.copy_(0.1 * torch.randn(E, H, I, generator=g))
    return ex, g


def test_experts_match_hf_fp32():
    ex, g = _hf_experts()
    x = torch.randn(5, 64, generator=g)
    idx = torch.stack([torch.randperm(8, generator=g)[:2] for _ in range(5)])
    wts = torch.rand(5, 2, generator=g)
    with torch.no_grad():
        y_hf = ex(x, idx, wts)
    gu = ex.gate_up_proj.detach()
    dn = ex.down_proj.detach()
    y_q = ref.qwen_experts(x, gu, dn, idx, wts, emulate_bf16=False)
    assert torch.allclose(y_q, y_hf, rtol=1e-5, atol=1e-6)
    # the generic moe_tkg over the reference layouts [E,H,2,I] / [E,I,H], POST_SCALE
    I = 32
    gu_ref = torch.stack([gu[:, :I, :], gu[:, I:, :]], 2).permute(0, 3, 2, 1).contiguous()  # [E,H,2,I]
    dn_ref = dn.transpose(1, 2).contiguous()                                                # [E,I,H]
    aff = torch.zeros(5, 8).scatter_(1, idx, wts)
    y_g = ref.moe_tkg(x, gu_ref, dn_ref, aff, idx, scaling_mode="post", emulate_bf16=False)
    assert torch.allclose(y_g, y_hf, rtol=1e-5, atol=1e-6)


def test_one_hot_routing_is_dense_swiglu():
    ex, g = _hf_experts(seed=7)
    x = torch.randn(4, 64, generator=g)
    e = 3
    idx = torch.full((4, 1), e)
    y = ref.qwen_experts(x, ex.gate_up_proj.detach(), ex.down_proj.detach(), idx,
                         torch.ones(4, 1), emulate_bf16=False)
    W = ex.gate_up_proj.detach()[e]
    gte, up = (x @ W.t()).chunk(2, -1)
    dense = (torch.nn.functional.silu(gte) * up) @ ex.down_proj.detach()[e].t()
    assert torch.allclose(y, dense, rtol=1e-5, atol=1e-6)


def test_moe_gelu_activations_closed_form():
    """One expert per token with weight 1: the oracle's GELU-gated expert equals
    g/2 (1 + erf(g / sqrt 2)) * u (math.erf) and the tanh form
    g/2 (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))) (math.tanh), element by element."""
    g = torch.Generator().manual_seed(5)
    T, E, H, I = 3, 4, 32, 16
    x = torch.randn(T, H, generator=g)
    gu = 0.3 * torch.randn(E, H, 2, I, generator=g)
    dn = 0.3 * torch.randn(E, I, H, generator=g)
    idx = torch.tensor([[1], [3], [0]])
    aff = torch.zeros(T, E).scatter_(1, idx, 1.0)
    for act, f in [("gelu", lambda v: 0.5 * v * (1 + math.erf(v / math.sqrt(2)))),
                   ("gelu_tanh", lambda v: 0.5 * v * (1 + math.tanh(math.sqrt(2 / math.pi) * (v + 0.044715 * v ** 3))))]:
        y = ref.moe_tkg(x, gu, dn, aff, idx, None, None, "post", act, emulate_bf16=False)
        for t in range(T):
            e = int(idx[t, 0])
            gv = x[t] @ gu[e, :, 0, :]
            uv = x[t] @ gu[e, :, 1, :]
            h = torch.tensor([f(float(a)) for a in gv]) * uv
            assert torch.allclose(y[t], h @ dn[e], atol=1e-5), act


def test_moe_clamps_and_swish():
    # GPT-OSS semantics: gate <= 7, up in [-7, 7], g * sigmoid(1.702 g) (HF modeling_gpt_oss.py:82-88)
    g = torch.Generator().manual_seed(8)
    E, H, I = 4, 32, 32
    x = 3 * torch.randn(2, H, generator=g)
    gu = torch.randn(E, H, 2, I, generator=g)
    dn = 0.1 * torch.randn(E, I, H, generator=g)
    idx = torch.tensor([[0, 2], [1, 3]])
    aff = torch.zeros(2, E).scatter_(1, idx, torch.tensor([[0.7, 0.3], [0.4, 0.6]]))
    y = ref.moe_tkg(x, gu, dn, aff, idx, scaling_mode="post", act="swish",
                    gate_clamp_upper=7.0, up_clamp_upper=7.0, up_clamp_lower=-7.0,
                    emulate_bf16=False)
    exp = torch.zeros(2, H)
    for t in range(2):
        for j in range(2):
            e = int(idx[t, j])
            gt = (x[t] @ gu[e, :, 0, :]).clamp(max=7.0)
            up = (x[t] @ gu[e, :, 1, :]).clamp(min=-7.0, max=7.0)
            exp[t] += aff[t, e] * ((gt * torch.sigmoid(1.702 * gt) * up) @ dn[e])
    assert torch.allclose(y, exp, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------ rope / attention
def test_rope_matches_hf_and_identity_at_zero():
    M, _ = _hf()
    g = torch.Generator().manual_seed(9)
    q = torch.randn(2, 4, 1, 64, generator=g)
    k = torch.randn(2, 2, 1, 64, generator=g)
    pos = torch.tensor([5, 1000])
    cos, sin = ref.rope_cos_sin(pos, 64, 1e6)
    qh, kh = M.apply_rotary_pos_emb(q, k, cos[:, None, :], sin[:, None, :], unsqueeze_dim=1)
    qo = ref.rope_apply(q[:, :, 0], cos[:, None], sin[:, None], emulate_bf16=False)
    assert torch.allclose(qo, qh[:, :, 0], atol=1e-6)
    c0, s0 = ref.rope_cos_sin(torch.tensor([0]), 64, 1e6)
    assert torch.equal(ref.rope_apply(q[0, :, 0], c0, s0, emulate_bf16=False), q[0, :, 0])


def _generic_attn_inputs(B=2, H=128, nq=4, d=32, S_ctx=20, S_max=24, seed=10):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(B, 1, H, generator=g)
    W = 0.1 * torch.randn(H, d * (nq + 2), generator=g)
    Kc = torch.randn(B, S_max, d, generator=g)
    Vc = torch.randn(B, S_max, d, generator=g)
    mask = torch.ones(S_ctx, B, nq, 1)
    return X, W, Kc, Vc, mask, g


def test_generic_attention_matches_sdpa():
    X, W, Kc, Vc, mask, g = _generic_attn_inputs()
    B, nq, d, S_ctx = 2, 4, 32, 20
    mask[5:9, 1] = 0      # knock out a span for sequence 1
    out, Kn, Vn = ref.attention_block_tkg(X, W, None, None, None, None, None, 1e-6, None, None,
                                          Kc.clone(), Vc.clone(), mask, None, False, None,
                                          None, None)
    qkv = X.reshape(B, -1) @ W
    q = qkv[:, :nq * d].reshape(B, nq, d)
    k = qkv[:, nq * d:(nq + 1) * d]
    v = qkv[:, (nq + 1) * d:]
    for b in range(B):
        keys = torch.cat([Kc[b, :S_ctx - 1], k[b:b + 1]], 0)
        vals = torch.cat([Vc[b, :S_ctx - 1], v[b:b + 1]], 0)
        am = mask[:, b, :, 0].t().bool()                         # [nq, S_ctx]
        o = torch.nn.functional.scaled_dot_product_attention(
            q[b][:, None, :], keys[None].expand(nq, -1, -1), vals[None].expand(nq, -1, -1),
            attn_mask=am[:, None, :])
        assert torch.allclose(out[b].reshape(nq, d), o[:, 0], atol=1e-5)


def test_generic_attention_special_cases():
    X, W, Kc, Vc, mask, g = _generic_attn_inputs(S_ctx=1)
    # S_ctx = 1: only the active token -> output = its V
    out, _, _ = ref.attention_block_tkg(X, W, None, None, None, None, None, 1e-6, None, None,
                                        Kc, Vc, mask, None, False, None, None, None)
    v = (X.reshape(2, -1) @ W)[:, 5 * 32:]
    assert torch.allclose(out.reshape(2, 4, 32), v[:, None, :].expand(2, 4, 32), atol=1e-6)
    # uniform scores (zero queries) -> mean of V over the window
    W0 = W.clone()
    W0[:, :4 * 32] = 0
    X, _, Kc, Vc, mask, _ = _generic_attn_inputs(S_ctx=9)
    out, _, _ = ref.attention_block_tkg(X, W0, None, None, None, None, None, 1e-6, None, None,
                                        Kc, Vc, mask, None, False, None, None, None)
    v = (X.reshape(2, -1) @ W0)[:, 5 * 32:]
    for b in range(2):
        mean = torch.cat([Vc[b, :8], v[b:b + 1]], 0).mean(0)
        assert torch.allclose(out[b].reshape(4, 32), mean.expand(4, 32), atol=1e-5)


def test_attention_sink_matches_hf_gpt_oss_formula():
    # sink: extra logit per head in the softmax denominator, dropped afterwards
    # (HF modeling_gpt_oss.py eager_attention_forward: cat sinks, softmax, drop last column)
    X, W, Kc, Vc, mask, g = _generic_attn_inputs(S_ctx=12)
    sink = torch.randn(4, generator=g)
    out, _, _ = ref.attention_block_tkg(X, W, None, None, None, None, None, 1e-6, None, None,
                                        Kc, Vc, mask, sink, False, None, None, None)
    qkv = X.reshape(2, -1) @ W
    for b in range(2):
        q = qkv[b, :128].reshape(4, 32)
        keys = torch.cat([Kc[b, :11], qkv[b, 128:160][None]], 0)
        vals = torch.cat([Vc[b, :11], qkv[b, 160:][None]], 0)
        sc = q @ keys.t() / math.sqrt(32)
        comb = torch.cat([sc, sink[:, None]], 1)
        p = torch.softmax(comb, -1)[:, :-1]
        assert torch.allclose(out[b].reshape(4, 32), p @ vals, atol=1e-5)


def test_kv_scatter_only_target_rows_change():
    X, W, Kc, Vc, mask, g = _generic_attn_inputs(S_ctx=10)
    K0, V0 = Kc.clone(), Vc.clone()
    idx = torch.tensor([[9], [0xFFFFFFFF]], dtype=torch.int64)   # seq 1: uint32 max = skip
    ref.attention_block_tkg(X, W, None, None, None, None, None, 1e-6, None, None, Kc, Vc, mask,
                            None, True, idx, None, None)
    qkv = X.reshape(2, -1) @ W
    changed = (Kc != K0).any(-1)
    assert changed[0].nonzero().flatten().tolist() == [9]
    assert not changed[1].any()
    assert torch.equal(Kc[0, 9], qkv[0, 128:160])
    assert torch.equal(Vc[0, 9], qkv[0, 160:])


def test_multi_token_window_equals_token_by_token():
    """S_tkg new tokens in one call (window = the cache positions, then the new
    tokens; causal among them) equal S_tkg one-token calls that each write their
    k / v row at the next position -- the multi-token form reduces to the
    one-token form pinned above."""
    g = torch.Generator().manual_seed(11)
    B, S, H, nq, d, P, S_max = 2, 4, 64, 4, 32, 9, 16
    X = torch.randn(B, S, H, generator=g)
    W = 0.2 * torch.randn(H, d * (nq + 2), generator=g)
    qn = 1 + 0.1 * torch.randn(d, generator=g)
    kn = 1 + 0.1 * torch.randn(d, generator=g)
    Kc = torch.randn(B, S_max, d, generator=g)
    Vc = torch.randn(B, S_max, d, generator=g)
    cos, sin = ref.rope_cos_sin(torch.arange(P, P + S).repeat(B), d, 1e4)
    cos_r = cos[:, :d // 2].reshape(B, S, d // 2).permute(2, 0, 1).contiguous()   # [d/2, B, S]
    sin_r = sin[:, :d // 2].reshape(B, S, d // 2).permute(2, 0, 1).contiguous()
    prior = (torch.rand(P, B, nq, S, generator=g) > 0.3).float()
    causal = (torch.arange(S)[:, None] <= torch.arange(S)[None, :]).float()     # [key i, query s]
    mask = torch.cat([prior, causal[:, None, None, :].expand(S, B, nq, S)], 0)   # [P + S, B, nq, S]
    idx = torch.full((B, 1), P, dtype=torch.int64)
    K1, V1 = Kc.clone(), Vc.clone()
    out, _, _ = ref.attention_block_tkg(X, W, None, None, None, qn, kn, 1e-6, cos_r, sin_r, K1, V1,
                                        mask, None, True, idx, None, None)
    K2, V2 = Kc.clone(), Vc.clone()
    for i in range(S):
        m_i = torch.cat([prior[:, :, :, i:i + 1], torch.ones(i + 1, B, nq, 1)], 0)
        o_i, _, _ = ref.attention_block_tkg(X[:, i:i + 1], W, None, None, None, qn, kn, 1e-6,
                                            cos_r[:, :, i:i + 1], sin_r[:, :, i:i + 1], K2, V2, m_i,
                                            None, True, idx + i, None, None)
        assert torch.allclose(out.reshape(B, S, -1)[:, i], o_i, atol=1e-5), i
    assert torch.allclose(K1, K2, atol=1e-6) and torch.allclose(V1, V2, atol=1e-6)
    assert (K1 != Kc).any(-1).nonzero()[:, 1].unique().tolist() == list(range(P, P + S))


def test_post_rope_norm_reduces_to_pre_rope_norm():
    """Post-RoPE per-head RMSNorm (attention_block_tkg.py:906-910) against the
    pre-RoPE norm pinned above: the contiguous-halves rotation keeps the rms, so
    with the identity rotation (cos 1, sin 0) the post norm with weights w is
    the pre norm with w, and with the quarter turn (cos 0, sin 1: x -> [-x2, x1])
    it is the pre norm with w's halves swapped -- a norm applied before RoPE, or
    a weight index off by the half, fails the second.  With eps = 0 the post norm
    also makes the block blind to the scale of the Q and K projections."""
    g = torch.Generator().manual_seed(23)
    B, S, H, nq, d, P, S_max = 2, 2, 48, 4, 16, 5, 10
    X = torch.randn(B, S, H, generator=g)
    W = 0.3 * torch.randn(H, d * (nq + 2), generator=g)
    w_q = 1 + 0.5 * torch.randn(d, generator=g)
    w_k = 1 + 0.5 * torch.randn(d, generator=g)
    Kc = torch.randn(B, S_max, d, generator=g)
    Vc = torch.randn(B, S_max, d, generator=g)
    prior = (torch.rand(P, B, nq, S, generator=g) > 0.3).float()
    causal = (torch.arange(S)[:, None] <= torch.arange(S)[None, :]).float()
    mask = torch.cat([prior, causal[:, None, None, :].expand(S, B, nq, S)], 0)
    idx = torch.full((B, 1), P, dtype=torch.int64)
    swap = lambda w: torch.cat([w[d // 2:], w[:d // 2]])

    def run(Wm, cosv, sinv, pre=None, post=None, eps=1e-5):
        c = torch.full((d // 2, B, S), float(cosv))
        s_ = torch.full((d // 2, B, S), float(sinv))
        K1, V1 = Kc.clone(), Vc.clone()
        o, K2, _ = ref.attention_block_tkg(
            X, Wm, None, None, None, pre[0] if pre else None, pre[1] if pre else None, eps, c, s_,
            K1, V1, mask, None, True, idx, None, None,
            q_norm_post_w=post[0] if post else None, k_norm_post_w=post[1] if post else None,
            qk_post_eps=eps)
        return o, K2[:, P:P + S]

    o_post, k_post = run(W, 1, 0, post=(w_q, w_k))
    o_pre, k_pre = run(W, 1, 0, pre=(w_q, w_k))
    assert torch.allclose(o_post, o_pre, atol=1e-5) and torch.allclose(k_post, k_pre, atol=1e-5)
    o_post, k_post = run(W, 0, 1, post=(w_q, w_k))
    o_pre, k_pre = run(W, 0, 1, pre=(swap(w_q), swap(w_k)))
    assert torch.allclose(o_post, o_pre, atol=1e-5) and torch.allclose(k_post, k_pre, atol=1e-5)
    o_wrong, _ = run(W, 0, 1, pre=(w_q, w_k))
    assert not torch.allclose(o_post, o_wrong, atol=1e-3)
    # scale blindness (eps = 0): Q columns x3, K columns x0.25
    cs = torch.ones(d * (nq + 2))
    cs[:nq * d] = 3.0
    cs[nq * d:(nq + 1) * d] = 0.25
    c0, s0 = 0.6, 0.8
    o1, _ = run(W, c0, s0, post=(w_q, w_k), eps=0.0)
    o2, _ = run(W * cs, c0, s0, post=(w_q, w_k), eps=0.0)
    assert torch.allclose(o1, o2, atol=1e-5)
    n1, _ = run(W, c0, s0, eps=0.0)
    n2, _ = run(W * cs, c0, s0, eps=0.0)
    assert not torch.allclose(n1, n2, atol=1e-3)


# ------------------------------------------------------------------ whole layer vs HF
def _load_golden():
    from safetensors.torch import load_file
    from safetensors import safe_open
    t = load_file(GOLDEN)
    with safe_open(GOLDEN, "pt") as f:
        meta = f.metadata()
    return t, meta


def golden_layer(t, meta):
    H, nq, nkv, d = int(meta["H"]), int(meta["nq"]), int(meta["nkv"]), int(meta["d"])
    E, K, I = int(meta["E"]), int(meta["K"]), int(meta["I"])
    lw = ref.QwenLayer(
        wq=t["w.self_attn.q_proj.weight"], wk=t["w.self_attn.k_proj.weight"],
        wv=t["w.self_attn.v_proj.weight"], wo=t["w.self_attn.o_proj.weight"],
        q_norm=t["w.self_attn.q_norm.weight"], k_norm=t["w.self_attn.k_norm.weight"],
        ln_in=t["w.input_layernorm.weight"], ln_post=t["w.post_attention_layernorm.weight"],
        router=t["w.mlp.gate.weight"], gate_up=t["w.mlp.experts.gate_up_proj"],
        down=t["w.mlp.experts.down_proj"])
    shape = ref.QwenShape(H=H, q_heads=nq, kv_heads=nkv, d=d, E=E, K=K, I=I, eps=1e-6, theta=1e6)
    return lw, shape


def test_qwen_layer_fp32_matches_hf_golden():
    t, meta = _load_golden()
    lw, shape = golden_layer(t, meta)
    kc, vc = t["k_cache"].float().clone(), t["v_cache"].float().clone()
    cos, sin = ref.rope_cos_sin(t["pos"], shape.d, shape.theta)
    assert torch.allclose(cos, t["cos"], atol=1e-6) and torch.allclose(sin, t["sin"], atol=1e-6)
    y, aux = ref.qwen_decoder_layer(t["x"].float(), lw, kc, vc, cos, sin, t["pos"], shape,
                                    emulate_bf16=False)
    assert torch.allclose(y, t["y"], rtol=1e-4, atol=1e-5), (y - t["y"]).abs().max()
    for b, p in enumerate(t["pos"].tolist()):
        assert torch.allclose(kc[b, :, p], t["k_new"][b], atol=1e-5)
        assert torch.allclose(vc[b, :, p], t["v_new"][b], atol=1e-5)
        # rows other than pos[b] untouched
        mask = torch.ones(kc.shape[2], dtype=torch.bool)
        mask[p] = False
        assert torch.equal(kc[b, :, mask], t["k_cache"].float()[b, :, mask])


def test_qwen_layer_bf16_flow_within_tolerance_of_fp32():
    # the reference's bf16 rounding points move the result by O(bf16 eps), well inside 2e-2
    t, meta = _load_golden()
    lw, shape = golden_layer(t, meta)
    cos, sin = ref.rope_cos_sin(t["pos"], shape.d, shape.theta)
    y, _ = ref.qwen_decoder_layer(t["x"].float(), lw, t["k_cache"].float().clone(),
                                  t["v_cache"].float().clone(), cos, sin, t["pos"], shape,
                                  emulate_bf16=True)
    err = (y - t["y"]).abs().max() / t["y"].abs().max()
    assert err < 2e-2, err


def test_block_kv_gather_identity_and_permutation():
    """block_kv_to_flat: an identity table is a reshape; a permuted table moves
    whole blocks; an entry outside the pool reads as zeros."""
    from oracle import ref
    cache = torch.randn(6, 4, 3)
    ident = torch.arange(6).reshape(2, 3)
    assert torch.equal(ref.block_kv_to_flat(cache, ident), cache.reshape(2, 12, 3))
    perm = torch.tensor([[5, 0], [-1, 2]])
    flat = ref.block_kv_to_flat(cache, perm)
    assert torch.equal(flat[0, :4], cache[5]) and torch.equal(flat[0, 4:], cache[0])
    assert torch.equal(flat[1, :4], torch.zeros(4, 3)) and torch.equal(flat[1, 4:], cache[2])


@pytest.mark.parametrize("pos,window", [(5, 0), (11, 8), (3, 8)])
def test_gpt_oss_layer_oracle_matches_hf(pos, window):
    """oracle.ref.gpt_oss_decoder_layer (fp32, no bf16 rounding) == HF
    GptOssDecoderLayer on the last token of a causal (optionally sliding-window)
    prefill, with the decode oracle's KV cache built from the earlier tokens
    (ring rows t % (W-1) for a sliding layer)."""
    from transformers import GptOssConfig
    from transformers.models.gpt_oss import modeling_gpt_oss as M
    from oracle import ref
    torch.manual_seed(pos * 10 + window)
    H, nq, nkv, d, E, K, I = 128, 4, 2, 32, 4, 2, 64
    cfg = GptOssConfig(hidden_size=H, num_attention_heads=nq, num_key_value_heads=nkv, head_dim=d,
                       num_local_experts=E, num_experts_per_tok=K, intermediate_size=I,
                       num_hidden_layers=2, sliding_window=window or 8,
                       layer_types=["sliding_attention" if window else "full_attention"] * 2,
                       rms_norm_eps=1e-5, attn_implementation="eager")
    layer = M.GptOssDecoderLayer(cfg, 0).float().eval()
    with torch.no_grad():
        for p_ in layer.parameters():
            p_.copy_(0.1 * torch.randn_like(p_))
        layer.input_layernorm.weight.add_(1.0)
        layer.post_attention_layernorm.weight.add_(1.0)
    rot = M.GptOssRotaryEmbedding(cfg)
    S = pos + 1
    X = torch.randn(1, S, H)
    ids = torch.arange(S)[None]
    cos, sin = rot(X, ids)
    # HF causal (+ sliding) mask for the prefill, additive
    mask = torch.full((S, S), float("-inf"))
    for i in range(S):
        for j in range(S):
            if j <= i and (not window or i - j < window):
                mask[i, j] = 0.0
    with torch.no_grad():
        y_hf = layer(X, attention_mask=mask[None, None], position_ids=ids,
                     position_embeddings=(cos, sin))
        y_hf = y_hf[0] if isinstance(y_hf, tuple) else y_hf
    a = layer.self_attn
    lw = ref.GptOssLayer(
        wq=a.q_proj.weight.data, bq=a.q_proj.bias.data, wk=a.k_proj.weight.data, bk=a.k_proj.bias.data,
        wv=a.v_proj.weight.data, bv=a.v_proj.bias.data, wo=a.o_proj.weight.data, bo=a.o_proj.bias.data,
        sinks=a.sinks.data, ln_in=layer.input_layernorm.weight.data,
        ln_post=layer.post_attention_layernorm.weight.data,
        router_w=layer.mlp.router.weight.data, router_b=layer.mlp.router.bias.data,
        gate_up=layer.mlp.experts.gate_up_proj.data, gate_up_b=layer.mlp.experts.gate_up_proj_bias.data,
        down=layer.mlp.experts.down_proj.data, down_b=layer.mlp.experts.down_proj_bias.data)
    shape = ref.GptOssShape(H=H, nq=nq, nkv=nkv, d=d, E=E, K=K, I=I)
    # decode cache from tokens 0..pos-1: rmsnorm -> k/v proj (+bias) -> RoPE
    rows = window if window else S
    kc = torch.zeros(1, nkv, rows, d)
    vc = torch.zeros(1, nkv, rows, d)
    for t in range(pos):
        h = ref.rmsnorm_tkg(X[0, t][None], lw.ln_in, shape.eps)
        k = (h @ lw.wk.t() + lw.bk).reshape(1, nkv, d)
        v = (h @ lw.wv.t() + lw.bv).reshape(1, nkv, d)
        k = ref.gpt_oss_rope(k, cos[0, t][None, : d // 2], sin[0, t][None, : d // 2])
        r = t % (window - 1) if window else t
        kc[0, :, r] = k[0]
        vc[0, :, r] = v[0]
    y, _ = ref.gpt_oss_decoder_layer(X[0, pos][None], lw, kc, vc, cos[0, pos][None, : d // 2],
                                     sin[0, pos][None, : d // 2], torch.tensor([pos]), window, shape,
                                     emulate_bf16=False)
    torch.testing.assert_close(y[0], y_hf[0, pos], rtol=2e-5, atol=2e-5)


def test_forced_routing_identity_and_pairing():
    """force_idx (routing teacher-forcing in the GPU tests): forcing the oracle's own
    top-k reproduces it exactly; forcing the same experts in another rank order
    gives the same layer output in the fp32 flow (each weight stays with its
    expert; only the order of the fp32 sum over k changes)."""
    t, meta = _load_golden()
    lw, shape = golden_layer(t, meta)
    cos, sin = ref.rope_cos_sin(t["pos"], shape.d, shape.theta)
    x = t["x"].float()

    def run(force, emulate):
        return ref.qwen_decoder_layer(x, lw, t["k_cache"].float().clone(), t["v_cache"].float().clone(),
                                      cos, sin, t["pos"], shape, emulate_bf16=emulate, force_idx=force)

    for emulate in (True, False):
        y0, aux = run(None, emulate)
        y1, aux1 = run(aux["idx"], emulate)
        assert torch.equal(y0, y1) and torch.equal(aux["w"], aux1["w"])
    y0, aux = run(None, False)
    perm = aux["idx"].flip(-1)
    y2, aux2 = run(perm, False)
    assert torch.allclose(y2, y0, rtol=0, atol=1e-5)
    assert torch.allclose(aux2["w"], aux["w"].flip(-1), atol=1e-7)
    # a different expert set moves the output
    other = (aux["idx"] + 1) % shape.E
    y3, _ = run(other, False)
    assert (y3 - y0).abs().max() > 1e-3


# ------------------------------------------------------------ KV cache formats
def test_kv_fp8_quant_matches_independent_e4m3_and_known_answers():
    """kv_fp8_quant (torch's float8_e4m3fn cast after the clip) against the
    independent numpy e4m3 quantiser of oracle/mx.py, over the whole range,
    plus known answers: the +-240 clip, round-to-nearest-even ties, subnormals."""
    import numpy as np
    from oracle import mx
    g = torch.Generator().manual_seed(11)
    x = torch.cat([torch.randn(4096, generator=g) * 10 ** torch.empty(4096).uniform_(-4, 3, generator=g),
                   torch.tensor([0.0, -0.0, 1e-12, 300.0, -1e4])])
    for scale in (1.0, 0.37, 16.0):
        q = ref.kv_fp8_quant(x, scale)
        y = (x * scale).clamp(-240, 240).numpy().astype(np.float64)
        codes = mx.quantize_elements(y, "e4m3")
        assert np.array_equal(q.view(torch.uint8).numpy() & 0x7f, codes & 0x7f)
        nz = y != 0
        assert np.array_equal(q.view(torch.uint8).numpy()[nz], codes[nz])
    kat = {1000.0: 240.0, -1000.0: -240.0, 239.0: 240.0, 1.0625: 1.0, 1.1875: 1.25,
           2.0 ** -10: 0.0, 3 * 2.0 ** -10: 2.0 ** -8, 2.0 ** -9: 2.0 ** -9, 0.0: 0.0}
    for xin, want in kat.items():
        assert ref.kv_fp8_quant(torch.tensor([xin]), 1.0).float().item() == want, xin


def _attn_case(seed, B=2, S=1, nq=4, d=64, H=128, P=20, S_max=40):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    W = (0.05 * torch.randn(H, d * (nq + 2), generator=g))
    Kc = torch.randn(B, S_max, d, generator=g)
    Vc = torch.randn(B, S_max, d, generator=g)
    mask = (torch.rand(P + S, B, nq, S, generator=g) > 0.2).float()
    mask[P:] = 1
    upd = torch.tensor([[P]] * B)
    return X, W, Kc, Vc, mask, upd


def _run_attn(X, W, Kc, Vc, mask, upd, **kw):
    return ref.attention_block_tkg(X, W, None, None, None, None, None, 1e-6, None, None,
                                   Kc, Vc, mask, None, True, upd, None, None, **kw)


def test_transposed_k_cache_equals_row_layout():
    """K_cache_transposed reads and writes the same logical cache: results and
    the written column equal the [S, d] layout's on the same data."""
    X, W, Kc, Vc, mask, upd = _attn_case(3, S=2)
    K1, V1 = Kc.clone(), Vc.clone()
    o1, _, _ = _run_attn(X, W, K1, V1, mask, upd)
    Kt, V2 = Kc.transpose(1, 2).contiguous(), Vc.clone()
    o2, _, _ = _run_attn(X, W, Kt, V2, mask, upd, K_cache_transposed=True)
    assert torch.equal(o1, o2)
    assert torch.equal(Kt.transpose(1, 2), K1) and torch.equal(V1, V2)
    p = int(upd[0, 0])
    assert not torch.equal(Kt[:, :, p], Kc.transpose(1, 2)[:, :, p])   # the column was written


def test_fp8_kv_scales_multiply_and_are_not_undone():
    """FP8 KV: the scales multiply the stored values and the attention does not
    divide them out.  With power-of-two scales (no clipping, no subnormals),
    quantisation commutes with the scale, so k_scale = 2 with softmax_scale / 2
    equals k_scale = 1, and v_scale = 2 doubles the output (up to the few new
    elements below 2^-6, whose subnormal quantum does not scale).  An oracle
    that dequantised (or divided by the scale) is off by O(1) in both."""
    X, W, Kc, Vc, mask, upd = _attn_case(5)
    Kq = ref.kv_fp8_quant(Kc, 1.0)
    Vq = ref.kv_fp8_quant(Vc, 1.0)
    s = 1.0 / 8.0
    o1, K1, V1 = _run_attn(X, W, Kq.clone(), Vq.clone(), mask, upd, k_scale=1.0, v_scale=1.0,
                           softmax_scale=s)
    # the cache doubled for K (exact in e4m3), scores rescaled back
    o2, K2, _ = _run_attn(X, W, ref.kv_fp8_quant(Kq.float() * 2, 1.0), Vq.clone(), mask, upd,
                          k_scale=2.0, v_scale=1.0, softmax_scale=s / 2)
    assert torch.allclose(o1, o2, rtol=2e-3, atol=2e-4)
    assert (o1 - o2).abs().max() < 1e-2 * o1.abs().max()
    o3, _, V3 = _run_attn(X, W, Kq.clone(), ref.kv_fp8_quant(Vq.float() * 2, 1.0), mask, upd,
                          k_scale=1.0, v_scale=2.0, softmax_scale=s)
    assert torch.allclose(o3, 2 * o1, rtol=2e-3, atol=2e-4)
    # the new row is stored quantised, and a fp8 cache of exactly representable
    # values with unit scales gives the bf16-valued attention of those values
    p = int(upd[0, 0])
    assert K1.dtype == torch.float8_e4m3fn
    assert not torch.equal(K1[:, p].float(), Kq[:, p].float())


# ------------------------------------------------- static FP8 projections
def _fp8_values(g, *shape, std=1.0):
    return ref.kv_fp8_quant(std * torch.randn(*shape, generator=g), 1.0).float()


def test_static_fp8_projection_reduces_to_plain_on_e4m3_values():
    """Inputs and weights that are e4m3 values, unit scales: the static path is the
    plain projection (quantisation is the identity there, the scales neutral);
    power-of-two input scales that keep x / s_in in range do not change the
    result (s_in divides the input and multiplies the output back); the weight
    scale multiplies.  Clipping saturates at +-240."""
    g = torch.Generator().manual_seed(21)
    x = _fp8_values(g, 4, 64)
    W = _fp8_values(g, 64, 48, std=0.1)
    b = torch.randn(48, generator=g).to(torch.bfloat16)
    plain = x @ W + b.float()
    ones = torch.ones(48)
    assert torch.allclose(ref.static_fp8_linear(x, W, ones, 1.0, b), plain, rtol=1e-6, atol=1e-5)
    for s_in in (0.5, 0.25):    # x / s_in stays below 240 and normal
        assert torch.allclose(ref.static_fp8_linear(x, W, ones, s_in, b), plain, rtol=1e-6, atol=1e-5)
    assert torch.allclose(ref.static_fp8_linear(x, W, 3 * ones, 1.0), 3 * (x @ W), rtol=1e-6, atol=1e-5)
    big = ref.static_fp8_linear(torch.full((1, 64), 1e4), torch.eye(64)[:, :16], torch.ones(16), 1.0)
    assert torch.equal(big, torch.full((1, 16), 240.0))


def test_static_fp8_qkv_segments_map_to_q_k_v():
    """Weight scale j of the QKV projection scales the Q (j=0), K (1), V (2)
    columns: doubling the V scale doubles the attention output (linear in V);
    doubling the Q or the K scale with the softmax scale halved leaves it
    unchanged.  A wrong segment order fails one of the three."""
    g = torch.Generator().manual_seed(23)
    B, nq, d, H, P, S_max = 2, 4, 32, 64, 12, 20
    X = ref.kv_fp8_quant(torch.randn(B, 1, H, generator=g), 1.0).to(torch.bfloat16)
    W = ref.kv_fp8_quant(0.1 * torch.randn(H, d * (nq + 2), generator=g), 1.0)
    Kc = torch.randn(B, S_max, d, generator=g)
    Vc = torch.randn(B, S_max, d, generator=g)
    mask = torch.ones(P + 1, B, nq, 1)
    upd = torch.tensor([[P]] * B)

    def run(ws, sm):
        o, _, _ = ref.attention_block_tkg(X, W, None, None, None, None, None, 1e-6, None, None,
                                          Kc.clone(), Vc.clone(), mask, None, False, upd, None, None,
                                          softmax_scale=sm, qkv_static=(ws, 1.0))
        return o
    s = 1.0 / math.sqrt(d)
    base = run([1.0, 1.0, 1.0], s)
    assert torch.allclose(run([2.0, 1.0, 1.0], s / 2), base, rtol=1e-4, atol=1e-5)
    assert not torch.allclose(run([2.0, 1.0, 1.0], s), base, rtol=1e-3, atol=1e-4)
    # K: only the new token's key is projected; the cache keys are not rescaled, so
    # scale them by hand for the comparison
    o_k, _, _ = ref.attention_block_tkg(X, W, None, None, None, None, None, 1e-6, None, None,
                                        2 * Kc, Vc.clone(), mask, None, False, upd, None, None,
                                        softmax_scale=s / 2, qkv_static=([1.0, 2.0, 1.0], 1.0))
    assert torch.allclose(o_k, base, rtol=1e-4, atol=1e-5)
    o_v, _, _ = ref.attention_block_tkg(X, W, None, None, None, None, None, 1e-6, None, None,
                                        Kc.clone(), 2 * Vc, mask, None, False, upd, None, None,
                                        softmax_scale=s, qkv_static=([1.0, 1.0, 2.0], 1.0))
    assert torch.allclose(o_v, 2 * base, rtol=1e-4, atol=1e-5)


def test_fp8_row_experts_equal_experts_on_dequantised_weights():
    """Per-column dequantisation commutes with the projection: the FP8 row-
    quantised experts equal the bf16-flow experts on weights * column scale (the
    gate and up halves scaled by their own [E, 2, I] rows, down by [E, H]).  With
    unit scales they equal the experts on the e4m3 values.  A scale applied to
    the wrong axis (rows instead of columns, or the gate scale on up) fails."""
    g = torch.Generator().manual_seed(29)
    T, E, K, H, I = 3, 6, 2, 64, 32
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    gu = ref.kv_fp8_quant(10 * torch.randn(E, H, 2, I, generator=g), 1.0)
    dn = ref.kv_fp8_quant(10 * torch.randn(E, I, H, generator=g), 1.0)
    gs = 0.003 * (1 + torch.rand(E, 2, I, generator=g))
    ds = 0.003 * (1 + torch.rand(E, H, generator=g))
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)])
    aff = torch.zeros(T, E).scatter_(1, idx, torch.rand(T, K, generator=g))
    gub = 0.1 * torch.randn(E, 2, I, generator=g)
    y = ref.moe_tkg_fp8_row(x, gu, dn, gs, ds, aff, idx, gub, None, "post")
    y_deq = ref.moe_tkg(x, gu.float() * gs[:, None, :, :], dn.float() * ds[:, None, :], aff, idx,
                        gub, None, "post")
    assert torch.allclose(y, y_deq, rtol=1e-4, atol=1e-5 * y.abs().max().item())
    y1 = ref.moe_tkg_fp8_row(x, gu, dn, torch.ones(E, 2, I), torch.ones(E, H), aff, idx)
    assert torch.allclose(y1, ref.moe_tkg(x, gu.float(), dn.float(), aff, idx), rtol=1e-5, atol=1e-4)
    y_swapped = ref.moe_tkg_fp8_row(x, gu, dn, gs.flip(1), ds, aff, idx, gub, None, "post")
    assert not torch.allclose(y_swapped, y, rtol=1e-2, atol=1e-3 * y.abs().max().item())
