"""GPU parity of attention_block_tkg's optional KV cache formats against the CPU
oracle (through the C ABI): the FP8 e4m3 KV cache (k_scale / v_scale,
attention_block_tkg.py:133-134, :749-754, :1694-1737) and the transposed K
cache (K_cache_transposed, :112, :197-202), flat and block caches, one and
several new tokens per sequence.

Tolerances: output max-abs-rel <= 2e-2 (the oracle runs the same stored fp8
values in fp32).  Written cache rows: exactly the target rows change; bf16 rows
within 2e-2 of the oracle's; e4m3 codes equal the oracle's except where the
GPU's bf16 k / v differs from the oracle's fp32 one by a rounding and lands on
the other side of an e4m3 rounding boundary -- such codes differ by one step
(<= 1/8 relative, or one subnormal quantum 2^-9) and are at most 3 % of a row.
"""
import pytest
import torch

from conftest import max_abs_rel
from oracle import ref

pytestmark = pytest.mark.gpu

TOL = 2e-2


def bf(t):
    return t.to(torch.bfloat16)


def _rope_rows(B, S, P, d):
    cos, sin = ref.rope_cos_sin((torch.arange(S)[None, :] + P + 3 * torch.arange(B)[:, None]).reshape(-1), d, 1e6)
    cos_r = cos[:, :d // 2].reshape(B, S, d // 2).permute(2, 0, 1).contiguous()   # [d/2, B, S]
    sin_r = sin[:, :d // 2].reshape(B, S, d // 2).permute(2, 0, 1).contiguous()
    return cos_r, sin_r


def _mask(g, P, B, nq, S, keep=0.8):
    """[P + S, B, nq, S]: random prior slots, then causal among the S new tokens."""
    prior = (torch.rand(P, B, nq, S, generator=g) < keep).to(torch.bfloat16)
    causal = (torch.arange(S)[:, None] <= torch.arange(S)[None, :]).to(torch.bfloat16)
    return torch.cat([prior, causal[:, None, None, :].expand(S, B, nq, S)], 0).contiguous()


def _assert_codes_close(got, want):
    """e4m3 rows: equal codes, or one rounding step apart on a small fraction."""
    gb, wb = got.view(torch.uint8), want.view(torch.uint8)
    diff = gb != wb
    assert diff.float().mean().item() <= 0.03, f"{int(diff.sum())} of {diff.numel()} codes differ"
    if diff.any():
        gv, wv = got.float()[diff], want.float()[diff]
        assert ((gv - wv).abs() <= wv.abs() / 8 + 2.0 ** -9 + 1e-12).all()


def _call(mk, dev, X, W, Wo, qn, kn, cos_r, sin_r, Kg, Vg, mask, sk, upd, table, kt, ks, vs, scale):
    from nki_moe_megakernel_amd.common_types import QuantizationType
    return mk.attention_block_tkg(
        X.to(dev), None, False, 1e-6, None, W.to(dev), None,
        QuantizationType.NONE, None, None, qn is not None, 1e-6,
        qn.to(dev) if qn is not None else None, kn.to(dev) if kn is not None else None,
        cos_r.to(dev), sin_r.to(dev), True, False, 1e-6, None, None,
        kt, table.to(dev) if table is not None else None, Kg, Vg, mask.to(dev),
        sk.to(dev) if sk is not None else None, True, upd.to(dev),
        Wo.to(dev) if Wo is not None else None, None, QuantizationType.NONE, None, None, False, False,
        softmax_scale=scale, k_scale=ks.to(dev) if ks is not None else None,
        v_scale=vs.to(dev) if vs is not None else None)


@pytest.mark.parametrize("fp8,kt,B,H,nq,nkv,d,S,P,S_max,qknorm,sink,wout", [
    (True, False, 2, 512, 8, 1, 128, 1, 300, 384, True, False, True),
    (True, False, 3, 256, 8, 2, 64, 1, 70, 96, False, True, True),
    (False, True, 2, 512, 8, 1, 128, 1, 500, 512, True, False, True),
    (False, True, 2, 256, 16, 2, 64, 2, 40, 64, False, True, False),
    (True, True, 1, 2048, 32, 4, 128, 1, 1000, 1024, True, False, True),
    (True, False, 2, 512, 16, 2, 128, 4, 200, 256, True, True, True),
    (True, True, 2, 256, 4, 1, 128, 3, 9, 16, False, False, True),
])
def test_attention_kv_formats_flat(mk, dev, fp8, kt, B, H, nq, nkv, d, S, P, S_max, qknorm, sink, wout):
    """Flat caches ([B, S_max, d] / [B, kv_heads, S_max, d]; K as [.., d, S_max]
    when transposed) against the oracle per kv head; the last sequence skips its
    cache update (uint32 max)."""
    print(f"kv formats flat: fp8={fp8} kt={kt} B={B} nq={nq} nkv={nkv} d={d} S={S} P={P}", flush=True)
    g = torch.Generator().manual_seed(B * 131 + S * 17 + P + 7 * fp8 + 3 * kt)
    X = bf(torch.randn(B, S, H, generator=g))
    W = bf(0.03 * torch.randn(H, d * (nq + 2 * nkv), generator=g))
    Wo = bf(0.03 * torch.randn(nq * d, H, generator=g)) if wout else None
    qn = bf(1 + 0.1 * torch.randn(1, d, generator=g)) if qknorm else None
    kn = bf(1 + 0.1 * torch.randn(1, d, generator=g)) if qknorm else None
    k_val = 0.5 if fp8 else 1.0
    v_val = 2.0 if fp8 else 1.0
    # caches as [B, nkv, S_max, d] logical values
    K4 = torch.randn(B, nkv, S_max, d, generator=g)
    V4 = torch.randn(B, nkv, S_max, d, generator=g)
    if fp8:
        K4 = ref.kv_fp8_quant(K4, k_val)
        V4 = ref.kv_fp8_quant(V4, v_val)
        ks = torch.tensor([[k_val]], dtype=torch.float32)
        vs = torch.full((128, 1), v_val, dtype=torch.bfloat16)     # (PMAX, 1) replicated
    else:
        K4, V4 = bf(K4), bf(V4)
        ks = vs = None
    Kst = K4.transpose(2, 3).contiguous() if kt else K4          # stored K layout
    Kdev = Kst if nkv > 1 else Kst[:, 0]
    Vdev = V4 if nkv > 1 else V4[:, 0]
    cos_r, sin_r = _rope_rows(B, S, P, d)
    mask = _mask(g, P, B, nq, S)
    sk = torch.randn(nq, 1, generator=g) if sink else None
    upd = torch.full((B, 1), P, dtype=torch.int64)
    if B > 1:
        upd[-1, 0] = 0xFFFFFFFF
    scale = 1.0 / ((d ** 0.5) * k_val)
    Kg, Vg = Kdev.contiguous().to(dev), Vdev.contiguous().to(dev)
    out, K2, V2 = _call(mk, dev, X, W, Wo, qn, kn, cos_r, sin_r, Kg, Vg, mask, sk, upd, None, kt,
                        ks, vs, scale)
    assert K2 is Kg and V2 is Vg
    gqa = nq // nkv
    attn = torch.zeros(B * S, nq * d)
    Kr, Vr = Kst.clone(), V4.clone()
    for h in range(nkv):
        cols = torch.cat([torch.arange(h * gqa * d, (h + 1) * gqa * d),
                          nq * d + h * d + torch.arange(d),
                          (nq + nkv) * d + h * d + torch.arange(d)])
        Kh, Vh = Kr[:, h].clone(), Vr[:, h].clone()
        o, Kh2, Vh2 = ref.attention_block_tkg(
            X.float(), W.float()[:, cols], None, 1e-6, None,
            qn.float() if qknorm else None, kn.float() if qknorm else None, 1e-6, cos_r, sin_r,
            Kh, Vh, mask[:, :, h * gqa:(h + 1) * gqa].float(),
            sk[h * gqa:(h + 1) * gqa] if sink else None, True, upd, None, None,
            softmax_scale=scale, k_scale=k_val if fp8 else None, v_scale=v_val if fp8 else None,
            K_cache_transposed=kt)
        attn[:, h * gqa * d:(h + 1) * gqa * d] = o
        Kr[:, h], Vr[:, h] = Kh2, Vh2
    y_ref = attn @ Wo.float() if wout else attn.reshape(B, S, nq, d).permute(0, 2, 3, 1)
    assert max_abs_rel(out, y_ref) < TOL
    # the cache: exactly rows P .. P+S-1 of the updated sequences changed
    Kn = Kg.cpu().reshape(Kst.shape)
    Vn = Vg.cpu().reshape(V4.shape)
    Kn_rows = Kn.transpose(2, 3) if kt else Kn                     # [B, nkv, S_max, d]
    Kr_rows = Kr.transpose(2, 3) if kt else Kr
    K0_rows = K4
    for b in range(B):
        ch = (Kn_rows[b].view(torch.uint8 if fp8 else torch.int16) !=
              K0_rows[b].view(torch.uint8 if fp8 else torch.int16)).any(-1).any(0)
        chv = (Vn[b].view(torch.uint8 if fp8 else torch.int16) !=
               V4[b].view(torch.uint8 if fp8 else torch.int16)).any(-1).any(0)
        expect = [] if int(upd[b, 0]) == 0xFFFFFFFF else list(range(P, P + S))
        # a new row may equal the old one only by chance: compare against the oracle's rows
        assert set(ch.nonzero().flatten().tolist()) <= set(expect)
        assert set(chv.nonzero().flatten().tolist()) <= set(expect)
        if not expect:
            continue
        if fp8:
            _assert_codes_close(Kn_rows[b, :, P:P + S], Kr_rows[b, :, P:P + S])
            _assert_codes_close(Vn[b, :, P:P + S], Vr[b, :, P:P + S])
        else:
            assert max_abs_rel(Kn_rows[b, :, P:P + S], Kr_rows[b, :, P:P + S]) < TOL
            assert max_abs_rel(Vn[b, :, P:P + S], Vr[b, :, P:P + S]) < TOL
        # every other row untouched (bitwise)
        keep = torch.ones(S_max, dtype=torch.bool)
        keep[P:P + S] = False
        assert torch.equal(Kn_rows[b, :, keep].contiguous().view(torch.uint8),
                           K0_rows[b, :, keep].contiguous().view(torch.uint8))


def test_attention_fp8_block_kv(mk, dev):
    """FP8 e4m3 block cache [num_blocks, block_len, kv_heads, d] through a block
    table (one sequence's table with an invalid entry), global write rows."""
    print("kv formats: fp8 block cache", flush=True)
    B, H, nq, nkv, d, blk, n_act, nb = 2, 512, 8, 2, 128, 16, 5, 14
    g = torch.Generator().manual_seed(99)
    X = bf(torch.randn(B, 1, H, generator=g))
    W = bf(0.03 * torch.randn(H, d * (nq + 2 * nkv), generator=g))
    Wo = bf(0.03 * torch.randn(nq * d, H, generator=g))
    Kc = ref.kv_fp8_quant(torch.randn(nb, blk, nkv, d, generator=g), 0.75)
    Vc = ref.kv_fp8_quant(torch.randn(nb, blk, nkv, d, generator=g), 1.5)
    perm = torch.randperm(nb, generator=g)                 # disjoint blocks per sequence
    table = torch.stack([perm[b * n_act:(b + 1) * n_act] for b in range(B)]).to(torch.int32)
    table[1, 4] = -1                                      # an absent block reads as zero rows
    S_ctx = n_act * blk
    P = S_ctx - 1 - 20                                     # the new token's slot index
    cos_r, sin_r = _rope_rows(B, 1, P, d)
    mask = torch.zeros(S_ctx, B, nq, 1, dtype=torch.bfloat16)
    mask[:P] = (torch.rand(P, B, nq, 1, generator=g) < 0.8).to(torch.bfloat16)
    mask[-1] = 1
    # the new token of sequence b goes to its position P: block table[b, P // blk]
    rows = [int(table[b, P // blk]) * blk + P % blk for b in range(B)]
    upd = torch.tensor(rows, dtype=torch.int64).reshape(B, 1)
    ks = torch.tensor([[0.75]], dtype=torch.float32)
    vs = torch.tensor([[1.5]], dtype=torch.float16)
    scale = 1.0 / (d ** 0.5 * 0.75)
    Kg, Vg = Kc.to(dev), Vc.to(dev)
    out, _, _ = _call(mk, dev, X, W, Wo, None, None, cos_r, sin_r, Kg, Vg, mask, None, upd, table,
                      False, ks, vs, scale)
    # oracle on the flat view (mask slots P .. S_ctx-2 are masked; slot S_ctx-1 is the new token)
    Kf = ref.block_kv_to_flat(Kc, table)                   # [B, S_ctx, nkv, d]
    Vf = ref.block_kv_to_flat(Vc, table)
    gqa = nq // nkv
    attn = torch.zeros(B, nq * d)
    newk = torch.zeros(B, nkv, d, dtype=torch.float8_e4m3fn)
    newv = torch.zeros(B, nkv, d, dtype=torch.float8_e4m3fn)
    for h in range(nkv):
        cols = torch.cat([torch.arange(h * gqa * d, (h + 1) * gqa * d),
                          nq * d + h * d + torch.arange(d),
                          (nq + nkv) * d + h * d + torch.arange(d)])
        Kh = Kf[:, :, h].contiguous()
        Vh = Vf[:, :, h].contiguous()
        slot = torch.full((B, 1), S_ctx - 1)
        o, Kh2, Vh2 = ref.attention_block_tkg(
            X.float(), W.float()[:, cols], None, 1e-6, None, None, None, 1e-6, cos_r, sin_r,
            Kh, Vh, mask[:, :, h * gqa:(h + 1) * gqa].float(), None, True, slot, None, None,
            softmax_scale=scale, k_scale=0.75, v_scale=1.5)
        attn[:, h * gqa * d:(h + 1) * gqa * d] = o
        newk[:, h], newv[:, h] = Kh2[:, S_ctx - 1], Vh2[:, S_ctx - 1]
    assert max_abs_rel(out, attn @ Wo.float()) < TOL
    Kn, Vn = Kg.cpu(), Vg.cpu()
    flat_rows = (Kn.view(torch.uint8) != Kc.view(torch.uint8)).reshape(nb * blk, -1).any(-1)
    assert set(flat_rows.nonzero().flatten().tolist()) <= set(rows)
    for b in range(B):
        r = rows[b]
        _assert_codes_close(Kn.reshape(nb * blk, nkv, d)[r], newk[b])
        _assert_codes_close(Vn.reshape(nb * blk, nkv, d)[r], newv[b])


def test_attention_kv_formats_reject(mk, dev):
    """A transposed K cache with a block table, and an fp8 cache without both
    scales, are rejected before any launch."""
    from nki_moe_megakernel_amd.common_types import QuantizationType
    B, H, nq, d, S_max = 1, 256, 4, 64, 32
    X = torch.zeros(B, 1, H, dtype=torch.bfloat16, device=dev)
    W = torch.zeros(H, d * (nq + 2), dtype=torch.bfloat16, device=dev)
    mask = torch.ones(S_max, B, nq, 1, dtype=torch.bfloat16, device=dev)
    upd = torch.zeros(B, 1, dtype=torch.int64, device=dev)
    Kb = torch.zeros(4, 8, d, dtype=torch.bfloat16, device=dev)
    table = torch.zeros(B, 4, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="block KV"):
        mk.attention_block_tkg(X, None, False, 1e-6, None, W, None, QuantizationType.NONE, None, None,
                               False, 1e-6, None, None, None, None, True, False, 1e-6, None, None,
                               True, table, Kb, Kb.clone(), mask, None, True, upd, None, None,
                               QuantizationType.NONE, None, None, False, False)
    K8 = torch.zeros(B, S_max, d, dtype=torch.uint8, device=dev).view(torch.float8_e4m3fn)
    with pytest.raises(ValueError, match="float8_e4m3 needs k_scale"):
        mk.attention_block_tkg(X, None, False, 1e-6, None, W, None, QuantizationType.NONE, None, None,
                               False, 1e-6, None, None, None, None, True, False, 1e-6, None, None,
                               False, None, K8, K8.clone(), mask, None, True, upd, None, None,
                               QuantizationType.NONE, None, None, False, False,
                               k_scale=torch.ones(1, 1, device=dev))


@pytest.mark.parametrize("B,H,nq,nkv,d,S,P,S_max,norm,bias,q_st,o_st,fp8kv", [
    (2, 512, 8, 1, 128, 1, 100, 128, True, True, True, True, False),
    (3, 256, 8, 2, 64, 2, 30, 64, False, False, True, False, True),
    (1, 2048, 32, 4, 128, 1, 500, 512, True, True, False, True, False),
    (48, 256, 4, 1, 64, 2, 10, 16, True, True, True, True, False),
])
def test_attention_static_fp8_projections(mk, dev, B, H, nq, nkv, d, S, P, S_max, norm, bias,
                                          q_st, o_st, fp8kv):
    """quantization_type_qkv / _out = STATIC: e4m3 weights, the input quantised
    by 1 / input scale and clipped to +-240, per-segment (Q / K / V) weight
    scales, bias after the dequantisation -- against the oracle per kv head."""
    from nki_moe_megakernel_amd.common_types import QuantizationType
    print(f"static fp8 projections: B={B} S={S} nq={nq} nkv={nkv} q={q_st} o={o_st} fp8kv={fp8kv}", flush=True)
    g = torch.Generator().manual_seed(B * 7 + S * 3 + P + 11 * q_st + 5 * o_st)
    X = bf(torch.randn(B, S, H, generator=g))
    I = d * (nq + 2 * nkv)
    gamma = bf(1 + 0.1 * torch.randn(1, H, generator=g)) if norm else None
    wsq = torch.tensor([0.002, 0.003, 0.0025])
    s_in_q, s_in_o, ws_o = 1.0 / 32, 1.0 / 16, 0.0015
    if q_st:
        Wq = ref.kv_fp8_quant(0.03 * torch.randn(H, I, generator=g), 1.0 / 0.0025)
    else:
        Wq = bf(0.03 * torch.randn(H, I, generator=g))
    if o_st:
        Wo = ref.kv_fp8_quant(0.03 * torch.randn(nq * d, H, generator=g), 1.0 / ws_o)
    else:
        Wo = bf(0.03 * torch.randn(nq * d, H, generator=g))
    bq = bf(0.1 * torch.randn(1, I, generator=g)) if bias else None
    bo = bf(0.1 * torch.randn(1, H, generator=g)) if bias else None
    K4 = torch.randn(B, nkv, S_max, d, generator=g)
    V4 = torch.randn(B, nkv, S_max, d, generator=g)
    if fp8kv:
        K4, V4 = ref.kv_fp8_quant(K4, 1.0), ref.kv_fp8_quant(V4, 1.0)
    else:
        K4, V4 = bf(K4), bf(V4)
    cos_r, sin_r = _rope_rows(B, S, P, d)
    mask = _mask(g, P, B, nq, S)
    upd = torch.full((B, 1), P, dtype=torch.int64)
    one = torch.ones(1, 1)
    Kg = (K4 if nkv > 1 else K4[:, 0]).contiguous().to(dev)
    Vg = (V4 if nkv > 1 else V4[:, 0]).contiguous().to(dev)
    out, _, _ = mk.attention_block_tkg(
        X.to(dev), None, norm, 1e-6, gamma.to(dev) if norm else None, Wq.to(dev),
        bq.to(dev) if bias else None,
        QuantizationType.STATIC if q_st else QuantizationType.NONE,
        wsq.reshape(1, 3).expand(128, 3).contiguous().to(dev) if q_st else None,
        torch.full((1, 1), s_in_q).to(dev) if q_st else None,
        False, 1e-6, None, None, cos_r.to(dev), sin_r.to(dev), True, False, 1e-6, None, None,
        False, None, Kg, Vg, mask.to(dev), None, True, upd.to(dev), Wo.to(dev),
        bo.to(dev) if bias else None,
        QuantizationType.STATIC if o_st else QuantizationType.NONE,
        torch.full((128, 1), ws_o).to(dev) if o_st else None,
        torch.full((128, 1), s_in_o).to(dev) if o_st else None, False, False,
        k_scale=one.to(dev) if fp8kv else None, v_scale=one.to(dev) if fp8kv else None)
    gqa = nq // nkv
    attn = torch.zeros(B * S, nq * d)
    for h in range(nkv):
        cols = torch.cat([torch.arange(h * gqa * d, (h + 1) * gqa * d),
                          nq * d + h * d + torch.arange(d),
                          (nq + nkv) * d + h * d + torch.arange(d)])
        o, _, _ = ref.attention_block_tkg(
            X.float(), Wq[:, cols] if q_st else Wq.float()[:, cols], gamma.float() if norm else None,
            1e-6, bq.reshape(-1)[cols] if bias else None, None, None, 1e-6, cos_r, sin_r,
            K4[:, h].clone(), V4[:, h].clone(), mask[:, :, h * gqa:(h + 1) * gqa].float(), None, True,
            upd, None, None, k_scale=1.0 if fp8kv else None, v_scale=1.0 if fp8kv else None,
            qkv_static=(wsq, s_in_q) if q_st else None)
        attn[:, h * gqa * d:(h + 1) * gqa * d] = o
    if o_st:
        y_ref = ref.static_fp8_linear(attn, Wo, torch.full((H,), ws_o), s_in_o, bo)
    else:
        y_ref = attn @ Wo.float() + (bo.float() if bias else 0.0)
    assert max_abs_rel(out, y_ref) < TOL


@pytest.mark.parametrize("T,E,K,H,I,act,bias", [
    (1, 128, 8, 2048, 768, "silu", False),
    (5, 16, 4, 512, 128, "silu", True),
    (40, 32, 4, 256, 64, "swish", True),
    (128, 8, 2, 128, 32, "gelu", False),
])
def test_moe_tkg_fp8_row(mk, dev, T, E, K, H, I, act, bias):
    """moe_tkg with FP8 row-quantised experts (e4m3 [E, H, 2, I] / [E, I, H],
    fp32 scales [E, 2, I] / [E, H]) against the oracle; STATIC (input scales)
    is rejected as by the reference (moe_tkg.py:405-408)."""
    from nki_moe_megakernel_amd.common_types import ActFnType, ExpertAffinityScaleMode
    print(f"moe fp8 row: T={T} E={E} K={K} H={H} I={I} act={act}", flush=True)
    g = torch.Generator().manual_seed(T * 13 + E + H)
    x = bf(torch.randn(T, H, generator=g))
    gs = 0.003 * (1 + torch.rand(E, 2, I, generator=g))
    ds = 0.003 * (1 + torch.rand(E, H, generator=g))
    gu = ref.kv_fp8_quant(0.03 * torch.randn(E, H, 2, I, generator=g) / gs[:, None, :, :], 1.0)
    dn = ref.kv_fp8_quant(0.03 * torch.randn(E, I, H, generator=g) / ds[:, None, :], 1.0)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    aff = torch.zeros(T, E).scatter_(1, idx.long(), torch.rand(T, K, generator=g))
    gub = bf(0.1 * torch.randn(E, 2, I, generator=g)) if bias else None
    dnb = bf(0.1 * torch.randn(E, H, generator=g)) if bias else None
    actf = {"swish": ActFnType.Swish, "gelu": ActFnType.GELU}.get(act, ActFnType.SiLU)
    out = mk.moe_tkg(x.to(dev), gu.to(dev), dn.to(dev), aff.to(dev), idx.to(dev), False,
                     expert_gate_up_bias=gub.to(dev) if bias else None,
                     expert_down_bias=dnb.to(dev) if bias else None,
                     expert_gate_up_weights_scale=gs.to(dev), expert_down_weights_scale=ds.to(dev),
                     expert_affinities_scaling_mode=ExpertAffinityScaleMode.POST_SCALE,
                     activation_fn=actf)
    y_ref = ref.moe_tkg_fp8_row(x, gu, dn, gs, ds, aff, idx.long(), gub, dnb, "post", act)
    assert out.shape == (T, H)
    assert max_abs_rel(out, y_ref) < TOL
    with pytest.raises(ValueError, match="Static quantization"):
        mk.moe_tkg(x.to(dev), gu.to(dev), dn.to(dev), aff.to(dev), idx.to(dev), False,
                   expert_gate_up_weights_scale=gs[:, :, :1].to(dev), expert_down_weights_scale=ds[:, :1].to(dev),
                   gate_up_input_scale=torch.ones(E, 1, device=dev), down_input_scale=torch.ones(E, 1, device=dev))
