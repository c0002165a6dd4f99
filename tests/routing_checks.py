"""Routing-log checks shared by the GPU parity tests (imported, not collected).

A routing record is what one layer's router produced on the GPU (the model's
route log): idx [B, K] int32, w [B, K] fp32, logits [B, E] fp32 and the
post-attention residual r [B, H] bf16 the router normalised.  The contract
(megakernels/qwen3_moe/moe_fused_nki.py:159-276, nki_kernels/moe/
router_topk.py:626-646): expert indices bit-exact, excluding fp32 router-logit
near-ties (gap < 1e-4); ties go to the lowest expert index.
"""
import torch

from oracle import ref

TIE = 1e-4


def stable_order(x):
    """Indices sorted by value descending, lowest index first among equal values."""
    return torch.sort(-x, dim=-1, stable=True).indices


def check_selection(rec, K):
    """The GPU's indices are exactly the stable top-k of the GPU's own logits."""
    want = stable_order(rec["logits"])[:, :K].to(torch.int32)
    assert torch.equal(rec["idx"], want), (rec["idx"], want)


def check_against_oracle_logits(idx_gpu, logits_ref, K, tie=TIE):
    """Indices equal to the stable top-k of the oracle logits, except rows whose
    order is decided by a near-tie (gap < tie) at or above the K-th position."""
    order = stable_order(logits_ref)
    vals = torch.gather(logits_ref, 1, order)
    flips = 0
    for t in range(idx_gpu.shape[0]):
        if torch.equal(idx_gpu[t].long(), order[t, :K]):
            continue
        gaps = (vals[t, :-1] - vals[t, 1:])[:K]
        assert (gaps < tie).any(), f"token {t}: gpu {idx_gpu[t].tolist()} vs oracle {order[t, :K].tolist()}"
        assert set(idx_gpu[t].tolist()) <= set(order[t, :K + 2].tolist())
        flips += 1
    return flips


def check_qwen_routing(rec, lw, eps, K):
    """Qwen3 flow: router on the fp32 norm of the logged residual
    (moe_fused_nki.py:70-153, 159-276), weights softmax-at-top-k -> bf16 -> bf16
    L1 renormalisation (:252-272, :404-418)."""
    check_selection(rec, K)
    n32 = ref.rmsnorm_tkg(rec["r"].float(), lw.ln_post, eps)
    lg_o, idx_o, w_o = ref.qwen_router(n32, lw.router.float().t(), K)
    # fp32 normed rows carried as bf16 hi + lo: ~2^-16 relative per element
    assert (rec["logits"] - lg_o).abs().max().item() < 5e-5
    check_against_oracle_logits(rec["idx"], lg_o, K)
    _, _, w_gpu_formula = ref.qwen_router_from_logits(rec["logits"], K)
    assert torch.allclose(rec["w"], w_gpu_formula, rtol=2 ** -7, atol=1e-6)
    assert torch.allclose(rec["w"].sum(-1), torch.ones(rec["w"].shape[0]), atol=2e-2)


def check_oracle_flips(idx_gpu, logits_gpu, logits_own, K):
    """Tokens whose routing by the oracle's own top-k (on its own residual)
    differs from the GPU's: each GPU expert outside the oracle's top-k must sit
    within twice the measured logit difference of the oracle's K-th logit."""
    dl = (logits_gpu - logits_own).abs().max().item()
    order = stable_order(logits_own)
    flips = 0
    for t in range(idx_gpu.shape[0]):
        own = set(order[t, :K].tolist())
        extra = [e for e in idx_gpu[t].tolist() if e not in own]
        if not extra:
            continue
        flips += 1
        kth = logits_own[t, order[t, K - 1]].item()
        for e in extra:
            assert kth - logits_own[t, e].item() <= 2 * dl + 1e-6, (t, e, kth, dl)
    return flips, dl
