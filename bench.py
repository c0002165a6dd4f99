"""Decode throughput benchmark (one JSON line on stdout).

Workload: 48-layer Qwen3-30B-A3B-shaped MoE model,
random bf16 weights, batch 1, KV context prefilled to 2048 positions with
seeded N(0,1), then greedy decode steps from uniformly drawn token ids.  A
step = embedding -> 48 decoder layers (RMSNorm, QKV, qk-norm, RoPE, split-K
GQA attention + KV scatter, o_proj + residual, RMSNorm, router top-8,
grouped expert GEMMs, residual) -> final norm -> lm_head -> arg-max -> feed
back.  The whole step is captured once as a HIP graph and replayed.

Also reported:
  roofline      -- the dominant kernel (MoE gate/up grouped GEMM) timed live
                   with HIP events carried by each of its dispatch packets, in
                   one eager step of the same workload right after the timed
                   region; algorithmic bytes per launch = distinct experts *
                   2*I*H*2 (weights; activations are < 0.1%).  `traffic` is
                   the HBM bytes per launch measured by rocprofv3 counter runs
                   (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel of
                   known size, `--calib-copy`) and read from
                   profiles/gate_up_traffic.json when its workload matches.
  cpu_baseline  -- the CPU oracle (oracle/ref.py, fp32 torch on the host) on a
                   bounded sample: decode steps over 2 distinct layers' weights
                   (each used for 24 of the 48 layer slots), scaled to tok/s.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--batch B]
       python bench.py --moe-prefill T   (MFMA regime of the expert GEMMs)
       python bench.py --prefill T       (context encoding of a T-token prompt)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_model(Q, cfg, B, dev, seed):
    import torch
    layers = []
    for l in range(cfg.num_hidden_layers):
        hf = Q.random_layer_hf(cfg, l, seed, dev)
        layers.append(Q.pack_layer(hf, cfg.expert_format))
        del hf
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 1)
    emb = (0.02 * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g, device=dev)).to(torch.bfloat16)
    lm = (0.02 * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g, device=dev)).to(torch.bfloat16)
    lnf = (1 + 0.02 * torch.randn(cfg.hidden_size, generator=g, device=dev)).to(torch.bfloat16)
    model = Q.Qwen3MoeMegakernelModel(cfg, layers, B, dev, embed=emb, ln_f=lnf, lm_head=lm)
    del lm
    return model


def build_gpt_oss(G, cfg, B, dev, seed):
    import torch
    layers = []
    for l in range(cfg.num_hidden_layers):
        hf = G.random_layer_hf(cfg, l, seed, dev)
        layers.append(G.pack_layer(hf, cfg))
        del hf
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 1)
    emb = (0.02 * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g, device=dev)).to(torch.bfloat16)
    lm = (0.02 * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g, device=dev)).to(torch.bfloat16)
    lnf = (1 + 0.02 * torch.randn(cfg.hidden_size, generator=g, device=dev)).to(torch.bfloat16)
    model = G.GptOssMegakernelModel(cfg, layers, B, dev, embed=emb, ln_f=lnf, lm_head=lm)
    del lm, emb
    return model


def prefill_kv(model, cfg, ctx, seed, dev):
    import torch
    g = torch.Generator(device=dev)
    g.manual_seed(seed + 2)
    for l in range(cfg.num_hidden_layers):
        for t in (model.kv_mgr.k(l), model.kv_mgr.v(l)):
            if getattr(cfg, "kv_block_len", 0) or t.shape[2] < ctx:   # block pool / ring: every row
                t.copy_(torch.randn(t.shape, generator=g, device=dev))
            else:
                t[:, :, :ctx].copy_(torch.randn(t[:, :, :ctx].shape, generator=g, device=dev))


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(cfg, lens, seconds_budget=20.0):
    """Time the CPU oracle's decode step on host cores (bounded sample).

    The batch and per-sequence KV lengths are the GPU workload's.  Weights of 2
    distinct layers are reused for all layer slots.  When a full 48-layer step
    does not fit the budget, a pass over fewer layers is timed and scaled to 48
    layers (said in `sample`).  Expert math is the bf16-weight oracle in every
    mode (an MX run's CPU leg does not dequantise).
    """
    import torch
    from oracle import ref
    from importlib import import_module
    Q = import_module("nki_moe_megakernel_amd.qwen_with_megakernel")
    torch.set_num_threads(os.cpu_count() or 1)
    cores = torch.get_num_threads()
    B = int(lens.numel())
    n_distinct = 2
    hfs = [Q.random_layer_hf(cfg, l, 77, "cpu") for l in range(n_distinct)]
    lws = [ref.QwenLayer(wq=h["q_proj"], wk=h["k_proj"], wv=h["v_proj"], wo=h["o_proj"],
                         q_norm=h["q_norm"], k_norm=h["k_norm"], ln_in=h["input_layernorm"],
                         ln_post=h["post_attention_layernorm"], router=h["gate"],
                         gate_up=h["gate_up_proj"], down=h["down_proj"]) for h in hfs]
    g = torch.Generator().manual_seed(5)
    S = int(lens.max()) + 64
    kcs = [torch.randn(B, cfg.num_key_value_heads, S, cfg.head_dim, generator=g).to(torch.bfloat16)
           for _ in range(n_distinct)]
    vcs = [torch.randn(B, cfg.num_key_value_heads, S, cfg.head_dim, generator=g).to(torch.bfloat16)
           for _ in range(n_distinct)]
    lm = (0.02 * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g)).to(torch.bfloat16)
    lnf = torch.ones(cfg.hidden_size, dtype=torch.bfloat16)
    shape = ref.QwenShape()
    x0 = torch.randn(B, cfg.hidden_size, generator=g).to(torch.bfloat16).float()
    pos = lens.clone()
    L = cfg.num_hidden_layers

    def layers(x, n, p):
        cos, sin = ref.rope_cos_sin(p, cfg.head_dim, cfg.rope_theta)
        for l in range(n):
            j = l % n_distinct
            x, _ = ref.qwen_decoder_layer(x, lws[j], kcs[j], vcs[j], cos, sin, p, shape)
        return x

    t0 = time.perf_counter()
    layers(x0, 1, pos)
    t1 = time.perf_counter() - t0
    if t1 * L <= seconds_budget:
        steps, t_total = 0, 0.0
        while t_total < seconds_budget and steps < 8:
            t0 = time.perf_counter()
            x = layers(x0, L, pos)
            ref.final_norm_lm_head(x, lnf, lm, cfg.rms_norm_eps)
            t_total += time.perf_counter() - t0
            steps += 1
            pos = pos + 1
        step_s = t_total / steps
        sample = (f"{steps} full {L}-layer bs={B} decode steps of the fp32 torch oracle")
    else:
        n = max(2, min(L, int(seconds_budget / t1)))
        t0 = time.perf_counter()
        x = layers(x0, n, pos)
        t_layers = time.perf_counter() - t0
        t0 = time.perf_counter()
        ref.final_norm_lm_head(x, lnf, lm, cfg.rms_norm_eps)
        t_lm = time.perf_counter() - t0
        t_total = t_layers + t_lm
        step_s = t_layers * L / n + t_lm
        sample = (f"one pass of {n} of {L} layers at bs={B} of the fp32 torch oracle, scaled by "
                  f"{L}/{n}, + lm_head")
    return {"value": B / step_s, "unit": "tok/s", "cores": cores, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{sample}, KV lengths mean {float(lens.float().mean()):.0f} "
                      f"({n_distinct} distinct layers' weights reused for all layer slots), "
                      f"{t_total:.1f} s on {cores} host threads"}


def cpu_baseline_gpt_oss(cfg, lens, seconds_budget=20.0):
    """Time the CPU oracle's GPT-OSS decode layers (bf16 experts, same batch and KV
    lengths, 2 distinct layers' weights reused); a pass over a bounded number of
    layers is scaled to all layers (said in `sample`)."""
    import torch
    from oracle import ref
    from importlib import import_module
    G = import_module("nki_moe_megakernel_amd.gpt_oss_with_megakernel")
    torch.set_num_threads(os.cpu_count() or 1)
    cores = torch.get_num_threads()
    B = int(lens.numel())
    hfs = [G.random_layer_hf(cfg, l, 77, "cpu") for l in range(2)]
    lws = [ref.GptOssLayer(
        wq=h["q_proj.weight"], bq=h["q_proj.bias"], wk=h["k_proj.weight"], bk=h["k_proj.bias"],
        wv=h["v_proj.weight"], bv=h["v_proj.bias"], wo=h["o_proj.weight"], bo=h["o_proj.bias"],
        sinks=h["sinks"], ln_in=h["input_layernorm"], ln_post=h["post_attention_layernorm"],
        router_w=h["router.weight"], router_b=h["router.bias"], gate_up=h["experts.gate_up_proj"],
        gate_up_b=h["experts.gate_up_proj_bias"], down=h["experts.down_proj"],
        down_b=h["experts.down_proj_bias"]) for h in hfs]
    g = torch.Generator().manual_seed(5)
    S = int(lens.max()) + 64
    caches = []
    for l in range(2):
        rows = cfg.sliding_window if cfg.is_sliding(l) else S
        caches.append((torch.randn(B, cfg.num_key_value_heads, rows, cfg.head_dim, generator=g).to(torch.bfloat16),
                       torch.randn(B, cfg.num_key_value_heads, rows, cfg.head_dim, generator=g).to(torch.bfloat16)))
    inv, scl = G.yarn_inv_freq(cfg)
    freqs = lens.reshape(-1, 1).float() * inv[None, :]
    cos, sin = freqs.cos() * scl, freqs.sin() * scl
    shape = ref.GptOssShape(H=cfg.hidden_size, nq=cfg.num_attention_heads, nkv=cfg.num_key_value_heads,
                            d=cfg.head_dim, E=cfg.num_experts, K=cfg.num_experts_per_tok,
                            I=cfg.intermediate_size, eps=cfg.rms_norm_eps)
    x = torch.randn(B, cfg.hidden_size, generator=g).to(torch.bfloat16).float()
    L = cfg.num_hidden_layers
    n, t_layers = 0, 0.0
    while n < L and (n < 2 or t_layers < seconds_budget):
        j = n % 2
        t0 = time.perf_counter()
        x, _ = ref.gpt_oss_decoder_layer(x, lws[j], caches[j][0], caches[j][1], cos, sin, lens,
                                         cfg.sliding_window if cfg.is_sliding(j) else 0, shape)
        t_layers += time.perf_counter() - t0
        n += 1
    lm = (0.02 * torch.randn(cfg.vocab_size, cfg.hidden_size, generator=g)).to(torch.bfloat16)
    t0 = time.perf_counter()
    ref.final_norm_lm_head(x, torch.ones(cfg.hidden_size, dtype=torch.bfloat16), lm, cfg.rms_norm_eps)
    t_lm = time.perf_counter() - t0
    step_s = t_layers * L / n + t_lm
    return {"value": B / step_s, "unit": "tok/s", "cores": cores, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{n} of {L} GPT-OSS layers at bs={B} of the fp32 torch oracle (bf16 experts), "
                      f"scaled by {L}/{n}, + lm_head; KV lengths mean {float(lens.float().mean()):.0f}; "
                      f"{t_layers + t_lm:.1f} s on {cores} host threads"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--batch", type=int, default=1)
    ap.add_argument("--ctx", type=int, default=2048)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=20.0)
    ap.add_argument("--calib-copy", action="store_true",
                    help="after the JSON line, run a copy kernel of known size (counter calibration)")
    ap.add_argument("--ragged", action="store_true",
                    help="per-sequence KV lengths drawn uniformly from [512, 8192] (configs[2])")
    ap.add_argument("--experts", choices=["bf16", "mxfp8", "mxfp4"], default="bf16",
                    help="expert weight format (mxfp8 at --batch 32 is configs[3])")
    ap.add_argument("--kv-block", type=int, default=0,
                    help="paged KV cache with blocks of this many positions (0: flat)")
    ap.add_argument("--model", choices=["qwen3", "gpt-oss"], default="qwen3",
                    help="gpt-oss: GPT-OSS-20B shape, 24 layers, MXFP4 experts (configs[4]; "
                         "use --batch 32 --ragged --experts mxfp4)")
    ap.add_argument("--persistent", action="store_true",
                    help="run each decoder layer as one persistent kernel launch (batches <= 4)")
    ap.add_argument("--prefill", type=int, default=0, metavar="T",
                    help="measure context encoding instead: model.prefill of a T-token prompt "
                         "(passes of --prefill-chunk tokens through all layers)")
    ap.add_argument("--prefill-chunk", type=int, default=4096,
                    help="tokens per prefill pass (<= 4096; above 128 the experts run as tiled MFMA GEMMs)")
    ap.add_argument("--moe-prefill", type=int, default=0, metavar="T",
                    help="measure the MFMA regime instead: moe_prefill (LDS-tiled grouped GEMMs) "
                         "on T tokens of the Qwen3 expert shape (E=128, K=8), T*K/E tokens/expert")
    args = ap.parse_args()
    if args.moe_prefill and args.gpus == 1:
        return bench_moe_prefill(args)
    if args.prefill and args.gpus == 1:
        return bench_context_prefill(args)
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (--gpus {args.gpus} requested); "
              "multi-GPU sharding is a design note, not a measured path", file=sys.stderr)
        sys.exit(2)

    import torch
    import __graft_entry__ as ge
    ge.load_package()
    from nki_moe_megakernel_amd import _lib as L
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q

    dev = torch.device("cuda:0")
    Q.set_decode_path("persistent" if args.persistent else "multi_kernel")
    B, ctx = args.batch, args.ctx
    oss = args.model == "gpt-oss"
    lo, hi = (1024, 4096) if oss else (512, 8192)
    if args.ragged:
        gl = torch.Generator().manual_seed(4321)
        lens = torch.randint(lo, hi + 1, (B,), generator=gl, dtype=torch.int32)
    else:
        lens = torch.full((B,), ctx, dtype=torch.int32)
    S_max = ((int(lens.max()) + args.warmup + args.steps + 8 + 127) // 128) * 128
    if args.kv_block:
        S_max = (S_max + args.kv_block - 1) // args.kv_block * args.kv_block
    t0 = time.time()
    if oss:
        from nki_moe_megakernel_amd import gpt_oss_with_megakernel as G
        if args.kv_block:
            raise SystemExit("--kv-block applies to the qwen3 model only")
        cfg = G.GptOssMKConfig(num_hidden_layers=24 if args.layers == 48 else args.layers,
                               max_batch=B, max_seq=S_max, expert_format=args.experts)
        model = build_gpt_oss(G, cfg, B, dev, seed=1234)
        width = cfg.hidden_pad
    else:
        cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=args.layers, max_batch=B, max_seq=S_max,
                                 expert_format=args.experts, kv_block_len=args.kv_block)
        model = build_model(Q, cfg, B, dev, seed=1234)
        width = cfg.hidden_size
    prefill_kv(model, cfg, int(lens.max()), 1234, dev)
    torch.cuda.synchronize()
    log(f"model built in {time.time() - t0:.1f}s "
        f"({torch.cuda.memory_allocated() / 2**30:.1f} GiB allocated)")

    g = torch.Generator(device=dev)
    g.manual_seed(99)
    ids = torch.randint(0, cfg.vocab_size, (B,), generator=g, device=dev, dtype=torch.int32)
    pos = lens.to(dev)
    hidden = torch.empty(B, width, dtype=torch.bfloat16, device=dev)
    logits = torch.empty(B, cfg.vocab_size, dtype=torch.float32, device=dev)
    nxt = torch.empty(B, dtype=torch.int32, device=dev)
    lib = L.load()

    # events for the dominant kernel: one pair per layer of one step
    n_ev = cfg.num_hidden_layers
    ev_s = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    ev_e = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    arr = lambda evs: (L.vp * n_ev)(*[e.cuda_event for e in evs])
    for e in ev_s + ev_e:
        e.record()      # materialise the underlying hipEvent_t

    def step():
        model.step(ids, pos, hidden, logits, nxt)
        L.check(lib.mkd_decode_advance(ids.data_ptr(), pos.data_ptr(), nxt.data_ptr(), B,
                                       L.stream_ptr(dev)), "decode_advance")

    graph = None
    step()                            # first step eager (also surfaces errors)
    torch.cuda.synchronize()
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        run = graph.replay
    else:
        run = step
    for _ in range(args.warmup):
        run()
    # one event between consecutive steps: the whole region and every step's own time
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    w0 = time.perf_counter()
    marks[0].record()
    for i in range(args.steps):
        run()
        marks[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - w0
    ms_total = marks[0].elapsed_time(marks[-1])
    ms_step = ms_total / args.steps
    tok_s = B * args.steps / (ms_total / 1e3)
    per_step = sorted(a.elapsed_time(b) for a, b in zip(marks[:-1], marks[1:]))
    ms_median = per_step[len(per_step) // 2] if len(per_step) % 2 else \
        0.5 * (per_step[len(per_step) // 2 - 1] + per_step[len(per_step) // 2])
    ms_p99 = per_step[min(len(per_step) - 1, int(math.ceil(0.99 * len(per_step))) - 1)]

    # Dominant kernel: the persistent layer kernel when the step runs one launch
    # per layer, else the MoE gate/up GEMM.  HIP events recorded by each of its
    # dispatch packets on the launch stream (hipExtLaunchKernel), so a pair
    # times the kernel alone, in one eager step right after the timed region (a
    # captured graph keeps no timing events).
    plan = model.decode_plan(B)
    layer_kernel = plan == "persistent"
    joined = plan == "joined_experts"      # gate/up and down in one launch
    if model.layer_kernel_status(B)[1]:
        raise RuntimeError("an in-launch wait (grid barrier or expert flags) timed out")
    kcls = "layer" if layer_kernel else "moe_gate_up"
    n_prof = 1 if layer_kernel else n_ev      # the persistent kernel: one launch for all layers
    L.check(lib.mkd_profile_events(L.KCLASS[kcls], arr(ev_s), arr(ev_e), n_prof), "profile_events")
    step()
    torch.cuda.synchronize()
    n_rec = lib.mkd_profile_count()
    L.check(lib.mkd_profile_events(-1, None, None, 0), "profile off")
    if n_rec != n_prof:
        raise RuntimeError(f"expected {n_prof} profiled {kcls} launches, got {n_rec}")
    durs = [a.elapsed_time(b) for a, b in zip(ev_s[:n_prof], ev_e[:n_prof])]
    avg_ms = sum(durs) / len(durs)
    H, E, K = cfg.hidden_size, cfg.num_experts, cfg.num_experts_per_tok
    I = cfg.intermediate_size if oss else cfg.moe_intermediate_size
    # expected number of distinct experts a layer touches (near-uniform routing)
    distinct = E * (1 - (1 - K / E) ** B) if B > 1 else K
    # bytes per expert weight element: bf16 2; MX codes + one scale byte per 32
    wbytes = {"bf16": 2.0, "mxfp8": 1.0 + 1 / 32, "mxfp4": 0.5 + 1 / 32}[args.experts]
    n_mats = 3 if joined else 2                       # gate + up (+ down when joined)
    alg_bytes = distinct * n_mats * I * H * wbytes
    achieved = alg_bytes / (avg_ms / 1e3) / 1e9
    gu_flops = 2.0 * B * K * n_mats * I * H            # one launch
    gu_tflops = gu_flops / (avg_ms / 1e3) / 1e12
    # dense MFMA peaks: bf16 2.5, MXFP8 5.0, MXFP4 10.1 PFLOP/s
    mfma_peak = {"bf16": MFMA_BF16_PEAK_TFLOPS, "mxfp8": 5000.0, "mxfp4": 10100.0}[args.experts]
    # whole-step algorithmic bytes (weights + KV read + lm_head) for reference
    attn_b = 2 * H * (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim + \
        2 * cfg.num_attention_heads * cfg.head_dim * H
    kv_row = 2 * cfg.num_key_value_heads * cfg.head_dim * 2       # K + V bytes per position
    kv_full = kv_row * float((lens.float() + args.steps / 2).sum())
    if oss:   # sliding layers read at most window - 1 prior rows
        kv_win = kv_row * float((lens.float() + args.steps / 2).clamp(max=cfg.sliding_window - 1).sum())
        n_win = sum(cfg.is_sliding(l) for l in range(cfg.num_hidden_layers))
        kv_b = (n_win * kv_win + (cfg.num_hidden_layers - n_win) * kv_full) / cfg.num_hidden_layers
    else:
        kv_b = kv_full
    layer_b = attn_b + 2 * E * H + distinct * 3 * H * I * wbytes + kv_b
    step_b = cfg.num_hidden_layers * layer_b + 2 * H * cfg.vocab_size
    step_gbs = step_b / (ms_step / 1e3) / 1e9
    if layer_kernel:   # the launch streams every layer: their algorithmic bytes
        alg_bytes = cfg.num_hidden_layers * layer_b
        achieved = alg_bytes / (avg_ms / 1e3) / 1e9

    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline_gpt_oss(cfg, lens, args.cpu_seconds) if oss else \
                cpu_baseline(cfg, lens, args.cpu_seconds)
        except Exception as e:  # report, never fail the GPU number on it
            log(f"cpu baseline failed: {e!r}")
    log(f"step {ms_step:.3f} ms ({tok_s:.1f} tok/s), wall {wall:.2f}s; whole-step algorithmic "
        f"{step_b / 1e9:.3f} GB -> {step_gbs:.0f} GB/s ({step_gbs / HBM_PEAK_GBS:.1%} of HBM); "
        f"{kcls} avg {avg_ms * 1e3:.1f} us over {len(durs)} launches -> {achieved:.0f} GB/s")
    out = {
        "metric": "decode tok/s/GPU, Qwen3-30B-A3B shape bs=1/16/64; % of HBM & MFMA roofline",
        "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "ms_per_step_median": round(ms_median, 4), "ms_per_step_p99": round(ms_p99, 4),
        "higher_is_better": True,
        "scaling": "weak", "vs_baseline": vs_baseline(tok_s, cfg, B, ctx, args), "dtype": "bf16",
        "data": "synthetic (seeded random bf16 weights N(0,0.02)" +
                (f", experts quantised to {args.experts}" if args.experts != "bf16" else "") +
                ", KV N(0,1), uniform token ids)",
        "config": {"workload": workload_name(cfg, B, ctx, lens, args),
                   "batch": B, "kv_context": ctx if not args.ragged else f"U[{lo},{hi}]",
                   "kv_lengths_mean": round(float(lens.float().mean()), 1),
                   "layers": cfg.num_hidden_layers, "experts": args.experts,
                   "kv_block": args.kv_block,
                   "graph": graph is not None,
                   "attention_launch": attention_launch(model, B),
                   "step_algorithmic_GB": round(step_b / 1e9, 4),
                   "step_GBps": round(step_gbs, 1),
                   "step_hbm_frac": round(step_gbs / HBM_PEAK_GBS, 4),
                   "gate_up_TFLOPs": round(gu_tflops, 2),
                   "gate_up_mfma_frac": round(gu_tflops / mfma_peak, 5)},
        "roofline": {"bound": "hbm",
                     "kernel": ("persistent decoder (layer_kernel<%d,%d>), one launch for all layers"
                                % (cfg.head_dim, 2 if cfg.num_experts <= 128 else 8)) if layer_kernel else
                               ("moe_fused_kernel: router top-k, grouped gate/up + SwiGLU and down in one "
                                "launch (down blocks wait in-launch for their expert's gate/up blocks)")
                               if joined else
                               "moe gate_up grouped GEMM (" + (
                                   "gemm_mx_kernel<2,fmt,3>" if args.experts != "bf16" else
                                   "gemm_frag_sel_kernel<2>: router top-k formed in every block"
                                   if B == 1 and not oss else "gemm_frag_kernel<2,1,0,3>") + ")",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic(B, ctx, cfg.num_hidden_layers, kcls, joined)
                     if (args.model == "qwen3" and args.experts == "bf16" and not args.ragged
                         and not args.kv_block) else None,
                     "traffic_source": "committed rocprofv3 FETCH_SIZE + WRITE_SIZE summary of this kernel "
                                       "and workload (profiles/), not measured in this run",
                     "avg_us": round(avg_ms * 1e3, 2), "bytes_per_launch": int(alg_bytes)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    if args.calib_copy:
        calib_copy(dev)


# The reference's published decode throughput for this workload: Qwen3-30B-A3B,
# bs = 1, 48 fused layers, 122.7 tok/s on one Trainium 3 chip
# (megakernels/qwen3_moe/README.md:12).
REF_TOK_S_BS1 = 122.7


def bench_moe_prefill(args):
    """MFMA-regime measurement of the expert GEMMs: moe_prefill on a
    prefill-shaped batch (T tokens, Qwen3-30B-A3B expert shape, uniform
    seeded routing), timed with events around K calls and per kernel through
    the dispatch-packet profile events.  FLOPs: gate/up 2*T*K*H*2I, down
    2*T*K*I*H."""
    import torch
    import __graft_entry__ as ge
    mk = ge.load_package()
    from nki_moe_megakernel_amd import _lib as L
    from nki_moe_megakernel_amd.common_types import ExpertAffinityScaleMode
    dev = torch.device("cuda:0")
    lib = L.load()
    T, E, K, H, I = args.moe_prefill, 128, 8, 2048, 768
    g = torch.Generator(device=dev).manual_seed(1)
    x = torch.randn(T, H, device=dev, generator=g).to(torch.bfloat16)
    gu = (0.02 * torch.randn(E, H, 2, I, device=dev, generator=g)).to(torch.bfloat16)
    dn = (0.02 * torch.randn(E, I, H, device=dev, generator=g)).to(torch.bfloat16)
    idx = torch.argsort(torch.rand(T, E, device=dev, generator=g), dim=1)[:, :K].to(torch.int32)
    aff = torch.zeros(T, E, device=dev).scatter_(1, idx.long(), 1.0 / K)
    post = ExpertAffinityScaleMode.POST_SCALE
    run = lambda: mk.moe_prefill(x, gu, dn, aff, idx, expert_affinities_scaling_mode=post)
    for _ in range(max(args.warmup, 2)):
        run()
    torch.cuda.synchronize()
    n = max(args.steps, 4)
    kern = {}
    for cls in ("moe_gate_up", "moe_down"):
        st = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
        sp = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
        for e in st + sp:
            e.record()                         # creates the events
        torch.cuda.synchronize()
        arr = lambda es: (L.vp * n)(*[e.cuda_event for e in es])
        L.check(lib.mkd_profile_events(L.KCLASS[cls], arr(st), arr(sp), n), "arm")
        try:
            for _ in range(n):
                run()
            torch.cuda.synchronize()
        finally:
            L.check(lib.mkd_profile_events(-1, None, None, 0), "off")
        kern[cls] = sum(a.elapsed_time(b) for a, b in zip(st, sp)) / n * 1e3   # us
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(n):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / n
    fl_gu, fl_dn = 2.0 * T * K * H * 2 * I, 2.0 * T * K * I * H
    gu_tf = fl_gu / kern["moe_gate_up"] / 1e6
    dn_tf = fl_dn / kern["moe_down"] / 1e6
    # the same per-expert gate/up shape through torch.matmul (hipBLASLt), one call per expert
    xs = torch.randn(T * K // E, H, device=dev).to(torch.bfloat16)
    wt = torch.randn(2 * I, H, device=dev).to(torch.bfloat16).t().contiguous()
    for _ in range(3):
        torch.matmul(xs, wt)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(E):
        torch.matmul(xs, wt)
    e1.record()
    torch.cuda.synchronize()
    bl_tf = fl_gu / (e0.elapsed_time(e1) * 1e3) / 1e6
    line = {
        "metric": "MoE expert GEMM throughput in the MFMA regime (moe_prefill, grouped bf16 GEMMs)",
        "value": round((fl_gu + fl_dn) / (ms * 1e3) / 1e6, 1), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": n, "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded random bf16 weights N(0,0.02), hidden N(0,1), uniform top-8 routing)",
        "config": {"workload": f"Qwen3-30B-A3B expert shape (E=128, K=8, H=2048, I=768), "
                               f"{T} tokens = ~{T * K // E} tokens/expert, whole moe_prefill",
                   "tokens": T, "tokens_per_expert": T * K // E,
                   "gate_up_us": round(kern["moe_gate_up"], 1), "down_us": round(kern["moe_down"], 1),
                   "down_TFLOPs": round(dn_tf, 1), "down_mfma_frac": round(dn_tf / MFMA_BF16_PEAK_TFLOPS, 4),
                   "hipblaslt_per_expert_gate_up_TFLOPs": round(bl_tf, 1)},
        "roofline": {"bound": "mfma", "kernel": "gate/up grouped GEMM (gemm_tile_kernel<3>)",
                     "achieved": round(gu_tf, 1), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gu_tf / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
                     "flops_per_launch": fl_gu, "avg_us": round(kern["moe_gate_up"], 1)},
    }
    print(json.dumps(line), flush=True)


def bench_context_prefill(args):
    """Context encoding: model.prefill of a T-token prompt (one sequence, passes of
    --prefill-chunk tokens through all 48 layers), each step re-encoding the same prompt into
    cache rows 0..T-1.  Algorithmic HBM bytes per pass: the attention / router
    weights once, each expert's weights once if any token of the pass routes to
    it (expected distinct experts under uniform routing), and the K/V rows each
    16-token query tile of the prefill attention reads (every row up to the
    tile's last position, once per tile); reported against HBM peak for the whole
    pass (several kernels), with the pass's FLOPs against the bf16 MFMA peak
    beside it (config.mfma_TFLOPs / mfma_frac)."""
    import torch
    import __graft_entry__ as ge
    ge.load_package()
    from nki_moe_megakernel_amd import qwen_with_megakernel as Q
    dev = torch.device("cuda:0")
    T, CH = args.prefill, max(1, min(args.prefill_chunk, 4096))
    cfg = Q.Qwen3MoeMKConfig(num_hidden_layers=args.layers, max_batch=1,
                             max_seq=(T + 127) // 128 * 128 + 128)
    t0 = time.time()
    model = build_model(Q, cfg, 1, dev, seed=1234)
    torch.cuda.synchronize()
    log(f"model built in {time.time() - t0:.1f}s")
    g = torch.Generator(device=dev).manual_seed(7)
    ids = torch.randint(0, cfg.vocab_size, (T,), generator=g, device=dev, dtype=torch.int32)
    for _ in range(max(args.warmup, 1)):
        model.prefill(ids, start_pos=0, chunk=CH)
    torch.cuda.synchronize()
    n = max(1, min(args.steps, 16))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(n):
        model.prefill(ids, start_pos=0, chunk=CH)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / n
    H, E, K, I, d, nq, nkv = (cfg.hidden_size, cfg.num_experts, cfg.num_experts_per_tok,
                              cfg.moe_intermediate_size, cfg.head_dim, cfg.num_attention_heads,
                              cfg.num_key_value_heads)
    dense_b = 2 * ((nq + 2 * nkv) * d * H + H * nq * d + E * H)
    expert_b = 2 * 3 * I * H
    passes = [(c0, min(CH, T - c0)) for c0 in range(0, T, CH)]
    alg = 0.0
    flops = 0.0
    for c0, nt in passes:
        distinct = E * (1 - (1 - K / E) ** nt)
        kv = sum(2 * nkv * min(c0 + 16 * (q + 1), c0 + nt) * d * 2 for q in range((nt + 15) // 16))
        alg += cfg.num_hidden_layers * (dense_b + distinct * expert_b + kv)
        # dense projections + router, the experts' three matrices, and QK / PV
        # over each token's prefix (itself included)
        attn_f = sum(4 * nq * d * (c0 + t + 1) for t in range(nt))
        flops += cfg.num_hidden_layers * (nt * (dense_b + K * expert_b) + attn_f)
    gbs = alg / (ms * 1e-3) / 1e9
    tflops = flops / (ms * 1e-3) / 1e12
    line = {
        "metric": "context-encoding throughput (prefill of one sequence)", "value": round(T / (ms * 1e-3), 1),
        "unit": "tokens/s", "n_gpus": 1, "steps": n, "warmup": args.warmup, "ms_per_step": round(ms, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded random bf16 weights, random prompt ids)",
        "config": {"workload": f"Qwen3-30B-A3B shape, {cfg.num_hidden_layers} layers, {T}-token prompt "
                               f"in {len(passes)} passes of <= {CH} tokens", "tokens": T, "chunk": CH,
                   "flops_per_step": round(flops), "mfma_TFLOPs": round(tflops, 1),
                   "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)},
        "roofline": {"bound": "hbm", "kernel": "whole prefill pass (all kernels)",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_step": round(alg)},
    }
    print(json.dumps(line), flush=True)


def vs_baseline(tok_s, cfg, B, ctx, args):
    if (args.model == "qwen3" and args.experts == "bf16" and not args.ragged and B == 1
            and ctx == 2048 and cfg.num_hidden_layers == 48 and not args.kv_block):
        return round(tok_s / REF_TOK_S_BS1, 3)
    return None


def workload_name(cfg, B, ctx, lens, args):
    kv = "KV lengths U[512,8192] (ragged)" if args.ragged else f"KV context {ctx}"
    if args.kv_block:
        kv += f", paged KV (blocks of {args.kv_block})"
    tag = ""
    if args.experts == "bf16" and not args.ragged and B == 1 and ctx == 2048 and cfg.num_hidden_layers == 48:
        tag = " (BASELINE configs[1])"
    elif args.experts == "bf16" and args.ragged and B in (16, 64):
        tag = " (BASELINE configs[2])"
    elif args.experts == "mxfp8" and B == 32:
        tag = " (BASELINE configs[3] expert format)"
    if args.model == "gpt-oss":
        kv = kv.replace("U[512,8192]", "U[1024,4096]")
        tag = " (BASELINE configs[4])" if (B == 32 and args.experts == "mxfp4" and args.ragged) else ""
        return (f"GPT-OSS-20B-shaped {cfg.num_hidden_layers}-layer greedy decode (sliding-window 128 / "
                f"full alternating, sinks), bs={B}, {kv}, {args.experts} experts{tag}")
    return (f"Qwen3-30B-A3B-shaped {cfg.num_hidden_layers}-layer greedy decode, bs={B}, {kv}, "
            f"{args.experts} experts{tag}")


def attention_launch(model, B):
    """How the decode step runs attention for this batch (the decode plan)."""
    if not (hasattr(model, "joined_attention") and model.joined_attention(B)):
        return "separate launches"
    if model.router_in_attention(B):
        return ("joined (attention, chunk merge + o_proj, residual + post norm + router GEMM)" if B == 1
                else "joined (attention, combine, o_proj, residual + post norm + router GEMM)")
    return "joined (attention + combine + o_proj)"


def measured_traffic(B, ctx, layers, kcls="moe_gate_up", joined=False):
    """HBM bytes per launch of the dominant kernel, read from the committed
    counter summary for that kernel and workload (profiles/*_traffic.json, made
    by two rocprofv3 --pmc runs of this bench), or None.  Not measured in this run."""
    name = "layer_kernel_traffic.json" if kcls == "layer" else (
        "moe_joined_traffic.json" if joined else "gate_up_traffic.json")
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    w = t.get("workload", {})
    if (w.get("batch"), w.get("kv_context"), w.get("layers")) != (B, ctx, layers):
        return None
    return t.get("bytes_per_launch")


def calib_copy(dev, nbytes=256 << 20, reps=3):
    """A plain copy kernel of known size (reads and writes `nbytes` each) for
    scaling the FETCH_SIZE / WRITE_SIZE counters of a rocprofv3 --pmc run."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(reps):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    log(f"calib copy: {reps} x neg over {nbytes} bytes")


if __name__ == "__main__":
    main()
