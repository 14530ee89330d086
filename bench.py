#!/usr/bin/env python3
"""Benchmark of the complexity-deep hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]

Default workload ("1b-forward", configuration 4): one full ComplexityModel forward of
the 1B preset (hidden 2048, 24 layers, 16 Q / 8 KV heads, intermediate 5632, 8 routed
experts + shared expert, vocab 32000) in bf16 over batch 8 x seq 2048 token ids drawn
from Zipf(1.1), with the greedy bin-packed expert map installed in every layer and
random-normal weights (seed 1).  A step is one forward returning logits; `value` is
tokens per second with inputs already in HBM.

The other workloads run one configuration each:
  "readme-forward"  configuration 1: the reference README's model (hidden 768, 18
                    layers, 12/4 heads, E=4 + shared), batch 4 x seq 512, seed 0
  "readme-forward-graph"  the same forward replayed from a HIP graph recorded once
                    (GraphedForward; at this size Python's launch rate paces eager)
  "moe-layer"       configuration 2: TokenRoutedMLP, 16384 x 768, E=4, Ie=512 + shared
  "qkv-norm"        configuration 3: add+RMSNorm then mu-QKV, 32768 x 2048, 16q/8kv x 128
  "route-stress"    configuration 5: routing plan + MoE layer, 65536 tokens, 90% skew
  "route-permute"   configuration 5's token rows (65536 x 2048 bf16) permuted into
                    expert order and back (cdx_permute_rows / cdx_unpermute_rows)
  "rmsnorm-1b"      configuration 4's plain RMSNorm, 49 launches per step over 8
                    rotating inputs (every launch reads from HBM; region-timed)
  "attention-1b"    configuration 4's causal GQA attention core, one layer (region-timed)
After the headline workload (and its CPU baselines) the default run also times each
of these for a few steps and reports them under "workloads" (skip: --no-extras).

Printed: ONE JSON line on stdout.  Besides the contract keys it carries
  roofline      the dominant hot-path kernel's achieved rate against the MI355X peak
                (2.5 PFLOP/s dense bf16 MFMA, 8 TB/s HBM), from HIP events recorded
                around each launch on the stream it runs on, over a second pass of
                the timed steps;
  kernels       the same for every hot-path entry point;
  cpu_baseline  the fp32 CPU restatement (oracle/) timed on this host over a bounded
                sample of the same workload, plus its agreement with the GPU logits;
                under "readme_forward" the same for configuration 1's whole batch;
  workloads     per extra workload: tokens/s, ms per step, roofline and kernels;
  hbm_ceiling   measured streaming read / write / copy rates of this GPU's HBM
                (cdx_hbm_probe), the practical ceilings of the HBM-bound kernels.
Everything else goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from collections import defaultdict
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "complexity-deep_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

METRIC = "fwd tokens/sec at 1B bf16; MFMA util % (MoE/QKV GEMM), HBM % (route/norm)"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def measured_traffic(workload: str) -> dict:
    """HBM bytes per launch of each hot-path kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE runs of this workload (profiles/hbm_traffic_<workload>.json,
    each counter scaled by its reading for a 1 GiB copy).  Empty if none is committed."""
    path = REPO / "profiles" / f"hbm_traffic_{workload.replace('-', '_')}.json"
    try:
        with open(path) as f:
            data = json.load(f)
    except (OSError, ValueError):
        return {}
    return {k: v["hbm_bytes_per_launch"] for k, v in data.get("kernels", {}).items()}


# ---------------------------------------------------------------------------
# algorithmic work per entry-point call (the units roofline.achieved is priced on)
# ---------------------------------------------------------------------------

def work_of(name: str, s: dict):
    """(amount, kind) per call: FLOP for MFMA-bound calls, bytes for HBM-bound ones."""
    if name == "mu_qkv":
        K = 2 * s["H"] if s["mu"] else s["H"]
        return 2.0 * s["M"] * K * s["N"], "flop"
    if name == "mu_qkv_bcast":
        # layer 0: the broadcast mu row's product folded into one 64-column K block
        return 2.0 * s["M"] * (s["H"] + 64) * s["N"], "flop"
    if name == "moe_swiglu":
        blocks = 2 if s["shared"] else 1
        # gate + up + down per block, each token sees one routed expert (+ shared)
        return 6.0 * s["T"] * s["H"] * s["Ie"] * blocks, "flop"
    if name == "add_rmsnorm":
        rows = s["T"] * s["H"] * 2
        return float(rows * (4 if s["store_residual"] else 3) + 2 * s["H"]), "byte"
    if name == "rmsnorm":
        return float(2 * s["T"] * s["H"] * 2 + 2 * s["H"]), "byte"
    if name == "mu_guidance":
        return 2.0 * s["T"] * s["H"] * s["H"], "flop"
    if name == "attention":
        # causal: query s sees s + 1 keys; QK^T and PV are 2 * D FLOP per (query, key) each
        S = s["S"]
        return 4.0 * s["B"] * s["nq"] * s["D"] * S * (S + 1) / 2, "flop"
    if name in ("lm_head", "o_proj"):
        return 2.0 * s["M"] * s["K"] * s["N"], "flop"
    if name == "embedding":
        # ids in; one table row read and one output row written per token
        return float(s["T"] * (8 + 2 * 2 * s["H"])), "byte"
    if name == "route_plan":
        # ids in; expert_id, perm, inv_perm out; the map is read once per token at most.
        # A few hundred KB in two launches: bound by launch latency, not by HBM.
        return float(s["T"] * (8 + 4 + 4 + 4) + 2 * 4 * (s["E"] + 1)), "latency"
    if name in ("permute_rows", "unpermute_rows"):
        # every row read once and written once (plus the int32 permutation)
        return float(s["T"] * (2 * s["row_bytes"] + 4)), "byte"
    if name == "swiglu":
        return float(3 * s["n"] * s["elt"]), "byte"
    if name == "grouped_gemm":
        return 2.0 * s["T"] * s["K"] * s["N"], "flop"
    return 0.0, "none"


class KernelTimer:
    """Collects (name, start, end, shape) from the package's launch hook."""

    def __init__(self):
        self.events = []
        self.active = False

    def __call__(self, name, e0, e1, shape):
        if self.active:
            self.events.append((name, e0, e1, shape))

    def summary(self, steps: int):
        import torch
        torch.cuda.synchronize()
        acc = defaultdict(lambda: {"calls": 0, "ms": 0.0, "work": 0.0, "kind": "none"})
        for name, e0, e1, shape in self.events:
            a = acc[name]
            a["calls"] += 1
            a["ms"] += e0.elapsed_time(e1)
            w, kind = work_of(name, shape)
            a["work"] += w
            a["kind"] = kind
        out = {}
        for name, a in acc.items():
            avg_us = 1e3 * a["ms"] / a["calls"]
            rec = {"launches_per_step": a["calls"] / steps, "avg_us": round(avg_us, 2),
                   "ms_per_step": round(a["ms"] / steps, 4)}
            if a["kind"] == "flop":
                tf = a["work"] / (a["ms"] * 1e-3) / 1e12
                rec.update(bound="mfma", achieved=round(tf, 1), unit="TFLOP/s",
                           frac=round(tf / PEAK_BF16_TFLOPS, 4), work_per_launch=a["work"] / a["calls"])
            elif a["kind"] == "byte":
                gbs = a["work"] / (a["ms"] * 1e-3) / 1e9
                rec.update(bound="hbm", achieved=round(gbs, 1), unit="GB/s",
                           frac=round(gbs / PEAK_HBM_GBS, 4), work_per_launch=a["work"] / a["calls"])
            elif a["kind"] == "latency":
                rec.update(bound="launch latency", bytes_per_launch=a["work"] / a["calls"])
            out[name] = rec
        return out


# ---------------------------------------------------------------------------
# workloads
# ---------------------------------------------------------------------------

def build_1b(dev):
    import torch
    import complexity_deep as cd
    from complexity_deep import synthetic as syn
    cfg = cd.ComplexityConfig.complexity_1b()
    cfg.vocab_size = 32000
    torch.manual_seed(1)
    with torch.device(dev):
        model = cd.ComplexityModel(cfg)
    tmap = syn.binpacked_map(cfg.vocab_size, cfg.num_experts)
    syn.install_expert_map(model, tmap)
    model = model.to(torch.bfloat16).eval()
    ids = syn.zipf_token_ids(8, 2048, cfg.vocab_size, seed=1)
    return cfg, model, ids


def workload_1b(args, dev):
    import torch
    cfg, model, ids_cpu = build_1b(dev)
    ids = ids_cpu.to(dev)
    T = ids.numel()

    def step():
        return model(ids).logits

    config = {"workload": "configuration 4: 1B ComplexityModel forward (logits)", "preset": "complexity_1b",
              "hidden": cfg.hidden_size, "layers": cfg.num_hidden_layers,
              "heads_q_kv_dim": [cfg.num_attention_heads, cfg.num_key_value_heads,
                                 cfg.hidden_size // cfg.num_attention_heads],
              "intermediate": cfg.intermediate_size, "experts": cfg.num_experts,
              "expert_width": cfg.intermediate_size // cfg.num_experts, "shared_expert": True,
              "vocab": cfg.vocab_size, "global_batch": 8, "seq_len": 2048, "tokens_per_step": T,
              "token_ids": "Zipf(1.1) over 32000, seed 1", "expert_map": "greedy bin-packing of the Zipf pmf",
              "weights": "random normal init (std 0.02, residual 0.02/sqrt(48)), seed 1, cast to bf16",
              "parallelism": "single GPU"}
    return step, T, config, ("mu_qkv",), (cfg, model, ids_cpu)


def build_readme(dev):
    import torch
    import complexity_deep as cd
    from complexity_deep import synthetic as syn
    cfg = cd.ComplexityConfig(vocab_size=32000, hidden_size=768, intermediate_size=2048, num_hidden_layers=18,
                              num_attention_heads=12, num_key_value_heads=4, num_experts=4, shared_expert=True,
                              use_mu_guidance=True)
    torch.manual_seed(0)
    model = cd.ComplexityModel(cfg)
    syn.install_expert_map(model, syn.binpacked_map(cfg.vocab_size, cfg.num_experts))
    ids = syn.zipf_token_ids(4, 512, cfg.vocab_size, seed=0)
    return cfg, model, ids


def workload_readme(args, dev):
    import torch
    cfg, model, ids_cpu = build_readme(dev)
    model = model.to(dev, torch.bfloat16).eval()
    ids = ids_cpu.to(dev)

    def step():
        return model(ids).logits

    config = {"workload": "configuration 1: the reference README model forward (logits)", "hidden": 768,
              "layers": 18, "heads_q_kv_dim": [12, 4, 64], "intermediate": 2048, "experts": 4, "shared_expert": True,
              "vocab": 32000, "global_batch": 4, "seq_len": 512, "tokens_per_step": ids.numel(),
              "token_ids": "Zipf(1.1) over 32000, seed 0", "expert_map": "greedy bin-packing of the Zipf pmf",
              "weights": "random normal init (std 0.02, residual 0.02/sqrt(36)), seed 0, cast to bf16"}
    return step, ids.numel(), config, ("mu_qkv",), None


def workload_readme_graph(args, dev):
    import torch
    cfg, model, ids_cpu = build_readme(dev)
    model = model.to(dev, torch.bfloat16).eval()
    ids = ids_cpu.to(dev)
    graphed = model.capture_forward(*ids.shape)

    def step():
        return graphed(ids)

    config = {"workload": "configuration 1 (as readme-forward), each forward replayed from a HIP graph "
                          "recorded once (GraphedForward): the same kernels on the same buffers, issued from the "
                          "device queue instead of by Python", "hidden": 768, "layers": 18,
              "global_batch": 4, "seq_len": 512, "tokens_per_step": ids.numel(),
              "note": "no per-launch events in a replay: no kernels table"}
    return step, ids.numel(), config, (), None


def workload_route_permute(args, dev):
    import torch
    from complexity_deep import synthetic as syn
    from complexity_deep.token_routed_mlp import permute_rows, route_plan, unpermute_rows
    T, H, E = 65536, 2048, 8
    tmap = syn.binpacked_map(32000, E)
    ids = syn.routing_stress_ids(T, tmap, E, heavy=1, seed=0).to(dev)
    x = syn.normal_bf16((T, H), seed=2, device=dev)
    plan = route_plan(ids, tmap.to(dev), E)

    def step():
        return unpermute_rows(permute_rows(x, plan.perm), plan.perm)

    config = {"workload": "configuration 5 token rows permuted into expert order and back", "tokens_per_step": T,
              "row_bytes": 2 * H, "token_ids": "90% heavy expert 1, 1% each other, rest id 0, seed 0"}
    return step, T, config, ("permute_rows", "unpermute_rows"), None


def workload_rmsnorm(args, dev):
    """The 1B forward's plain RMSNorm (16384 x 2048 bf16), 49 launches per step as in one
    forward, over 8 distinct inputs (537 MB, more than the 256 MB last-level cache) so
    that every launch reads its input from HBM."""
    import torch
    from complexity_deep import synthetic as syn
    from complexity_deep.normalization import rms_norm
    T, H, n_in = 16384, 2048, 8
    xs = [syn.normal_bf16((T, H), seed=10 + i, device=dev) for i in range(n_in)]
    w = torch.ones(H, dtype=torch.bfloat16, device=dev)

    def step():
        out = None
        for i in range(49):
            out = rms_norm(xs[i % n_in], w, 1e-6)
        return out

    config = {"workload": "configuration 4's plain RMSNorm: 49 back-to-back launches of 16384 x 2048 bf16 per step, "
                          "inputs rotating over 8 buffers (537 MB)", "tokens_per_step": 49 * T, "hidden": H,
              "region_timed": "rmsnorm"}
    return step, 49 * T, config, ("rmsnorm",), None


def workload_moe(args, dev):
    import torch
    import complexity_deep as cd
    from complexity_deep import synthetic as syn
    T, H, I, E = 16384, 768, 2048, 4
    torch.manual_seed(0)
    with torch.device(dev):
        m = cd.TokenRoutedMLP(H, I, num_experts=E, vocab_size=32000)
        m.token_to_expert.copy_(syn.binpacked_map(32000, E))
    m = m.to(torch.bfloat16)
    ids = syn.zipf_token_ids(1, T, 32000, seed=0).to(dev)
    x = syn.normal_bf16((1, T, H), seed=1, device=dev)

    def step():
        return m(x, token_ids=ids)

    config = {"workload": "configuration 2: one TokenRoutedMLP layer (route plan + grouped SwiGLU + shared)",
              "tokens_per_step": T, "hidden": H, "experts": E, "expert_width": I // E, "shared_expert": True,
              "token_ids": "Zipf(1.1) over 32000, seed 0", "expert_map": "greedy bin-packing"}
    return step, T, config, ("moe_swiglu",), None


def workload_qkv_norm(args, dev):
    import torch
    import complexity_deep as cd
    from complexity_deep import synthetic as syn
    from complexity_deep.normalization import add_rms_norm
    B, S, H, nq, nkv = 16, 2048, 2048, 16, 8
    torch.manual_seed(0)
    with torch.device(dev):
        attn = cd.ComplexityAttention(H, nq, nkv)
        w = torch.ones(H)
    attn = attn.to(torch.bfloat16)
    w = w.to(torch.bfloat16)
    x = syn.normal_bf16((B, S, H), seed=1, device=dev)
    res = syn.normal_bf16((B, S, H), seed=2, device=dev)
    mu = syn.normal_bf16((B, S, H), seed=3, device=dev)
    h = torch.empty_like(res)

    def step():
        n, _ = add_rms_norm(x, res, w, 1e-6, residual_out=h)
        return attn.project_qkv(n, mu)

    config = {"workload": "configuration 3: residual add + RMSNorm, then the mu-QKV projection",
              "tokens_per_step": B * S, "hidden": H, "heads_q_kv_dim": [nq, nkv, H // nq], "eps": 1e-6}
    return step, B * S, config, ("mu_qkv", "add_rmsnorm"), None


def workload_attention(args, dev):
    """Configuration 4's causal GQA attention core, one layer: q [8, 16, 2048, 128] and
    k / V^T of 8 KV heads, as the fused QKV + RoPE epilogue leaves them."""
    from complexity_deep import synthetic as syn
    from complexity_deep.attention import causal_attention, to_vt_layout
    B, S, nq, nkv, D = 8, 2048, 16, 8, 128
    q = syn.normal_bf16((B, nq, S, D), seed=1, device=dev)
    k = syn.normal_bf16((B, nkv, S, D), seed=2, device=dev)
    vt = to_vt_layout(syn.normal_bf16((B, nkv, S, D), seed=3, device=dev))

    def step():
        return causal_attention(q, k, vt)

    config = {"workload": "configuration 4's causal GQA attention core (one layer, B 8 x S 2048, 16 q / 8 kv "
                          "heads of 128)", "tokens_per_step": B * S, "region_timed": "attention"}
    return step, B * S, config, ("attention",), None


def workload_route_stress(args, dev):
    import torch
    import complexity_deep as cd
    from complexity_deep import synthetic as syn
    T, H, I, E = 65536, 2048, 5632, 8
    tmap = syn.binpacked_map(32000, E)
    torch.manual_seed(0)
    with torch.device(dev):
        m = cd.TokenRoutedMLP(H, I, num_experts=E, vocab_size=32000)
        m.token_to_expert.copy_(tmap)
    m = m.to(torch.bfloat16)
    ids = syn.routing_stress_ids(T, tmap, E, heavy=1, seed=0).to(dev)
    x = syn.normal_bf16((T, H), seed=2, device=dev)

    def step():
        return m(x, token_ids=ids)

    config = {"workload": "configuration 5: routing plan + MoE layer under 90% skew", "tokens_per_step": T,
              "hidden": H, "experts": E, "expert_width": I // E,
              "token_ids": "90% heavy expert 1, 1% each other, rest id 0, seed 0"}
    return step, T, config, ("moe_swiglu", "route_plan"), None


WORKLOADS = {"1b-forward": workload_1b, "readme-forward": workload_readme,
             "readme-forward-graph": workload_readme_graph, "moe-layer": workload_moe,
             "qkv-norm": workload_qkv_norm, "route-stress": workload_route_stress,
             "route-permute": workload_route_permute, "rmsnorm-1b": workload_rmsnorm,
             "attention-1b": workload_attention}
EXTRAS = ("readme-forward", "readme-forward-graph", "moe-layer", "qkv-norm", "route-stress", "route-permute", "rmsnorm-1b", "attention-1b")


# ---------------------------------------------------------------------------
# CPU baseline: the fp32 oracle on this host's cores, bounded sample
# ---------------------------------------------------------------------------

def cpu_model_name() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _logit_agreement(gpu, ref):
    d = gpu.float().cpu() - ref
    return {"max_rel": float(d.abs().max() / ref.abs().max()),
            "rel_rms": float(d.pow(2).mean().sqrt() / ref.pow(2).mean().sqrt())}


def cpu_baseline_1b(ctx, gpu_logits0, seqs: int):
    import torch
    from oracle import oracle as orc
    cfg, model, ids_cpu = ctx
    log("cpu baseline: copying weights to host fp32")
    sd = {k: v.detach().float().cpu() for k, v in model.state_dict().items()}
    sample = ids_cpu[:seqs]
    threads = torch.get_num_threads()
    with torch.no_grad():
        orc.forward(sd, cfg.to_dict(), sample[:, :64])  # warm-up (allocator, BLAS threads)
        t0 = time.perf_counter()
        ref = orc.forward(sd, cfg.to_dict(), sample)
        dt = time.perf_counter() - t0
    tok = sample.numel()
    agree = _logit_agreement(gpu_logits0[:seqs], ref)
    log(f"cpu baseline: {tok} tokens in {dt:.2f} s ({tok / dt:.1f} tok/s, {threads} threads); "
        f"GPU logits vs CPU fp32: max_rel={agree['max_rel']:.3e} rel_rms={agree['rel_rms']:.3e}")
    return {"value": round(tok / dt, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{seqs} x 2048 tokens (the first {seqs} sequence(s) of the workload batch), the full "
                      f"24-layer 1B forward in fp32 through oracle.forward (torch CPU, {threads} threads)",
            "seconds": round(dt, 3), "cpu_model": cpu_model_name(), "affinity_cores": len(os.sched_getaffinity(0)),
            "gpu_vs_cpu_logits": agree}


def cpu_baseline_readme(dev):
    """Configuration 1 (the reference README model, 4 x 512 tokens) through the fp32
    oracle on this host, and the same batch through the bf16 GPU model for agreement
    and for the GPU rate of the same workload."""
    import torch
    from oracle import oracle as orc
    cfg, model, ids = build_readme(dev)
    # the oracle sees the bf16-rounded weights the GPU model holds
    sd = {k: (v.detach().to(torch.bfloat16).float() if v.is_floating_point() else v.detach())
          for k, v in model.state_dict().items()}
    threads = torch.get_num_threads()
    with torch.no_grad():
        orc.forward(sd, cfg.to_dict(), ids[:1, :64])  # warm-up
        t0 = time.perf_counter()
        ref = orc.forward(sd, cfg.to_dict(), ids)
        dt = time.perf_counter() - t0
    gpu_model = model.to(dev, torch.bfloat16).eval()
    with torch.inference_mode():
        logits = gpu_model(ids.to(dev)).logits
    agree = _logit_agreement(logits, ref)
    tok = ids.numel()
    log(f"cpu baseline (configuration 1): {tok} tokens in {dt:.2f} s ({tok / dt:.1f} tok/s, {threads} threads); "
        f"GPU logits vs CPU fp32: max_rel={agree['max_rel']:.3e} rel_rms={agree['rel_rms']:.3e}")
    return {"value": round(tok / dt, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"configuration 1 whole: the README model (768 hidden, 18 layers, E=4 + shared) over "
                      f"4 x 512 Zipf tokens in fp32 through oracle.forward (torch CPU, {threads} threads)",
            "seconds": round(dt, 3), "gpu_vs_cpu_logits": agree}


# ---------------------------------------------------------------------------

def hbm_ceilings(dev) -> dict:
    """Measured streaming ceilings of this GPU's HBM (cdx_hbm_probe: plain read, write
    and copy kernels, 16-byte non-temporal accesses), in TB/s of algorithmic bytes,
    for a copy of the 1B RMSNorm's size (64 MB each way) and for buffers beyond the
    256 MB last-level cache (512 MB).  Back-to-back launches rotating over four
    buffers, timed by HIP events around the whole pass."""
    import torch
    from complexity_deep import _native as nat
    lib = nat.lib()
    out = {}
    for label, mb in (("64MB", 64), ("512MB", 512)):
        nbytes = mb << 20
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(1) for _ in range(4)]
        dsts = [torch.empty(nbytes, dtype=torch.uint8, device=dev) for _ in range(4)]
        sink = torch.zeros(4, dtype=torch.int32, device=dev)
        s = torch.cuda.current_stream(dev).cuda_stream
        res = {}
        for mode, name, moved in ((0, "read", 1), (1, "write", 1), (2, "copy", 2)):
            def call(i):
                src = bufs[i % 4].data_ptr() if mode != 1 else 0
                dst = dsts[i % 4].data_ptr() if mode != 0 else sink.data_ptr()
                nat.check(lib.cdx_hbm_probe(mode, src, dst, nbytes, s), "cdx_hbm_probe")
            call(0)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            iters = 20
            e0.record()
            for i in range(iters):
                call(i)
            e1.record()
            torch.cuda.synchronize()
            us = 1e3 * e0.elapsed_time(e1) / iters
            res[name] = {"us": round(us, 2), "TBps": round(moved * nbytes / us / 1e6, 3),
                         "frac_of_8TBps": round(moved * nbytes / us / 1e6 / 8.0, 4)}
        out[label] = res
        del bufs, dsts
        torch.cuda.empty_cache()
    log(f"HBM ceilings: {json.dumps(out)}")
    return out


def roofline_of(kernels: dict, dominant, workload: str):
    dom = next((d for d in dominant if d in kernels), None)
    if dom is None:
        return None
    k = kernels[dom]
    traffic = measured_traffic(workload)
    return {"kernel": dom, "bound": k["bound"], "achieved": k["achieved"],
            "peak": PEAK_BF16_TFLOPS if k["bound"] == "mfma" else PEAK_HBM_GBS,
            "unit": k["unit"], "frac": k["frac"], "traffic": traffic.get(dom),
            "traffic_source": f"profiles/hbm_traffic_{workload.replace('-', '_')}.json" if dom in traffic else None,
            "work_per_launch": k["work_per_launch"], "avg_launch_us": k["avg_us"],
            "timing": "HIP events around each launch on its stream, over a second pass of the same K steps "
                      "run right after the timed (event-free) pass"}


def run(step, steps: int, warmup: int, kernel_timing: bool):
    """Warm-up, then `steps` timed steps bracketed by synchronisations (no events in
    them), then the same steps again with events around every launch.  Also returns
    the GPU time of the timed pass from a pair of HIP events around it (on the
    current stream, which every entry point launches on)."""
    import torch
    from complexity_deep import _native as nat
    timer = KernelTimer()
    with torch.inference_mode():
        out = None
        for _ in range(warmup):
            out = step()
        torch.cuda.synchronize()
        r0 = torch.cuda.Event(enable_timing=True)
        r1 = torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        r0.record()
        for _ in range(steps):
            out = step()
        r1.record()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        region_ms = r0.elapsed_time(r1)
        if kernel_timing:
            # A second pass of the same K steps with a pair of HIP events around every
            # launch, kept out of the timed pass (the events cost about 1 ms of GPU
            # time per 1B step).
            nat.set_launch_hook(timer)
            timer.active = True
            for _ in range(steps):
                step()
            torch.cuda.synchronize()
            timer.active = False
            nat.set_launch_hook(None)
    kernels = timer.summary(steps) if kernel_timing else {}
    return out, t1 - t0, kernels, region_ms


def log_kernels(kernels: dict):
    for name, k in sorted(kernels.items()):
        log(f"  {name:14s} {k['launches_per_step']:5.1f}/step avg {k['avg_us']:9.2f} us  "
            f"{k.get('achieved', 0):9.1f} {k.get('unit', '')}  frac {k.get('frac', 0):.3f}")


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", choices=sorted(WORKLOADS), default="1b-forward")
    ap.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU oracle timings")
    ap.add_argument("--cpu-seqs", type=int, default=1, help="sequences of 2048 tokens in the CPU sample")
    ap.add_argument("--no-kernel-timing", action="store_true", help="do not record per-launch events")
    ap.add_argument("--no-extras", action="store_true", help="time only the selected workload")
    ap.add_argument("--extra-steps", type=int, default=10, help="timed steps of each extra workload")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run one plain 1 GiB device copy (read 1 GiB, write 1 GiB): the reference "
                         "dispatch that scales FETCH_SIZE / WRITE_SIZE counter runs")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE {world}); "
              "the multi-GPU sharding of this path is a design, not a measured configuration", file=sys.stderr)
        return 2

    import torch
    from complexity_deep import _native as nat
    if not torch.cuda.is_available():
        log("bench.py needs a ROCm GPU")
        return 1
    nat.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_calibration:
        src = torch.empty(1 << 30, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    log(f"device: {torch.cuda.get_device_name(dev)}; workload {args.workload}")
    step, tokens, config, dominant, ctx = WORKLOADS[args.workload](args, dev)
    out, elapsed, kernels, _ = run(step, args.steps, args.warmup, not args.no_kernel_timing)
    ms = 1e3 * elapsed / args.steps
    value = tokens * args.steps / elapsed
    log(f"timed {args.steps} steps: {ms:.3f} ms/step, {value:.1f} tokens/s")
    log_kernels(kernels)
    hot_ms = sum(k["ms_per_step"] for k in kernels.values())
    roofline = roofline_of(kernels, dominant, args.workload)

    cpu = None
    if args.workload == "1b-forward" and not args.no_cpu_baseline:
        cpu = cpu_baseline_1b(ctx, out, args.cpu_seqs)
        cpu["readme_forward"] = cpu_baseline_readme(dev)
    del step, out, ctx
    torch.cuda.empty_cache()

    workloads = {}
    if not args.no_extras and args.workload == "1b-forward":
        for name in EXTRAS:
            w_step, w_tokens, w_config, w_dom, _ = WORKLOADS[name](args, dev)
            _, w_elapsed, w_kernels, w_region_ms = run(w_step, args.extra_steps, 2, True)
            w_ms = 1e3 * w_elapsed / args.extra_steps
            rt = w_config.get("region_timed")
            if rt in w_kernels:
                # Back-to-back launches of one kernel: its rate over the event-timed pass
                # (no event pair per launch, whose own cost would dominate a 20 us kernel).
                k = w_kernels[rt]
                n = k["launches_per_step"] * args.extra_steps
                avg_us = 1e3 * w_region_ms / n
                rate = k["work_per_launch"] / (avg_us * 1e-6)
                if k["bound"] == "mfma":
                    achieved, unit, peak = rate / 1e12, "TFLOP/s", PEAK_BF16_TFLOPS
                else:
                    achieved, unit, peak = rate / 1e9, "GB/s", PEAK_HBM_GBS
                w_kernels[rt + "_region"] = {"launches_per_step": k["launches_per_step"], "avg_us": round(avg_us, 2),
                                             "bound": k["bound"], "achieved": round(achieved, 1), "unit": unit,
                                             "frac": round(achieved / peak, 4),
                                             "work_per_launch": k["work_per_launch"],
                                             "timing": "HIP events around the whole timed pass / launches"}
                w_dom = (rt + "_region",) + tuple(w_dom)
            log(f"workload {name}: {w_ms:.3f} ms/step, {w_tokens * args.extra_steps / w_elapsed:.1f} tokens/s")
            log_kernels(w_kernels)
            workloads[name] = {"value": round(w_tokens * args.extra_steps / w_elapsed, 1), "unit": "tokens/s",
                               "ms_per_step": round(w_ms, 4), "steps": args.extra_steps, "warmup": 2,
                               "config": w_config, "roofline": roofline_of(w_kernels, w_dom, name),
                               "kernels": w_kernels}
            del w_step
            torch.cuda.empty_cache()

    ceilings = hbm_ceilings(dev) if not args.no_extras and args.workload == "1b-forward" else None

    rec = {"metric": METRIC, "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16", "data": "synthetic", "config": config,
           "roofline": roofline, "cpu_baseline": cpu,
           "kernels": kernels, "hot_path_ms_per_step": round(hot_ms, 4),
           "workloads": workloads, "hbm_ceiling": ceilings, "device": torch.cuda.get_device_name(dev)}
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
