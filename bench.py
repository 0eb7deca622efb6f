#!/usr/bin/env python3
"""LUCID attention fwd+bwd throughput on one MI355X (north-star workload).

Workload (BASELINE.json metric "at T=32K bf16"): B=1, H=16 (MHA), T=32768,
d=64, bf16, causal; Q, K, V ~ N(0,1)/sqrt(64), dO ~ N(0,1), synthetic, seeded.
One step = one forward + one backward through ``lucid_amd.lucid_attention``
with the inputs already resident in HBM.

Reported: tokens/s (whole job), TFLOP/s by the frozen algorithmic count
7*T^2*d*B*(Hq+Hkv) (causal halves, 1 FMA = 2 flop; exp, RMSNorm and the
diagonal-block inverses excluded), the roofline of the dominant kernel timed
with HIP events on its launch stream inside the timed region (events around that
kernel only; the per-kernel breakdown "kernels" comes from K untimed steps before
it with events around every launch, which would otherwise add two event records
per launch to the timed steps), plain causal
attention at the same shape as a comparator (this build's own attention kernels
with V' = V, and torch SDPA; the ratio is taken against the faster), and a CPU
baseline (the float32 torch restatement of the reference's dense path, one head
at the full length, on every core the process may use).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
HBM_PEAK_GBS = 8000.0


def lucid_flops(B, Hq, Hkv, T, D):
    """Algorithmic fwd+bwd FLOPs of LUCID attention: 7 T^2 d per query head + 7 T^2 d per kv head."""
    return 7.0 * T * T * D * B * (Hq + Hkv)


def causal_flops(B, Hq, T, D):
    return 7.0 * T * T * D * B * Hq


# algorithmic FLOPs per launch of each kernel (same counting rules; recomputed
# scores and the preprocessing kernels count zero)
KERNEL_FLOPS = {
    "lucid_precond_fwd_kernel": lambda B, Hq, Hkv, T, D: 2.0 * T * T * D * B * Hkv,   # K^K^T, P V'
    "lucid_precond_fwd_wide_kernel": lambda B, Hq, Hkv, T, D: 2.0 * T * T * D * B * Hkv,  # the same, 256 rows/WG
    "lucid_attn_fwd_kernel": lambda B, Hq, Hkv, T, D: 2.0 * T * T * D * B * Hq,       # QK^T, P V'
    # chain (K^K^T, P V') and attention (QK^T, P V') of each block in one kernel (Hq == Hkv)
    "lucid_fused_fwd_kernel": lambda B, Hq, Hkv, T, D: 2.0 * T * T * D * B * (Hkv + Hq),
    "lucid_attn_fwd_wide_kernel": lambda B, Hq, Hkv, T, D: 2.0 * T * T * D * B * Hq,  # the same at head dim 128
    "lucid_attn_bwd_dkdv_kernel": lambda B, Hq, Hkv, T, D: 4.0 * T * T * D * B * Hq,  # S, dV', dP, dK
    "lucid_attn_bwd_dq_kernel": lambda B, Hq, Hkv, T, D: 1.0 * T * T * D * B * Hq,    # dQ
    "lucid_precond_bwd_col_kernel": lambda B, Hq, Hkv, T, D: 4.0 * T * T * D * B * Hkv,  # P, P^T dV, dV V'^T, M^T K^
    "lucid_precond_bwd_col_wide_kernel": lambda B, Hq, Hkv, T, D: 4.0 * T * T * D * B * Hkv,  # the same, 256 columns/WG
    "lucid_precond_bwd_row_kernel": lambda B, Hq, Hkv, T, D: 1.0 * T * T * D * B * Hkv,  # M K^
}
# fp32 inputs: the same algorithmic counts (at the caller's head dim; the kernels run on rows
# padded to 64 or 128 and take every product as three or four bf16 MFMAs)
for _n in ("lucid_precond_fwd", "lucid_attn_fwd", "lucid_attn_bwd_dkdv", "lucid_attn_bwd_dq", "lucid_precond_bwd_col",
           "lucid_precond_bwd_row"):
    KERNEL_FLOPS[_n + "_f32_kernel"] = KERNEL_FLOPS[_n + "_kernel"]


def warm_up(step, warmup):
    """Untimed warmup: exactly `warmup` steps when given; by default at least 3 steps and at
    least 0.5 s of GPU work (the clocks of an idle GPU take that long to come up: a 2 ms step
    timed after three warmup steps reads ~2 % slow).  Returns the number of steps run."""
    import torch
    if warmup is not None:
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        return warmup
    n, t0 = 0, time.perf_counter()
    while n < 3 or time.perf_counter() - t0 < 0.5:
        step()
        torch.cuda.synchronize()
        n += 1
    return n


def profiled_timing(lib, prefix, step, steps, dom=None):
    """Per-kernel breakdown and the timed region, kept apart so that the events do not slow the
    step they time: K untimed steps with every launch bracketed by HIP events (the breakdown;
    the dominant kernel = the largest total unless `dom` names it), then the timed region of
    K steps (barrier + synchronize on both sides) with events around the dominant kernel's
    launches only (one pair per launch, on its own stream).  Returns (ms per step, breakdown
    totals {name: (total_ms, launches)}, dominant kernel, its average ms in the timed region)."""
    import torch

    from lucid_amd import _lib
    getattr(lib, prefix + "profile_reset")()
    getattr(lib, prefix + "profile_only")(None)
    getattr(lib, prefix + "profile_enable")(1)
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    getattr(lib, prefix + "profile_enable")(0)
    totals = _lib.profile_totals(lib, prefix)
    if dom is None:
        dom = max(totals.items(), key=lambda kv: kv[1][0])[0]
    getattr(lib, prefix + "profile_reset")()
    getattr(lib, prefix + "profile_only")(dom.encode())
    getattr(lib, prefix + "profile_enable")(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / steps * 1e3
    getattr(lib, prefix + "profile_enable")(0)
    getattr(lib, prefix + "profile_only")(None)
    timed = _lib.profile_totals(lib, prefix)
    getattr(lib, prefix + "profile_reset")()
    tot, cnt = timed[dom]
    return ms, totals, dom, tot / cnt


def _cpu_info():
    """Host CPU facts for the record: model name (lscpu), os.cpu_count(), the cores this process
    may run on (sched affinity) and the thread cap of the environment (OMP_NUM_THREADS)."""
    import subprocess
    model = None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model = line.split(":", 1)[1].strip()
    except Exception:  # lscpu missing: the record says so
        model = None
    affinity = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    omp = os.environ.get("OMP_NUM_THREADS")
    return {"model": model, "cpu_count": os.cpu_count(), "affinity": affinity,
            "omp_num_threads": int(omp) if omp and omp.isdigit() else None}


def cpu_baseline(T=32768, H_full=16, D=64):
    """Time the float32 torch restatement of the reference dense path on the host cores.

    One head at the full sequence length (fwd + bwd through autograd: dense P,
    solve_triangular, SDPA), times the head count -- all 16 heads at once need 64 GiB of
    fp32 P alone.  Threads: every core this process may run on, capped by OMP_NUM_THREADS
    where the host sets it (the GPU box's CPU share).  One untimed warm-up at T=1024; the
    median of three runs, or one run when it takes over 20 s.
    """
    import statistics

    import torch

    from oracle.lucid_ref import lucid_attention_torch

    info = _cpu_info()
    threads = info["affinity"]
    if info["omp_num_threads"]:
        threads = min(threads, info["omp_num_threads"])
    torch.set_num_threads(threads)

    def run(T_):
        g = torch.Generator().manual_seed(0)
        q, k, v = ((torch.randn(1, 1, T_, D, generator=g) / D ** 0.5).requires_grad_() for _ in range(3))
        do = torch.randn(1, T_, 1, D, generator=g)
        t0 = time.perf_counter()
        o, _ = lucid_attention_torch(q, k, v)
        o.backward(do)
        return time.perf_counter() - t0

    run(1024)  # warm-up
    times = [run(T)]
    if times[0] < 20.0:
        times += [run(T), run(T)]
    t = statistics.median(times)
    return {
        "value": T / (t * H_full),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"1 head of the workload (B1 H1 T{T} d{D}), fp32, torch CPU dense P + solve_triangular + SDPA, "
                   f"fwd+bwd: {'median of 3' if len(times) == 3 else 'one run'} {t:.2f} s "
                   f"({', '.join(f'{x:.2f}' for x in times)}); x {H_full} heads"),
        "host": info,
    }


def _bench_inputs(B, Hq, Hkv, T, D, dev, grad=True, keys="iid", dtype=None):
    import torch
    dt = dtype or torch.bfloat16
    g = torch.Generator().manual_seed(0)
    mk = lambda *shape: (torch.randn(*shape, generator=g) / D ** 0.5).to(dt).to(dev)  # noqa: E731
    q, k, v = mk(B, Hq, T, D), mk(B, Hkv, T, D), mk(B, Hkv, T, D)
    if keys == "correlated":  # a shared direction per head + 0.1 N(0,1) noise
        base = torch.randn(B, Hkv, 1, D, generator=g)
        k = ((base + 0.1 * torch.randn(B, Hkv, T, D, generator=g)) / D ** 0.5).to(dt).to(dev)
    if grad:
        for x in (q, k, v):
            x.requires_grad_()
    do = torch.randn(B, T, Hq, D, generator=g).to(dt).to(dev)
    return q, k, v, do


def _path_inputs(B, H, T, D, dev, dtype=None):
    import torch
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, T, H, D, generator=g) for _ in range(3))
    w = torch.randn(B, T, H, D, generator=g)
    w = w / w.norm(dim=-1, keepdim=True)
    beta = 2 * torch.sigmoid(torch.randn(B, T, H, generator=g))
    do = torch.randn(B, T, H, D, generator=g)
    xs = [x.to(dtype or torch.bfloat16).to(dev) for x in (q, k, v, w, beta, do)]
    for x in xs[:5]:
        x.requires_grad_()
    return xs


# LUCID-Path kernel FLOPs of this implementation's algorithm (per query head, in T^2 d,
# causal halves): the two-level transport makes every inter-chunk logit block one GEMM.
# Executed per step: LUCID-Path 10 T^2 d per query head (solve 2 + dV 2 + row 3 + col 3),
# PaTH softmax 9 (2 + 3 + 4), against the reference algorithm's 16 T^2 d (the bench's
# headline count, which also charges the per-pair query propagation).
PATH_EXECUTED = {"path": 10.0, "path_softmax": 9.0}
PATH_KERNEL_FLOPS = {
    "path_solve_fwd_kernel": 2.0,  # A = Q K^T, L O
    "path_dv_kernel": 2.0,         # A, L^T dV
    "path_bwd_row_kernel": 3.0,    # A, dV O^T, dA K
    "path_bwd_col_kernel": 3.0,    # A, dV O^T, dA^T Q
    # PaTH softmax attention
    "path_softmax_fwd_kernel": 2.0,      # A, P V
    "path_softmax_bwd_row_kernel": 3.0,  # A, dO V^T, dA K
    "path_softmax_bwd_col_kernel": 4.0,  # A, dO V^T, dA^T Q, P^T dO
}


def copy_calibration(nbytes: int, reps: int = 3) -> None:
    """A plain copy of ``nbytes`` (reads nbytes, writes nbytes) so that per-dispatch
    HBM counters can be scaled to bytes: factor = nbytes / counter reading."""
    import torch
    x = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        y.copy_(x)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) / reps * 1e3
    print(json.dumps({"copy_bytes": nbytes, "ms": round(ms, 4), "GB/s": round(2 * nbytes / ms / 1e6, 1)}),
          flush=True)


def measured_traffic(workload, kernel):
    """Calibrated HBM bytes per launch of `kernel` at `workload`'s shape, from
    profiles/traffic.json (rocprofv3 FETCH_SIZE + WRITE_SIZE runs); None if not measured."""
    tfile = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")
    if not os.path.exists(tfile):
        return None
    with open(tfile) as fh:
        return json.load(fh).get(workload, {}).get(kernel)


def bench_decode(args, dev):
    """One LUCID decoding step (one layer's attention for ``--decode-tokens`` L new tokens per
    sequence, default 1) against a full cache at the long-context shape of config 5: B=1,
    Hq=32 over Hkv=8, d=128, T=131072 cached rows.  HBM-bound: the K and V' caches are read
    once per pass of up to 32 / (Hq/Hkv + 1) = 6 tokens."""
    import torch

    from lucid_amd import _lib, lucid_decode

    B, Hq, Hkv, T, D = 1, 32, 8, 131072, 128
    g = torch.Generator().manual_seed(0)
    s = D ** -0.5
    L = args.decode_tokens
    kc = (torch.randn(B, Hkv, T + L, D, generator=g) * s).to(torch.bfloat16).to(dev)
    vc = (torch.randn(B, Hkv, T + L, D, generator=g) * s).to(torch.bfloat16).to(dev)
    q = (torch.randn(B, Hq, L, D, generator=g) * s).to(torch.bfloat16).to(dev)
    k = (torch.randn(B, Hkv, L, D, generator=g) * s).to(torch.bfloat16).to(dev)
    v = (torch.randn(B, Hkv, L, D, generator=g) * s).to(torch.bfloat16).to(dev)
    lib = _lib.load()

    def step():  # every step decodes rows T .. T+L-1 against rows [0, T) (same work each time)
        lucid_decode(q, k, v, kc, vc, T)

    args.warmup = warm_up(step, args.warmup)
    ms, totals, dom, dom_avg = profiled_timing(lib, "lucid_", step, args.steps, "lucid_decode_split_kernel")
    kernels = {n: {"avg_ms": round(tot / cnt, 4), "launches": cnt} for n, (tot, cnt) in
               sorted(totals.items(), key=lambda kv: -kv[1][0])}
    nbytes = 2.0 * B * Hkv * T * D * 2  # K and V' caches, bf16, read once per split pass
    achieved = nbytes / (dom_avg / 1e3) / 1e9
    traffic = measured_traffic("decode", dom) if L == 1 else None
    out = {
        "metric": "LUCID decode step (one layer, L new tokens) tokens/s at T=128K cache (config-5 shape)",
        "value": round(B * L / (ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)/sqrt(d) caches and token)",
        "config": {"workload": "lucid_decode_step", "B": B, "Hq": Hq, "Hkv": Hkv, "T_cache": T, "head_dim": D,
                   "new_tokens": L, "parallelism": "single GPU"},
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": nbytes},
        "kernels": kernels,
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def bench_c3(args, dev):
    """Decoder training step: 16 layers, hidden 2048, 32 x 64 heads, SwiGLU 5632, vocab 32000,
    bf16 weights, random init N(0, 0.02); tokens uniform over the vocabulary, labels = tokens.
    One step = forward + loss + backward + AdamW update (lucid_amd.optim.AdamW).  The same
    model with the attention core swapped for PyTorch's causal SDPA is timed beside it (plain
    Llama: the same GEMMs, fused RMSNorm, RoPE, SwiGLU, loss and optimizer kernels)."""
    import torch

    from lucid_amd import _lib, modeling_lucid as M
    from lucid_amd.optim import AdamW

    cfg = M.c3_config()
    B, T = 1, 8192
    torch.manual_seed(0)
    model = M.LlamaForCausalLM(cfg).to(dev, torch.bfloat16)
    opt = AdamW(model.parameters(), lr=1e-4)  # torch.optim.AdamW's update on one HIP pass per step
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=torch.Generator().manual_seed(1)).to(dev)
    lib = _lib.load()
    losses = []

    def step():
        opt.zero_grad(set_to_none=True)
        loss, _ = model(ids, labels=ids)
        loss.backward()
        opt.step()
        return loss

    first = step().item()
    args.warmup = 1 + warm_up(step, None if args.warmup is None else max(0, args.warmup - 1))
    ms, totals, dom, dom_avg = profiled_timing(lib, "lucid_", lambda: losses.append(step()), args.steps)
    model_ops = ("lucid_rmsnorm", "lucid_rope", "lucid_swiglu", "lucid_ce_", "lucid_adamw")  # not attention
    attn_ms = sum(tot for n, (tot, _) in totals.items() if not n.startswith(model_ops)) / args.steps
    layers_ms = sum(tot for n, (tot, _) in totals.items() if n.startswith(model_ops)) / args.steps
    kernels = {n: {"avg_ms": round(tot / cnt, 4), "launches": cnt} for n, (tot, cnt) in
               sorted(totals.items(), key=lambda kv: -kv[1][0])}
    H, D = cfg.num_attention_heads, cfg.head_dim
    achieved = KERNEL_FLOPS[dom](B, H, H, T, D) / (dom_avg / 1e3) / 1e12
    n_params = M.count_parameters(model)
    # 6 N per token for the dense layers and head, plus the attention core's count
    flops = 6.0 * n_params * B * T + cfg.num_hidden_layers * lucid_flops(B, H, H, T, D)

    # comparator: identical model and optimizer, attention core = causal SDPA on (q, k, v)
    saved = M.lucid_attention

    def sdpa_core(q, k, v, scaling=None, eps=1e-5, return_vprime=False):
        o = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scaling)
        o = o.transpose(1, 2)
        return (o, None) if return_vprime else o

    cms = None
    if not args.no_causal:
        M.lucid_attention = sdpa_core
        try:
            for _ in range(max(1, args.warmup)):
                step()
            torch.cuda.synchronize()
            c0 = time.perf_counter()
            for _ in range(args.steps):
                step()
            torch.cuda.synchronize()
            cms = (time.perf_counter() - c0) / args.steps * 1e3
        finally:
            M.lucid_attention = saved

    out = {
        "metric": "Llama-LUCID decoder training step tokens/s (config 3)",
        "value": round(B * T / (ms / 1e3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (tokens uniform over the vocabulary, seeded; random-init weights N(0, 0.02))",
        "config": {"workload": "llama_lucid_train_step", "layers": cfg.num_hidden_layers,
                   "hidden": cfg.hidden_size, "heads": H, "head_dim": D, "ffn": cfg.intermediate_size,
                   "vocab": cfg.vocab_size, "params": n_params, "global_batch": B, "seq_len": T,
                   "optimizer": "AdamW (lucid_amd.optim: torch.optim.AdamW's update, one HIP pass)",
                   "parallelism": "single GPU"},
        "loss_first_step": round(first, 4),
        "loss_last_step": round(losses[-1].item(), 4),
        "tflops": round(flops / (ms / 1e3) / 1e12, 1),
        "attention_ms_per_step": round(attn_ms, 3),
        "fused_layers_and_optimizer_ms_per_step": round(layers_ms, 3),
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None},
        "kernels": kernels,
        "causal_comparator": None if cms is None else {
            "impl": "same model, attention core = torch SDPA causal (ROCm)", "ms_per_step": round(cms, 3),
            "lucid_over_causal": round(ms / cms, 3)},
        "cpu_baseline": None,
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed warmup steps (default: at least 3 steps and 0.5 s of GPU work)")
    ap.add_argument("--workload", default="lucid",
                    choices=["lucid", "c2", "c3", "c5", "gqa128", "ref_f32", "ref_bf16", "path", "path128", "path_f32",
                             "path_softmax", "decode"],
                    help="lucid: north star B1 H16 T32768 d64 fwd+bwd (default); c2: B4 H16 T4096 d64 "
                         "fwd+bwd; c3: 16-layer Llama-LUCID decoder, one training step (fwd+bwd+AdamW) "
                         "on B1 x T8192; c5: B1 T131072 Hq32/Hkv8 d128 forward only; gqa128: the config-5 heads "
                         "(Hq32/Hkv8 d128) at B1 T32768, fwd+bwd; ref_f32: the attention layer of the reference's shipped "
                         "LUCID model config (fp32, head dim 68, 32 query / 4 kv heads) at B8 T2048, fwd+bwd; ref_bf16: "
                         "the same shape in bf16; path: LUCID-Path "
                         "B1 H16 T32768 d64 fwd+bwd; path128: the same at head dim 128; path_f32: config 4 on fp32 "
                         "inputs; path_softmax: PaTH softmax attention on the config-4 "
                         "shape, fwd+bwd; decode: one decoding step against a 128K cache (config-5 heads)")
    ap.add_argument("--precision", default="auto", choices=["auto", "fast", "exact"],
                    help="LUCID chain precision (lucid_amd.set_precision): auto picks per head from the row "
                         "mass; exact forces the hi/lo split chains for every head")
    ap.add_argument("--keys", default="iid", choices=["iid", "correlated"],
                    help="iid: the BASELINE inputs; correlated: every key = a shared direction + 0.1 N(0,1) "
                         "(row mass ~T, the exact chains under --precision auto)")
    ap.add_argument("--decode-tokens", type=int, default=1,
                    help="new tokens per decoding call (--workload decode)")
    ap.add_argument("--no-fused-fwd", action="store_true",
                    help="time the two-kernel forward (chain, then attention) instead of the fused kernel "
                         "(lucid_amd.set_fused_forward)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-causal", action="store_true")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="calibration only: time a plain device copy of this many bytes (the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings) and exit")
    args = ap.parse_args()

    if args.copy_bytes:
        copy_calibration(args.copy_bytes)
        return
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only; --gpus {args.gpus} is not supported "
              "(heads shard across GPUs with no exchange; no multi-GPU run is part of this build)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    from lucid_amd import _lib, lucid_attention, set_fused_forward, set_precision

    dev = torch.device("cuda:0")
    wl = args.workload
    set_precision(args.precision)
    set_fused_forward(not args.no_fused_fwd)
    if wl == "c3":
        bench_c3(args, dev)
        return
    if wl == "decode":
        bench_decode(args, dev)
        return
    fwd_only = wl == "c5"
    path_kind = {"path": "path", "path128": "path", "path_f32": "path", "path_softmax": "path_softmax"}.get(wl)
    executed = None
    if path_kind:
        from lucid_amd.lucid_path import parallel_lucid_path_attention, parallel_path_attention
        B, Hq, Hkv, T, D = 1, 16, 16, 32768, (128 if wl == "path128" else 64)
        q, k, v, w, beta, do = _path_inputs(B, Hq, T, D, dev, torch.float32 if wl == "path_f32" else None)
        lib, prefix = _lib.load("liblucid_path.so"), "lucid_path_"

        def step():
            for x in (q, k, v, w, beta):
                x.grad = None
            if path_kind == "path":
                o, _ = parallel_lucid_path_attention(k, v, w, beta, q=q)
            else:
                o, _ = parallel_path_attention(q, k, v, w, beta)
            o.backward(do)
        # count of the reference algorithm (query propagated through every chunk pair):
        # fwd 4 T^2 d (A, L O, 2x propagation) + bwd 12 T^2 d per query head
        flops = 16.0 * T * T * D * B * Hq
        executed = PATH_EXECUTED[path_kind] * T * T * D * B * Hq
        kflops = {n: f * T * T * D * B * Hq for n, f in PATH_KERNEL_FLOPS.items()}
        metric = {"path": "LUCID-Path fwd+bwd tokens/s & TFLOP/s at T=32K bf16 (config 4)",
                  "path128": "LUCID-Path fwd+bwd tokens/s & TFLOP/s at T=32K bf16, head dim 128",
                  "path_f32": "LUCID-Path fwd+bwd tokens/s & TFLOP/s at T=32K fp32 (config 4, fp32 inputs)",
                  "path_softmax": "PaTH softmax attention fwd+bwd tokens/s & TFLOP/s at T=32K bf16 "
                                  "(config-4 shape)"}[wl]
    else:
        B, Hq, Hkv, T, D = {"lucid": (1, 16, 16, 32768, 64), "c2": (4, 16, 16, 4096, 64),
                            "c5": (1, 32, 8, 131072, 128), "gqa128": (1, 32, 8, 32768, 128),
                            "ref_f32": (8, 32, 4, 2048, 68), "ref_bf16": (8, 32, 4, 2048, 68)}[wl]
        q, k, v, do = _bench_inputs(B, Hq, Hkv, T, D, dev, grad=not fwd_only, keys=args.keys,
                                    dtype=torch.float32 if wl == "ref_f32" else None)
        lib, prefix = _lib.load(), "lucid_"

        def step():
            if fwd_only:
                with torch.no_grad():
                    lucid_attention(q, k, v)
                return
            q.grad = k.grad = v.grad = None
            o = lucid_attention(q, k, v)
            o.backward(do)
        if fwd_only:
            flops = 2.0 * T * T * D * B * (Hq + Hkv)
            kflops = {n: KERNEL_FLOPS[n](B, Hq, Hkv, T, D) for n in
                      ("lucid_precond_fwd_kernel", "lucid_precond_fwd_wide_kernel", "lucid_attn_fwd_kernel",
                       "lucid_attn_fwd_wide_kernel", "lucid_fused_fwd_kernel")}
        else:
            flops = lucid_flops(B, Hq, Hkv, T, D)
            kflops = {n: f(B, Hq, Hkv, T, D) for n, f in KERNEL_FLOPS.items()}
        metric = "LUCID attn fwd+bwd tokens/s & TFLOP/s at T=32K bf16; % MFMA peak; vs CPU ref"
        if wl != "lucid":
            metric = f"LUCID attention {'forward' if fwd_only else 'fwd+bwd'} tokens/s & TFLOP/s ({wl})"

    args.warmup = warm_up(step, args.warmup)
    ms, totals, dom, dom_avg = profiled_timing(lib, prefix, step, args.steps)
    tokens_s = B * T / (ms / 1e3)

    kernels = {}
    for name, (tot, cnt) in sorted(totals.items(), key=lambda kv: -kv[1][0]):
        avg = tot / cnt
        kf = kflops.get(name, 0.0)
        kernels[name] = {"avg_ms": round(avg, 4), "launches": cnt,
                         "tflops": round(kf / (avg / 1e3) / 1e12, 1) if kf else None}
    achieved = kflops.get(dom, 0.0) / (dom_avg / 1e3) / 1e12
    traffic = measured_traffic(wl, dom)

    causal = None
    if not args.no_causal and wl in ("lucid", "c2", "path_softmax"):
        import torch.nn.functional as F

        from lucid_amd import causal_attention
        if wl == "path_softmax":  # [B, T, H, D] inputs
            qc, kc, vc = (t.detach().transpose(1, 2).contiguous().requires_grad_() for t in (q, k, v))
            doc = do.transpose(1, 2).contiguous()
        else:
            qc, kc, vc = (t.detach().clone().requires_grad_() for t in (q, k, v))
            doc = do.transpose(1, 2)

        def sdpa_step():
            qc.grad = kc.grad = vc.grad = None
            F.scaled_dot_product_attention(qc, kc, vc, is_causal=True).backward(doc)

        def own_step():  # the build's attention kernels with V' = V (outputs [B, T, H, D])
            qc.grad = kc.grad = vc.grad = None
            causal_attention(qc, kc, vc).backward(do)

        def timed(fn):
            for _ in range(max(1, args.warmup)):
                fn()
            torch.cuda.synchronize()
            c0 = time.perf_counter()
            for _ in range(args.steps):
                fn()
            torch.cuda.synchronize()
            return (time.perf_counter() - c0) / args.steps * 1e3

        sdpa_ms = timed(sdpa_step)
        set_precision("fast")  # plain attention has no preconditioner: skip the row-mass pass
        try:
            own_ms = timed(own_step)
        finally:
            set_precision(args.precision)
        best = min(sdpa_ms, own_ms)
        cf = causal_flops(B, Hq, T, D)
        causal = {"sdpa": {"impl": "torch.nn.functional.scaled_dot_product_attention (ROCm)",
                           "ms_per_step": round(sdpa_ms, 3), "tflops": round(cf / (sdpa_ms / 1e3) / 1e12, 1)},
                  "own": {"impl": "lucid_amd.causal_attention (this build's attention kernels, V' = V)",
                          "ms_per_step": round(own_ms, 3), "tflops": round(cf / (own_ms / 1e3) / 1e12, 1)},
                  "faster": "own" if own_ms <= sdpa_ms else "sdpa",
                  "lucid_over_causal": round(ms / best, 3)}

    cpu = None
    if not args.no_cpu_baseline and wl == "lucid":
        cpu = cpu_baseline(T=T, H_full=B * Hq, D=D)

    out = {
        "metric": metric,
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if wl in ("path_f32", "ref_f32") else "bf16",
        "data": "synthetic (seeded N(0,1)/sqrt(d) q,k,v; N(0,1) dO)" if not path_kind
                else "synthetic (seeded N(0,1) q,k,v,w; w L2-normalised; beta=2 sigmoid(N(0,1)); N(0,1) dO)",
        "precision": args.precision, "keys": args.keys, "fused_forward": not args.no_fused_fwd,
        "config": {"workload": {"lucid": "lucid_attention_fwd_bwd", "c2": "lucid_attention_fwd_bwd",
                                "c5": "lucid_attention_fwd", "gqa128": "lucid_attention_fwd_bwd",
                                "ref_f32": "lucid_attention_fwd_bwd", "ref_bf16": "lucid_attention_fwd_bwd",
                                "path": "lucid_path_fwd_bwd", "path128": "lucid_path_fwd_bwd",
                                "path_f32": "lucid_path_fwd_bwd",
                                "path_softmax": "path_softmax_attention_fwd_bwd"}[wl],
                   "B": B, "Hq": Hq, "Hkv": Hkv, "T": T, "head_dim": D, "causal": True,
                   "parallelism": "single GPU"},
        "tflops": round(flops / (ms / 1e3) / 1e12, 1),
        "frac_mfma_peak": round(flops / (ms / 1e3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4),
        # path workloads: the work this implementation executes (see PATH_EXECUTED), beside the
        # reference algorithm's count above
        "tflops_executed": round(executed / (ms / 1e3) / 1e12, 1) if executed else None,
        "frac_mfma_peak_executed": (round(executed / (ms / 1e3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 4)
                                    if executed else None),
        "roofline": {"kernel": dom, "bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": traffic},
        "kernels": kernels,
        "causal_comparator": causal,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
