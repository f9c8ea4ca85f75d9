"""Benchmark of the quantized scoring path on one MI355X.

Workload (one step): the option-row scoring pass of 8 requests through a random-init 36-layer 9B-class decoder
(hidden 4096, FFN 12288, 32 query / 8 KV heads, head_dim 128), every request scoring 32 options of 16 tokens against
its own cached 2048-token state held as int8 K/V with per-token-per-head fp32 scales (one cache per layer), ending in
per-request log-probabilities over the 32 options and 'none'. Per layer: RMSNorm+int8 quantize, W8A8 QKV GEMM,
q/k norm + RoPE, branched attention over the int8 state + own tokens, W8A8 O GEMM (+residual), RMSNorm+quantize,
W8A8 gate+up GEMM, SwiGLU+quantize, W8A8 down GEMM (+residual). The states' K/V are synthetic (bf16 N(0,1)
quantized by the append kernel) and resident in HBM before timing; so are the option token ids.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]

Prints ONE JSON line: metric / value (decisions/s) / timing, the roofline of the dominant kernel (the W8A8 GEMM,
int8 MFMA), the branched attention's figures, and a CPU baseline (the oracle, on this host's cores, on a bounded
sample of the same workload, scaled).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decisions/sec (2k-tok state, 32 opts, 9B dims); int8 GEMM TOPS; attn HBM GB/s"
INT8_PEAK_TOPS = 5000.0      # MI355X dense int8 MFMA
BF16_PEAK_TFLOPS = 2500.0    # MI355X dense bf16 / fp16 MFMA
HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--requests", type=int, default=8)
    ap.add_argument("--options", type=int, default=32)
    ap.add_argument("--tokens", type=int, default=16)
    ap.add_argument("--state", type=int, default=2048)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-repeats", type=int, default=3)
    return ap.parse_args()


class KernelTimer:
    """Wraps a kernels.* entry point and brackets every call with HIP events on the current stream (the stream the
    kernel is launched on), accumulating its algorithmic work."""

    def __init__(self, fn, work):
        import torch
        self.fn, self.work, self.torch = fn, work, torch
        self.events, self.units, self.active = [], [], False

    def __call__(self, *a, **k):
        if not self.active:
            return self.fn(*a, **k)
        e0, e1 = self.torch.cuda.Event(enable_timing=True), self.torch.cuda.Event(enable_timing=True)
        e0.record()
        r = self.fn(*a, **k)
        e1.record()
        self.events.append((e0, e1))
        self.units.append(self.work(*a, **k))
        return r

    def summary(self):
        ms = [e0.elapsed_time(e1) for e0, e1 in self.events]
        n = len(ms)
        tot_ms = sum(ms)
        tot_units = [sum(u[i] for u in self.units) for i in range(len(self.units[0]))] if n else []
        return n, tot_ms, tot_units


def gemm_work(a, sa, w, sw, bias=None, residual=None, out=None, want_out=True, want_acc=False):
    M, K = a.shape
    N = w.shape[0]
    return (2 * M * N * K, M * K + N * K + 2 * M * N + (2 * M * N if residual is not None else 0))


def attn_work(q, k_own, v_own, kq, ks, vq, vs, scale, kvalid=None, row_counts=None, length=None, out=None,
              return_lse=False, row_start=None, max_rows=None):
    R, Hq, t, D = q.shape
    Ns, Hkv, cap, _ = kq.shape
    T = length
    rows_per_state = R // Ns
    flops_prefix = 4 * Ns * Hq * rows_per_state * t * T * D
    flops_own = 4 * R * Hq * t * (t + 1) // 2 * D
    # algorithmic HBM bytes: int8 state K/V + fp32 scales once, q / own k,v / out once
    bytes_ = 2 * Ns * Hkv * T * D + 2 * Ns * Hkv * T * 4 + 2 * R * Hq * t * D * 2 + 2 * R * Hkv * t * D * 2
    return (flops_prefix + flops_own, bytes_)


def cpu_baseline(args):
    """The oracle (CPU torch restatement of the path) on a bounded sample: ONE request (32 options x 16 tokens, its
    2048-token int8 state) through ONE 9B-dims layer, timed and scaled x36 layers x8 requests."""
    import torch

    from oracle import decoder as od
    from oracle import quant as oq
    torch.set_num_threads(os.cpu_count() or 1)
    cfg = od.DecoderConfig(n_layers=1, vocab=1000)
    w = od.make_weights(cfg, seed=1)
    lw = w["layers"][0]
    ql = od.quantize_layer(lw)
    g = torch.Generator().manual_seed(2)
    T, n_opt, t = args.state, args.options, args.tokens
    kv = torch.randn(2, 1, cfg.n_kv_heads, T, cfg.head_dim, generator=g).to(torch.bfloat16)
    kq, ks = oq.quantize_rows(kv[0])
    vq, vs = oq.quantize_rows(kv[1])
    h = torch.randn(n_opt * t, cfg.hidden, generator=g).to(torch.bfloat16)
    pos = (T + torch.arange(t)).repeat(n_opt)
    cos, sin = od.rope_tables(cfg, T + t)

    def run():
        return od.layer_forward(h, lw, ql, cfg, (kq, ks[..., 0]), (vq, vs[..., 0]), n_opt, t, pos, cos, sin)

    run()
    ts = []
    for _ in range(args.cpu_sample_repeats):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    per_layer = ts[len(ts) // 2]
    decision_s = per_layer * args.layers  # one request's scoring pass
    return {"value": 1.0 / decision_s, "unit": "decisions/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"1 request (32 options x 16 tokens, {T}-token int8 state) x 1 of {args.layers} layers, "
                       f"median of {args.cpu_sample_repeats} after a warm-up, {per_layer * 1e3:.0f} ms per layer, "
                       f"scaled x{args.layers} layers")}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from opendecider_amd import decoder as dmod
    from opendecider_amd import kernels
    from opendecider_amd.kv_cache import Int8KVCache

    dev = "cuda:0"
    torch.cuda.set_device(0)
    cfg = dmod.DecoderConfig(n_layers=args.layers)
    B, n_opt, t, T = args.requests, args.options, args.tokens, args.state
    dec = dmod.random_decoder(cfg, seed=0, device=dev, max_pos=T + t + 16)
    g = torch.Generator(device=dev).manual_seed(1)
    states = []
    for _ in range(cfg.n_layers):
        pair = []
        for _ in range(2):
            c = Int8KVCache(B, cfg.n_kv_heads, cfg.head_dim, T, dev)
            c.append(torch.randn(B, cfg.n_kv_heads, T, cfg.head_dim, generator=g, device=dev).to(torch.bfloat16))
            pair.append(c)
        states.append(tuple(pair))
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=g, device=dev)
    torch.cuda.synchronize()

    gemm_t = KernelTimer(kernels.w8a8_gemm, gemm_work)
    attn_t = KernelTimer(kernels.branched_attn, attn_work)
    kernels.w8a8_gemm, kernels.branched_attn = gemm_t, attn_t

    for _ in range(args.warmup):
        out = dec.score(ids, states)
    torch.cuda.synchronize()
    gemm_t.active = attn_t.active = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = dec.score(ids, states)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    gemm_t.active = attn_t.active = False
    assert torch.isfinite(out).all(), "non-finite log-probabilities"

    ms_per_step = dt / args.steps * 1e3
    n_g, ms_g, (ops_g, bytes_g) = gemm_t.summary()
    n_a, ms_a, (fl_a, by_a) = attn_t.summary()
    gemm_tops = ops_g / (ms_g * 1e-3) / 1e12
    attn_tflops = fl_a / (ms_a * 1e-3) / 1e12
    attn_gbs = by_a / (ms_a * 1e-3) / 1e9
    res = {
        "metric": METRIC,
        "value": B * args.steps / dt,
        "unit": "decisions/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": (f"option-row scoring pass: {B} requests x {n_opt} options x {t} tokens over cached "
                                f"{T}-token int8 K/V states, {cfg.n_layers}-layer 9B-dims decoder (hidden 4096, "
                                f"FFN 12288, 32/8 heads, head_dim 128), W8A8 linears, random init"),
                   "requests": B, "options": n_opt, "tokens_per_option": t, "state_tokens": T,
                   "layers": cfg.n_layers, "tokens_per_layer": B * n_opt * t},
        "roofline": {"kernel": "od_w8a8_gemm (all 4 layer GEMMs)", "bound": "mfma",
                     "achieved": gemm_tops, "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": gemm_tops / INT8_PEAK_TOPS, "traffic": None,
                     "note": "int8 ops (TOPS) per launch over launch duration (HIP events, timed region)",
                     "launches": n_g, "avg_launch_us": ms_g / max(n_g, 1) * 1e3},
        "attention": {"kernel": "od_branched_attn", "tflops": attn_tflops, "frac_of_bf16_mfma": attn_tflops /
                      BF16_PEAK_TFLOPS, "algorithmic_gbs": attn_gbs, "frac_of_hbm": attn_gbs / HBM_PEAK_GBS,
                      "launches": n_a, "avg_launch_us": ms_a / max(n_a, 1) * 1e3},
        "time_share": {"gemm": ms_g / (ms_per_step * args.steps), "attention": ms_a / (ms_per_step * args.steps)},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(args)
    print(json.dumps(res))


if __name__ == "__main__":
    main()
