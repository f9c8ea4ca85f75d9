"""Benchmark of the quantized scoring path on one MI355X.

Workload (one step): the option-row scoring pass of 8 requests through a random-init 36-layer 9B-class decoder
(hidden 4096, FFN 12288, 32 query / 8 KV heads, head_dim 128), every request scoring 32 options of 16 tokens against
its own cached 2048-token state held as int8 K/V with per-token-per-head fp32 scales (one cache per layer), ending in
per-request log-probabilities over the 32 options and 'none'. Per layer: RMSNorm+int8 quantize, W8A8 QKV GEMM,
q/k norm + RoPE, branched attention over the int8 state + own tokens, W8A8 O GEMM (+residual), RMSNorm+quantize,
W8A8 gate+up GEMM, SwiGLU+quantize, W8A8 down GEMM (+residual). The states' K/V are synthetic (bf16 N(0,1)
quantized by the append kernel) and resident in HBM before timing; so are the option token ids.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline] [--scoring-only]
                    [--workload scoring|decision|wide_choice|gemm|gemm_traffic|attention|lm_logprob|
                                qcache_rows|mfma_ceiling|hybrid]

Prints ONE JSON line: metric / value (decisions/s) / timing, the roofline of the dominant kernel (the W8A8 GEMM,
int8 MFMA), the branched attention's figures, and a CPU baseline (the oracle, on this host's cores, on a bounded
sample of the same workload, scaled). The default line also carries the full decision forward from token ids
("decision": 4096-token states prefilled, 64 options x 24 tokens), the wide-choice growing state ("wide_choice":
a 32768-token int8 state + 256-token records, 2 x 255 options x 12 tokens) and the decision on the Qwen3.5 hybrid
stack ("hybrid": 24 Gated DeltaNet + 8 full-attention layers), each with its own CPU baseline, and the kernel-level
figures: the few-slot KV-bound attention ("attention_kv_bound", 16 query slots per KV head) beside the KV-bound probe
("attention_kv_probe": the same 32768-token states with 2 options x 16 tokens, 128 slots per KV head, near the
HBM / bf16 ridge),
the single 256 x 4096 x 4096 W8A8 linear with the reference's CPU linear path ("config0_linear"), the reference's
scripts/bench_gemm.py sweep beside the vendor int8 GEMM ("gemm_sweep") and scripts/bench_qcache_rows.py's question
cache shapes with a CPU baseline ("qcache_rows"). --scoring-only leaves all sub-objects out. Every CPU baseline is
the median of --cpu-sample-repeats timed runs after one warm-up and names the host CPU model.
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

PROBE_MODES = {0: ("int8", "constant operands"), 1: ("int8", "operands changing every round"),
               2: ("int8", "operands read from LDS (6 fragment reads per 8 MFMAs)"),
               3: ("bf16", "operands changing every round"), 4: ("bf16", "operands read from LDS")}


def mfma_ceiling(modes=(0, 1, 2, 3, 4), iters=100000):
    """Matrix-core throughput the chip sustains (od_probe_mfma in libod_probe.so): per mode, dense TOPS (int8) or
    TFLOP/s (bf16) and the mean core clock in MHz under that load (s_memtime over s_memrealtime)."""
    import ctypes

    from opendecider_amd import build as _b
    L = ctypes.CDLL(_b.PROBE_LIB)
    L.od_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                                ctypes.POINTER(ctypes.c_double)]
    L.od_probe_mfma.restype = ctypes.c_int
    out = {}
    for m in modes:
        tops, mhz = ctypes.c_double(), ctypes.c_double()
        rc = L.od_probe_mfma(m, iters, ctypes.byref(tops), ctypes.byref(mhz))
        if rc != 0:
            raise RuntimeError(f"od_probe_mfma({m}) failed: {rc}")
        dt, what = PROBE_MODES[m]
        peak = INT8_PEAK_TOPS if dt == "int8" else BF16_PEAK_TFLOPS
        out[f"mode{m}"] = {"dtype": dt, "operands": what, "value": tops.value, "frac_of_peak": tops.value / peak,
                           "clock_mhz": mhz.value}
    return out


def hbm_ceiling(gib: int = 2, reps: int = 10):
    """HBM read rate the chip sustains (od_probe_hbm_read in libod_probe.so): a buffer of `gib` GiB (well past the
    256 MB Infinity Cache) read with 16-byte non-temporal loads, by a grid-stride kernel at 4, 8 and 16 workgroups
    per CU and as contiguous per-workgroup chunks at 1 and 2 workgroups of 8 waves per CU; the best, in GB/s."""
    import ctypes

    from opendecider_amd import build as _b
    L = ctypes.CDLL(_b.PROBE_LIB)
    L.od_probe_hbm_read.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.POINTER(ctypes.c_double)]
    L.od_probe_hbm_read.restype = ctypes.c_int
    gbs = ctypes.c_double()
    rc = L.od_probe_hbm_read(gib << 30, reps, ctypes.byref(gbs))
    if rc != 0:
        raise RuntimeError(f"od_probe_hbm_read failed: {rc}")
    return {"value": gbs.value, "unit": "GB/s", "frac_of_peak": gbs.value / HBM_PEAK_GBS,
            "probe": f"od_probe_hbm_read: {gib} GiB read with 16-byte non-temporal loads, best of a grid-stride "
                     "kernel (4/8/16 workgroups per CU) and contiguous chunks (1/2 workgroups of 8 waves per CU)"}


def _sustained(ceil, mode):
    c = ceil[f"mode{mode}"]
    return {"value": c["value"], "clock_mhz": c["clock_mhz"], "frac_of_peak": c["frac_of_peak"],
            "probe": f"od_probe_mfma mode {mode}: {c['dtype']} MFMAs, {c['operands']}, 8 waves per CU"}


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
    ap.add_argument("--workload", choices=["scoring", "decision", "wide_choice", "gemm", "gemm_traffic",
                                           "attention", "lm_logprob", "qcache_rows", "mfma_ceiling", "hybrid"],
                    default="scoring",
                    help="scoring (default): the metric's option-row scoring pass over cached 2048-token states; "
                         "decision: full decision forward from token ids (4 requests, 4096-token states prefilled, "
                         "64 options x 24 tokens); wide_choice: a 32768-token int8 state growing by 256-token "
                         "records, 2 requests x 255 options x 12 tokens scored after each record; gemm_traffic: "
                         "the run the GEMM traffic counters are read on (a 256 MiB device copy to calibrate them, "
                         "then two scoring passes through 2 layers, i.e. each M = 4096 GEMM shape twice); "
                         "attention: the branched attention alone on the 8-state option-row shape and on the KV-bound probe "
                         "(32768-token states, 2 options x 16 tokens per state); lm_logprob: the LM head's token "
                         "log-prob of 1024 rows over a 151936 x 4096 int8 table; gemm: the W8A8 linear alone over "
                         "the reference's (K, N) x M sweep (scripts/bench_gemm.py) and the 9B layer shapes at M = 4096; "
                         "qcache_rows: decide latency with and without the question cache over the reference's "
                         "(questions, options) shapes (scripts/bench_qcache_rows.py); mfma_ceiling: what the "
                         "matrix cores sustain (int8 and bf16 MFMAs on constant, changing and LDS-fed operands, one "
                         "8-wave workgroup per CU) with the core clock under that load; hybrid: the decision "
                         "workload on the Qwen3.5 hybrid stack (32 layers, 24 Gated DeltaNet + 8 full attention)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--scoring-only", action="store_true",
                    help="the default line without its decision / wide_choice sub-objects")
    ap.add_argument("--cpu-sample-repeats", type=int, default=5)
    return ap.parse_args()


class AbiTimer:
    """Brackets calls of one C-ABI entry point with HIP events on the current stream (the stream its kernels are
    launched on) and accumulates the call's algorithmic work, computed from the ABI arguments. It replaces the
    entry point on the loaded library, so the events enclose the launch only (not the Python argument checks
    around it). every = k times the 1st, (k+1)th, ... call while active: a pair of timing events costs a few us of
    GPU time, and the scoring pass makes ~250 timed calls, so timing all of them would slow the pass by ~3%."""

    def __init__(self, name, work, every=1):
        import torch

        from opendecider_amd import _lib
        self.L = _lib.lib()
        self.name, self.fn, self.work, self.torch = name, getattr(self.L, name), work, torch
        self.events, self.units, self.active, self.every, self.calls = [], [], False, every, 0
        setattr(self.L, name, self)

    def __call__(self, *a):
        if not self.active:
            return self.fn(*a)
        self.calls += 1
        if (self.calls - 1) % self.every:
            return self.fn(*a)
        e0, e1 = self.torch.cuda.Event(enable_timing=True), self.torch.cuda.Event(enable_timing=True)
        e0.record()
        r = self.fn(*a)
        e1.record()
        self.events.append((e0, e1))
        self.units.append(self.work(*a))
        return r

    def summary(self):
        ms = [e0.elapsed_time(e1) for e0, e1 in self.events]
        n = len(ms)
        tot = [sum(u[i] for u in self.units) for i in range(len(self.units[0]))] if n else [0, 0]
        return n, sum(ms), tot

    def reset(self):
        self.events, self.units, self.calls = [], [], 0


# (work units from the raw arguments of each entry point, in include/od_mi355x.h order)
def gemm_work(a, lda, sa, w, ldw, sw, bias, residual, ldr, out, ldo, acc, ldacc, M, N, K, stream):
    return (2 * M * N * K, M * K + N * K + 2 * M * N + (2 * M * N if residual else 0))


def swiglu_work(a, lda, sa, w, ldw, sw, out, ldo, M, N, K, stream):
    # od_w8a8_gemm_swiglu: the gate+up GEMM (N = 2F weight rows), output bf16 [M, F]
    return (2 * M * N * K, M * K + N * K + M * N)


class GemmTimers:
    """The W8A8 GEMM entry points timed together (od_w8a8_gemm for QKV / O / down, od_w8a8_gemm_swiglu for
    gate+up); `shapes` records the shape key of every timed launch."""

    def __init__(self, every=1):
        self.shapes = []
        self.timers = [AbiTimer("od_w8a8_gemm", gemm_work, every), AbiTimer("od_w8a8_gemm_swiglu", swiglu_work, every)]
        plain, fused = (t.work for t in self.timers)
        self.timers[0].work = lambda *a: (self.shapes.append((a[14], a[15])), plain(*a))[1]
        self.timers[1].work = lambda *a: (self.shapes.append(("swiglu", a[9], a[10])), fused(*a))[1]
        self.every = every

    @property
    def active(self):
        return self.timers[0].active

    @active.setter
    def active(self, v):
        for t in self.timers:
            t.active = v

    def summary(self):
        n, ms, tot = 0, 0.0, [0, 0]
        for t in self.timers:
            tn, tms, ttot = t.summary()
            n, ms, tot = n + tn, ms + tms, [tot[0] + ttot[0], tot[1] + ttot[1]]
        return n, ms, tot

    def reset(self):
        self.shapes = []
        for t in self.timers:
            t.reset()


def attn_work(*a):
    R, Hq, Hkv, t, D, Ns, T = a[24:31]
    rows_per_state = R // Ns
    flops_prefix = 4 * Ns * Hq * rows_per_state * t * T * D
    flops_own = 4 * R * Hq * t * (t + 1) // 2 * D
    # algorithmic HBM bytes: int8 state K/V + fp32 scales once, q / own k,v / out once
    bytes_ = 2 * Ns * Hkv * T * D + 2 * Ns * Hkv * T * 4 + 2 * R * Hq * t * D * 2 + 2 * R * Hkv * t * D * 2
    return (flops_prefix + flops_own, bytes_)


def staged_work(*a):
    # od_branched_attn_staged: the same work as od_branched_attn (its arguments sit three places earlier)
    R, Hq, Hkv, t, D, Ns, T = a[21:28]
    return attn_work(*([None] * 24 + [R, Hq, Hkv, t, D, Ns, T]))


def stage_work(*a):
    # od_attn_stage: part of the same attention (its work is counted once, on the attention call)
    return (0, 0)


ATTN_KERNELS = ("od_attn_stage + od_branched_attn_staged (or od_branched_attn / od_branched_attn_split / "
                "od_branched_attn_stream)")


class AttnTimers:
    """The branched attention's entry points timed together: od_branched_attn and od_branched_attn_split (direct
    path), od_attn_stage and od_branched_attn_staged (staged path), od_branched_attn_stream (few slots)."""

    def __init__(self, every=1):
        # one stage and one attention call per layer: the same `every` times both on the same layers
        self.timers = [AbiTimer("od_branched_attn", attn_work, every), AbiTimer("od_attn_stage", stage_work, every),
                       AbiTimer("od_branched_attn_staged", staged_work, every),
                       AbiTimer("od_branched_attn_split", attn_work, every),  # same leading arguments
                       AbiTimer("od_branched_attn_stream", attn_work, every)]

    @property
    def active(self):
        return self.timers[0].active

    @active.setter
    def active(self, v):
        for t in self.timers:
            t.active = v

    def summary(self):
        n, ms, tot = 0, 0.0, [0, 0]
        for t in self.timers:
            tn, tms, ttot = t.summary()
            if t.name != "od_attn_stage":
                n += tn
            ms += tms
            tot = [tot[0] + ttot[0], tot[1] + ttot[1]]
        return n, ms, tot

    def reset(self):
        for t in self.timers:
            t.reset()


def wide_work(*a):
    B, H, G, T, S, DK, DV, causal = a[19:27]
    pairs = B * H * (T * S - (T * (T - 1) // 2 if causal and T == S else 0))
    return (2 * pairs * (DK + DV), 2 * (B * H * T * DK + 2 * B * G * S * DK + B * H * T * DV))


def append_work(x, B, H, n, D, *rest):
    return (B * H * n * D, B * H * n * D * 3 + B * H * n * 4)


def rope_append_work(qkv, ld, B, S, Hq, Hk, D, *rest):
    # od_qk_norm_rope_kv_append(_ex): q/k/v heads read, q/k heads written back, int8 K/V + scales written
    tok = B * S
    return (tok * (Hq + 2 * Hk) * D, tok * ((Hq + 2 * Hk) * D * 2 + (Hq + Hk) * D * 2 + 2 * Hk * (D + 4)))


# HBM-side traffic of the layer GEMMs per launch at M = 4096 (bytes), from two rocprofv3 --pmc passes (FETCH_SIZE,
# then WRITE_SIZE) over the four layer GEMMs (gate+up through od_w8a8_gemm_swiglu), each counter scaled by its
# reading for a plain 256 MiB device copy (fetch x2.000, write x1.000); the summary is
# profiles/w8a8_gemm_traffic_M4096.md.
GEMM_TRAFFIC_M4096 = {(6144, 4096): 218.5e6, (4096, 4096): 168.0e6, ("swiglu", 24576, 4096): 705.5e6,
                      (4096, 12288): 369.3e6}


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo, what lscpu prints as 'Model name')."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_timed(fn, repeats: int):
    """One warm-up call, then `repeats` timed calls (time.perf_counter); returns (median seconds, all times)."""
    fn()
    ts = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2], ts


def cpu_fields(torch, repeats: int) -> dict:
    """The host description every CPU baseline carries."""
    return {"cores": torch.get_num_threads(), "host_cpus": os.cpu_count(), "cpu_model": cpu_model(),
            "repeats": repeats, "statistic": f"median of {repeats} after one warm-up"}


def cpu_baseline(args):
    """The oracle (CPU torch restatement of the path) on a bounded sample: ONE request (32 options x 16 tokens, its
    2048-token int8 state) through ONE 9B-dims layer, timed and scaled x36 layers. A decision is one request, so
    the CPU's decisions/s is 1 / (36 x the layer time) whatever the batch (8 requests take 8 times as long)."""
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

    per_layer, _ = cpu_timed(run, args.cpu_sample_repeats)
    decision_s = per_layer * args.layers  # one request's scoring pass
    return {"value": 1.0 / decision_s, "unit": "decisions/s", **cpu_fields(torch, args.cpu_sample_repeats),
            "kind": "port",
            "sample": (f"1 request (32 options x 16 tokens, {T}-token int8 state) x 1 of {args.layers} layers, "
                       f"median of {args.cpu_sample_repeats} after a warm-up, {per_layer * 1e3:.0f} ms per layer, "
                       f"scaled x{args.layers} layers")}


def cpu_baseline_decision(args):
    """The oracle on a bounded sample of the decision forward: ONE request (a 4096-token state of random ids
    prefilled, then 64 options x 24 tokens scored) through ONE 9B-dims layer, the median of the timed runs after a
    warm-up, scaled x36 layers."""
    import torch

    from oracle import decoder as od
    torch.set_num_threads(os.cpu_count() or 1)
    cfg = od.DecoderConfig(n_layers=1)
    w = od.make_weights(cfg, seed=1)
    emb = torch.randn(4096, cfg.hidden, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    g = torch.Generator().manual_seed(2)
    S, n_opt, t = 4096, 64, 24
    ids_s = torch.randint(0, 4096, (1, S), generator=g)
    ids_o = torch.randint(0, 4096, (1, n_opt, t), generator=g)
    def run():
        _, kv = od.prefill_forward(ids_s, w, emb, cfg)
        od.decision_forward(ids_o, w, emb, cfg, kv, S)

    n = args.cpu_sample_repeats
    per_layer, _ = cpu_timed(run, n)
    per_request = per_layer * args.layers
    return {"value": 1.0 / per_request, "unit": "decisions/s", **cpu_fields(torch, n), "kind": "port",
            "sample": (f"1 request ({S}-token state prefilled + {n_opt} options x {t} tokens) x 1 of {args.layers} "
                       f"layers, median of {n} after a warm-up, {per_layer:.2f} s per layer, scaled x{args.layers} "
                       "layers")}


def cpu_baseline_wide(args):
    """The oracle on a bounded sample of the wide-choice workload: ONE 256-token record appended to a 32768-token
    int8 state through ONE 9B-dims layer (attention over the cached state + itself, only the new K/V quantized),
    the median of the timed runs after a warm-up, scaled x36 layers: the full-record append cost."""
    import torch

    from oracle import decoder as od
    from oracle import quant as oq
    torch.set_num_threads(os.cpu_count() or 1)
    cfg = od.DecoderConfig(n_layers=1)
    w = od.make_weights(cfg, seed=1)
    emb = torch.randn(4096, cfg.hidden, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    g = torch.Generator().manual_seed(4)
    S0, rec = 32768, 256
    kv = torch.randn(2, 1, cfg.n_kv_heads, S0, cfg.head_dim, generator=g).to(torch.bfloat16)
    kq, ks = oq.quantize_rows(kv[0])
    vq, vs = oq.quantize_rows(kv[1])
    state = [((kq, ks[..., 0]), (vq, vs[..., 0]))]
    ids = torch.randint(0, 4096, (1, rec), generator=g)
    n = args.cpu_sample_repeats
    per_layer, _ = cpu_timed(lambda: od.prefill_forward(ids, w, emb, cfg, state_kv=state, n0=S0), n)
    return {"value": per_layer * args.layers * 1e3, "unit": "ms per appended record (full prefill)",
            **cpu_fields(torch, n), "kind": "port",
            "sample": (f"1 record of {rec} tokens onto a {S0}-token int8 state x 1 of {args.layers} layers, median "
                       f"of {n} after a warm-up, {per_layer:.2f} s per layer, scaled x{args.layers} layers")}


# Qwen3.5's full-attention layer geometry (transformers' Qwen3_5TextConfig): 16 / 4 heads of 256, rotary on the
# first 64 dims (partial_rotary_factor 0.25), zero-centred RMSNorms, the output gate
QWEN35_ATTENTION = dict(n_heads=16, n_kv_heads=4, head_dim=256, rot_dim=64, norm_offset=True, gated=True)


def cpu_baseline_hybrid(args):
    """The oracle on a bounded sample of the hybrid decision: ONE request (a 4096-token state of random ids prefilled,
    then 64 options x 24 tokens scored) through ONE Gated DeltaNet layer (the gated delta rule in fp32, the
    reference's own CPU arithmetic) and ONE gated full-attention layer, each the median of the timed runs after a
    warm-up, scaled to the 24 + 8 layers of the stack."""
    import torch

    from oracle import decoder as od
    torch.set_num_threads(os.cpu_count() or 1)
    emb = torch.randn(4096, 4096, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
    g = torch.Generator().manual_seed(2)
    S, n_opt, t = 4096, 64, 24
    ids_s = torch.randint(0, 4096, (1, S), generator=g)
    ids_o = torch.randint(0, 4096, (1, n_opt, t), generator=g)
    per = {}
    n = args.cpu_sample_repeats
    for kind, cfg in (("gdn", od.DecoderConfig(n_layers=1, full_attention_interval=4, **QWEN35_ATTENTION)),
                      ("attention", od.DecoderConfig(n_layers=1, **QWEN35_ATTENTION))):
        w = od.make_weights(cfg, seed=1)

        def run():
            _, st = od.prefill_forward(ids_s, w, emb, cfg, gdn_dtype=torch.float32)
            od.decision_forward(ids_o, w, emb, cfg, st, S, gdn_dtype=torch.float32)

        per[kind], _ = cpu_timed(run, n)
    per_request = 24 * per["gdn"] + 8 * per["attention"]
    return {"value": 1.0 / per_request, "unit": "decisions/s", **cpu_fields(torch, n), "kind": "port",
            "sample": (f"1 request ({S}-token state prefilled + {n_opt} options x {t} tokens) through 1 Gated DeltaNet "
                       f"layer ({per['gdn']:.2f} s) and 1 gated attention layer ({per['attention']:.2f} s), median of "
                       f"{n} after a warm-up each, scaled to 24 + 8 layers")}


def cpu_baseline_qcache(args, n_q: int = 2, k: int = 16):
    """The oracle on a bounded sample of the question-cache decide (scripts/bench_qcache_rows.py's measurement):
    one decide of n_q questions x k options over one 900-token int8 state, with the cache (question pass, then the
    option rows over [state ; question]), through ONE 9B-dims layer, the median of the timed runs after a warm-up,
    scaled x36 layers."""
    import torch

    from oracle import decoder as od
    from oracle import quant as oq
    torch.set_num_threads(os.cpu_count() or 1)
    cfg = od.DecoderConfig(n_layers=1, vocab=4096)
    w = od.make_weights(cfg, seed=1)
    emb = od.make_embedding(cfg, seed=3)
    g = torch.Generator().manual_seed(7)
    S, t = 900, 6
    Lq = min(256 - t, 24 + 4 * k)
    kv = torch.randn(2, 1, cfg.n_kv_heads, S, cfg.head_dim, generator=g).to(torch.bfloat16)
    kq, ks = oq.quantize_rows(kv[0])
    vq, vs = oq.quantize_rows(kv[1])
    state = [((kq, ks[..., 0]), (vq, vs[..., 0]))]
    ids_q = torch.randint(0, cfg.vocab, (n_q, Lq), generator=g)
    ids_o = torch.randint(0, cfg.vocab, (n_q, k, t), generator=g)
    gs = [0] * n_q

    def run():
        q_kv = od.question_forward(ids_q, w, emb, cfg, state, S, gs)
        od.qcache_decision_forward(ids_o, w, emb, cfg, state, S, q_kv, [Lq] * n_q, gs)

    n = args.cpu_sample_repeats
    per_layer, _ = cpu_timed(run, n)
    return {"value": per_layer * args.layers * 1e3, "unit": f"ms per decide ({n_q} questions x {k} options)",
            **cpu_fields(torch, n), "kind": "port",
            "sample": (f"1 decide with the question cache ({n_q} questions of {Lq} tokens, {k} options x {t} tokens "
                       f"each, {S}-token int8 state) x 1 of {args.layers} layers, median of {n} after a warm-up, "
                       f"{per_layer * 1e3:.0f} ms per layer, scaled x{args.layers} layers")}


def _gemm_roofline(gemm_t):
    n_g, ms_g, (ops_g, _) = gemm_t.summary()
    tops = ops_g / (ms_g * 1e-3) / 1e12 if n_g else 0.0
    return {"kernel": "od_w8a8_gemm + od_w8a8_gemm_swiglu", "bound": "mfma", "achieved": tops, "peak": INT8_PEAK_TOPS,
            "unit": "TFLOP/s",
            "frac": tops / INT8_PEAK_TOPS, "traffic": None, "launches": n_g,
            "avg_launch_us": ms_g / max(n_g, 1) * 1e3}, ms_g


def run_decision(args):
    """Full decision forward from token ids: 4 requests, each a 4096-token state prefilled through the 36 layers
    (causal wide_attention, K/V quantized into int8 caches) and 64 options x 24 tokens scored against it."""
    import torch

    from opendecider_amd import decoder as dmod
    from opendecider_amd import kernels
    dev = "cuda:0"
    cfg = dmod.DecoderConfig(n_layers=args.layers)
    B, S, n_opt, t = 4, 4096, 64, 24
    dec = dmod.random_decoder(cfg, seed=0, device=dev, max_pos=S + t + 16)
    g = torch.Generator(device=dev).manual_seed(3)
    ids_state = torch.randint(0, cfg.vocab, (B, S), generator=g, device=dev)
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=g, device=dev)
    caches = dec.new_state_caches(B, S)
    gemm_t = GemmTimers()
    wide_t = AbiTimer("od_wide_attn", wide_work)
    attn_t = AttnTimers()

    def decide():
        caches.set_length(0)
        dec.prefill(ids_state, caches)
        return dec.score(ids, caches)

    for _ in range(args.warmup):
        out = decide()
    torch.cuda.synchronize()
    gemm_t.active = wide_t.active = attn_t.active = True
    lat = []
    for _ in range(args.steps):
        t0 = time.perf_counter()
        out = decide()
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - t0)
    gemm_t.active = wide_t.active = attn_t.active = False
    assert torch.isfinite(out).all(), "non-finite log-probabilities"
    lat_sorted = sorted(lat)
    p50 = lat_sorted[len(lat) // 2]
    roof, ms_g = _gemm_roofline(gemm_t)
    n_w, ms_w, (fl_w, _) = wide_t.summary()
    n_a, ms_a, (fl_a, by_a) = attn_t.summary()
    tot_ms = sum(lat) * 1e3
    return {
        "metric": "decisions/sec (4 requests, 4096-token states prefilled from ids, 64 options x 24 tokens, 9B dims)",
        "value": B / p50, "unit": "decisions/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": sum(lat) / len(lat) * 1e3, "p50_latency_ms": p50 * 1e3,
        "p90_latency_ms": lat_sorted[min(len(lat) - 1, int(0.9 * len(lat)))] * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": (f"full decision forward: {B} requests, {S}-token states of random ids prefilled "
                                f"through {cfg.n_layers} layers, {n_opt} options x {t} tokens scored, 'none' "
                                "appended; 9B dims, random init"),
                   "requests": B, "state_tokens": S, "options": n_opt, "tokens_per_option": t,
                   "layers": cfg.n_layers},
        "roofline": roof,
        "state_attention": {"kernel": "od_wide_attn (causal)", "tflops": fl_w / (ms_w * 1e-3) / 1e12 if n_w else 0,
                            "frac_of_bf16_mfma": fl_w / (ms_w * 1e-3) / 1e12 / BF16_PEAK_TFLOPS if n_w else 0,
                            "launches": n_w, "avg_launch_us": ms_w / max(n_w, 1) * 1e3},
        "row_attention": {"kernel": ATTN_KERNELS, "tflops": fl_a / (ms_a * 1e-3) / 1e12 if n_a else 0,
                          "algorithmic_gbs": by_a / (ms_a * 1e-3) / 1e9 if n_a else 0, "launches": n_a},
        "time_share": {"gemm": ms_g / tot_ms, "state_attention": ms_w / tot_ms, "row_attention": ms_a / tot_ms},
    }


def gdn_prep_work(proj, ldp, conv_w, conv_in, seq_state, n_states, seq_len, A_log, dt_bias, S, L, n_k, n_v, dk, dv,
                  *rest):
    # od_gdn_prep_ex: the projection's qkv / b / a columns read once, q k v written bf16, g and beta fp32, the 3-row
    # conv windows read per sequence (when continuing) and written (when asked); the taps' 4 rows hit the cache
    M, C = S * L, 2 * n_k * dk + n_v * dv
    conv_out = rest[4]
    by = M * (C + 2 * n_v) * 2 + M * C * 2 + M * n_v * 8 + (S * 3 * C * 2 if conv_in else 0) + \
        (S * 3 * C * 2 if conv_out else 0)
    return (M * C * 9, by)


def gdn_rec_work(qk, v, g, beta, init, seq_state, n_states, S, L, n_k, n_v, dk, dv, o, final_state, *rest):
    # od_gdn_recurrence(_chunked), counted as the token-by-token recurrence: per token and value head, decay (dk dv),
    # kv = S^T k (2 dk dv), the rank-1 update (2 dk dv), o = S^T q (2 dk dv) (the chunked form does more arithmetic,
    # on the matrix cores); bytes: the token inputs and o once, the fp32 state read once per sequence that starts
    # from one and written once per sequence that keeps one
    M = S * L
    st = n_v * dk * dv * 4
    by = M * (2 * n_k * dk * 2 + n_v * dv * 2 + n_v * 8 + n_v * dv * 2) + (S * st if init else 0) + \
        (S * st if final_state else 0)
    return (7 * M * n_v * dk * dv, by)


def gdn_norm_work(o, ldo, z, ldz, w, inv_s, eps, M, n_v, dv, *rest):
    V = n_v * dv
    return (M * V * 8, M * V * (2 + 2 + 1) + M * 4)


def _rate(t, flops_key=None):
    n, ms, (fl, by) = t.summary()
    out = {"launches": n, "avg_launch_us": ms / max(n, 1) * 1e3, "ms_total": ms}
    if n:
        out["algorithmic_gbs"] = by / (ms * 1e-3) / 1e9
        out["frac_of_hbm"] = out["algorithmic_gbs"] / HBM_PEAK_GBS
        if flops_key:
            out[flops_key] = fl / (ms * 1e-3) / 1e12
    return out


def run_hybrid(args):
    """The full decision forward on the Qwen3.5 hybrid stack: 32 layers (hidden 4096, FFN 12288), every 4th a
    full-attention layer in Qwen3.5's geometry (16 / 4 heads of 256, rotary on the first 64 dims, zero-centred
    RMSNorms, output gate), the others Gated DeltaNet layers (16 key / 32 value heads of 128, conv 4); 4 requests,
    each a 4096-token state of random ids prefilled (GDN layers: conv windows and recurrent states; attention layers:
    int8 K/V), then 64 options x 24 tokens scored against it, the rows reading their request's GDN states in
    place."""
    import torch

    from opendecider_amd import decoder as dmod
    dev = "cuda:0"
    cfg = dmod.DecoderConfig(n_layers=32, full_attention_interval=4, vocab=248320, **QWEN35_ATTENTION)
    B, S, n_opt, t = 4, 4096, 64, 24
    dec = dmod.random_decoder(cfg, seed=0, device=dev, max_pos=S + t + 16)
    g = torch.Generator(device=dev).manual_seed(3)
    ids_state = torch.randint(0, cfg.vocab, (B, S), generator=g, device=dev)
    ids = torch.randint(0, cfg.vocab, (B, n_opt, t), generator=g, device=dev)
    st = dec.new_state_caches(B, S)
    gemm_t = GemmTimers()
    wide_t = AbiTimer("od_wide_attn", wide_work)
    attn_t = AttnTimers()
    prep_t = AbiTimer("od_gdn_prep_ex", gdn_prep_work)
    rec_t = AbiTimer("od_gdn_recurrence_chunked", gdn_rec_work)
    norm_t = AbiTimer("od_gdn_norm_quant", gdn_norm_work)
    timers = (gemm_t, wide_t, attn_t, prep_t, rec_t, norm_t)

    def reset():
        st.kv.set_length(0)
        for it in st:
            if isinstance(it, dmod.GDNState):
                it.length = 0

    def decide():
        reset()
        dec.prefill(ids_state, st)
        return dec.score(ids, st)

    for _ in range(args.warmup):
        out = decide()
    torch.cuda.synchronize()
    # the scoring pass alone, over the prefilled states
    for tm in timers:
        tm.active = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = dec.score(ids, st)
    torch.cuda.synchronize()
    score_ms = (time.perf_counter() - t0) / args.steps * 1e3
    for tm in timers:
        tm.active = False
    score_rates = {"gemm": _gemm_roofline(gemm_t)[0], "row_attention": _rate(attn_t),
                   "gdn_prep": _rate(prep_t), "gdn_recurrence": _rate(rec_t, "recurrent_equivalent_tflops"),
                   "gdn_norm_quant": _rate(norm_t)}
    for tm in timers:
        tm.reset()
    # the whole decision: prefill + scoring
    for tm in timers:
        tm.active = True
    lat = []
    for _ in range(args.steps):
        t0 = time.perf_counter()
        out = decide()
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - t0)
    for tm in timers:
        tm.active = False
    assert torch.isfinite(out).all(), "non-finite log-probabilities"
    lat_sorted = sorted(lat)
    p50 = lat_sorted[len(lat) // 2]
    roof, ms_g = _gemm_roofline(gemm_t)
    tot_ms = sum(lat) * 1e3
    parts = {"gemm": ms_g, "state_attention": wide_t.summary()[1], "row_attention": attn_t.summary()[1],
             "gdn_prep": prep_t.summary()[1], "gdn_recurrence": rec_t.summary()[1],
             "gdn_norm_quant": norm_t.summary()[1]}
    return {
        "metric": "decisions/sec (Qwen3.5 hybrid stack: 4096-token states prefilled from ids, 64 options x 24 "
                  "tokens)",
        "value": B / p50, "unit": "decisions/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": sum(lat) / len(lat) * 1e3, "p50_latency_ms": p50 * 1e3,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": (f"full decision forward, hybrid stack: {B} requests, {S}-token states of random ids "
                                f"prefilled through {cfg.n_layers} layers ({sum(cfg.is_gdn(i) for i in range(32))} "
                                "Gated DeltaNet + 8 full attention), 64 options x 24 tokens scored, 'none' appended; "
                                "hidden 4096, FFN 12288, attention 16 / 4 heads of 256 with rotary on 64 dims and "
                                "zero-centred norms, random init"),
                   "requests": B, "state_tokens": S, "options": n_opt, "tokens_per_option": t,
                   "layers": cfg.n_layers, "full_attention_interval": 4, "attention_heads": "16/4 x 256",
                   "rotary_dims": cfg.rotary_dims},
        "roofline": roof,
        "gdn_prep": _rate(prep_t), "gdn_recurrence": _rate(rec_t, "recurrent_equivalent_tflops"),
        "gdn_norm_quant": _rate(norm_t),
        "state_attention": {"kernel": "od_wide_attn (causal)", **_rate(wide_t)},
        "time_share": {k: v / tot_ms for k, v in parts.items()},
        "scoring_pass": {"ms": score_ms, **score_rates},
    }


def run_wide_choice(args):
    """A 32768-token shared state cached as int8 K/V (36 layers; synthetic bf16 N(0,1) K/V quantized by the append
    kernel), grown by 8 records of 256 tokens (each prefilled through the decoder on top of the cache, only the new
    K/V quantized and appended); after each record 2 requests x 255 options x 12 tokens are scored against it."""
    import torch

    from opendecider_amd import decoder as dmod
    from opendecider_amd import kernels
    dev = "cuda:0"
    cfg = dmod.DecoderConfig(n_layers=args.layers)
    S0, n_rec, rec, n_req, n_opt, t = 32768, 8, 256, 2, 255, 12
    cap = S0 + n_rec * rec
    dec = dmod.random_decoder(cfg, seed=0, device=dev, max_pos=cap + t + 16)
    g = torch.Generator(device=dev).manual_seed(4)
    caches = dec.new_state_caches(1, cap)
    for kc, vc in caches:
        for c in (kc, vc):
            for j in range(0, S0, 8192):  # synthetic state K/V, quantized by the append kernel in pieces
                c.append(torch.randn(1, cfg.n_kv_heads, 8192, cfg.head_dim, generator=g, device=dev)
                         .to(torch.bfloat16))
    records = [torch.randint(0, cfg.vocab, (1, rec), generator=g, device=dev) for _ in range(n_rec + args.warmup)]
    ids = torch.randint(0, cfg.vocab, (1, n_req * n_opt, t), generator=g, device=dev)
    app_t = AbiTimer("od_qk_norm_rope_kv_append_ex", rope_append_work)
    attn_t = AttnTimers()
    # warm-up: one record + one scoring pass, then rewind the caches
    for i in range(args.warmup):
        dec.prefill(records[n_rec + i], caches)
        dec.score(ids, caches)
        caches.set_length(S0)
    torch.cuda.synchronize()
    rec_ms, score_ms = [], []
    app_ms = []
    for r in range(n_rec):
        app_t.active = True
        t0 = time.perf_counter()
        dec.prefill(records[r], caches)
        torch.cuda.synchronize()
        rec_ms.append((time.perf_counter() - t0) * 1e3)
        app_t.active = False
        n_ap, ms_ap, _ = app_t.summary()
        app_ms.append(ms_ap)
        app_t.reset()
        attn_t.active = True
        t0 = time.perf_counter()
        out = dec.score(ids, caches)
        torch.cuda.synchronize()
        score_ms.append((time.perf_counter() - t0) * 1e3)
        attn_t.active = False
    assert torch.isfinite(out).all(), "non-finite log-probabilities"
    n_a, ms_a, (fl_a, by_a) = attn_t.summary()
    gbs = by_a / (ms_a * 1e-3) / 1e9
    tflops = fl_a / (ms_a * 1e-3) / 1e12
    # 2 x 255 x 12 x 4 = 24,480 query slots per KV head read each state key: ~1,500 FLOP per K/V byte, so the row
    # attention is bf16-MFMA-bound and its rate is quoted in TFLOP/s (the HBM figure stays beside it)
    return {
        "metric": "row-attention TFLOP/s and append cost per record (32k int8 state + 8 x 256-token "
                  "records, 2 x 255 options x 12 tokens)",
        "value": tflops, "unit": "TFLOP/s", "n_gpus": 1, "steps": n_rec, "warmup": args.warmup,
        "ms_per_step": sum(rec_ms) / n_rec + sum(score_ms) / n_rec, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": (f"{S0}-token shared int8 state (36 layers) + {n_rec} records x {rec} tokens, "
                                f"{n_req} requests x {n_opt} options x {t} tokens after each record; 9B dims"),
                   "state_tokens": S0, "records": n_rec, "record_tokens": rec, "requests": n_req,
                   "options": n_opt, "tokens_per_option": t, "layers": cfg.n_layers},
        "attention": {"kernel": ATTN_KERNELS, "bound": "mfma", "tflops": tflops,
                      "frac_of_bf16_mfma": tflops / BF16_PEAK_TFLOPS, "algorithmic_gbs": gbs,
                      "frac_of_hbm": gbs / HBM_PEAK_GBS, "launches": n_a, "avg_launch_us": ms_a / max(n_a, 1) * 1e3},
        "append_per_record": {"full_prefill_ms": sum(rec_ms) / n_rec,
                              "kernel_only_us": sum(app_ms) / n_rec * 1e3,
                              "kernel": ("od_qk_norm_rope_kv_append (q/k norm + RoPE and the K/V quantize-append "
                                         "in one pass, 36 layers)")},
        "scoring_ms": sum(score_ms) / n_rec,
    }


def run_gemm(args):
    """The W8A8 linear alone: od_act_quant + od_w8a8_gemm on the reference's sweep (scripts/bench_gemm.py:22-23:
    (K, N) in {(2048, 6144), (6144, 2048), (2048, 2048)} x M in {64, 512, 2048, 8192}) and on the 9B layer shapes at
    M = 4096 (QKV 4096 -> 6144, O 4096 -> 4096, gate+up 4096 -> 24576 also with SwiGLU in the epilogue, down
    12288 -> 4096), and the single 256 x 4096 x 4096 linear. Inputs as the layer shapes: X bf16 N(0, 1) with 1% outlier channels x20, W N(0, 0.02) with SmoothQuant
    factors U(0.5, 2) folded in, per-channel int8; 1/s fused into the activation quantizer. HIP events over 20 calls
    of each kernel after 3 warm-up calls; the vendor int8 GEMM (torch._int_mm, hipBLASLt, int32 output, no
    epilogue) beside it. Each timing is a replay of a HIP graph of the 20 calls (GPU time, no host launch gaps): warm
    caches, the weights of the smaller shapes staying in the Infinity Cache between calls. gemm_us_cold: the median
    of 5 single calls, each after a 512 MB buffer has been read and written (no operand in L2 or the Infinity
    Cache; the 36-layer passes see the weights this way, 36 layers of them being far larger than the cache).
    CPU baselines on the single linear (M = 256, 4096 x 4096): the reference's CPU linear path
    (Int8Linear.forward: dequantize + F.linear in bf16, quant.py:156-157) and the W8A8 oracle."""
    import torch

    from opendecider_amd import kernels
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(6)
    reps = 20

    def timed(fn):
        # the reps calls captured in one HIP graph and replayed: GPU time only (at small M the host's launch
        # overhead would otherwise be what is measured)
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(reps):
                fn()
        graph.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps * 1e3  # us

    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)  # twice the 256 MB Infinity Cache

    def timed_cold(fn, n=5):
        # one call after 512 MB have been read and written (L2 and Infinity Cache hold none of its operands); median
        # of n such calls
        ts = []
        for _ in range(n):
            flush.add_(1)
            c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            c0.record()
            fn()
            c1.record()
            torch.cuda.synchronize()
            ts.append(c0.elapsed_time(c1) * 1e3)
        return sorted(ts)[n // 2]

    def operands(M, K, N):
        x = torch.randn(M, K, device=dev, generator=g)
        idx = torch.randperm(K, device=dev, generator=g)[: (K + 99) // 100]
        x[:, idx] *= 20
        x = x.to(torch.bfloat16)
        s = torch.rand(K, device=dev, generator=g) * 1.5 + 0.5
        wt = (torch.randn(N, K, device=dev, generator=g) * 0.02 * s[None, :]).to(torch.bfloat16)
        wq, sw = kernels.act_quant(wt)
        inv = (1.0 / s).to(torch.bfloat16)
        return x, inv, wq, sw

    rows = []
    shapes = [("bench_gemm", K, N, M) for K, N in ((2048, 6144), (6144, 2048), (2048, 2048))
              for M in (64, 512, 2048, 8192)]
    shapes += [("config0", 4096, 4096, 256)]
    shapes += [("9b_qkv", 4096, 6144, 4096), ("9b_o", 4096, 4096, 4096), ("9b_gate_up", 4096, 24576, 4096),
               ("9b_down", 12288, 4096, 4096)]
    for name, K, N, M in shapes:
        x, inv, wq, sw = operands(M, K, N)
        xq, sx = kernels.act_quant(x, inv)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        us_q = timed(lambda: kernels.act_quant(x, inv, xq=xq, sx=sx))
        us_g = timed(lambda: kernels.w8a8_gemm(xq, sx, wq, sw, out=out))
        us_v = timed(lambda: torch._int_mm(xq, wq.t()))
        us_c = timed_cold(lambda: kernels.w8a8_gemm(xq, sx, wq, sw, out=out))
        ops = 2 * M * N * K
        row = {"shape": name, "M": M, "K": K, "N": N, "act_quant_us": us_q, "gemm_us": us_g,
               "gemm_tops": ops / us_g / 1e6, "frac": ops / us_g / 1e6 / INT8_PEAK_TOPS,
               "gemm_us_cold": us_c, "gemm_tops_cold": ops / us_c / 1e6,
               "linear_tops": ops / (us_q + us_g) / 1e6, "vendor_int_mm_us": us_v}
        if name == "9b_gate_up":
            hm = torch.empty(M, N // 2, dtype=torch.bfloat16, device=dev)
            wi = kernels.interleave_gate_up(wq)
            si = kernels.interleave_gate_up(sw)
            us_s = timed(lambda: kernels.w8a8_gemm_swiglu(xq, sx, wi, si, out=hm))
            row["swiglu_gemm_us"] = us_s
            row["swiglu_gemm_tops"] = ops / us_s / 1e6
        rows.append(row)
        del x, xq, wq, out
    nine = [r for r in rows if r["shape"].startswith("9b_")]
    ops9 = sum(2 * r["M"] * r["N"] * r["K"] for r in nine)
    us9 = sum(r.get("swiglu_gemm_us", r["gemm_us"]) for r in nine)
    res = {"metric": "int8 GEMM TOPS (W8A8 linear, per shape)", "value": ops9 / us9 / 1e6, "unit": "TOPS",
           "n_gpus": 1, "steps": reps, "warmup": 3, "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8", "data": "synthetic",
           "config": {"workload": "W8A8 linear sweep: scripts/bench_gemm.py shapes and the 9B layer GEMMs at M = 4096"},
           "roofline": {"kernel": "od_w8a8_gemm (gate+up: od_w8a8_gemm_swiglu)", "bound": "mfma",
                        "achieved": ops9 / us9 / 1e6, "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                        "frac": ops9 / us9 / 1e6 / INT8_PEAK_TOPS, "traffic": None,
                        "note": "the four 9B layer GEMMs at M = 4096 together"},
           "shapes": rows}
    us9c = sum(r["gemm_us_cold"] for r in nine)
    res["cold"] = {"tops": ops9 / us9c / 1e6, "frac": ops9 / us9c / 1e6 / INT8_PEAK_TOPS,
                   "note": "the four 9B layer GEMMs at M = 4096 (gate+up without the SwiGLU epilogue), each timed "
                           "alone after a 512 MB cache flush"}
    ceil = mfma_ceiling(modes=(1, 2))
    res["roofline"]["sustained"] = _sustained(ceil, 2)
    res["roofline"]["frac_of_sustained"] = res["roofline"]["achieved"] / ceil["mode2"]["value"]
    if not args.no_cpu_baseline:
        import torch as _t
        from oracle import quant as oq
        _t.set_num_threads(os.cpu_count() or 1)
        cg = _t.Generator().manual_seed(0)
        M, K, N = 256, 4096, 4096
        x = _t.randn(M, K, generator=cg).to(_t.bfloat16)
        wq = _t.randint(-127, 128, (N, K), generator=cg, dtype=_t.int8)
        sw = _t.rand(N, generator=cg) * 1.5e-3 + 0.5e-3
        ops = 2 * M * N * K
        n = args.cpu_sample_repeats
        ref, _ = cpu_timed(lambda: oq.int8_linear_dequant(x, wq, sw), n)
        port, _ = cpu_timed(lambda: oq.w8a8_linear(x, wq, sw), n)
        res["cpu_baseline"] = {"value": ops / ref / 1e12, "unit": "TOPS", **cpu_fields(_t, n), "kind": "port",
                               "reference_linear_ms": ref * 1e3, "w8a8_port_ms": port * 1e3,
                               "w8a8_port_tops": ops / port / 1e12,
                               "sample": (f"the single linear (M={M}, K={K}, N={N}), median of {n} after a warm-up: the "
                                          f"reference's CPU linear path (Int8Linear.forward: dequantize + F.linear, "
                                          f"quant.py:156-157) {ref * 1e3:.1f} ms; the W8A8 oracle (act-quant, int32 "
                                          f"GEMM, epilogue) {port * 1e3:.1f} ms")}
    return res


def run_mfma_ceiling(args):
    """What the matrix cores sustain on this chip: od_probe_mfma's five modes (int8 on constant / changing /
    LDS-fed operands, bf16 on changing / LDS-fed operands), one 8-wave workgroup per CU, 100000 rounds of 8 MFMAs
    per wave, with the core clock under that load. `value` is the int8 LDS-fed rate, the ceiling the W8A8 GEMM's
    inner loop has without any global traffic."""
    ceil = mfma_ceiling()
    ceil["hbm_read"] = hbm_ceiling()
    return {"metric": "int8 MFMA sustained TOPS (LDS-fed operands)", "value": ceil["mode2"]["value"], "unit": "TOPS",
            "n_gpus": 1, "steps": 1, "warmup": 1, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "int8", "data": "synthetic",
            "config": {"workload": "matrix-core ceiling probe: one 8-wave workgroup per CU, 100000 rounds of 8 "
                                   "independent 32x32 MFMAs per wave"},
            "roofline": {"bound": "mfma", "achieved": ceil["mode2"]["value"], "peak": INT8_PEAK_TOPS,
                         "unit": "TFLOP/s", "frac": ceil["mode2"]["frac_of_peak"], "traffic": None},
            "modes": ceil}


def run_qcache_rows(args):
    """Where the question cache pays off (scripts/bench_qcache_rows.py): the latency of one decision with and
    without it, over the reference's (questions, options) shapes, on a 36-layer 9B-dims decoder with one cached
    900-token int8 state (synthetic K/V). A question is its prompt plus the listing of its options: 24 + 4 k tokens
    for k options (capped at 256); an option is 6 tokens. With the cache: one question pass (each question's tokens
    over the state; every layer's question K/V kept as second-level block images) and then the option rows over
    [state ; question]. Without: every option row carries its question's tokens followed by its own, over the state
    alone, pooled over the option tokens. Median of 3 after a warm-up, each call synchronized."""
    import torch

    from opendecider_amd import decoder as dmod
    dev = "cuda:0"
    cfg = dmod.DecoderConfig(n_layers=args.layers)
    S, t = 900, 6
    shapes = [(1, 4), (3, 4), (2, 16), (4, 16), (2, 32), (8, 16), (4, 32), (16, 8), (8, 32), (16, 16), (16, 32)]
    dec = dmod.random_decoder(cfg, seed=0, device=dev, max_pos=S + 256 + t + 16)
    g = torch.Generator(device=dev).manual_seed(7)
    states = dec.new_state_caches(1, S)
    for kc, vc in states:
        for c in (kc, vc):
            c.append(torch.randn(1, cfg.n_kv_heads, S, cfg.head_dim, generator=g, device=dev).to(torch.bfloat16))

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            ts.append(time.perf_counter() - t0)
        return sorted(ts)[1] * 1e3

    rows = []
    for n, k in shapes:
        Lq = min(256 - t, 24 + 4 * k)
        ids_q = torch.randint(0, cfg.vocab, (n, Lq), generator=g, device=dev)
        ids_o = torch.randint(0, cfg.vocab, (n, k, t), generator=g, device=dev)
        gs = [0] * n

        def with_cache():
            qc = dec.question_pass(ids_q, [Lq] * n, states, gs)
            return dec.score_qcache(ids_o, qc, states)

        rows_ids = torch.cat([ids_q[:, None, :].expand(n, k, Lq), ids_o], 2).reshape(1, n * k, Lq + t)

        def without_cache():
            return dec.score(rows_ids, states, pool_last=t)

        w_ms, wo_ms = timed(with_cache), timed(without_cache)
        rows.append({"questions": n, "options": k, "rows": n * k, "question_tokens": Lq, "option_tokens": t,
                     "with_qcache_ms": w_ms, "without_qcache_ms": wo_ms, "speedup": wo_ms / w_ms})
        dec._ws.clear()
        torch.cuda.empty_cache()
    last = rows[-1]
    return {"metric": "decide latency with / without the question cache (speedup at 16 questions x 32 options)",
            "value": last["speedup"], "unit": "x", "n_gpus": 1, "steps": 3, "warmup": 1, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
            "config": {"workload": (f"one {S}-token int8 state, {cfg.n_layers}-layer 9B-dims decoder; questions of "
                                    f"24 + 4 k tokens, options of {t} tokens; scripts/bench_qcache_rows.py shapes"),
                       "state_tokens": S, "layers": cfg.n_layers},
            "shapes": rows}


def run_gemm_traffic(args):
    """The run profiled with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE for roofline.traffic: a 256 MiB device copy
    (known bytes, to calibrate the counters), then two scoring passes through 2 layers (M = 4096: QKV, O, gate+up,
    down each twice)."""
    import torch

    from opendecider_amd import decoder as dmod
    from opendecider_amd.kv_cache import Int8KVCache
    dev = "cuda:0"
    x = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    cfg = dmod.DecoderConfig(n_layers=2)
    dec = dmod.random_decoder(cfg, seed=0, device=dev, max_pos=2048 + 32)
    g = torch.Generator(device=dev).manual_seed(1)
    states = []
    for _ in range(cfg.n_layers):
        pair = []
        for _ in range(2):
            c = Int8KVCache(8, cfg.n_kv_heads, cfg.head_dim, 2048, dev)
            c.append(torch.randn(8, cfg.n_kv_heads, 2048, cfg.head_dim, generator=g, device=dev).to(torch.bfloat16))
            pair.append(c)
        states.append(tuple(pair))
    ids = torch.randint(0, cfg.vocab, (8, 32, 16), generator=g, device=dev)
    for _ in range(2):
        dec.score(ids, states)
    torch.cuda.synchronize()
    return {"workload": "gemm_traffic", "copy_bytes": 256 << 20, "layers": 2, "passes": 2, "tokens_per_layer": 4096}


ATTN_SHAPES = (("config1", 8, 32, 2048, 16), ("kv_probe", 8, 2, 32768, 16), ("kv_stream", 8, 2, 32768, 2))


def run_attention(args, only=None):
    """The branched attention alone on the shapes its rooflines are quoted on: the 8-state option-row shape (8 states of
    2048 int8 K/V tokens, 32 options x 16 tokens each, 32/8 heads, head_dim 128: bf16-MFMA-bound), the ridge probe
    (the same dims with 32768-token states and 2 options x 16 tokens each: about 250 FLOP per K/V byte, at the
    MFMA/HBM ridge) and the KV-bound few-slot probe (32768-token states, 2 options x 2 tokens each: 16 query slots
    per KV head, about 31 FLOP per K/V byte, od_branched_attn_stream). K/V int8 uniform in [-127, 127] with fp32
    scales, queries and own K/V bf16 N(0, 1); HIP events around every call. only: a subset of the shape names."""
    import torch

    from opendecider_amd import kernels
    dev = "cuda:0"
    g = torch.Generator(device=dev).manual_seed(5)
    Hq, Hkv, t, D = 32, 8, 16, 128
    res = {}
    for name, Ns, rows, T, t in ATTN_SHAPES:
        if only is not None and name not in only:
            continue
        R = Ns * rows
        q = torch.randn(R, Hq, t, D, device=dev, generator=g).to(torch.bfloat16)
        k = torch.randn(R, Hkv, t, D, device=dev, generator=g).to(torch.bfloat16)
        v = torch.randn(R, Hkv, t, D, device=dev, generator=g).to(torch.bfloat16)
        kq = torch.randint(-127, 128, (Ns, Hkv, T, D), device=dev, dtype=torch.int8, generator=g)
        vq = torch.randint(-127, 128, (Ns, Hkv, T, D), device=dev, dtype=torch.int8, generator=g)
        ks = torch.rand(Ns, Hkv, T, device=dev, generator=g) * 0.02
        vs = torch.rand(Ns, Hkv, T, device=dev, generator=g) * 0.02
        rs, mr = kernels.row_start_of([rows] * Ns, dev)
        out = torch.empty_like(q)
        timers = AttnTimers()

        def call():
            kernels.branched_attn(q, k, v, kq, ks, vq, vs, D ** -0.5, out=out, row_start=rs, max_rows=mr, length=T)

        for _ in range(args.warmup):
            call()
        torch.cuda.synchronize()
        timers.active = True
        for _ in range(args.steps):
            call()
        torch.cuda.synchronize()
        timers.active = False
        n, ms, (fl, by) = timers.summary()
        kv_bytes = 2 * Ns * Hkv * T * (D + 4)
        res[name] = {"states": Ns, "state_tokens": T, "options_per_state": rows, "tokens_per_option": t,
                     "avg_launch_us": ms / n * 1e3, "tflops": fl / (ms * 1e-3) / 1e12,
                     "frac_of_bf16_mfma": fl / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                     "kv_gbs": kv_bytes / (ms / n * 1e-3) / 1e9,
                     "kv_frac_of_hbm": kv_bytes / (ms / n * 1e-3) / 1e9 / HBM_PEAK_GBS,
                     "algorithmic_gbs": by / (ms * 1e-3) / 1e9, "launches": n,
                     "path": ("stream" if rows * t * (Hq // Hkv) <= kernels.STREAM_MAX_SLOTS else
                              "staged" if kernels.uses_staging(rows, t, Hq, Hkv) else "direct")}
    if only is not None:
        return {"shapes": res}
    out = {"metric": "branched attention: KV GB/s on the KV-bound few-slot probe (TFLOP/s on the 8-state option-row shape "
                     "and the ridge probe beside it)",
           "value": res["kv_stream"]["kv_gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": res["kv_stream"]["avg_launch_us"] / 1e3, "higher_is_better": True,
           "scaling": "weak", "vs_baseline": None, "dtype": "int8 K/V, bf16 MFMA", "data": "synthetic",
           "config": {"workload": "branched attention alone: 8-state option-row shape, ridge probe, KV-bound few-slot probe"},
           "shapes": res}
    if not args.no_cpu_baseline:
        # the reference's CPU branch of _split_attention (prefix_attn.py:58-76) on K/V materialized in bf16, as the
        # oracle restates it, for 1 of the 8 states (32 options x 16 tokens over 2048 keys), scaled x8
        from oracle import attention as oa
        torch.set_num_threads(os.cpu_count() or 1)
        cg = torch.Generator().manual_seed(5)
        T, rows = 2048, 32
        q = torch.randn(rows, Hq, t, D, generator=cg).to(torch.bfloat16)
        k = torch.randn(rows, Hkv, t, D, generator=cg).to(torch.bfloat16)
        v = torch.randn(rows, Hkv, t, D, generator=cg).to(torch.bfloat16)
        kq = torch.randint(-127, 128, (1, Hkv, T, D), generator=cg, dtype=torch.int8)
        vq = torch.randint(-127, 128, (1, Hkv, T, D), generator=cg, dtype=torch.int8)
        ks, vs = torch.rand(1, Hkv, T, generator=cg) * 0.02, torch.rand(1, Hkv, T, generator=cg) * 0.02
        n = args.cpu_sample_repeats
        per_state, _ = cpu_timed(lambda: oa.branched_attention_int8(q, k, v, kq, ks, vq, vs, D ** -0.5), n)
        out["cpu_baseline"] = {"value": 1e3 * per_state * 8, "unit": "ms per 8-state option-row call", **cpu_fields(torch, n),
                               "kind": "port",
                               "sample": (f"1 of the 8 states (32 options x 16 tokens over 2048 int8 keys, K/V "
                                          f"materialized in bf16), median of {n} after a warm-up: "
                                          f"{per_state * 1e3:.0f} ms, scaled x8"),
                               "gpu_speedup": per_state * 8 / (res["config1"]["avg_launch_us"] * 1e-6)}
    return out


def run_lm_logprob(args):
    """The LM head's token log-prob (the option-token LM feature, backbone.py:164-178) over a Qwen-size int8
    vocabulary table: 151936 rows x 4096 (Int8Table of random N(0, 0.03) rows, bf16 scales), 1024 rows of bf16 h
    N(0, 2) (16 options x 64 tokens) with random target tokens. One call = od_lm_head_logprob (the bf16-MFMA logit
    tiles with the table dequantized on the fly and the log-sum-exp in their epilogue, then the per-row combine);
    HIP events around the timed calls. The same rows against the table re-quantized as Q4_0 are reported beside
    (od_lm_head_logprob_q4). CPU baseline: the oracle on 2 rows over the whole vocabulary."""
    import torch

    from opendecider_amd import Int8Table, token_logprob
    dev = "cuda:0"
    V, K, M = 151936, 4096, 1024
    g = torch.Generator(device=dev).manual_seed(7)
    w = (torch.randn(V, K, device=dev, generator=g) * 0.03).to(torch.bfloat16)
    table = Int8Table(w)
    del w
    h = (torch.randn(M, K, device=dev, generator=g) * 2.0).to(torch.bfloat16)
    tok = torch.randint(0, V, (M,), device=dev, generator=g)
    out = None
    for _ in range(args.warmup):
        out = token_logprob(table, h, tok)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(args.steps):
        out = token_logprob(table, h, tok)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / args.steps
    assert torch.isfinite(out).all()
    flops = 2.0 * M * V * K
    tflops = flops / (ms * 1e-3) / 1e12
    table_bytes = V * K + V * 2
    res = {"metric": "LM-head token log-probs/s over an int8 151936 x 4096 table (bf16 MFMA TFLOP/s beside it)",
           "value": M / (ms * 1e-3), "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "int8 table, bf16 MFMA", "data": "synthetic",
           "config": {"workload": f"token_logprob: {M} rows of h (bf16, hidden {K}) against a {V}-row int8 LM-head "
                                  "table, one target token per row"},
           "roofline": {"kernel": "od_lm_head_logprob (lm_logits_kernel + lm_combine_kernel)", "bound": "mfma",
                        "achieved": tflops, "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                        "frac": tflops / BF16_PEAK_TFLOPS, "traffic": None,
                        "algorithmic_bytes": table_bytes + M * K * 2 + M * 8,
                        "note": "2 x rows x vocabulary x hidden FLOP per call over the call's duration (HIP events)",
                        "avg_launch_us": ms * 1e3}}
    # the same rows against the same table held as Q4_0 (4.5 bits per value)
    from opendecider_amd import Q4Table
    t4 = Q4Table(table.weight)
    for _ in range(args.warmup):
        token_logprob(t4, h, tok)
    torch.cuda.synchronize()
    s.record()
    for _ in range(args.steps):
        out4 = token_logprob(t4, h, tok)
    e.record()
    torch.cuda.synchronize()
    ms4 = s.elapsed_time(e) / args.steps
    assert torch.isfinite(out4).all()
    res["q4_table"] = {"ms_per_call": ms4, "rows_per_s": M / (ms4 * 1e-3), "tflops": flops / (ms4 * 1e-3) / 1e12,
                       "frac_of_bf16_mfma": flops / (ms4 * 1e-3) / 1e12 / BF16_PEAK_TFLOPS}
    del t4
    if not args.no_cpu_baseline:
        from oracle import lm_head as ol
        torch.set_num_threads(os.cpu_count() or 1)
        q, sc = table.qweight.cpu(), table.scale.cpu().reshape(-1)
        hs, ts = h[:2].cpu(), tok[:2].cpu()
        rows = lambda idx, dt: ol.int8_rows(q, sc, idx, dt)
        ol.token_logprob(hs[:1], rows, V, ts[:1])
        t0 = time.perf_counter()
        ol.token_logprob(hs, rows, V, ts)
        dt = time.perf_counter() - t0
        res["cpu_baseline"] = {"value": 2 / dt, "unit": "rows/s", "cores": torch.get_num_threads(), "kind": "port",
                               "sample": f"the oracle (float64 logits of the bf16 operands, chunked logaddexp) on 2 "
                                         f"rows over the whole {V}-row table, {dt:.1f} s, after a 1-row warm-up"}
    return res


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if args.workload != "scoring":
        torch.cuda.set_device(0)
        fn = {"decision": run_decision, "wide_choice": run_wide_choice, "gemm": run_gemm,
              "gemm_traffic": run_gemm_traffic, "attention": run_attention,
              "lm_logprob": run_lm_logprob, "qcache_rows": run_qcache_rows,
              "mfma_ceiling": run_mfma_ceiling, "hybrid": run_hybrid}[args.workload]
        print(json.dumps(fn(args)))
        return

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

    # every 5th call of each GEMM entry point (5 is prime to the 3 od_w8a8_gemm calls of a layer, so the timed
    # calls cycle through the shapes evenly) and every 3rd layer's attention carry timing events
    gemm_t = GemmTimers(every=5)
    attn_t = AttnTimers(every=3)

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
    known = [GEMM_TRAFFIC_M4096.get(sh) for sh in gemm_t.shapes]
    traffic = sum(known) / len(known) if known and None not in known and args.tokens * args.options * args.requests == 4096 else None
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
        "roofline": {"kernel": "od_w8a8_gemm + od_w8a8_gemm_swiglu (all 4 layer GEMMs)", "bound": "mfma",
                     "achieved": gemm_tops, "peak": INT8_PEAK_TOPS, "unit": "TFLOP/s",
                     "frac": gemm_tops / INT8_PEAK_TOPS, "traffic": traffic,
                     "traffic_unit": "bytes per launch (calibrated FETCH_SIZE + WRITE_SIZE)",
                     "algorithmic_bytes": bytes_g / max(n_g, 1),
                     "note": "int8 ops (TOPS) per launch over launch duration (HIP events, timed region)",
                     "launches": n_g, "timed_every": gemm_t.every, "avg_launch_us": ms_g / max(n_g, 1) * 1e3},
        "attention": {"kernel": ATTN_KERNELS, "tflops": attn_tflops, "frac_of_bf16_mfma": attn_tflops /
                      BF16_PEAK_TFLOPS, "algorithmic_gbs": attn_gbs, "frac_of_hbm": attn_gbs / HBM_PEAK_GBS,
                      "launches": n_a, "timed_every": attn_t.timers[0].every,
                      "avg_launch_us": ms_a / max(n_a, 1) * 1e3},
        "time_share": {"gemm": ms_g * gemm_t.every / (ms_per_step * args.steps),
                       "attention": ms_a * attn_t.timers[0].every / (ms_per_step * args.steps)},
    }
    ceil = mfma_ceiling(modes=(2, 4))
    res["roofline"]["sustained"] = _sustained(ceil, 2)
    res["roofline"]["frac_of_sustained"] = gemm_tops / ceil["mode2"]["value"]
    res["attention"]["sustained_bf16"] = _sustained(ceil, 4)
    res["attention"]["frac_of_sustained_bf16"] = attn_tflops / ceil["mode4"]["value"]
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(args)
    if not args.scoring_only:
        del states, dec
        torch.cuda.empty_cache()
        # the int8-KV option-row attention where it is HBM-bound: the few-slot probe (od_branched_attn_stream)
        # it runs after the CPU baseline has left the GPU idle: 300 untimed calls (~35 ms) bring the clocks back up
        kvb = run_attention(_sub_args(args, steps=20, warmup=300), only=("kv_stream",))["shapes"]["kv_stream"]
        res["attention_kv_bound"] = {
            "kernel": "od_branched_attn_stream (split merge fused in the kernel)", "bound": "hbm", "achieved": kvb["kv_gbs"],
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": kvb["kv_frac_of_hbm"],
            "avg_launch_us": kvb["avg_launch_us"], "launches": kvb["launches"],
            "config": {"workload": "8 states x 32768 int8 K/V tokens (fp32 per-token scales), 2 options x 2 tokens "
                                   "per state, 32/8 heads, head_dim 128", "slots_per_kv_head": 16},
            "note": "K/V bytes (int8 + fp32 scales) per call over the call's duration (HIP events)"}
        hbm = hbm_ceiling()
        res["attention_kv_bound"]["sustained"] = hbm
        res["attention_kv_bound"]["frac_of_sustained"] = kvb["kv_gbs"] / hbm["value"]
        # the KV-bound probe near the HBM / bf16 ridge: the same states with 2 options x 16 tokens per state (128
        # query slots per KV head, ~250 FLOP per K/V byte: at the bf16-MFMA / HBM ridge, so both fractions apply)
        kvp = run_attention(_sub_args(args, steps=20, warmup=50), only=("kv_probe",))["shapes"]["kv_probe"]
        res["attention_kv_probe"] = {
            "kernel": f"branched attention, {kvp['path']} path", "bound": "hbm and bf16 mfma (ridge)",
            "achieved": kvp["kv_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": kvp["kv_frac_of_hbm"],
            "tflops": kvp["tflops"], "frac_of_bf16_mfma": kvp["frac_of_bf16_mfma"],
            "avg_launch_us": kvp["avg_launch_us"], "launches": kvp["launches"],
            "config": {"workload": "8 states x 32768 int8 K/V tokens (fp32 per-token scales), 2 options x 16 tokens "
                                   "per state, 32/8 heads, head_dim 128", "slots_per_kv_head": 128,
                       "definition": "the KV-bound ridge probe (S=32768, 2 rows x 16 tokens, 128 slots per KV head)"},
            "frac_of_sustained_hbm": kvp["kv_gbs"] / hbm["value"],
            "note": "K/V bytes (int8 + fp32 scales) per call over the call's duration (HIP events)"}
        torch.cuda.empty_cache()
        # the single 256 x 4096 x 4096 W8A8 linear and the reference's scripts/bench_gemm.py sweep, with the vendor int8
        # GEMM (torch._int_mm, hipBLASLt) beside each shape and the single linear's CPU baselines
        gm = run_gemm(args)
        c0 = next(r for r in gm["shapes"] if r["shape"] == "config0")
        res["config0_linear"] = {
            "config": {"workload": "single W8A8 linear: X bf16 [256, 4096] (1% outlier channels x20), W int8 "
                                   "[4096, 4096] per-channel, per-token dynamic activation quantizer"},
            "act_quant_us": c0["act_quant_us"], "gemm_us": c0["gemm_us"], "linear_us": c0["act_quant_us"] + c0["gemm_us"],
            "gemm_tops": c0["gemm_tops"], "frac": c0["frac"], "linear_tops": c0["linear_tops"],
            "gemm_us_cold": c0["gemm_us_cold"], "vendor_int_mm_us": c0["vendor_int_mm_us"],
            "note": "HIP-graph replays of 20 calls (warm caches); gemm_us_cold: after a 512 MB cache flush"}
        if "cpu_baseline" in gm:
            res["config0_linear"]["cpu_baseline"] = gm["cpu_baseline"]
        keep = ("shape", "M", "K", "N", "gemm_us", "gemm_tops", "frac", "gemm_us_cold", "vendor_int_mm_us",
                "swiglu_gemm_us", "swiglu_gemm_tops")
        res["gemm_sweep"] = {
            "kernel": "od_w8a8_gemm (gate+up also od_w8a8_gemm_swiglu)",
            "config": {"workload": "scripts/bench_gemm.py (K, N) x M sweep and the 9B layer GEMMs at M = 4096"},
            "nine_b_tops": gm["value"], "nine_b_frac": gm["roofline"]["frac"], "cold": gm["cold"],
            "sustained": gm["roofline"]["sustained"],
            "shapes": [{k: r[k] for k in keep if k in r} | {"vendor_tops": 2 * r["M"] * r["N"] * r["K"] /
                                                           r["vendor_int_mm_us"] / 1e6} for r in gm["shapes"]]}
        del gm
        torch.cuda.empty_cache()
        res["decision"] = _sub(run_decision(_sub_args(args, steps=10, warmup=2)),
                               ("value", "unit", "p50_latency_ms", "p90_latency_ms", "config", "roofline",
                                "state_attention", "row_attention", "time_share"))
        if not args.no_cpu_baseline:
            res["decision"]["cpu_baseline"] = cpu_baseline_decision(args)
        torch.cuda.empty_cache()
        res["wide_choice"] = _sub(run_wide_choice(_sub_args(args, warmup=1)),
                                  ("value", "unit", "config", "attention", "append_per_record", "scoring_ms"))
        if not args.no_cpu_baseline:
            res["wide_choice"]["cpu_baseline"] = cpu_baseline_wide(args)
        torch.cuda.empty_cache()
        res["hybrid"] = _sub(run_hybrid(_sub_args(args, steps=5, warmup=2)),
                             ("value", "unit", "p50_latency_ms", "config", "roofline", "gdn_prep", "gdn_recurrence",
                              "gdn_norm_quant", "time_share", "scoring_pass"))
        if not args.no_cpu_baseline:
            res["hybrid"]["cpu_baseline"] = cpu_baseline_hybrid(args)
        torch.cuda.empty_cache()
        qc = run_qcache_rows(args)
        res["qcache_rows"] = {"value": qc["value"], "unit": qc["unit"], "metric": qc["metric"], "config": qc["config"],
                              "shapes": qc["shapes"]}
        if not args.no_cpu_baseline:
            cb = cpu_baseline_qcache(args)
            gpu_ms = next(r["with_qcache_ms"] for r in qc["shapes"] if (r["questions"], r["options"]) == (2, 16))
            res["qcache_rows"]["cpu_baseline"] = cb | {"gpu_with_qcache_ms": gpu_ms,
                                                       "gpu_speedup": cb["value"] / gpu_ms}
    print(json.dumps(res))


def _sub_args(args, **kw):
    a = argparse.Namespace(**vars(args))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def _sub(d, keys):
    return {k: d[k] for k in keys if k in d}


if __name__ == "__main__":
    main()
