#!/usr/bin/env python3
"""Benchmark: MXFP4 routed-expert MoE decode layer on one MI355X.

Workload: DeepSeek-V3/V4 geometry, hidden 7168, 256
routed experts + 1 shared expert, each gate+up [2*2048, 7168] and down
[7168, 2048] in MXFP4 (weights N(0, 0.02) quantized with the ceil e8m0 recipe
and RNE E2M1, then MXT16-prepacked), tokens bf16 N(0, 1), router logits
N(0, 1), sigmoid scores, top-8, weights renormalized to 1, SwiGLU.  A step is
one full layer (routing, stable expert sort, gate/up+SwiGLU, down, combine) on
one batch of M tokens (default M=1; at M=1..4 the layer is two launches:
routing fused into gate/up+SwiGLU, then down fused with the combine).  Inputs are
resident in HBM before the timed region.  Three independent 6 GB layer banks
rotate step by step and the routing changes every step, so a bank's bytes
(its shared expert included) are read again only after two other layers
(about 420 MB, more than the 256 MB MALL): weights come from HBM.

The timed region replays a HIP graph of the K steps (one replay = exactly K
layers), three times between synchronizations, and reports the median replay;
the same K steps run eagerly through the Python wrapper are reported beside it.  ``value`` is the algorithmic HBM throughput of the layer (every
distinct expert's bytes read once + x + y) in GB/s; ``roofline`` reports the
gate/up kernel (the dominant one) against 8 TB/s, timed with HIP events that
the kernel's own dispatch records; ``cpu_baseline`` times the reference's own
CPU kernel (the integer-exact A8 ``vnni_source_gemm`` built from the
reference's source) on single-token layers of the same weights, beside a
torch-CPU fp32 dequant-then-matmul of the A16 layer.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

H, I, E, K = 7168, 2048, 256, 8
GU_BYTES = 2 * I * (H // 2 + H // 32)   # gate+up codes and scales of one expert
DN_BYTES = H * (I // 2 + I // 32)       # down codes and scales of one expert
EXPERT_BYTES = GU_BYTES + DN_BYTES      # 23,396,352
HBM_PEAK_GBS = 8000.0
# HBM bytes per launch of moe_dec1_gateup_kernel (the M = 1 roofline kernel),
# from two rocprofv3 --pmc passes over this script (FETCH_SIZE, then
# WRITE_SIZE, KiB per dispatch, averaged over the timed dispatches), each
# scaled by what the same counter reads for --calibration-copy-mib 256:
# FETCH_SIZE x 2.0, WRITE_SIZE x 1.0.  The profile summary
# profiles/moe_decode_m1_traffic.md holds the commands and raw figures.
GATEUP_M1_TRAFFIC_BYTES = (68771.5 * 2.0 + 36.1) * 1024
N_BANKS = 3  # independent layers rotated step by step (reuse distance > the 256 MB MALL)
METRIC = "MXFP4 MoE-layer decode µs & HBM GB/s % peak; FP8/MXFP4 GEMM TFLOPS % peak"


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--m", type=int, default=1, help="tokens per decode step")
    ap.add_argument("--sweep", default="4,16,64", help="extra M values reported under m_sweep ('' to skip)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-configs", action="store_true", help="skip BASELINE.json configs 1, 3, 4, 5")
    ap.add_argument("--configs", default="",
                    help="comma-separated subset of config1_linear_m1, config3_fp8_gemm, config3_mxfp4_gemm, "
                         "config4_moe_prefill, config5_dsa to run (default: all); config3_vendor_fp8 and "
                         "config3_vendor_mx (the vendor library's per-tensor FP8 and MX block-scaled GEMMs at "
                         "the config-3 shapes, calibrations) and config3_w8a16 (fp8_linear's W8A16 path at the "
                         "config-3 weight shapes) run only when named")
    ap.add_argument("--no-headline", action="store_true",
                    help="skip the decode layer (one bank is still built for config 4); for profiling the configs")
    ap.add_argument("--no-graph", action="store_true",
                    help="time the K steps eagerly instead of replaying a HIP graph (for counter-collecting "
                         "profiler passes; the headline line is graph-timed)")
    ap.add_argument("--launch-table", default="",
                    help="write the per-launch table behind roofline (the event-timed durations of the M-token "
                         "gate/up and down dispatches and each launch's algorithmic bytes) to this Markdown file")
    ap.add_argument("--calibration-copy-mib", type=int, default=0,
                    help="after the line is printed, copy a buffer of this many MiB device to device three times "
                         "(a plain copy of known size that scales FETCH_SIZE / WRITE_SIZE counter passes)")
    return ap.parse_args()


def build_banks(torch, ops, n_banks: int, seed: int = 0):
    """n_banks independent layers: (gate_up MXT16 [E,2I,H/2], down MXT16 [E,H,I/2], shared pair)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    banks = []
    for _ in range(n_banks):
        gp = torch.empty(E + 1, 2 * I, H // 2, dtype=torch.uint8, device=dev)
        gs = torch.empty(E + 1, 2 * I, H // 32, dtype=torch.uint8, device=dev)
        dp = torch.empty(E + 1, H, I // 2, dtype=torch.uint8, device=dev)
        ds = torch.empty(E + 1, H, I // 32, dtype=torch.uint8, device=dev)
        for e in range(E + 1):
            w = (torch.randn(2 * I, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            p, s = ops.mx_quantize(w, "ceil")
            gp[e].copy_(p)
            gs[e].copy_(s)
            w = (torch.randn(H, I, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            p, s = ops.mx_quantize(w, "ceil")
            dp[e].copy_(p)
            ds[e].copy_(s)
        gu = ops.mxt16_prepack(gp[:E], gs[:E])
        dn = ops.mxt16_prepack(dp[:E], ds[:E])
        sgu = ops.mxt16_prepack(gp[E], gs[E])
        sdn = ops.mxt16_prepack(dp[E], ds[E])
        raw = (gp, gs, dp, ds)
        banks.append({"gu": gu, "dn": dn, "shared": (sgu, sdn), "raw": raw})
        # progress (a counter-collecting profiler makes each set-up launch slow)
        print(f"bench.py: weight bank {len(banks)}/{n_banks} built", file=sys.stderr, flush=True)
    torch.cuda.synchronize()
    return banks


def run_m(torch, ops, banks, m: int, steps: int, warmup: int, seed: int, graph: bool = True):
    """K layer steps at M tokens: eager warmup, the K steps eagerly (reported
    beside the headline), then the K steps captured in one HIP graph and timed
    by three replays (the median is the headline), then an instrumented eager
    pass with HIP events at the stage boundaries."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1000 + seed)
    pool = 16
    xs = [torch.randn(m, H, generator=g, device=dev).to(torch.bfloat16) for _ in range(pool)]
    ls = [torch.randn(m, E, generator=g, device=dev) for _ in range(pool)]
    ws = ops.MoEWorkspace()

    def step(i, se=None):
        b = banks[i % len(banks)]
        return ops.moe_a16_forward(xs[i % pool], b["gu"], b["dn"], logits=ls[i % pool], top_k=K, shared=b["shared"],
                                   workspace=ws, stage_events=se)

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    print(f"bench.py: M={m} warmup done", file=sys.stderr, flush=True)
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for i in range(steps):
        step(warmup + i)
    ev1.record()
    torch.cuda.synchronize()
    eager_ms = ev0.elapsed_time(ev1)
    ids_all = []
    if graph:
        # the same K steps in one graph: one replay = exactly K layers
        g_k = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g_k):
            for i in range(steps):
                ids_all.append(step(warmup + i)[1])
        g_k.replay()  # untimed: first replay
        torch.cuda.synchronize()
        # three timed replays, each exactly the K steps between synchronizations;
        # the median is reported (one replay moved by +-3 us per layer run to run)
        samples = []
        for _ in range(3):
            t0 = time.perf_counter()
            ev0.record()
            g_k.replay()
            ev1.record()
            torch.cuda.synchronize()
            samples.append((ev0.elapsed_time(ev1), time.perf_counter() - t0))
        samples.sort()
        gpu_ms, wall = samples[1]
        del g_k
    else:
        # counter passes: the eager K steps are the timed ones
        ids_all = [step(warmup + i)[1] for i in range(steps)]
        torch.cuda.synchronize()
        gpu_ms, wall = eager_ms, eager_ms / 1e3
    print(f"bench.py: M={m} timed steps done", file=sys.stderr, flush=True)
    # instrumented pass over the same steps: HIP events at the stage boundaries,
    # on the kernels' stream (at M = 1 the gate/up and down dispatches record
    # them, so they bracket those kernels' execution); the headline above is
    # timed without them
    stage = [ops.StageEvents() for _ in range(steps)]
    torch.cuda.synchronize()
    for i in range(steps):
        step(warmup + i, stage[i])
    torch.cuda.synchronize()
    times = [s.times() for s in stage]
    distinct = [len(set(ids.flatten().tolist())) for ids in ids_all]
    layer_bytes = [(u + 1) * EXPERT_BYTES + 2 * m * H * 2 + m * E * 4 for u in distinct]
    gu_bytes = [(u + 1) * GU_BYTES + m * H * 2 + (u + 1) * I * 2 for u in distinct]
    dn_bytes = [(u + 1) * DN_BYTES + (u + 1) * I * 2 + m * H * 2 for u in distinct]
    gu_s = sum(t["gu_sec"] for t in times)
    return {
        "m": m,
        "us_per_layer": gpu_ms * 1e3 / steps,
        "eager_us_per_layer": eager_ms * 1e3 / steps,
        "wall_ms": wall * 1e3,
        "gbs": sum(layer_bytes) / (gpu_ms / 1e3) / 1e9,
        "distinct_experts_avg": sum(distinct) / len(distinct),
        "layer_bytes_avg": sum(layer_bytes) / steps,
        "stage_us": {k: 1e6 * sum(t[k] for t in times) / steps for k in ops.MOE_STAGES},
        "gateup_us": 1e6 * gu_s / steps,
        "gateup_gbs": sum(gu_bytes) / gu_s / 1e9,
        "gateup_bytes_per_launch": sum(gu_bytes) / steps,
        "per_launch": [{"gu_us": 1e6 * t["gu_sec"], "down_us": 1e6 * t["down_sec"], "gu_bytes": gb, "down_bytes": db,
                        "distinct": u} for t, gb, db, u in zip(times, gu_bytes, dn_bytes, distinct)],
    }


def _graph_time(torch, fn, calls: int, reps: int = 5) -> float:
    """Average microseconds per fn() call, replaying a HIP graph of `calls` calls
    (launch overhead of the Python wrapper excluded)."""
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (reps * calls)


def config1_linear(torch, ops):
    """one MXFP4 linear [2048, 7168] at M=1 (A16, MXT16 weights);
    ~70 weight copies (> the 256 MB MALL) rotate through the graph."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    n, k = 2048, 7168
    w = (torch.randn(n, k, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    p, sc = ops.mx_quantize(w, "ceil")
    copies = [ops.mxt16_prepack(p.clone(), sc.clone()) for _ in range(70)]
    x = torch.randn(1, k, generator=g, device=dev).to(torch.bfloat16)
    it = iter(range(10 ** 9))
    cold = _graph_time(torch, lambda: ops.mxt16_linear_a16(x, copies[next(it) % len(copies)]), len(copies))
    warm = _graph_time(torch, lambda: ops.mxt16_linear_a16(x, copies[0]), 70)
    byts = n * (k // 2 + k // 32) + k * 2 + n * 2
    return {"shape": [1, n, k], "us": round(cold, 3), "GBs": round(byts / cold / 1e3, 1),
            "hbm_frac": round(byts / cold / 1e3 / HBM_PEAK_GBS, 4), "warm_mall_us": round(warm, 3),
            "bytes": byts}


def config3_fp8(torch, ops):
    """FP8 block-scaled GEMMs, 5 shapes x M in {1, 16, 128, 4096}
    (and M = 64, not in the config: the mid-size kernel's range).  Copies of the
    weight (over 512 MB in all, twice the 256 MB MALL) rotate through the graph,
    so every call reads its weight from HBM.  At M <= 64 the drop-ins
    (fp8_gemm, w8a8_block_fp8_matmul) read the weight's cached T16 prepack, so
    ``us`` times that (each copy prepacked once, outside the timed graph) and
    ``us_checkpoint_layout`` the same call over the [N, K] codes."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    out = {}
    for n, k in [(1536, 7168), (24576, 1536), (576, 7168), (7168, 16384), (18432, 7168)]:
        w = torch.randn(n, k, generator=g, device=dev) * 0.02
        wb = w.view((n + 127) // 128, 128, k // 128, 128) if n % 128 == 0 else None
        if wb is None:
            wp = torch.zeros((n + 127) // 128 * 128, k, device=dev)
            wp[:n] = w
            wb = wp.view(-1, 128, k // 128, 128)
        bs = (wb.abs().amax(dim=(1, 3)) / 448.0).clamp_min(1e-12)
        bq0 = (wb / bs[:, None, :, None]).reshape(-1, k)[:n].to(torch.float8_e4m3fn)
        nrot = (512 << 20) // (n * k) + 1
        bqs = [bq0] + [bq0.clone() for _ in range(nrot - 1)]
        tqs = [ops.fp8_t16_prepack(b) for b in bqs]
        for m in (1, 16, 64, 128, 4096):
            x = torch.randn(m, k, generator=g, device=dev)
            aq, a_s = ops.act_quant(x, 128, "amax")

            def timed(ws):
                it = iter(range(10 ** 9))
                return _graph_time(torch, lambda: ops.fp8_block_gemm(aq, a_s, ws[next(it) % nrot], bs), nrot,
                                   reps=3 if m < 4096 else 1)

            us = timed(tqs if m <= ops.FP8_T16_MAX_M else bqs)
            fl = 2 * m * n * k
            byts = m * k + 4 * m * (k // 128) + n * k + 4 * bs.numel() + 2 * m * n
            out[f"m{m}_n{n}_k{k}"] = {"us": round(us, 2), "TFLOPs": round(fl / us / 1e6, 1),
                                      "mfma_frac": round(fl / us / 1e6 / 5000.0, 4),
                                      "hbm_frac": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)}
            if m <= ops.FP8_T16_MAX_M:
                out[f"m{m}_n{n}_k{k}"]["us_checkpoint_layout"] = round(timed(bqs), 2)
        del bqs, bq0, tqs
    return out


def config3_vendor_fp8(torch, ops):
    """Calibration, not a path of this build: AMD's hipBLASLt FP8 GEMM (through
    torch._scaled_mm, one scale per tensor, so no per-128-block rescale; bf16 out)
    at the config-3 M = 4096 shapes, weights rotating past the MALL as in config 3.
    It shows what the vendor library reaches on this box for the simpler problem."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(16)
    one = torch.ones((), device=dev)
    out = {}
    for n, k in [(1536, 7168), (24576, 1536), (576, 7168), (7168, 16384), (18432, 7168)]:
        b0 = (torch.randn(n, k, generator=g, device=dev) * 8.0).clamp(-448, 448).to(torch.float8_e4m3fn)
        nrot = (512 << 20) // (n * k) + 1
        bs = [b0] + [b0.clone() for _ in range(nrot - 1)]
        a = (torch.randn(4096, k, generator=g, device=dev) * 8.0).clamp(-448, 448).to(torch.float8_e4m3fn)
        it = iter(range(10 ** 9))
        us = _graph_time(torch, lambda: torch._scaled_mm(a, bs[next(it) % nrot].t(), scale_a=one, scale_b=one,
                                                         out_dtype=torch.bfloat16), nrot, reps=1)
        fl = 2 * 4096 * n * k
        out[f"m4096_n{n}_k{k}"] = {"us": round(us, 2), "TFLOPs": round(fl / us / 1e6, 1),
                                   "mfma_frac": round(fl / us / 1e6 / 5000.0, 4)}
        del bs, b0
    return out


def config3_w8a16(torch, ops):
    """fp8_linear's W8A16 path (bench/fp8_core.py:160-231; not a BASELINE.json row): bf16
    activations against e4m3 weights with 128 x 128 fp32 block scales, the weight decoded
    inside the GEMM (ops.fp8_w8a16_linear, with its split-K workspace), at M = 1, 16, 64 and
    80 on the config-3 weight shapes, the weights rotating past the MALL as in config 3."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(17)
    out = {}
    for n, k in [(1536, 7168), (24576, 1536), (576, 7168), (7168, 16384), (18432, 7168)]:
        nrot = (512 << 20) // (n * k) + 1
        w0 = (torch.randn(n, k, generator=g, device=dev) * 0.02).clamp(-0.4, 0.4).to(torch.float8_e4m3fn)
        ws = [w0.view(torch.uint8)] + [w0.view(torch.uint8).clone() for _ in range(nrot - 1)]
        s = torch.rand((n + 127) // 128, k // 128, generator=g, device=dev) * 1e-3 + 1e-4
        for m in (1, 16, 64, 80):
            x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
            it = iter(range(10 ** 9))
            us = _graph_time(torch, lambda: ops.fp8_w8a16_linear(x, ws[next(it) % nrot], s), nrot, reps=3)
            byt = n * k + 4 * ((n + 127) // 128) * (k // 128) + 2 * m * k + 2 * m * n
            out[f"m{m}_n{n}_k{k}"] = {"us": round(us, 2), "GBs": round(byt / us / 1e3, 1),
                                      "hbm_frac": round(byt / us / 1e3 / 8000.0, 4)}
        del ws, w0
    return out


def config3_vendor_mx(torch, ops):
    """Calibration, not a path of this build: hipBLASLt's MX block-scaled GEMM (torch._scaled_mm
    with one e8m0 scale per 32 K on both operands, bf16 out) at the config-3 M = 4096 shapes,
    fp8 x fp8 (the scaled MFMA at the fp8 rate, as this build's fp8 x fp4 A8 GEMM runs) and
    fp4 x fp4 (twice that rate), weights rotating past the MALL as in config 3."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(17)
    out = {}
    for n, k in [(1536, 7168), (24576, 1536), (576, 7168), (7168, 16384), (18432, 7168)]:
        # unit scales; the library takes them in 128-row blocks (rows padded to a multiple of 128)
        sa = torch.full((4096, k // 32), 127, dtype=torch.uint8, device=dev).view(torch.float8_e8m0fnu)
        sb = torch.full(((n + 127) // 128 * 128, k // 32), 127, dtype=torch.uint8,
                        device=dev).view(torch.float8_e8m0fnu)
        fl = 2 * 4096 * n * k
        for fmt in ("fp8", "fp4"):
            if fmt == "fp8":
                a = (torch.randn(4096, k, generator=g, device=dev) * 8.0).clamp(-448, 448).to(torch.float8_e4m3fn)
                b0 = (torch.randn(n, k, generator=g, device=dev) * 8.0).clamp(-448, 448).to(torch.float8_e4m3fn)
                peak = 5000.0
            else:
                a = torch.randint(0, 256, (4096, k // 2), generator=g, device=dev,
                                  dtype=torch.uint8).view(torch.float4_e2m1fn_x2)
                b0 = torch.randint(0, 256, (n, k // 2), generator=g, device=dev,
                                   dtype=torch.uint8).view(torch.float4_e2m1fn_x2)
                peak = 10000.0
            nrot = (512 << 20) // (b0.numel() * b0.element_size()) + 1
            bs = [b0] + [b0.clone() for _ in range(nrot - 1)]
            it = iter(range(10 ** 9))
            us = _graph_time(torch, lambda: torch._scaled_mm(a, bs[next(it) % nrot].t(), scale_a=sa, scale_b=sb,
                                                             out_dtype=torch.bfloat16), nrot, reps=1)
            out[f"{fmt}_m4096_n{n}_k{k}"] = {"us": round(us, 2), "TFLOPs": round(fl / us / 1e6, 1),
                                             "mfma_frac": round(fl / us / 1e6 / peak, 4)}
            del bs, b0, a
    return out


def config3_mxfp4(torch, ops):
    """The config-3 shapes with MXFP4 weights (A8: 1x128 power-of-two e4m3
    activations, ceil-recipe MXFP4 weights N(0, 0.02)), the dense fp4_gemm of
    .mosaicvm/source/inference_kernel.py:441-536 at M in {128, 4096}; weight copies
    rotate past the MALL as in config 3.  Peaks: 5.0 PFLOP/s (the fp8 rate of the
    f8f6f4 MFMA) and 10.1 (the fp4 rate)."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(15)
    out = {}
    for n, k in [(1536, 7168), (24576, 1536), (576, 7168), (7168, 16384), (18432, 7168)]:
        w = (torch.randn(n, k, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        p, sc = ops.mx_quantize(w, "ceil")
        del w
        wbytes = n * (k // 2 + k // 32)
        nrot = (512 << 20) // wbytes + 1
        ws = [ops.mxt16_prepack(p.clone(), sc.clone()) for _ in range(nrot)]
        for m in (128, 4096):
            x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
            xq, sa = ops.act_quant(x, 128, "pow2")
            it = iter(range(10 ** 9))
            us = _graph_time(torch, lambda: ops.mxt16_linear_a8(None, ws[next(it) % nrot], prequant=(xq, sa)), nrot,
                             reps=3 if m < 4096 else 1)
            fl = 2 * m * n * k
            byts = m * k + 4 * m * (k // 128) + wbytes + 2 * m * n
            out[f"m{m}_n{n}_k{k}"] = {"us": round(us, 2), "TFLOPs": round(fl / us / 1e6, 1),
                                      "mfma_frac_fp8_rate": round(fl / us / 1e6 / 5000.0, 4),
                                      "mfma_frac_fp4_rate": round(fl / us / 1e6 / 10100.0, 4),
                                      "hbm_frac": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)}
        del ws, p, sc
    return out


def config4_prefill(torch, ops, bank, m: int = 4096, seed: int = 13):
    """MoE prefill at M=4096 with Zipf(1.1) expert popularity over a
    seeded permutation (8 experts pinned to zero), Gumbel-top-8, A8 contract."""
    import math
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    perm = torch.randperm(E, generator=g, device=dev)
    logp = torch.tensor([-1.1 * math.log(r + 1) for r in range(E)], device=dev)[torch.argsort(perm)]
    logp[perm[-8:]] = -1e4
    u = torch.rand(m, E, generator=g, device=dev).clamp(1e-9, 1 - 1e-9)
    logits = logp[None, :] - torch.log(-torch.log(u))
    x = torch.randn(m, H, generator=g, device=dev).to(torch.bfloat16)
    ws = ops.MoEWorkspace()
    fn = lambda: ops.moe_a8_forward(x, bank["gu"], bank["dn"], logits=logits, top_k=K, shared=bank["shared"],
                                    workspace=ws)
    _, ids, _ = fn()
    us = _graph_time(torch, fn, 3, reps=3)
    # per-stage times (eager, HIP events at the stage boundaries), 3 calls
    reps = [ops.StageEvents(ops.MOE_A8_STAGES) for _ in range(3)]
    torch.cuda.synchronize()
    for se in reps:
        ops.moe_a8_forward(x, bank["gu"], bank["dn"], logits=logits, top_k=K, shared=bank["shared"], workspace=ws,
                           stage_events=se)
    torch.cuda.synchronize()
    st = [se.times() for se in reps]
    stage_us = {k: round(1e6 * sum(t[k] for t in st) / len(st), 1) for k in ops.MOE_A8_STAGES}
    counts = torch.bincount(ids.flatten().long(), minlength=E)
    used = int((counts > 0).sum().item())
    fl = 2 * m * (K + 1) * 3 * H * I
    byts = (used + 1) * EXPERT_BYTES + m * H * 2 * 2
    return {"tokens": m, "us": round(us, 1), "tokens_per_s": round(m / us * 1e6, 1),
            "TFLOPs": round(fl / us / 1e6, 1), "mfma_frac": round(fl / us / 1e6 / 5000.0, 4),
            "hbm_GBs": round(byts / us / 1e3, 1), "hbm_frac": round(byts / us / 1e3 / HBM_PEAK_GBS, 4),
            "experts_used": used, "max_expert_rows": int(counts.max().item()), "contract": "A8 (fused_moe_mxint)",
            "stage_us": stage_us,
            "stage_note": "eager calls with stage events (the timed line replays a graph); sort/permute = "
                          "layout_sec, gate/up with the SwiGLU + z requant epilogue fused = gu_sec "
                          "(down_quant_sec ~ 0), scatter-combine = reduction_sec"}


def config5_dsa(torch, ops):
    """FP8 lightning indexer + top-2048 and MLA decode over the picks."""
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(14)
    out = {}
    ws = ops.MoEWorkspace()
    for b, l in [(1, 32768), (8, 131072)]:
        q8 = lambda *sh: (torch.randn(*sh, generator=g, device=dev) * 60).clamp(-448, 448).to(torch.float8_e4m3fn)
        nrot = max(1, (512 << 20) // (b * l * 132) + 1)
        ks = [q8(b, l, 128) for _ in range(nrot)]
        kss = [torch.rand(b, l, generator=g, device=dev) * 0.01 + 1e-3 for _ in range(nrot)]
        q, qs = q8(b, 64, 128), torch.rand(b, 64, generator=g, device=dev) * 0.01 + 1e-3
        w = torch.randn(b, 64, generator=g, device=dev) * 0.01
        it = iter(range(10 ** 9))

        def idx_fn():
            i = next(it) % nrot
            return ops.dsa_indexer_topk(q, qs, ks[i], kss[i], w, 2048, workspace=ws)
        us = _graph_time(torch, idx_fn, nrot, reps=3)
        byts = b * l * 132 + b * 64 * 136
        out[f"indexer_b{b}_l{l}"] = {"us": round(us, 1), "GBs": round(byts / us / 1e3, 1),
                                     "hbm_frac": round(byts / us / 1e3 / HBM_PEAK_GBS, 4)}
        del ks, kss
    ws = ops.MoEWorkspace()  # the MLA calls' own workspace (its placement does not follow the indexer's size)
    for b in (1, 8):
        n = 65536
        qh = torch.randn(b, 128, 576, generator=g, device=dev).to(torch.bfloat16)
        # KV caches rotate (over 512 MB in all), as each layer gathers from its own cache
        kv_bytes = b * n * (512 + 8 * 4 + 64 * 2)
        nrot = (512 << 20) // kv_bytes + 1
        kvs = []
        for _ in range(nrot):
            lat = (torch.randn(b, n, 512, generator=g, device=dev) * 60).clamp(-448, 448).to(torch.float8_e4m3fn)
            ls = torch.rand(b, n, 8, generator=g, device=dev) * 0.01
            rope = torch.randn(b, n, 64, generator=g, device=dev).to(torch.bfloat16)
            kvs.append((lat, ls, rope))
        idx = torch.stack([torch.randperm(n, generator=g, device=dev)[:2048] for _ in range(b)]).int()
        sink = torch.randn(128, generator=g, device=dev)
        it = iter(range(10 ** 9))

        def mla_fn():
            lat, ls, rope = kvs[next(it) % nrot]
            return ops.mla_sparse_decode(qh, lat, ls, rope, idx, 576 ** -0.5, sink, workspace=ws)
        us = _graph_time(torch, mla_fn, nrot * max(1, 10 // nrot), reps=3)
        fl = 2 * b * 128 * 2048 * (576 + 512)
        out[f"mla_b{b}"] = {"us": round(us, 1), "TFLOPs": round(fl / us / 1e6, 2)}
        del kvs
    return out


def _cpu_threads() -> int:
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    return min(n, int(env)) if env.isdigit() and int(env) > 0 else n


def _cpu_info() -> dict:
    model, phys, cores, siblings = "unknown", set(), 0, 0
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name":
                model = v
            elif k == "physical id":
                phys.add(v)
            elif k == "cpu cores":
                cores = int(v)
            elif k == "siblings":
                siblings = int(v)
    except OSError:
        pass
    return {"model": model, "sockets": max(1, len(phys)), "cores_per_socket": cores,
            "smt": (siblings // cores) if cores else None, "visible_cpus": os.cpu_count()}


def cpu_baseline(torch, ops, bank, tokens: int = 6, seed: int = 7, min_seconds: float = 10.0):
    """The reference's CPU path on the host cores, beside the GPU numbers.

    ``value``: the reference's own integer-exact A8 CPU kernel (``vnni_source_gemm``,
    ``bench/vnni_source_kernel.c:8-47``, built from the reference's source into
    ``oracle/_ref``) running the A8 MoE layer of ``fused_moe_mxint`` on ``tokens``
    single-token decode steps (8 routed + the shared expert each; weights tiled
    outside the timed region, as the reference's bench prepares them), the steps
    timed again until ``min_seconds`` of CPU work are measured.  Also
    timed: the A16 layer as torch-CPU fp32 dequant-then-matmul (weights
    dequantized outside the timed region), the config-1 linear both ways, and
    the config-3 FP8 shapes as torch-CPU fp32 dequant-then-matmul at every M.
    Without a VNNI-capable build the numpy oracle stands in (kind "port")."""
    import numpy as np

    from oracle import codecs as C
    from oracle import moe as MO
    from oracle import ref_c

    cores = _cpu_threads()
    torch.set_num_threads(cores)
    rng = np.random.default_rng(seed)
    gp, gs, dp, ds = bank["raw"]
    lib = ref_c.library()
    host = {}

    def expert(e):
        if e not in host:
            host[e] = (gp[e].cpu().numpy(), gs[e].cpu().numpy(), dp[e].cpu().numpy(), ds[e].cpu().numpy())
        return host[e]

    steps = []
    for _ in range(tokens):
        x = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).to(torch.bfloat16).float().numpy()
        ids, w = MO.route_topk(rng.standard_normal((1, E)).astype(np.float32), K, "sigmoid")
        steps.append((x, ids, w))
    used = sorted({int(e) for _, ids, _ in steps for e in ids.flatten()})
    out = {"cores": cores, "cpu": _cpu_info()}

    # (1) A8 layer on the reference's own CPU kernel
    if lib is not None:
        tiles = {e: (ref_c.prepare_weights(*expert(e)[:2]), ref_c.prepare_weights(*expert(e)[2:]))
                 for e in used + [E]}

        def a8_expert(codes, sa, e, wt):
            g = C.round_bf16(ref_c.gemm(codes, sa, tiles[e][0], lib))
            z = C.round_bf16((MO.swiglu(g[:, :I], g[:, I:], 0.0) * np.float32(wt)).astype(np.float32))
            zc, zs = C.act_quant(z, 128, "pow2")
            return C.round_bf16(ref_c.gemm(zc, zs, tiles[e][1], lib))

        # the same layers are timed again until at least min_seconds of CPU work
        # (their tiled weights, ~0.4 GB a layer, stream from DRAM every pass)
        t_a8, nbytes, passes, layers = 0.0, 0, 0, 0
        while passes == 0 or (t_a8 < min_seconds and passes < 400):
            for x, ids, w in steps:
                t0 = time.perf_counter()
                codes, sa = C.act_quant(x, 128, "pow2")
                acc = np.zeros((1, H), dtype=np.float32)
                for s_ in np.argsort(ids[0], kind="stable"):
                    acc = (acc + a8_expert(codes, sa, int(ids[0, s_]), w[0, s_])).astype(np.float32)
                acc = (acc + a8_expert(codes, sa, E, 1.0)).astype(np.float32)
                C.round_bf16(acc)
                t_a8 += time.perf_counter() - t0
                nbytes += (len(set(ids.flatten().tolist())) + 1) * EXPERT_BYTES + 2 * H * 2
                layers += 1
            passes += 1
        out.update({"value": round(nbytes / t_a8 / 1e9, 3), "unit": "GB/s", "kind": "reference",
                    "us_per_layer": round(t_a8 / layers * 1e6, 1),
                    "sample": f"{tokens} single-token A8 decode layers (8 routed + 1 shared expert, hidden {H}, "
                              f"inter {I}) through vnni_source_gemm ({cores} OpenMP threads), each timed {passes} "
                              f"times: {layers} layers, {t_a8:.2f} s"})
    # (2) A16 layer, torch-CPU fp32 dequant-then-matmul
    deq = {e: tuple(torch.from_numpy(C.dequant_mxfp4(*expert(e)[2 * j:2 * j + 2])) for j in range(2))
           for e in used + [E]}
    t_a16 = 0.0
    for x, ids, w in steps:
        xt = torch.from_numpy(x)
        t0 = time.perf_counter()
        acc = torch.zeros(1, H)
        order = list(np.argsort(ids[0], kind="stable")) + [None]
        for s_ in order:
            e, wt = (E, 1.0) if s_ is None else (int(ids[0, s_]), float(w[0, s_]))
            gu = xt @ deq[e][0].T
            z = (torch.nn.functional.silu(gu[:, :I]) * gu[:, I:] * wt).to(torch.bfloat16).float()
            acc = acc + z @ deq[e][1].T
        acc.to(torch.bfloat16)
        t_a16 += time.perf_counter() - t0
    a16_bytes = sum((len(set(ids.flatten().tolist())) + 1) * EXPERT_BYTES + 2 * H * 2 for _, ids, _ in steps)
    out["a16_torch_fp32"] = {"us_per_layer": round(t_a16 / tokens * 1e6, 1),
                             "GBs_mxfp4_equiv": round(a16_bytes / t_a16 / 1e9, 3)}
    if "value" not in out:  # no VNNI build here: the A16 torch path is the baseline
        out.update({"value": out["a16_torch_fp32"]["GBs_mxfp4_equiv"], "unit": "GB/s", "kind": "port",
                    "us_per_layer": out["a16_torch_fp32"]["us_per_layer"],
                    "sample": f"{tokens} single-token A16 decode layers, torch-CPU fp32 dequant-then-matmul"})
    del deq

    # (3) config 1: MXFP4 linear [2048, 7168] at M = 1 (the first 2048 gate rows of expert 0)
    p1, s1 = expert(0)[0][:2048], expert(0)[1][:2048]
    x1 = steps[0][0]
    c1 = {}
    if lib is not None:
        t1 = ref_c.prepare_weights(np.ascontiguousarray(p1), np.ascontiguousarray(s1))
        codes, sa = C.act_quant(x1, 128, "pow2")
        t0 = time.perf_counter()
        for _ in range(20):
            ref_c.gemm(codes, sa, t1, lib)
        c1["a8_reference_us"] = round((time.perf_counter() - t0) / 20 * 1e6, 1)
    w1 = torch.from_numpy(C.dequant_mxfp4(p1, s1))
    xt = torch.from_numpy(x1)
    t0 = time.perf_counter()
    for _ in range(20):
        xt @ w1.T
    c1["a16_torch_fp32_us"] = round((time.perf_counter() - t0) / 20 * 1e6, 1)
    out["config1_linear_m1"] = c1

    # (4) config 3: FP8 block-scaled GEMMs, torch-CPU fp32 dequant-then-matmul
    c3 = {}
    g = torch.Generator().manual_seed(12)
    for n, k in [(1536, 7168), (24576, 1536), (576, 7168), (7168, 16384), (18432, 7168)]:
        wq = (torch.randn(n, k, generator=g) * 0.02 * 448 / 0.08).clamp(-448, 448).to(torch.float8_e4m3fn)
        bs = torch.rand((n + 127) // 128, k // 128, generator=g) * 1e-4
        wf = wq.float() * bs.repeat_interleave(128, 0)[:n].repeat_interleave(128, 1)
        for m in (1, 16, 128, 4096):
            xa = (torch.randn(m, k, generator=g) * 60).clamp(-448, 448).to(torch.float8_e4m3fn)
            asc = torch.rand(m, k // 128, generator=g) * 1e-2
            reps = 5 if m < 4096 else 1
            t0 = time.perf_counter()
            for _ in range(reps):
                (xa.float() * asc.repeat_interleave(128, 1)) @ wf.T
            us = (time.perf_counter() - t0) / reps * 1e6
            c3[f"m{m}_n{n}_k{k}"] = {"us": round(us, 1), "TFLOPs": round(2 * m * n * k / us / 1e6, 3)}
        del wq, wf
    out["config3_fp8_gemm_torch_fp32"] = c3

    # (5) config 4: the A8 prefill layer's experts on the reference's own CPU kernel (a sample)
    if lib is not None:
        out["config4_moe_prefill_reference"] = _cpu_config4(expert, lib, cores)
    # (6) config 5: indexer + top-2048 and MLA decode, torch-CPU fp32
    out["config5_dsa_torch_fp32"] = _cpu_config5(torch)
    return out


def _cpu_config4(expert, lib, cores: int, m: int = 4096, seed: int = 13) -> dict:
    """A bounded sample of BASELINE.json configs[3] on the reference's ``vnni_source_gemm``:
    config-4 routing (Zipf(1.1) popularity over a seeded permutation, 8 experts
    pinned to zero, Gumbel-top-8 of 4096 tokens), then the A8 layer
    (``fused_moe_mxint``: token act_quant, gate/up, SwiGLU limit 10 x route weight,
    bf16, z act_quant, down, bf16) for four experts across the popularity range:
    the most loaded one and those at ranks 16, 64 and 128.  Weights are tiled
    outside the timed region.  Reported as TFLOP/s over the sample and the
    whole layer's time projected at that rate."""
    import numpy as np

    from oracle import codecs as C
    from oracle import moe as MO
    from oracle import ref_c

    rng = np.random.default_rng(seed)
    perm = rng.permutation(E)
    logp = np.empty(E)
    logp[perm] = -1.1 * np.log(np.arange(1, E + 1))
    logp[perm[-8:]] = -1e4
    u = rng.uniform(1e-9, 1 - 1e-9, size=(m, E))
    logits = (logp[None, :] - np.log(-np.log(u))).astype(np.float32)
    ids = np.argsort(-logits, axis=1, kind="stable")[:, :K]
    sc = MO.score_fn(np.take_along_axis(logits, ids, 1), "sigmoid")
    w = (sc / sc.sum(1, keepdims=True)).astype(np.float32)
    counts = np.bincount(ids.ravel(), minlength=E)
    by_load = np.argsort(-counts, kind="stable")
    picks = [int(by_load[r]) for r in (0, 16, 64, 128)]
    x = C.round_bf16(rng.standard_normal((m, H)).astype(np.float32))
    tiles = {e: (ref_c.prepare_weights(*expert(e)[:2]), ref_c.prepare_weights(*expert(e)[2:])) for e in picks}
    t, flops, rows_all = 0.0, 0, 0
    for e in picks:
        tok, slot = np.nonzero(ids == e)
        t0 = time.perf_counter()
        codes, sa = C.act_quant(x[tok], 128, "pow2")
        g = C.round_bf16(ref_c.gemm(codes, sa, tiles[e][0], lib))
        z = C.round_bf16((MO.swiglu(g[:, :I], g[:, I:], 10.0) * w[tok, slot][:, None]).astype(np.float32))
        zc, zs = C.act_quant(z, 128, "pow2")
        C.round_bf16(ref_c.gemm(zc, zs, tiles[e][1], lib))
        t += time.perf_counter() - t0
        flops += 2 * len(tok) * 3 * H * I
        rows_all += len(tok)
    rate = flops / t / 1e12
    layer_flops = 2 * m * (K + 1) * 3 * H * I
    return {"TFLOPs": round(rate, 4), "projected_layer_ms": round(layer_flops / (rate * 1e12) * 1e3, 1),
            "cores": cores, "kind": "reference",
            "sample": f"experts {picks} (loads {[int(counts[e]) for e in picks]}, {rows_all} token rows, "
                      f"{flops / 1e9:.0f} GFLOP of the layer's {layer_flops / 1e9:.0f}) through vnni_source_gemm, "
                      f"{t:.2f} s"}


def _cpu_config5(torch) -> dict:
    """BASELINE.json configs[4] on the CPU in torch fp32, one repetition each: the
    lightning indexer (e4m3 q and k decoded, per-head dots scaled by q_s and
    k_s, ReLU, x head weight, summed over 64 heads) + top-2048 at (B, L) =
    (1, 32768) and (8, 131072), and MLA decode over 2048 picks of an FP8
    latent cache (128 heads, 512 latent e4m3 with per-64 scales + 64 bf16
    rope, sink in the denominator) at B = 1 and 8."""
    g = torch.Generator().manual_seed(14)
    q8 = lambda *sh: (torch.randn(*sh, generator=g) * 60).clamp(-448, 448).to(torch.float8_e4m3fn)
    out = {}
    for b, l in [(1, 32768), (8, 131072)]:
        k, ks = q8(b, l, 128), torch.rand(b, l, generator=g) * 0.01 + 1e-3
        q, qs = q8(b, 64, 128), torch.rand(b, 64, generator=g) * 0.01 + 1e-3
        w = torch.randn(b, 64, generator=g) * 0.01
        t0 = time.perf_counter()
        dots = torch.bmm(k.float(), q.float().transpose(1, 2).contiguous())          # [b, l, 64]
        score = (torch.relu(dots * qs[:, None, :] * ks[:, :, None]) * w[:, None, :]).sum(-1)
        score.topk(2048, dim=-1)
        us = (time.perf_counter() - t0) * 1e6
        byts = b * l * 132 + b * 64 * 136
        out[f"indexer_b{b}_l{l}"] = {"us": round(us, 1), "GBs": round(byts / us / 1e3, 3)}
        del k, dots, score
    for b in (1, 8):
        n, t_ = 65536, 2048
        qh = torch.randn(b, 128, 576, generator=g).to(torch.bfloat16)
        lat, lsc = q8(b, n, 512), torch.rand(b, n, 8, generator=g) * 0.01
        rope = torch.randn(b, n, 64, generator=g).to(torch.bfloat16)
        idx = torch.stack([torch.randperm(n, generator=g)[:t_] for _ in range(b)])
        sink = torch.randn(128, generator=g)
        t0 = time.perf_counter()
        gi = idx[:, :, None]
        latd = (torch.gather(lat.float(), 1, gi.expand(-1, -1, 512)).view(b, t_, 8, 64) *
                torch.gather(lsc, 1, gi.expand(-1, -1, 8))[..., None]).view(b, t_, 512).to(torch.bfloat16).float()
        kv = torch.cat([latd, torch.gather(rope, 1, gi.expand(-1, -1, 64)).float()], -1)   # [b, t, 576]
        s_ = torch.bmm(qh.float(), kv.transpose(1, 2).contiguous()) * 576 ** -0.5      # [b, 128, t]
        mx = s_.amax(-1, keepdim=True)
        p_ = torch.exp(s_ - mx)
        den = p_.sum(-1, keepdim=True) + torch.exp(sink[None, :, None] - mx)
        torch.bmm(p_.to(torch.bfloat16).float(), latd) / den
        us = (time.perf_counter() - t0) * 1e6
        out[f"mla_b{b}"] = {"us": round(us, 1), "TFLOPs": round(2 * b * 128 * t_ * (576 + 512) / us / 1e6, 4)}
    return out


def write_launch_table(path: str, argv: list, r: dict, line: dict) -> None:
    """The per-launch table behind ``roofline``: every event-timed gate/up (and
    down) dispatch of the instrumented pass, its algorithmic bytes and rate."""
    import statistics
    rows = r["per_launch"]
    gu = [p["gu_us"] for p in rows]
    out = [f"# Event-timed launches behind bench.py's roofline: MoE decode, M = {r['m']}", "",
           "Command (from the repository root on one MI355X):", "", "```",
           "python3 " + " ".join(argv), "```", "",
           "The gate/up dispatch of each instrumented step records HIP events itself "
           "(`hipExtLaunchKernelGGL` start/stop on the kernel's stream), so its duration is the kernel's "
           "execution.  The down dispatch records only its end, so the down column runs from the gate/up "
           "kernel's end to the down kernel's end (the dependent-launch gap included).  Algorithmic bytes "
           "per launch: (distinct experts + shared) x each expert's codes and scales, + x + z (gate/up) or "
           "z + y (down).", "",
           "| step | distinct experts | gate/up µs | gate/up bytes | gate/up GB/s | gap + down µs | down bytes | "
           "down GB/s |", "|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for i, p in enumerate(rows):
        out.append(f"| {i} | {p['distinct']} | {p['gu_us']:.2f} | {p['gu_bytes']:,} | "
                   f"{p['gu_bytes'] / p['gu_us'] / 1e3:.0f} | {p['down_us']:.2f} | {p['down_bytes']:,} | "
                   f"{p['down_bytes'] / p['down_us'] / 1e3:.0f} |")
    gb = sum(p["gu_bytes"] for p in rows)
    db = sum(p["down_bytes"] for p in rows)
    dn = [p["down_us"] for p in rows]
    out += ["", "| kernel | launches | avg µs | median µs | min µs | max µs | bytes / time | of 8 TB/s |",
            "|---|---:|---:|---:|---:|---:|---:|---:|",
            f"| gate/up | {len(gu)} | {statistics.mean(gu):.2f} | {statistics.median(gu):.2f} | {min(gu):.2f} | "
            f"{max(gu):.2f} | {gb / sum(gu) / 1e3:.1f} GB/s | {gb / sum(gu) / 1e3 / HBM_PEAK_GBS:.4f} |",
            f"| gap + down | {len(dn)} | {statistics.mean(dn):.2f} | {statistics.median(dn):.2f} | {min(dn):.2f} | "
            f"{max(dn):.2f} | {db / sum(dn) / 1e3:.1f} GB/s | {db / sum(dn) / 1e3 / HBM_PEAK_GBS:.4f} |", "",
            f"The line's `roofline` (the gate/up kernel): achieved {line['roofline']['achieved']} GB/s, frac "
            f"{line['roofline']['frac']}, avg_launch_us {line['roofline']['avg_launch_us']}: the gate/up row "
            f"above.  The headline layer time of the same run: {line['us_per_layer']} µs "
            f"({line['config']['timing']}).", ""]
    with open(path, "w") as f:
        f.write("\n".join(out))


def _gateup_kernel_name(m: int) -> str:
    """The gate/up kernel the A16 forward launches for M tokens (routing on the device)."""
    return "moe_dec1_gateup_kernel" if m == 1 else ("moe_small_gateup_kernel" if m <= 4 else "moe_a16_gateup_kernel")


def _stage_view(m: int, st: dict) -> dict:
    """Per-stage microseconds of the instrumented pass.  At M = 1 the layer is
    two launches whose dispatches record their own start/end events, so only
    the two kernels are stages (routing is fused into gate/up, the combine
    into down); the other event gaps are dispatch latency, not work."""
    if 2 <= m <= 4:
        return {"gateup_kernel_with_routing": round(st["gu_sec"], 2),
                "down_kernel_with_combine": round(st["down_sec"], 2),
                "note": "2..4 tokens: two launches (routing in gate/up, the combine in down); "
                        "the other event gaps are dispatch latency"}
    if m != 1:
        return {k: round(v, 2) for k, v in st.items()}
    return {"gateup_kernel_with_routing": round(st["gu_sec"], 2),
            "gap_and_down_kernel_with_combine": round(st["down_sec"], 2),
            "note": "events recorded by the two dispatches themselves; M=1 has no separate layout or combine stage"}


def _config_fns(torch, ops, banks):
    return [("config1_linear_m1", lambda: config1_linear(torch, ops)),
            ("config3_fp8_gemm", lambda: config3_fp8(torch, ops)),
            ("config3_mxfp4_gemm", lambda: config3_mxfp4(torch, ops)),
            ("config4_moe_prefill", lambda: config4_prefill(torch, ops, banks[0])),
            ("config5_dsa", lambda: config5_dsa(torch, ops))]


# run only when named in --configs (calibration lines and the W8A16 drop-in, not BASELINE.json configs)
def _optional_config_fns(torch, ops):
    return [("config3_vendor_fp8", lambda: config3_vendor_fp8(torch, ops)),
            ("config3_vendor_mx", lambda: config3_vendor_mx(torch, ops)),
            ("config3_w8a16", lambda: config3_w8a16(torch, ops))]


def _selected_configs(args, torch, ops, banks):
    names = [v for v in args.configs.split(",") if v]
    fns = [(n, f) for n, f in _config_fns(torch, ops, banks) if not names or n in names]
    fns += [(n, f) for n, f in _optional_config_fns(torch, ops) if n in names]
    return fns


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported: this build runs on one GPU only "
              f"(no collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch

    from mosaic_amd import ops

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    need_bank = not args.no_headline or (not args.no_configs and (
        not args.configs or "config4_moe_prefill" in args.configs.split(",")))
    banks = build_banks(torch, ops, n_banks=1 if args.no_headline else N_BANKS) if need_bank else []
    if args.no_headline:
        configs = {}
        if not args.no_configs:
            for name, fn in _selected_configs(args, torch, ops, banks):
                print(f"bench.py: {name}", file=sys.stderr, flush=True)
                configs[name] = fn()
        print(json.dumps({"metric": METRIC, "profiling_run": True, "configs": configs}), flush=True)
        return
    main_r = run_m(torch, ops, banks, args.m, args.steps, args.warmup, seed=0, graph=not args.no_graph)
    sweep = {}
    for mv in [int(v) for v in args.sweep.split(",") if v.strip()]:
        if mv != args.m:
            r = run_m(torch, ops, banks, mv, max(6, args.steps // 5), 2, seed=mv, graph=not args.no_graph)
            sweep[str(mv)] = {k: (round(v, 2) if isinstance(v, float) else v) for k, v in r.items()
                              if k in ("us_per_layer", "eager_us_per_layer", "gbs", "distinct_experts_avg")}
            sweep[str(mv)]["hbm_frac"] = round(r["gbs"] / HBM_PEAK_GBS, 4)
    configs = {}
    if not args.no_configs:
        for name, fn in _selected_configs(args, torch, ops, banks):
            print(f"bench.py: {name}", file=sys.stderr, flush=True)
            configs[name] = fn()
    cpu = None if args.no_cpu_baseline else cpu_baseline(torch, ops, banks[0])
    gu_gbs = main_r["gateup_gbs"]
    line = {
        "metric": METRIC,
        "value": round(main_r["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_r["us_per_layer"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "mxfp4 weights x bf16 activations, fp32 accumulate",
        "data": "synthetic (seeded N(0,1) tokens/logits, N(0,0.02) weights quantized to MXFP4)",
        "config": {"workload": "MXFP4 MoE decode layer (BASELINE.json configs[1])", "tokens": args.m, "hidden": H,
                   "inter": I, "experts": E, "top_k": K, "shared_experts": 1, "score": "sigmoid",
                   "contract": "A16 dequant-then-matmul", "weight_layout": "MXT16 prepacked", "banks": N_BANKS,
                   "bank_reuse_distance_bytes": round((N_BANKS - 1) * main_r["layer_bytes_avg"]),
                   "timing": ("the K steps run eagerly (--no-graph)" if args.no_graph
                              else "median of three HIP-graph replays, each of exactly the K steps")},
        "us_per_layer": round(main_r["us_per_layer"], 2),
        "eager_us_per_layer": round(main_r["eager_us_per_layer"], 2),
        "hbm_frac": round(main_r["gbs"] / HBM_PEAK_GBS, 4),
        "tokens_per_s": round(args.m / (main_r["us_per_layer"] / 1e6), 1),
        "distinct_experts_avg": main_r["distinct_experts_avg"],
        "stage_us": _stage_view(args.m, main_r["stage_us"]),
        "roofline": {"kernel": _gateup_kernel_name(args.m), "bound": "hbm",
                     "achieved": round(gu_gbs, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": round(GATEUP_M1_TRAFFIC_BYTES) if args.m == 1 else None,
                     "avg_launch_us": round(main_r["gateup_us"], 2),
                     "algorithmic_bytes_per_launch": round(main_r["gateup_bytes_per_launch"])},
        "cpu_baseline": cpu,
        "m_sweep": sweep,
        "configs": configs,
    }
    print(json.dumps(line), flush=True)
    if args.launch_table:
        write_launch_table(args.launch_table, sys.argv, main_r, line)
    if args.calibration_copy_mib > 0:
        src = torch.ones(args.calibration_copy_mib << 18, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()


if __name__ == "__main__":
    main()
