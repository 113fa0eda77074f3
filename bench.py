#!/usr/bin/env python3
"""Benchmark of the MI355X MXFP4 W4A8 linear path (one GPU).

Headline workload: the speculative-verify decode GEMM, M=8 tokens x N=17408 x K=5120 (fused
gate/up of a 5120-hidden, 8704-intermediate MLP), HBM-bound, reported in GB/s of algorithmic bytes
  bytes = N*K/2 (e2m1) + N*K/32 (e8m0) + M*K (e4m3 activations) + 4*M (token scales) + 2*M*N (bf16)
with fp8 activations and repacked weights resident in HBM before the timed region. A step is one
GEMM launch over one batch of synthetic tokens. Weights rotate over 16 distinct copies (757 MB, about
3x the 256 MB MALL) so no launch is served from the last-level cache. The timed loop replays a HIP
graph of launches (a single launch is shorter than the host's launch overhead); the kernel's own
duration comes from HIP event pairs around individual launches on the launch stream.

Alongside: the M=4096 prefill GEMMs (gate_up 17408x5120, down 5120x8704) in TFLOP/s against the
fp8 x fp4 MFMA peak, the M=1 per-layer linear set, the fused producers and the per-token quantizer
at M=8 and M=4096 in GB/s, the register-resident MFMA rate, a streaming read of the verify
GEMM's bytes in its launch shape and over a sweep of launch shapes (the HBM ceiling it is held
against), and the CPU baseline (a torch restatement of the reference's dequant + fp32 matmul,
timed on this host's cores). Prints ONE JSON line.

  python bench.py [--gpus 1] [--steps 1024] [--warmup 64]

--steps K times exactly K verify-GEMM launches (one HIP graph of K launches between two events);
--warmup W runs W untimed launches first. Before those, the same graph replays for one second to
bring the clocks up; the line reports that separately (clock_warmup).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "W4A8 GEMM GB/s (M=8) & TFLOPS (M=4096), % of MI355X roofline"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
MFMA_PEAK_TFLOPS = 5000.0      # dense fp8 rate; the mixed fp8 x fp4 scaled MFMA issues at it
VERIFY = dict(M=8, N=17408, K=5120)
PREFILL = [("gate_up", 4096, 17408, 5120), ("down", 4096, 5120, 8704)]
LAYER_M1 = [("qkv", 10240, 5120), ("o_proj", 5120, 6144), ("gate_up", 17408, 5120),
            ("down", 5120, 8704)]
COPIES = 16


def gemm_bytes(M, N, K):
    return N * K // 2 + N * K // 32 + M * K + 4 * M + 2 * M * N


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024,
                    help="verify-GEMM launches timed (exactly this many)")
    ap.add_argument("--warmup", type=int, default=64,
                    help="untimed verify-GEMM launches before them (after the clock warm-up)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only-verify", action="store_true", help="skip prefill and M=1 legs")
    ap.add_argument("--sweep", action="store_true",
                    help="the 64-layer sweep instead of the headline: one-time repack cost per "
                         "layer, linear ms per forward at M in {1, 8, 16, 64, 512, 4096}, and the "
                         "M where the macro-tile GEMM overtakes the decode kernels; prints its own "
                         "JSON line")
    ap.add_argument("--sweep-layers", type=int, default=64)
    ap.add_argument("--profile", action="store_true",
                    help="counter-run workload: the verify-GEMM graph replay, 4 launches of each "
                         "prefill GEMM, fused producer and quantizer shape at M=4096, 8 of each "
                         "decode-band GEMM and M=1 linear, and one 256 MiB device copy (the "
                         "counter calibration); prints no JSON")
    return ap.parse_args()


class Gemm:
    """Device operands of one GEMM shape with `copies` distinct repacked weight copies."""

    def __init__(self, M, N, K, copies, seed):
        import torch
        from vllm_sly_radiance_amd import _native, radiance_mxfp4 as R, synthetic
        self.M, self.N, self.K = M, N, K
        w, ws = synthetic.weights(N, K, seed)
        x = synthetic.activations(M, K, seed + 1)
        self.x = torch.from_numpy(x.view(np.int16)).cuda().view(torch.bfloat16)
        self.q, self.s = R.quant_per_token(self.x)
        wq, sq = R.repack_weights(torch.from_numpy(w).cuda(), torch.from_numpy(ws).cuda())
        self.w = [wq] + [wq.clone() for _ in range(copies - 1)]
        self.ws = [sq] + [sq.clone() for _ in range(copies - 1)]
        self.out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        self.plan = _native.plan(M, N, K)
        self._native = _native
        torch.cuda.synchronize()

    def launch(self, i, stream):
        self._native.gemm(self.q.data_ptr(), self.s.data_ptr(), self.w[i].data_ptr(),
                          self.ws[i].data_ptr(), self.out.data_ptr(), self.M, self.N, self.K,
                          stream)


class QuantGemm(Gemm):
    """The linear as radiance::mxfp4_linear runs it: the per-token quantizer on bf16 activations,
    then the GEMM (two launches per step)."""

    def launch(self, i, stream):
        self._native.quant_per_token(self.x.data_ptr(), self.K, self.q.data_ptr(),
                                     self.s.data_ptr(), self.M, self.K, stream)
        super().launch(i, stream)


class Linear:
    """A Gemm's operands run as radiance::mxfp4_linear runs them through w4a8_linear: bf16
    activations in, one launch where the quantizer runs inside the streaming GEMM
    (w4a8_linear_fused), else two."""

    def __init__(self, g):
        self.g, self.w = g, g.w

    def launch(self, i, stream):
        g = self.g
        g._native.linear(g.x.data_ptr(), g.K, g.q.data_ptr(), g.s.data_ptr(), g.w[i].data_ptr(),
                         g.ws[i].data_ptr(), g.out.data_ptr(), g.M, g.N, g.K, stream)


def per_launch_us(g, n, stream_obj):
    """Median and mean duration of single launches, each bracketed by its own HIP event pair on the
    launch stream (includes the event overhead; a cross-check only)."""
    import torch
    st = stream_obj.cuda_stream
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(n)]
    for i, (a, b) in enumerate(ev):
        a.record(stream_obj)
        g.launch(i % len(g.w), st)
        b.record(stream_obj)
    torch.cuda.synchronize()
    t = np.array([a.elapsed_time(b) * 1000.0 for a, b in ev])
    return float(np.median(t)), float(np.mean(t))


WARM_SECONDS = 1.0


def graph_timed(g, steps, warmup, warm_seconds=WARM_SECONDS, direct=False):
    """Time exactly `steps` launches after `warmup` untimed ones, on one side stream.

    The timed launches are one HIP graph of `steps` launches (weight copies rotating), replayed
    once between two events on the stream the kernels run on, or with `direct` the same launches
    put on the stream one by one (no graph). Before the warmup launches the graph replays for at
    least `warm_seconds` (MI355X raises its clocks over the first few hundred milliseconds of
    load; a cold GEMM reads up to 20 % slow), reported separately as the clock warm-up. Its last
    four replays, the warmup launches, the first event and the timed launches are queued without
    a synchronization in between, so the GPU never idles (and never drops its clocks) before the
    timed launches start; the four replays keep the GPU busy for four times the timed work while
    the host queues the rest. Returns (seconds, clock warm-up dict, per-launch event median,
    mean)."""
    import torch
    stream = torch.cuda.Stream()
    n = len(g.w)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        g.launch(0, stream.cuda_stream)           # code objects loaded before capture
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(steps):
            g.launch(i % n, stream.cuda_stream)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        t0, replays = time.perf_counter(), 0
        while True:
            for _ in range(4):
                graph.replay()
            replays += 4
            if time.perf_counter() - t0 >= warm_seconds:
                break
            stream.synchronize()
        clock = dict(seconds=round(time.perf_counter() - t0, 3), launches=replays * steps)
        for i in range(warmup):
            g.launch(i % n, stream.cuda_stream)
        e0.record(stream)
        if direct:
            for i in range(steps):
                g.launch(i % n, stream.cuda_stream)
        else:
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    sec = e0.elapsed_time(e1) * 1e-3
    with torch.cuda.stream(stream):
        med_us, mean_us = per_launch_us(g, 64, stream)
    del graph
    return sec, clock, med_us, mean_us


def bench_verify(args):
    """The headline: exactly --steps launches of the verify GEMM, timed as direct stream launches
    behind the warm-up. A HIP graph replay adds ~5 us of its own on the GPU (measured on MI355X:
    graphs of 20 launches 10.20-10.27 us per launch, of 1024 launches 9.82; 20 direct launches
    9.87-10.01, 64-256 9.81-9.84), which at the driver's 20 steps would be 0.25 us per launch
    that no kernel spends; the gap between consecutive kernels is the same either way."""
    M, N, K = VERIFY["M"], VERIFY["N"], VERIFY["K"]
    g = Gemm(M, N, K, COPIES, seed=1)
    sec, clock, med_us, mean_us = graph_timed(g, args.steps, args.warmup, direct=True)
    nbytes = gemm_bytes(M, N, K)
    us = sec / args.steps * 1e6
    return dict(M=M, N=N, K=K, steps=args.steps, warmup=args.warmup, clock_warmup=clock,
                ms_per_step=us * 1e-3, gbs=nbytes / (us * 1e-6) / 1e9, bytes=nbytes,
                kernel_us=us, event_pair_us_median=med_us, event_pair_us_mean=mean_us,
                plan=g.plan)


# the fused producer that makes each prefill GEMM's input in the model
PREFILL_PRODUCER = {"gate_up": "add_rms", "down": "silu"}


def bench_prefill():
    """The M=4096 prefill GEMMs alone, and as config 4 states them: the per-token quantizer on
    bf16 activations fused ahead of the GEMM (quant + GEMM per step, timed as one unit); then
    the model's own chain, the fused producer + GEMM, with q row-major and fragment-tiled."""
    import torch
    from vllm_sly_radiance_amd import _native
    res = []
    for name, M, N, K in PREFILL:
        copies = max(2, -(-512 * 2 ** 20 // (N * K * 17 // 32)))
        flop = 2.0 * M * N * K
        row = dict(name=name, M=M, N=N, K=K)
        legs = (("gemm", lambda: Gemm(M, N, K, copies, seed=7)),
                ("quant_gemm", lambda: QuantGemm(M, N, K, copies, seed=7)),
                ("producer_gemm", lambda: ProducerGemm(PREFILL_PRODUCER[name], M, N, K, copies,
                                                       7, _native.Q_ROWS)),
                ("producer_gemm_tiled", lambda: ProducerGemm(PREFILL_PRODUCER[name], M, N, K,
                                                             copies, 7, _native.Q_TILED)))
        for key, make in legs:
            g = make()
            sec, _, _, _ = graph_timed(g, 8 * copies, 2 * copies)
            us = sec / (8 * copies) * 1e6
            tf = flop / (us * 1e-6) / 1e12
            if key == "gemm":
                row.update(us=round(us, 2), tflops=round(tf, 1),
                           frac=round(tf / MFMA_PEAK_TFLOPS, 4), plan=g.plan)
            else:
                row.update({f"{key}_us": round(us, 2), f"{key}_tflops": round(tf, 1),
                            f"{key}_frac": round(tf / MFMA_PEAK_TFLOPS, 4)})
            del g
            torch.cuda.empty_cache()
        row["producer"] = PREFILL_PRODUCER[name]
        util = measured_mfma_util(f"prefill_{name}")
        if util is not None:
            row["mfma_util"] = util
        res.append(row)
    return res


class SiluLinear:
    """The MLP's tail as radiance::silu_mul_mxfp4_linear runs it: gate_up bf16 [M, 2K] in, the
    down projection of silu(gate) * up out (w4a8_silu_mul_linear: one launch where
    w4a8_silu_mul_linear_fused says so, else the SiLU-mul producer and the GEMM)."""

    def __init__(self, g, prod):
        self.g, self.p, self.w = g, prod, g.w

    def launch(self, i, stream):
        g, p = self.g, self.p
        g._native.silu_mul_linear(p.w[i].data_ptr(), p.q.data_ptr(), p.s.data_ptr(),
                                  g.w[i].data_ptr(), g.ws[i].data_ptr(), g.out.data_ptr(), g.M,
                                  g.N, g.K, stream)


def bench_layer_m1():
    """The four linears of one layer at M = 1: the GEMM on pre-quantized activations (`us`), and
    the linear on bf16 activations as the op runs it (`linear_us`: one launch with the quantizer
    inside where `one_launch`, else quantizer + GEMM). For down also the MLP's tail from the
    gate_up output: SiLU-and-mul + down in one op (`silu_down_us`) against the SiLU-mul producer
    followed by the GEMM (`silu_then_down_us`)."""
    import torch
    out, tot_us, tot_lin, tot_bytes = [], 0.0, 0.0, 0
    for name, N, K in LAYER_M1:
        copies = max(2, -(-512 * 2 ** 20 // (N * K * 17 // 32)))
        g = Gemm(1, N, K, copies, seed=3)
        sec, _, _, _ = graph_timed(g, 32 * copies, 4 * copies, warm_seconds=0.5)
        us = sec / (32 * copies) * 1e6
        sec, _, _, _ = graph_timed(Linear(g), 32 * copies, 4 * copies, warm_seconds=0.2)
        lin = sec / (32 * copies) * 1e6
        nb = gemm_bytes(1, N, K)
        tot_us += us
        tot_lin += lin
        tot_bytes += nb
        out.append(dict(name=name, N=N, K=K, us=round(us, 2),
                        gbs=round(nb / (us * 1e-6) / 1e9, 1), plan=g.plan,
                        linear_us=round(lin, 2),
                        one_launch=bool(g._native.linear_fused(1, N, K, K))))
        if name == "down":
            prod = Producer("silu", 1, K, copies, seed=41)
            sec, _, _, _ = graph_timed(SiluLinear(g, prod), 32 * copies, 4 * copies,
                                       warm_seconds=0.2)
            out[-1]["silu_down_us"] = round(sec / (32 * copies) * 1e6, 2)
            out[-1]["silu_down_one_launch"] = bool(g._native.silu_mul_linear_fused(1, N, K))
            pg = ProducerGemm("silu", 1, N, K, copies, 41, 0)
            sec, _, _, _ = graph_timed(pg, 32 * copies, 4 * copies, warm_seconds=0.2)
            out[-1]["silu_then_down_us"] = round(sec / (32 * copies) * 1e6, 2)
            del prod, pg
        del g
        torch.cuda.empty_cache()
    return dict(layers=out, us_per_layer=round(tot_us, 2),
                gbs=round(tot_bytes / (tot_us * 1e-6) / 1e9, 1),
                linear_us_per_layer=round(tot_lin, 2))


class Producer:
    """Device operands of one fused producer (radiance::add_rms_quant / silu_mul_quant /
    gdn_norm_quant) with `copies` distinct input sets."""

    def __init__(self, kind, M, N, copies, seed, q_layout=0):
        import torch
        from vllm_sly_radiance_amd import _native, synthetic
        self.kind, self.M, self.N, self._native = kind, M, N, _native
        self.q_layout = q_layout

        def dev(bits):
            return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)
        width = {"add_rms": N, "silu": 2 * N, "gdn": N}[kind]
        self.w = [dev(synthetic.activations(M, width, seed + i)) for i in range(copies)]
        self.w2 = [dev(synthetic.activations(M, N, seed + 100 + i)) for i in range(copies)] \
            if kind in ("add_rms", "gdn") else None
        nw = 128 if kind == "gdn" else N
        self.weight = dev(synthetic.activations(1, nw, seed + 200)[0])
        qbytes = _native.tiled_bytes(M, N) if q_layout == _native.Q_TILED else M * N
        self.q = torch.empty((qbytes,), dtype=torch.uint8, device="cuda")
        self.s = torch.empty((M,), dtype=torch.float32, device="cuda")
        self.r = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        torch.cuda.synchronize()

    def bytes(self):
        M, N = self.M, self.N
        if self.kind == "add_rms":                       # y, res, weight in; res_out, q, s out
            return 7 * M * N + 2 * N + 4 * M
        if self.kind == "silu":                          # gate_up in; q, s out
            return 5 * M * N + 4 * M
        return 5 * M * N + 256 + 4 * M                   # x, z, weight in; q, s out

    def launch(self, i, stream):
        n = self._native
        if self.kind == "add_rms":
            n.add_rms_quant(self.w[i].data_ptr(), self.w2[i].data_ptr(), self.weight.data_ptr(),
                            self.q.data_ptr(), self.s.data_ptr(), self.r.data_ptr(), self.M,
                            self.N, 1e-6, stream, self.q_layout)
        elif self.kind == "silu":
            n.silu_mul_quant(self.w[i].data_ptr(), self.q.data_ptr(), self.s.data_ptr(), self.M,
                             self.N, stream, self.q_layout)
        else:
            n.gdn_norm_quant(self.w[i].data_ptr(), self.w2[i].data_ptr(), self.N,
                             self.weight.data_ptr(), self.q.data_ptr(), self.s.data_ptr(), self.M,
                             self.N, 1e-6, stream, self.q_layout)


class ProducerGemm(Gemm):
    """The linear as the model runs it at prefill: the fused producer that makes its input
    (add_rms_quant in front of gate_up, silu_mul_quant in front of down) writes (q, scale) and the
    GEMM reads them, one producer input set per weight copy. q_layout 1 writes q fragment-tiled
    and runs w4a8_gemm_at on it."""

    def __init__(self, kind, M, N, K, copies, seed, q_layout):
        super().__init__(M, N, K, copies, seed)
        self.prod = Producer(kind, M, K, copies, seed + 50, q_layout)

    def launch(self, i, stream):
        p = self.prod
        p.launch(i, stream)
        gemm = self._native.gemm_at if p.q_layout else self._native.gemm
        gemm(p.q.data_ptr(), p.s.data_ptr(), self.w[i].data_ptr(), self.ws[i].data_ptr(),
             self.out.data_ptr(), self.M, self.N, self.K, stream)


class Quant:
    """Device operands of the per-token quantizer (w4a8_quant_per_token) on `copies` distinct bf16
    activation sets."""

    def __init__(self, M, K, copies, seed):
        import torch
        from vllm_sly_radiance_amd import _native, synthetic
        self.M, self.K, self._native = M, K, _native
        self.w = [torch.from_numpy(synthetic.activations(M, K, seed + i).view(np.int16)).cuda()
                  for i in range(copies)]
        self.q = torch.empty((M, K), dtype=torch.uint8, device="cuda")
        self.s = torch.empty((M,), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()

    def bytes(self):
        return 3 * self.M * self.K + 4 * self.M          # bf16 in; codes and scales out

    def launch(self, i, stream):
        self._native.quant_per_token(self.w[i].data_ptr(), self.K, self.q.data_ptr(),
                                     self.s.data_ptr(), self.M, self.K, stream)


# the quantizer in front of every GEMM whose input no fused producer makes: (M, K)
QUANT_SHAPES = [(8, 5120), (4096, 5120), (4096, 8704)]


def bench_quant():
    import torch
    res = []
    for M, K in QUANT_SHAPES:
        copies = max(2, min(16, -(-512 * 2 ** 20 // (2 * M * K))))
        g = Quant(M, K, copies, seed=31)
        sec, _, _, _ = graph_timed(g, 8 * copies, 2 * copies, warm_seconds=0.2)
        us = sec / (8 * copies) * 1e6
        gbs = g.bytes() / (us * 1e-6) / 1e9
        res.append(dict(M=M, K=K, us=round(us, 2), gbs=round(gbs, 1),
                        frac=round(gbs / HBM_PEAK_GBS, 4)))
        del g
        torch.cuda.empty_cache()
    return res


# (op, width) at the benchmark model's shapes: the decoder norms feed K = 5120, the MLP activation
# N = 8704 (the gate_up GEMM's 17408 columns are gate and up; down has K = 8704), the GatedDeltaNet
# output projection N = 6144 (48 heads of 128)
PRODUCERS = [("add_rms", 5120), ("silu", 8704), ("gdn", 6144)]


def bench_producers():
    import torch
    from vllm_sly_radiance_amd import radiance_mxfp4 as R
    R.ensure_scratch("cuda")          # as after the plugin's first layer (silu's split path)
    res = []
    for M in (8, 4096):
        for kind, N in PRODUCERS:
            per_copy = 4 * M * N                         # bf16 input bytes per launch
            copies = max(2, min(16, -(-512 * 2 ** 20 // per_copy)))
            g = Producer(kind, M, N, copies, seed=21)
            sec, _, _, _ = graph_timed(g, 8 * copies, 2 * copies, warm_seconds=0.2)
            us = sec / (8 * copies) * 1e6
            gbs = g.bytes() / (us * 1e-6) / 1e9
            res.append(dict(op=kind, M=M, N=N, us=round(us, 2), gbs=round(gbs, 1),
                            frac=round(gbs / HBM_PEAK_GBS, 4)))
            del g
            torch.cuda.empty_cache()
    return res


class ReadProbe:
    """`copies` device buffers of `nbytes` each, read by w4a8_read_probe (the decode GEMM's launch
    shape over plain bytes)."""

    def __init__(self, nbytes, copies):
        import torch
        from vllm_sly_radiance_amd import _native
        self.n, self._native = nbytes, _native
        self.w = [torch.full((nbytes,), i + 1, dtype=torch.uint8, device="cuda")
                  for i in range(copies)]
        self.out = torch.zeros(1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()

    def launch(self, i, stream):
        self._native.read_probe(self.w[i].data_ptr(), self.n, self.out.data_ptr(), stream)


class ReadShape:
    """A ReadProbe's buffers read by w4a8_read_probe_shape: `blocks` workgroups of one variant."""

    def __init__(self, probe, blocks, variant):
        self.p, self.w, self.blocks, self.variant = probe, probe.w, blocks, variant

    def launch(self, i, stream):
        p = self.p
        p._native.read_probe_shape(p.w[i].data_ptr(), p.n, p.out.data_ptr(), self.blocks,
                                   self.variant, stream)


# (workgroups, read-probe variant) pairs of the launch-shape sweep over the verify GEMM's bytes:
# the GEMM's own grid (218 workgroups of 10 waves) and the 233-234 of the plain probe, fewer
# workgroups with more bytes each (136-182), grids that give every CU equal bytes (256) with 4-16
# waves, 12-46 KiB per wave, all loads issued at once or a window of 4-12 in flight, non-temporal
# or not, and two or four workgroups per CU
READ_SWEEP = [(234, 0), (218, 1), (136, 18), (160, 17), (182, 16), (240, 0), (248, 0), (256, 0),
              (256, 2), (256, 3), (256, 4), (256, 5), (256, 6), (256, 7), (256, 8), (256, 9),
              (256, 10), (256, 14), (256, 15), (512, 11), (512, 13), (1013, 12)]


def bench_read_probe(steps, warmup):
    """The HBM read ceiling for the verify GEMM: as many bytes per launch as its algorithmic
    traffic, the same rotation over 16 copies and the same timing (direct launches behind the
    graph warm-up), nothing but reads. First the fixed probe (the GEMM's launch shape), then the
    launch-shape sweep (READ_SWEEP, 256 launches each), whose fastest shape is the ceiling the
    GEMM is held against; last the GEMM against its own load pattern (bench_gemm_loads)."""
    import torch
    nbytes = gemm_bytes(VERIFY["M"], VERIFY["N"], VERIFY["K"])
    g = ReadProbe(nbytes, COPIES)
    sec, _, _, _ = graph_timed(g, steps, warmup, warm_seconds=0.5, direct=True)
    us = sec / steps * 1e6
    gbs = g.n / (us * 1e-6) / 1e9
    res = dict(bytes=nbytes, us=round(us, 3), gbs=round(gbs, 1), frac=round(gbs / HBM_PEAK_GBS, 4))
    variants = g._native.read_probe_variants()
    shapes = []
    for blocks, v in READ_SWEEP:
        waves, units, window, nt = variants[v]
        sec, _, _, _ = graph_timed(ReadShape(g, blocks, v), 256, 16, warm_seconds=0.2,
                                   direct=True)
        us_s = sec / 256 * 1e6
        shapes.append(dict(blocks=blocks, waves=waves, kib_per_wave=units, in_flight=window,
                           nontemporal=bool(nt), us=round(us_s, 3),
                           gbs=round(nbytes / (us_s * 1e-6) / 1e9, 1)))
        print(f"[bench] read sweep {shapes[-1]}", file=sys.stderr, flush=True)
    best = min(shapes, key=lambda r: r["us"])
    res["sweep"] = shapes
    res["best"] = dict(best, frac=round(best["gbs"] / HBM_PEAK_GBS, 4))
    del g
    torch.cuda.empty_cache()
    res["gemm_loads"] = bench_gemm_loads()
    return res


class StreamLoads:
    """A Gemm's operands read by w4a8_stream_load_probe: the streaming GEMM's own loads (one of
    the three load sets), without its math."""

    def __init__(self, g, parts):
        self.g, self.w, self.parts = g, g.w, parts

    def launch(self, i, stream):
        g = self.g
        g._native.stream_load_probe(g.q.data_ptr(), g.s.data_ptr(), g.w[i].data_ptr(),
                                    g.ws[i].data_ptr(), g.M, g.N, g.K, self.parts,
                                    g.probe_out.data_ptr(), stream)


def bench_gemm_loads(steps=256):
    """What the verify GEMM's load pattern costs without its math: the GEMM and its loads alone
    (weight granules; and scale dwords; and activation fragments with token scales, every load it
    issues), each `steps` direct launches over the same 16 weight copies, µs per launch."""
    import torch
    from vllm_sly_radiance_amd import _native
    M, N, K = VERIFY["M"], VERIFY["N"], VERIFY["K"]
    g = Gemm(M, N, K, COPIES, seed=1)
    g.probe_out = torch.zeros(1, dtype=torch.int32, device="cuda")
    res = dict(steps=steps)
    for key, obj in (("gemm_us", g), ("weights_us", StreamLoads(g, _native.STREAM_LOADS_WEIGHTS)),
                     ("weights_scales_us", StreamLoads(g, _native.STREAM_LOADS_SCALES)),
                     ("all_loads_us", StreamLoads(g, _native.STREAM_LOADS_ALL))):
        sec, _, _, _ = graph_timed(obj, steps, 16, warm_seconds=0.2, direct=True)
        res[key] = round(sec / steps * 1e6, 3)
    print(f"[bench] verify GEMM against its own loads: {res}", file=sys.stderr, flush=True)
    del g
    torch.cuda.empty_cache()
    return res


def mfma_probe():
    """Register-resident rate of the scaled MFMA the GEMMs issue (fp4 A x fp8 B), both shapes."""
    import torch
    from vllm_sly_radiance_amd import _native
    blocks, iters = 2048, 400
    out = torch.empty(blocks * 4, dtype=torch.float32, device="cuda")
    st = torch.cuda.current_stream()
    res = {}
    for shape, name in ((0, "16x16x128"), (1, "32x32x64")):
        _native.mfma_probe(shape, out.data_ptr(), blocks, 20, st.cuda_stream)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        flop = _native.mfma_probe(shape, out.data_ptr(), blocks, iters, st.cuda_stream)
        e1.record(st)
        torch.cuda.synchronize()
        res[name] = round(flop / (e0.elapsed_time(e1) * 1e-3) / 1e12, 1)
    return res


# the CPU baseline's configurations: (name, M, N, K, reps); reps 1 for the M = 4096 calls
CPU_CONFIGS = [("plumbing", 8, 5120, 5120, 5), ("verify", 8, 17408, 5120, 5),
               ("layer_qkv", 1, 10240, 5120, 5), ("layer_o_proj", 1, 5120, 6144, 5),
               ("layer_gate_up", 1, 17408, 5120, 5), ("layer_down", 1, 5120, 8704, 5),
               ("prefill_gate_up", 4096, 17408, 5120, 1), ("prefill_down", 4096, 5120, 8704, 1)]
# one layer of the 64-layer sweep at the M the other rows do not cover
CPU_SWEEP_M = [16, 64, 512]


def cpu_baseline():
    """The reference's CPU path, _exact_ref's dequant + fp32 matmul (sly/mxfp4/radiance_mxfp4.py:
    507-527) with _traced_quant in front (:392-396), restated in torch (oracle/torch_ref.py) and
    timed on this host's cores: quant, dequant and matmul separately, median of `reps` after one
    warm-up call, on every configuration at M <= 64, one M = 4096 call of gate_up and of down, and
    one layer of the sweep at M = 16, 64, 512. `value` is the verify GEMM's algorithmic bytes over
    its dequant + matmul time (activations already quantized, as for the GPU line)."""
    import torch
    from oracle import torch_ref as T
    from vllm_sly_radiance_amd import synthetic
    cores = os.cpu_count() or 1
    cores = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    torch.set_num_threads(cores)

    def med(fn, reps):
        fn()                                            # warm-up (allocations, thread pool)
        t = []
        for _ in range(reps):
            t0 = time.perf_counter()
            out = fn()
            t.append(time.perf_counter() - t0)
        return float(np.median(t)), out

    def one(M, N, K, reps, seed):
        x = torch.from_numpy(synthetic.activations(M, K, seed).view(np.int16)).view(torch.bfloat16)
        w, ws = synthetic.weights(N, K, seed + 1)
        w, ws = torch.from_numpy(w), torch.from_numpy(ws)
        tq, (q, s) = med(lambda: T.quant_per_token(x), reps)
        td, wd = med(lambda: T.dequant_weight(w, ws), reps)
        tm, _ = med(lambda: T.gemm(q, s, wd), reps)
        nb = gemm_bytes(M, N, K)
        return dict(M=M, N=N, K=K, reps=reps, quant_ms=round(tq * 1e3, 3),
                    dequant_ms=round(td * 1e3, 3), matmul_ms=round(tm * 1e3, 3),
                    gbs=round(nb / (td + tm) / 1e9, 3),
                    tflops=round(2.0 * M * N * K / (td + tm) / 1e12, 4))

    t_start = time.perf_counter()
    rows = {}
    for name, M, N, K, reps in CPU_CONFIGS:
        rows[name] = one(M, N, K, reps, seed=len(rows) + 1)
    sweep = {}
    for M in CPU_SWEEP_M:
        per = [one(M, N, K, 3, seed=100 + M) for _, N, K in LAYER_M1]
        sweep[M] = dict(ms_per_layer=round(sum(r["dequant_ms"] + r["matmul_ms"] for r in per), 2),
                        quant_ms_per_layer=round(sum(r["quant_ms"] for r in per), 3))
    layer = [rows[f"layer_{n}"] for n, _, _ in LAYER_M1]
    v = rows["verify"]
    return {"value": v["gbs"], "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"torch CPU dequant + fp32 matmul ({cores} threads) of the full M=8 N=17408 "
                      f"K=5120 GEMM, median of {v['reps']} after a warm-up: dequant "
                      f"{v['dequant_ms']} ms + matmul {v['matmul_ms']} ms (quant {v['quant_ms']} "
                      f"ms, not in value); the other configurations under 'configs'",
            "configs": rows,
            "layer_m1_ms": round(sum(r["dequant_ms"] + r["matmul_ms"] for r in layer), 2),
            "sweep_one_layer": sweep,
            "seconds": round(time.perf_counter() - t_start, 1)}


SWEEP_M = [1, 8, 16, 64, 512, 4096]
# the default run's sweep: 16 layers keep each shape's weight set (0.27-0.76 GB) above the 256 MB
# MALL, so no forward is served from the last-level cache; --sweep runs all 64
SWEEP_LAYERS_DEFAULT = 16
CROSSOVER_M = [8, 16, 17, 24, 32, 48, 64, 96, 128]


def _timed_graph(fn, reps, warm_seconds=0.2):
    """Capture fn() into a HIP graph on a side stream, replay it untimed for at least
    `warm_seconds` (and at least once), then `reps` times between events on that stream; returns
    ms per replay."""
    import torch
    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        fn()
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        t_end = time.perf_counter() + warm_seconds
        while True:
            graph.replay()
            torch.cuda.synchronize()
            if time.perf_counter() >= t_end:
                break
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / reps
    del graph
    return ms


def tiled_q(q):
    """Row-major e4m3 codes [M, K] (K % 128 == 0) -> the fragment-tiled bytes the producers write
    with Q_TILED: 16-token blocks, then k-tiles, then the two 64-byte halves, each 16 tokens x 4
    runs of 16 bytes in lane order (the last block's padding tokens zero)."""
    import torch
    M, K = q.shape
    Mp = -(-M // 16) * 16
    p = torch.zeros((Mp, K), dtype=torch.uint8, device=q.device)
    p[:M] = q.view(torch.uint8)
    return p.view(Mp // 16, 16, K // 128, 2, 4, 16).permute(0, 2, 3, 4, 1, 5).contiguous().view(-1)


def bench_sweep(n_layers):
    """64 stacked Qwen3.8-27B-shaped layers (qkv, o_proj, gate_up, down), random-init MXFP4
    checkpoint tensors generated on the device. Loads every linear through the plugin's
    process_weights_after_loading (the one-time repack, timed per layer), then times the linear
    part of a forward (per-token quant + GEMM per linear, through apply_weights as vLLM calls it)
    at each M, one HIP graph per shape over all layers. The crossover compares the decode
    kernels the plan uses up to M = 64 with the macro-tile kernel at the same M."""
    import torch
    from vllm_sly_radiance_amd import _native, radiance_mxfp4 as R, synthetic
    dev = torch.device("cuda", 0)
    R.ensure_scratch(dev)
    kern = R.kernel_class()()
    gen = torch.Generator(device=dev)
    gen.manual_seed(20251)
    layers = {name: [] for name, _, _ in LAYER_M1}
    repack_ms = []
    for _ in range(n_layers):
        t = 0.0
        for name, N, K in LAYER_M1:
            lin = torch.nn.Module()
            lin.weight = torch.nn.Parameter(
                torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=dev, generator=gen),
                requires_grad=False)
            lin.weight_scale = torch.nn.Parameter(
                torch.randint(synthetic.SCALE_LO, synthetic.SCALE_HI + 1, (N, K // 32),
                              dtype=torch.uint8, device=dev, generator=gen), requires_grad=False)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            kern.process_weights_after_loading(lin)
            e1.record()
            torch.cuda.synchronize()
            t += e0.elapsed_time(e1)
            layers[name].append(lin)
        repack_ms.append(t)
    weight_bytes = sum(N * K * 17 // 32 for _, N, K in LAYER_M1)
    print(f"[bench] sweep: {n_layers} layers loaded, {weight_bytes * n_layers / 1e9:.2f} GB of "
          f"repacked weights; repack {np.median(repack_ms):.3f} ms per layer (median)",
          file=sys.stderr, flush=True)

    xs = {}
    for K in sorted({K for _, _, K in LAYER_M1}):
        for M in SWEEP_M:
            x = synthetic.activations(M, K, 100 + M)
            xs[(M, K)] = torch.from_numpy(x.view(np.int16)).to(dev).view(torch.bfloat16)
    forward = []
    for M in SWEEP_M:
        per_shape = {}
        for name, N, K in LAYER_M1:
            x = xs[(M, K)]

            def fwd(x=x, name=name):
                for lin in layers[name]:
                    kern.apply_weights(lin, x)

            reps = 3 if M >= 512 else 10
            per_shape[name] = _timed_graph(fwd, reps)
        ms = sum(per_shape.values())
        flop = 2.0 * M * sum(N * K for _, N, K in LAYER_M1) * n_layers
        nbytes = n_layers * sum(gemm_bytes(M, N, K) for _, N, K in LAYER_M1)
        forward.append(dict(M=M, ms_per_forward=round(ms, 3),
                            us_per_layer=round(ms * 1e3 / n_layers, 2),
                            per_shape_us_per_layer={k: round(v * 1e3 / n_layers, 2)
                                                    for k, v in per_shape.items()},
                            tflops=round(flop / (ms * 1e-3) / 1e12, 1),
                            gbs=round(nbytes / (ms * 1e-3) / 1e9, 1),
                            plans={name: list(_native.plan(M, N, K)) for name, N, K in LAYER_M1}))
        print(f"[bench] sweep M={M}: {ms:.3f} ms per forward of {n_layers} layers "
              f"({forward[-1]['per_shape_us_per_layer']} us per layer)", file=sys.stderr,
              flush=True)

    # crossover: GEMM only (pre-quantized activations), up to 16 layers' weights rotating. The
    # decode family is the streaming kernel where it serves (M <= 16), else the pipelined ring
    # kernel with the fragments covering M (its first variant that serves the shape; a forced
    # plan, kept to show why the plan takes the tiles there), timed on row-major q and, as
    # ring_at_us, on the same codes fragment-tiled (contiguous 1 KiB activation loads instead of
    # 16 token rows x 64 bytes); the tile family is the macro tile the plan takes at M, or at
    # M = 17 below that, with the plan's K split (tile_split; tile_unsplit_us beside it). From 17
    # to 64 tokens band_us is the fastest band-kernel variant (weight waves and activation waves)
    # that serves the shape unsplit; where the plan takes the band kernel, plan_us is the plan.
    ring = _native.variants(_native.KERNEL_RING)
    band_cfg = _native.variants(_native.KERNEL_BAND)
    cross = {}
    for name, N, K in LAYER_M1:
        rows = []
        for M in CROSSOVER_M:
            q, sc = R.quant_per_token(xs[(4096, K)][:M].contiguous())
            out = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
            lins = layers[name][:16]
            per = len(lins)

            qt = tiled_q(q) if M <= 64 else q

            def run(kernel, variant, split, q=q, qt=qt, sc=sc, out=out, lins=lins, M=M):
                if kernel == _native.KERNEL_RING_AT:
                    q = qt
                for lin in lins:
                    _native.gemm(q.data_ptr(), sc.data_ptr(), lin.weight.data_ptr(),
                                 lin.weight_scale.data_ptr(), out.data_ptr(), M, N, K,
                                 torch.cuda.current_stream().cuda_stream, kernel, variant, split)

            k, v, sp = _native.plan(M, N, K)
            row = dict(M=M)
            if M > 16 and k == _native.KERNEL_BAND:
                # the plan takes the band kernel here; the tile beside it is the one the plan
                # takes otherwise (its tile rule is the same for 33 .. 64 tokens, so M = 64's plan
                # names it)
                row["plan_kernel"] = "band"
                row["plan_us"] = round(_timed_graph(
                    lambda: run(_native.KERNEL_AUTO, -1, 0), 5) * 1e3 / per, 2)
                tile_v, tile_sp = _native.plan(64, N, K)[1:]
            else:
                tile_v, tile_sp = (v, sp) if k == _native.KERNEL_TILE else \
                    _native.plan(max(M, 17), N, K)[1:]
            row["tile_us"] = round(_timed_graph(
                lambda: run(_native.KERNEL_TILE, tile_v, tile_sp), 5) * 1e3 / per, 2)
            if 16 < M <= 64:
                # every band variant that serves the shape unsplit; the fastest is reported
                band = []
                for bv in range(len(band_cfg)):
                    if _native.variant_serves(_native.KERNEL_BAND, bv, M, N, K, 1):
                        band.append((_timed_graph(lambda: run(_native.KERNEL_BAND, bv, 1), 5)
                                     * 1e3 / per, bv))
                if band:
                    t, bv = min(band)
                    row["band_us"] = round(t, 2)
                    row["band_variant"] = list(band_cfg[bv])
            if tile_sp > 1:
                # the plan splits K here: the same tile unsplit beside it
                row["tile_split"] = tile_sp
                row["tile_unsplit_us"] = round(_timed_graph(
                    lambda: run(_native.KERNEL_TILE, tile_v, 1), 5) * 1e3 / per, 2)
            if k != _native.KERNEL_STREAM and M <= 64:
                mf = -(-M // 16)
                k, sp = _native.KERNEL_RING, 1
                v = next((i for i, c in enumerate(ring) if c[0] == mf), None)
            if k != _native.KERNEL_TILE and v is not None:
                try:
                    row["decode_us"] = round(_timed_graph(lambda: run(k, v, sp), 5) * 1e3 / per,
                                             2)
                    row["decode_kernel"] = "stream" if k == _native.KERNEL_STREAM else "ring"
                    if k == _native.KERNEL_RING:
                        row["ring_at_us"] = round(_timed_graph(
                            lambda: run(_native.KERNEL_RING_AT, v, sp), 5) * 1e3 / per, 2)
                except RuntimeError:
                    pass
            rows.append(row)
        tile_wins = [r["M"] for r in rows if "decode_us" in r and r["tile_us"] <= r["decode_us"]]
        cross[name] = dict(rows=rows, tile_wins_from_M=min(tile_wins) if tile_wins else None)
        print(f"[bench] crossover {name}: {rows}", file=sys.stderr, flush=True)
    return dict(layers=n_layers, weight_gb=round(weight_bytes * n_layers / 1e9, 3),
                repack_ms_per_layer_median=round(float(np.median(repack_ms)), 4),
                repack_ms_total=round(float(np.sum(repack_ms)), 2), forward=forward,
                crossover=cross, plan_stream_max_M=16)


CALIBRATION_BYTES = 256 * 2 ** 20
# decode-band GEMMs in the counter runs: gate_up at M = 32, 48 and 64, qkv at M = 48 (the band
# kernel's two plan points), down at M = 17, 32, 48 and 64 (the plan splits down's K three ways up
# to M = 48)
BAND_PROFILE = [(32, 17408, 5120), (48, 17408, 5120), (64, 17408, 5120), (48, 10240, 5120),
                (17, 5120, 8704), (32, 5120, 8704), (48, 5120, 8704), (64, 5120, 8704)]


def profile_workload():
    """The launches the committed rocprofv3 summaries are taken on: the verify GEMM (the bench's
    graph replay: one second of warmup replays, then 64 timed launches over 16 weight copies,
    plus 64 event-bracketed single launches), each prefill GEMM (4 launches, then 4 more on
    fragment-tiled q behind its fused producer), gate_up at M = 32, 48 and 64, qkv at M = 48 and
    down at M = 17, 32, 48 and 64 (8 launches over 4 weight copies each), the four linears of the
    M = 1 layer set on bf16 activations as the op runs them (8 launches over 4 weight copies
    each), each fused
    producer and the quantizer at M = 4096 (4 launches over 2 input copies each) and a plain
    256 MiB device copy
    (torch's copy kernel), whose FETCH_SIZE / WRITE_SIZE readings calibrate the counters: a copy
    of B bytes fetches B and writes B."""
    import torch
    from vllm_sly_radiance_amd import radiance_mxfp4 as R
    R.ensure_scratch(torch.device("cuda", 0))
    st = torch.cuda.current_stream()
    M, N, K = VERIFY["M"], VERIFY["N"], VERIFY["K"]
    g = Gemm(M, N, K, COPIES, seed=1)
    graph_timed(g, 64, 16, direct=True)   # the bench's warm-up replays and timed launches
    del g
    for _, M, N, K in PREFILL:
        g = Gemm(M, N, K, 2, seed=7)
        for i in range(4):
            g.launch(i % 2, st.cuda_stream)
        torch.cuda.synchronize()
        del g
    from vllm_sly_radiance_amd import _native
    for name, M, N, K in PREFILL:                  # the same GEMMs on fragment-tiled q
        g = ProducerGemm(PREFILL_PRODUCER[name], M, N, K, 2, 7, _native.Q_TILED)
        for i in range(4):
            g.launch(i % 2, st.cuda_stream)
        torch.cuda.synchronize()
        del g
    for M, N, K in BAND_PROFILE:                   # the decode band above 16 tokens
        g = Gemm(M, N, K, 4, seed=9)
        for i in range(8):
            g.launch(i % 4, st.cuda_stream)
        torch.cuda.synchronize()
        del g
    for _, N, K in LAYER_M1:                       # the M = 1 layer set as the op runs it
        g = Gemm(1, N, K, 4, seed=3)
        lin = Linear(g)
        for i in range(8):
            lin.launch(i % 4, st.cuda_stream)
        torch.cuda.synchronize()
        del g, lin
    for kind, N in PRODUCERS:                      # the fused producers at M = 4096
        g = Producer(kind, 4096, N, 2, seed=21)
        for i in range(4):
            g.launch(i % 2, st.cuda_stream)
        torch.cuda.synchronize()
        del g
    for M, K in QUANT_SHAPES[1:]:                  # the quantizer at M = 4096
        g = Quant(M, K, 2, seed=31)
        for i in range(4):
            g.launch(i % 2, st.cuda_stream)
        torch.cuda.synchronize()
        del g
    torch.cuda.empty_cache()
    src = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    print(f"[bench] profile workload done (calibration copy {CALIBRATION_BYTES} B)",
          file=sys.stderr)


def measured_traffic(kernel_prefix):
    """HBM bytes per launch of the verify GEMM from the committed counter summary, or None."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            t = json.load(f)
        k = t["kernels"][kernel_prefix]
        return int(round(k["fetch_bytes"] + k["write_bytes"]))
    except (OSError, KeyError, ValueError):
        return None


def measured_mfma_util(kernel_key):
    """MFMA-busy fraction (SQ_VALU_MFMA_BUSY_CYCLES over active cycles, rocprofv3) of a prefill
    GEMM's two launches and the clock they ran at, from the committed counter summary, or None:
    counters need their own profiler run, so the bench reports the committed measurement."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            k = json.load(f)["kernels"][kernel_key]
        return dict(main=k["mfma_util_main"], tail=k["mfma_util_tail"],
                    clock_ghz_main=k["clock_ghz_main"],
                    source="profiles/traffic.json (rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES "
                           "GRBM_GUI_ACTIVE)")
    except (OSError, KeyError, ValueError):
        return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box here has one, and this path is a single-GPU "
              f"kernel (sharding is described, not run). Got --gpus {args.gpus}.",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    from vllm_sly_radiance_amd import radiance_mxfp4 as R
    if args.profile:
        profile_workload()
        return
    R.ensure_scratch(torch.device("cuda", 0))
    if args.sweep:
        sw = bench_sweep(args.sweep_layers)
        print(json.dumps({"metric": "64-layer MXFP4 W4A8 linear sweep, ms per forward",
                          "n_gpus": 1, "data": "synthetic, random-init layers",
                          "config": {"workload": "Qwen3.8-27B-shaped linear set x "
                                                 f"{args.sweep_layers} layers",
                                     "M": SWEEP_M}, "sweep": sw}), flush=True)
        return
    v = bench_verify(args)
    print(f"[bench] verify M=8: {v['kernel_us']:.2f} us/launch in the graph-timed region, "
          f"event pairs {v['event_pair_us_median']:.2f} us median, plan {v['plan']}",
          file=sys.stderr, flush=True)
    prefill = layer = producers = quant = sweep = None
    if not args.only_verify:
        prefill = bench_prefill()
        print(f"[bench] prefill: {prefill}", file=sys.stderr, flush=True)
        layer = bench_layer_m1()
        print(f"[bench] M=1 layer: {layer}", file=sys.stderr, flush=True)
        producers = bench_producers()
        print(f"[bench] producers: {producers}", file=sys.stderr, flush=True)
        quant = bench_quant()
        print(f"[bench] quantizer: {quant}", file=sys.stderr, flush=True)
        sweep = bench_sweep(SWEEP_LAYERS_DEFAULT)
    probe = mfma_probe()
    print(f"[bench] MFMA probe TFLOP/s: {probe}", file=sys.stderr, flush=True)
    rprobe = bench_read_probe(args.steps, args.warmup)
    print(f"[bench] HBM read probe (verify-GEMM shape and bytes): {rprobe}", file=sys.stderr,
          flush=True)
    cpu = None if args.no_cpu else cpu_baseline()
    achieved = v["bytes"] / (v["kernel_us"] * 1e-6) / 1e9
    line = {
        "metric": METRIC,
        "value": round(v["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": v["steps"],
        "warmup": v["warmup"],
        "clock_warmup": v["clock_warmup"],
        "ms_per_step": round(v["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3 x fp4e2m1 (e8m0 block scales), fp32 accumulate, bf16 out",
        "data": "synthetic (bf16 N(0,1) activations with 0.1% x20 outliers; uniform e2m1 codes; "
                "e8m0 exponents uniform in [119, 125])",
        "config": {"workload": "speculative-verify decode W4A8 GEMM M=8 N=17408 K=5120",
                   "M": 8, "N": 17408, "K": 5120, "weight_copies": COPIES,
                   "plan": list(v["plan"])},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("verify"),
                     "traffic_source": "profiles/traffic.json (rocprofv3 --pmc FETCH_SIZE, then "
                                       "WRITE_SIZE, of bench.py --profile; not measured in this "
                                       "run)"},
        "cpu_baseline": cpu,
        "kernel_us": round(v["kernel_us"], 3),
        "event_pair_us_median": round(v["event_pair_us_median"], 3),
        "prefill_m4096": prefill,
        "mfma_probe_tflops": probe,
        "hbm_read_probe": rprobe,
        "value_vs_read_probe": round(v["gbs"] / rprobe["gbs"], 4),
        "value_vs_best_read_shape": round(v["gbs"] / rprobe["best"]["gbs"], 4),
        "decode_m1_layer": layer,
        "producers": producers,
        "quantizer": quant,
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
