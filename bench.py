#!/usr/bin/env python3
"""GRINQH quantized-linear benchmark on one MI355X.

Workload (the decode sweep): Llama-3-8B linear shapes
qkv 4096->6144, o_proj 4096->4096, gate_up 4096->28672, down 14336->4096 at
M in {1, 4, 16, 64}; fp16 activations N(0,1) with 1 % of channels x20; weights
0.02*N(0,1) RTN-quantised to int8 codes per 128-row group with fp16 scales;
union grading with thresholds [0, P50, P80, P95] of sigma_k = max_m |x[m,k]|.
One step = the 16 products once.

HBM-cold timing: every shape has a pool of weight copies of at least 3 GiB,
handed out least recently used first, so that no timed product reads a weight
copy that was read less than ~0.9 GB of weight traffic earlier (the MI355X
MALL holds 256 MB).  The smallest distance actually seen between two reads
of one copy, in bytes the products touched, is reported in ``config``.

value = whole-step HBM throughput in algorithmic bytes (planes actually needed
by the grading + scales + x + y) per second.  The JSON line also carries the
per-case product times, the roofline of the dominant kernel, the prefill
TFLOP/s at M=2048 (dense, the reference's dispatch for M > 1), the graded
prefill sweep of BASELINE configs[2] (M = 512, 2048, 8192, 70/20/8/2 % grade
mix), the M=2048 products without the library path (allocation-free entry
point: the hand-written large-batch kernel instead of the dense weight and the
library GEMM), the Llama-3-70B shapes of BASELINE configs[4] with every zone
active (M = 1, 64, 4096) and the CPU baseline (the reference's pure-PyTorch
math on the host cores).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "vllm-grinqh-plugin_amd"))
sys.path.insert(0, REPO)

METRIC = "GEMM TFLOP/s + HBM GB/s (% roofline) at Llama-3-8B shapes, M=1/16/2048"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
SHAPES = [("qkv", 4096, 6144), ("o_proj", 4096, 4096), ("gate_up", 4096, 28672), ("down", 14336, 4096)]
DECODE_M = [1, 4, 16, 64]
PREFILL_M = 2048
PREFILL_GRADED_M = (512, 2048, 8192)
# Llama-3-70B linear shapes, M in {1, 64, 4096}, every zone active
SHAPES_70B = [("qkv", 8192, 10240), ("gate_up", 8192, 57344), ("down", 28672, 8192)]
M_70B = (1, 64, 4096)
GS = 128
BITS = 8
MALL_BYTES = 256 << 20
POOL_BYTES = 3 << 30  # weight copies per shape: at least this many bytes


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def synth_weight(torch, K: int, N: int, seed: int, device):
    """0.02*N(0,1) weights, symmetric RTN per 128-row group to int8 codes with
    fp16 scales, in the loader's [K, N] / [K/128, N] layout."""
    g = torch.Generator(device=device).manual_seed(seed)
    wf = 0.02 * torch.randn((N, K), generator=g, device=device, dtype=torch.float32)
    wg = wf.view(N, K // GS, GS)
    lim = (1 << (BITS - 1)) - 1
    s = (wg.abs().amax(-1) / lim).clamp_min(1e-8).half()
    q = torch.clamp(torch.round(wg / s.float().unsqueeze(-1)), -lim - 1, lim).to(torch.int8)
    return q.view(N, K).t().contiguous(), s.t().contiguous()


def synth_x(torch, M: int, K: int, seed: int, device):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn((M, K), generator=g)
    out = torch.randperm(K, generator=g)[: math.ceil(K / 100)]
    x[:, out] *= 20
    return x.half().to(device)


def thresholds_for(x, q=(0.5, 0.8, 0.95)):
    sigma = x.abs().float().amax(0).cpu().numpy()
    return [0.0] + [float(v) for v in np.quantile(sigma, q)]


def prefill_kernel_name(M, K, N, mode, noalloc=False):
    """The kernel the dispatch picks for an fp16 product of this shape."""
    from grinqh import _lib
    kern, rows, splits = _lib.product_kernel(M, K, K, N, _lib.DTYPE_F16, BITS, GS,
                                             _lib.MODE_UNION if mode == "union" else _lib.MODE_DENSE, noalloc)
    name = _lib.KERNEL_NAMES[kern]
    return f"{name} ({rows}-row blocks, {splits} K ranges)" if kern == _lib.KERNEL_TALL else name


def library_free_product(torch, lib, x, P, s, t, mode):
    """One product through grinqh_gemm_or_gemv_noalloc (include/grinqh.h): no
    workspace, so no dense weight for the library GEMM; batches of 256 rows
    and more run the hand-written large-batch kernel (prefill_tall_kernel)
    where its shape rules allow, else the fused prefill kernel."""
    from grinqh import _lib
    M, K = x.shape
    N = s.shape[1]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    rc = lib.grinqh_gemm_or_gemv_noalloc(
        x.data_ptr(), M, K, x.stride(0), N, _lib.DTYPE_F16, P.data_ptr(), s.data_ptr(), None, y.data_ptr(), BITS,
        GS, _lib.thresholds_f32(t), _lib.MODE_UNION if mode == "union" else _lib.MODE_DENSE,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "grinqh_gemm_or_gemv_noalloc")
    return y


class ColdRotation:
    """Least-recently-used hand-out of weight copies with exact accounting of
    the bytes the products touch between two reads of one copy.

    ``take(shape, touched)`` returns the next copy of ``shape`` (round robin
    over its pool) for a product that touches ``touched`` bytes.  A graph
    replays the takes made while it was captured, so after capturing a
    sequence that is replayed cyclically, ``replay(takes)`` runs the same
    sequence through the accounting once more: the distances it records are
    the ones every timed replay sees, including the wrap from the end of the
    sequence back to its start."""

    def __init__(self, pools):
        self.pools = pools
        self.next = {k: 0 for k in pools}
        self.clock = 0
        self.last = {}
        self.min_gap = None
        self.log = None

    def _use(self, key, touched):
        if key in self.last:
            gap = self.clock - self.last[key]
            self.min_gap = gap if self.min_gap is None else min(self.min_gap, gap)
        self.clock += touched
        self.last[key] = self.clock

    def take(self, shape, touched):
        i = self.next[shape]
        self.next[shape] = (i + 1) % len(self.pools[shape])
        self._use((shape, i), touched)
        if self.log is not None:
            self.log.append(((shape, i), touched))
        return self.pools[shape][i]

    def record(self):
        self.log = []

    def stop(self):
        takes, self.log = self.log, None
        return takes

    def replay(self, takes):
        for key, touched in takes:
            self._use(key, touched)


def make_pool(base, nbytes_each: int, multiple: int = 4):
    """``base`` plus clones: at least POOL_BYTES in all, a multiple of ``multiple`` copies."""
    n = max(multiple, multiple * math.ceil(POOL_BYTES / (multiple * nbytes_each)))
    return [base] + [tuple(t.clone() for t in base) for _ in range(n - 1)]


def graph_time_us(torch, stream, call, n_it: int, replays: int = 3) -> float:
    """Per-call GPU time of call(0) .. call(n_it - 1) captured in one HIP graph
    and replayed `replays` times between two events, so the host's launch cost
    (Python, ctypes, the GEMM library's host side) is not counted: the time of
    the products themselves.  Two eager calls first size the workspace and
    plan the library GEMM."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        for j in range(2):
            call(j)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for j in range(n_it):
                call(j)
        g.replay()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(replays):
            g.replay()
        e1.record(stream)
    e1.synchronize()
    return e0.elapsed_time(e1) * 1e3 / (replays * n_it)


def decode_bytes(bits_per_row, K, N, M):
    planes = int(bits_per_row.sum()) * (N // 4)
    return planes + (K // GS) * N * 2 + M * K * 2 + M * N * 2


def kernel_name(M: int, Z: int, dtype: str = "F16", graded: bool = True) -> str:
    """Kernel instantiation a decode-sweep product of M rows runs (mirrors the
    library's dispatch: GEMV kernel up to 4 rows, decode kernel above)."""
    dense = "false" if graded else "true"
    if M <= 4:
        return f"gemv_kernel<{dtype},{1 if M == 1 else 4},{Z},{dense}>"
    mt = 1 if M <= 16 else (2 if M <= 32 else 4)
    return f"decode_kernel<{dtype},{mt},{Z},{dense}>"


def traffic_for(kernel: str):
    """HBM bytes per launch of `kernel` measured with rocprofv3 --pmc
    FETCH_SIZE / WRITE_SIZE (scaled by a copy-kernel calibration), read from
    the 'traffic:' lines of profiles/*.md; None when not measured."""
    prof = os.path.join(REPO, "profiles")
    if not os.path.isdir(prof):
        return None
    for f in sorted(os.listdir(prof)):
        if not f.endswith(".md"):
            continue
        with open(os.path.join(prof, f)) as fh:
            for line in fh:
                parts = line.strip().strip("`").split()
                if len(parts) == 3 and parts[0] == "traffic:" and parts[1] == kernel:
                    return int(parts[2])
    return None


def llama8b_decode_step(torch, dev, stream, batch: int = 32, layers: int = 32, replays: int = 5):
    """One-GPU stand-in for BASELINE configs[3] (not the vLLM end-to-end run):
    the 128 GRINQH linears of a Llama-3-8B decode step at ``batch`` tokens --
    per layer qkv_proj 4096->6144, o_proj 4096->4096, gate_up_proj
    4096->28672 and down_proj 14336->4096, every layer with weights of its own
    (7 GB of planes, so every read comes from HBM) -- through
    torch.ops.grinqh.gemm_or_gemv, with the glue that feeds them (RMSNorm,
    residual adds, SiLU(gate)*up; attention is replaced by the query part of
    the qkv output) in torch.  Per-layer thresholds are calibrated on the
    step's own activations (P50/P80/P95 of each layer's statistic, zone 0 at
    0.0) with grinqh.thresholds.  The whole step is captured in one HIP graph
    per grading mode; the 128 linears alone, on the inputs the step produces,
    in another."""
    from grinqh import kernel as gk
    from grinqh.producer import gemv_batch_union_sigma, rmsnorm_sigma, silu_mul_sigma
    from grinqh.thresholds import StatsRecorder, llama_prefixes, thresholds_from_statistics
    from grinqh.utils import grade, prepare_weight
    H, F = 4096, 14336
    shapes = {"self_attn.qkv_proj": (H, 6144), "self_attn.o_proj": (H, H), "mlp.gate_up_proj": (H, 2 * F),
              "mlp.down_proj": (F, H)}
    prefixes = llama_prefixes(layers)
    W = {}
    for i, pfx in enumerate(prefixes):
        K, N = shapes[pfx.split(".", 3)[3]]
        w, s = synth_weight(torch, K, N, 5000 + i, dev)
        W[pfx] = (prepare_weight(w, BITS), s, K, N)
        del w
    norm_w = torch.ones(H, device=dev, dtype=torch.float16)

    def rmsnorm(h):
        hf = h.float()
        return (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-5)).half() * norm_w

    thr = {pfx: [-1.0] * 4 for pfx in prefixes}
    inputs = {}

    def linear(pfx, x):
        P, s, K, N = W[pfx]
        inputs[pfx] = x
        return torch.ops.grinqh.gemm_or_gemv(x, P, s, None, BITS, GS, N // 4, thr[pfx])

    def step(h):
        for li in range(layers):
            base = f"model.layers.{li}."
            qkv = linear(base + "self_attn.qkv_proj", rmsnorm(h))
            h = h + linear(base + "self_attn.o_proj", qkv[:, :H].contiguous())
            gu = linear(base + "mlp.gate_up_proj", rmsnorm(h))
            h = h + linear(base + "mlp.down_proj", (torch.nn.functional.silu(gu[:, :F].float()) * gu[:, F:].float()).half())
        return h

    def linear_sig(pfx, x, sig):
        P, s, K, N = W[pfx]
        inputs[pfx] = x
        return gemv_batch_union_sigma(x, P, s, None, BITS, GS, N // 4, thr[pfx], sig)

    def step_fused(h):
        """Union grading with producer fusion: the RMSNorms (residual add
        included) and SiLU*mul emit the statistic their consumer grades on."""
        hn, sig, _ = rmsnorm_sigma(h, norm_w)
        res = h
        for li in range(layers):
            base = f"model.layers.{li}."
            qkv = linear_sig(base + "self_attn.qkv_proj", hn, sig)
            o = linear(base + "self_attn.o_proj", qkv[:, :H].contiguous())
            hn, sig, res = rmsnorm_sigma(o, norm_w, 1e-5, res)
            gu = linear_sig(base + "mlp.gate_up_proj", hn, sig)
            a, asig = silu_mul_sigma(gu)
            d = linear_sig(base + "mlp.down_proj", a, asig)
            hn, sig, res = rmsnorm_sigma(d, norm_w, 1e-5, res)
        return res

    h0 = synth_x(torch, batch, H, 77, dev) * 0.05
    out = {"batch": batch, "layers": layers, "linears": len(prefixes),
           "note": "stand-in for BASELINE configs[3]: the quantized linears of a Llama-3-8B decode step on one "
                   "GPU with torch glue and no attention; the vLLM end-to-end run was not done"}
    saved = gk.batch_grading_mode()
    try:
        gk.set_batch_grading_mode("reference")
        with torch.cuda.stream(stream):
            step(h0)  # calibration pass (dense, reference dispatch)
            torch.cuda.synchronize()
        rec = StatsRecorder()
        for pfx in prefixes:
            rec.update(pfx, inputs[pfx])
        calibrated = thresholds_from_statistics({p: rec.samples(p) for p in prefixes})
        for mode in ("reference", "union", "union_fused"):
            gk.set_batch_grading_mode("reference" if mode == "reference" else "union")
            thr.update(calibrated)
            fn = step_fused if mode == "union_fused" else step
            with torch.cuda.stream(stream):
                fn(h0)
                torch.cuda.synchronize()
                g_step = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g_step, stream=stream):
                    fn(h0)
                g_step.replay()  # fills the captured step's tensors, the linears' inputs among them
                torch.cuda.synchronize()
                xs = {p: inputs[p].clone() for p in prefixes}
                sigs = {}
                if mode == "union_fused":  # each graded input's chunk maxima, as its producer gives them
                    for p in prefixes:
                        if not p.endswith("o_proj"):
                            xv = xs[p].float().abs()
                            sigs[p] = torch.stack([xv[c:c + 16].amax(0) for c in range(0, batch, 16)])
                g_lin = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g_lin, stream=stream):
                    for p in prefixes:  # the linears alone (union_fused: each with its statistic given)
                        P, s, K, N = W[p]
                        if mode == "union_fused" and p in sigs:
                            gemv_batch_union_sigma(xs[p], P, s, None, BITS, GS, N // 4, thr[p], sigs[p])
                        else:
                            torch.ops.grinqh.gemm_or_gemv(xs[p], P, s, None, BITS, GS, N // 4, thr[p])
                times = {}
                for name, g in (("step", g_step), ("linears", g_lin)):
                    g.replay()
                    torch.cuda.synchronize()
                    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    for _ in range(replays):
                        g.replay()
                    e1.record(stream)
                    e1.synchronize()
                    times[name] = e0.elapsed_time(e1) * 1e3 / replays
            nbytes = 0
            for p in prefixes:
                P, s, K, N = W[p]
                if mode != "reference":
                    zb, _ = grade(xs[p], thr[p], BITS)
                    planes = int(np.unpackbits(zb.cpu().numpy()[:, None], axis=1).sum()) * (N // 4)
                else:
                    planes = K * N * BITS // 8
                nbytes += planes + (K // GS) * N * 2 + batch * (K + N) * 2
            out[mode] = {"step_us": round(times["step"], 1), "linears_us": round(times["linears"], 1),
                         "linear_bytes": nbytes, "linears_gbs": round(nbytes / (times["linears"] * 1e-6) / 1e9, 1),
                         "frac_of_hbm": round(nbytes / (times["linears"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
            log(f"llama-3-8b decode step batch {batch} ({mode}): step {times['step']:.0f} us, 128 linears "
                f"{times['linears']:.0f} us, {out[mode]['linears_gbs']:.0f} GB/s")
            del g_step, g_lin, xs
    finally:
        gk.set_batch_grading_mode(saved)
    del W
    torch.cuda.empty_cache()
    return out


def touched_bytes(rec) -> int:
    """Weight bytes a product reads: the planes its grading needs and the scales."""
    return rec["bytes"] - rec["M"] * rec["K"] * 2 - rec["M"] * rec["N"] * 2


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--reps", type=int, default=20, help="eager launches per case for the kernel-event timing")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-70b", action="store_true", help="skip the Llama-3-70B shape sweep (BASELINE configs[4])")
    ap.add_argument("--no-model-step", action="store_true",
                    help="skip the Llama-3-8B decode-step stand-in (BASELINE configs[3])")
    ap.add_argument("--prefill-case", default=None, metavar="SHAPE:M:MODE[:noalloc]",
                    help="profiling run: one prefill product (e.g. gate_up:2048:union; MODE dense or union with "
                         "t = [0, P70, P90, P98]; ':noalloc' through the allocation-free entry point, i.e. without "
                         "the library path) twice as warm-up and twice counted; prints no JSON line")
    ap.add_argument("--no-library-free", action="store_true",
                    help="skip the prefill products through the allocation-free entry point (no library path)")
    ap.add_argument("--pmc-pass", action="store_true",
                    help="counter-collection run: each decode case twice (eager, cold weight copies) and a 256 MiB "
                         "copy kernel of known traffic for calibrating FETCH_SIZE / WRITE_SIZE; prints no JSON line")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this build runs on one GPU only: the GRINQH hot path has no sharded path "
                                   "(one process, one MI355X); run with --gpus 1"}))
        return 2

    import torch
    from grinqh import _lib
    from grinqh.kernel import run_product
    from grinqh.utils import grade, prepare_weight

    _lib.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    log(f"device {torch.cuda.get_device_name(dev)}")

    if args.prefill_case:
        name, m_str, mode, *path = args.prefill_case.split(":")
        K, N = {n: (k, nn) for n, k, nn in SHAPES}[name]
        M = int(m_str)
        w, s = synth_weight(torch, K, N, 1000, dev)
        P = prepare_weight(w, BITS)
        x = synth_x(torch, M, K, 5, dev)
        t = thresholds_for(x, (0.7, 0.9, 0.98)) if mode == "union" else [0.0] * 4
        if path == ["noalloc"]:
            lib = _lib.load_library()
            call = lambda: library_free_product(torch, lib, x, P, s, t, mode)
        else:
            call = lambda: run_product(x, P, s, None, BITS, GS, N // 4, t, mode)
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            call()
        e1.record()
        e1.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / 10
        # the main kernel alone: events the dispatch records around its launch
        lib = _lib.load_library()
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(5)]
        for a, b in pairs:
            a.record()
            b.record()
        torch.cuda.synchronize()
        for a, b in pairs:
            _lib.check(lib.grinqh_time_next_product(ctypes.c_void_p(a.cuda_event), ctypes.c_void_p(b.cuda_event)),
                       "grinqh_time_next_product")
            call()
        torch.cuda.synchronize()
        k_us = float(np.mean([a.elapsed_time(b) * 1e3 for a, b in pairs]))
        kern, wm, splits = _lib.product_kernel(M, K, K, N, _lib.DTYPE_F16, BITS, GS,
                                               _lib.MODE_UNION if mode == "union" else _lib.MODE_DENSE,
                                               noalloc=path == ["noalloc"])
        log(f"prefill case {args.prefill_case}: {us:.1f} us {2 * M * K * N / us / 1e6:.1f} TFLOP/s; "
            f"main kernel {_lib.KERNEL_NAMES[kern]} (wm {wm}, splits {splits}) {k_us:.1f} us "
            f"{2 * M * K * N / k_us / 1e6:.1f} TFLOP/s")
        return 0

    # ---------------- weights: a pool of >= POOL_BYTES of copies per shape, handed out LRU
    pools = {}
    for i, (name, K, N) in enumerate(SHAPES):
        w, s = synth_weight(torch, K, N, 1000 + i, dev)
        base = (prepare_weight(w, BITS), s)
        del w
        pools[name] = make_pool(base, base[0].numel() * 4 + s.numel() * 2)
    rot = ColdRotation(pools)
    copies_per_shape = {n: len(p) for n, p in pools.items()}
    log("weight pools: " + ", ".join(f"{n} {len(p)} copies" for n, p in pools.items()))

    # ---------------- cases
    cases = []
    for i, (name, K, N) in enumerate(SHAPES):
        for M in DECODE_M:
            x = synth_x(torch, M, K, 17 * i + M, dev)
            t = thresholds_for(x)
            zb, _ = grade(x, t, BITS)
            bits = np.unpackbits(zb.cpu().numpy()[:, None], axis=1).sum(1)
            c = dict(shape=name, K=K, N=N, M=M, x=x, t=t, bytes=decode_bytes(bits, K, N, M),
                     mean_planes=float(bits.mean()))
            c["touched"] = touched_bytes(c)
            cases.append(c)

    def call(c):
        p, s = rot.take(c["shape"], c["touched"])
        return run_product(c["x"], p, s, None, BITS, GS, c["N"] // 4, c["t"], "union")

    stream = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for c in cases:  # size the per-stream workspace before any capture
            call(c)
    torch.cuda.synchronize()

    if args.pmc_pass:
        with torch.cuda.stream(stream):
            for c in cases:
                for r in range(2):
                    call(c)
                torch.cuda.synchronize()
                log(f"pmc pass: {c['shape']} M={c['M']} kernel {kernel_name(c['M'], BITS // 2)} "
                    f"bytes {c['bytes']}")
            src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
            dst = torch.empty_like(src)
            torch.neg(src, out=dst)  # calibration: reads and writes exactly 256 MiB
            torch.cuda.synchronize()
        log("pmc pass: calibration kernel (torch.neg, 256 MiB in, 256 MiB out) done")
        return 0

    # per-case product time: one graph with one launch per copy of the shape's
    # pool, so that every replay reads each copy once and a copy is re-read
    # only after the rest of the pool (>= 2 GiB of copies) has been read
    rot.min_gap = None
    for c in cases:
        reps = len(pools[c["shape"]])
        g = torch.cuda.CUDAGraph()
        rot.record()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                for _ in range(reps):
                    call(c)
        rot.replay(rot.stop())
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for _ in range(3):
                g.replay()
            e1.record(stream)
        e1.synchronize()
        c["us"] = e0.elapsed_time(e1) * 1e3 / (3 * reps)
        c["gbs"] = c["bytes"] / (c["us"] * 1e-6) / 1e9
        log(f"{c['shape']:8s} M={c['M']:3d} planes/row={c['mean_planes']:.2f} {c['bytes'] / 1e6:7.2f} MB "
            f"{c['us']:8.2f} us {c['gbs']:8.1f} GB/s ({100 * c['gbs'] / HBM_PEAK_GBS:.1f}% HBM)")
        del g

    # ---------------- the step: graphs of the 16 products, each product on its
    # own weight copy; enough graphs that every copy of the largest pool is
    # used once per cycle of replays
    n_graphs = max(len(p) for p in pools.values()) // len(DECODE_M)
    step_graphs = []
    rot.record()
    for r in range(n_graphs):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                for c in cases:
                    call(c)
        step_graphs.append(g)
    rot.replay(rot.stop())
    for i in range(max(args.warmup, n_graphs)):
        step_graphs[i % n_graphs].replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for i in range(args.steps):
            step_graphs[i % n_graphs].replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = e0.elapsed_time(e1) / args.steps
    step_bytes = sum(c["bytes"] for c in cases)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"step {ms_per_step * 1e3:.1f} us  {value:.1f} GB/s  (wall {wall:.3f} s, {n_graphs} step graphs)")
    del step_graphs

    # ---------------- kernel timing: HIP events that the dispatch of each
    # product's main kernel records as the kernel starts and ends (the
    # library launches it with hipExtLaunchKernelGGL), on the stream the
    # kernel runs on: its execution alone, without the split-K reduction
    lib = _lib.load_library()
    ev_pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                for _ in range(args.reps)]
    with torch.cuda.stream(stream):
        for a, b in ev_pairs:  # materialise the events before handing them over
            a.record(stream)
            b.record(stream)
    torch.cuda.synchronize()
    for c in cases:
        with torch.cuda.stream(stream):
            for a, b in ev_pairs:
                _lib.check(lib.grinqh_time_next_product(ctypes.c_void_p(a.cuda_event), ctypes.c_void_p(b.cuda_event)),
                           "grinqh_time_next_product")
                call(c)
        torch.cuda.synchronize()
        c["kernel_us"] = float(np.mean([a.elapsed_time(b) * 1e3 for a, b in ev_pairs]))
        c["kernel"] = kernel_name(c["M"], BITS // 2)
    decode_min_gap = rot.min_gap
    kernels = {}
    for c in cases:
        k = kernels.setdefault(c["kernel"], {"launches_per_step": 0, "bytes": 0, "us": 0.0})
        k["launches_per_step"] += 1
        k["bytes"] += c["bytes"]
        k["us"] += c["kernel_us"]
    for name, k in kernels.items():
        k["avg_launch_us"] = round(k["us"] / k["launches_per_step"], 3)
        k["bytes_per_launch"] = int(k["bytes"] / k["launches_per_step"])
        k["achieved_gbs"] = round(k["bytes"] / (k["us"] * 1e-6) / 1e9, 1)
        k["frac"] = round(k["achieved_gbs"] / HBM_PEAK_GBS, 4)
        k["share_of_step"] = round(k["us"] * 1e-3 / ms_per_step, 4)
        log(f"{name:40s} x{k['launches_per_step']} avg {k['avg_launch_us']:8.2f} us "
            f"{k['achieved_gbs']:8.1f} GB/s ({100 * k['frac']:.1f}% HBM) share {100 * k['share_of_step']:.1f}%")
    dom_name = max(kernels, key=lambda n: kernels[n]["us"])
    dom = kernels[dom_name]
    roofline = {"bound": "hbm", "achieved": dom["achieved_gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": dom["frac"], "traffic": traffic_for(dom_name), "kernel": "grinqh::" + dom_name,
                "bytes_per_launch": dom["bytes_per_launch"], "avg_launch_us": dom["avg_launch_us"]}
    for k in kernels.values():
        del k["us"], k["bytes"]

    def prefill_time_us(name, K, N, M, x, t, mode, n_it):
        """Graph-timed product on rotated copies (every plane fetched counts as
        touched); at least n_it launches and at most one per copy of the pool,
        so that a replay reads each copy once."""
        touched = K * N * BITS // 8 + (K // GS) * N * 2
        n_it = min(len(pools[name]), max(n_it, math.ceil((1 << 30) / touched)))
        rot.record()
        us = graph_time_us(torch, stream, lambda j: run_product(
            x, *rot.take(name, touched), None, BITS, GS, N // 4, t, mode), n_it)
        rot.replay(rot.stop()[2:])  # the captured calls (the two eager sizing calls are not replayed)
        return us

    # ---------------- prefill at M=2048 (dense dequantize-then-matmul, reference dispatch for M>1)
    rot.min_gap = None
    prefill = None
    if not args.no_prefill:
        prefill = []
        for i, (name, K, N) in enumerate(SHAPES):
            x = synth_x(torch, PREFILL_M, K, 99 + i, dev)
            us = prefill_time_us(name, K, N, PREFILL_M, x, [0.0] * 4, "dense", 5)
            tf = 2.0 * PREFILL_M * K * N / (us * 1e-6) / 1e12
            kern = prefill_kernel_name(M=PREFILL_M, K=K, N=N, mode="dense")
            prefill.append({"shape": name, "M": PREFILL_M, "us": round(us, 2), "tflops": round(tf, 1),
                            "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "kernel": kern})
            log(f"prefill {name:8s} M={PREFILL_M} {us:9.1f} us {tf:7.1f} TFLOP/s ({kern})")

    # ---------------- graded prefill sweep: union grading with the
    # 70/20/8/2% grade mix (t = [0, P70, P90, P98] of the batch statistic)
    prefill_graded = None
    if not args.no_prefill:
        prefill_graded = []
        for i, (name, K, N) in enumerate(SHAPES):
            for M in PREFILL_GRADED_M:
                x = synth_x(torch, M, K, 199 + i, dev)
                t = thresholds_for(x, (0.7, 0.9, 0.98))
                us = prefill_time_us(name, K, N, M, x, t, "union", 3)
                tf = 2.0 * M * K * N / (us * 1e-6) / 1e12
                kern = prefill_kernel_name(M=M, K=K, N=N, mode="union")
                prefill_graded.append({"shape": name, "M": M, "us": round(us, 2), "tflops": round(tf, 1),
                                       "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4), "kernel": kern})
                log(f"prefill graded {name:8s} M={M:5d} {us:9.1f} us {tf:7.1f} TFLOP/s ({kern})")
                del x
    # MFMA leg of the metric (M=2048): the largest product, gate_up, priced on
    # its whole graph-timed time (the default dispatch at 2048 rows: the
    # dequantization pass + library GEMM)
    roofline_prefill = None
    if prefill:
        g = max(prefill, key=lambda r: r["us"])
        roofline_prefill = {"bound": "mfma", "achieved": g["tflops"], "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
                            "frac": g["frac"], "traffic": None, "shape": g["shape"], "M": g["M"], "kernel": g["kernel"],
                            "measured": "graph-timed product, rotated weights"}

    # ---------------- the same products without the library path (allocation-free
    # entry point: no dense weight; the hand-written large-batch kernel
    # prefill_tall_kernel wherever its repacked x fits the fixed scratch),
    # eager, rotated copies
    prefill_library_free = None
    if not args.no_prefill and not args.no_library_free:
        prefill_library_free = []
        lib = _lib.load_library()
        for i, (name, K, N) in enumerate(SHAPES):
            for M, mode in ((PREFILL_M, "dense"), (PREFILL_M, "union")):
                x = synth_x(torch, M, K, 299 + i, dev)
                t = thresholds_for(x, (0.7, 0.9, 0.98)) if mode == "union" else [0.0] * 4
                touched = K * N * BITS // 8 + (K // GS) * N * 2
                n_it = min(len(pools[name]), 8)
                for _ in range(2):
                    P, sc = rot.take(name, touched)
                    library_free_product(torch, lib, x, P, sc, t, mode)
                torch.cuda.synchronize()
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
                for _ in range(n_it):
                    P, sc = rot.take(name, touched)
                    library_free_product(torch, lib, x, P, sc, t, mode)
                e1.record()
                e1.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / n_it
                tf = 2.0 * M * K * N / (us * 1e-6) / 1e12
                kernel = prefill_kernel_name(M=M, K=K, N=N, mode=mode, noalloc=True)
                prefill_library_free.append({"shape": name, "M": M, "mode": mode, "us": round(us, 2),
                                             "tflops": round(tf, 1), "frac": round(tf / MFMA_F16_PEAK_TFLOPS, 4),
                                             "kernel": kernel})
                log(f"prefill library-free {name:8s} M={M} {mode:5s} {us:9.1f} us {tf:7.1f} TFLOP/s ({kernel})")
                del x
    # the hand-written large-batch kernel on the largest product (without a
    # workspace: repack pass + kernel, whole tiles)
    roofline_prefill_tall = None
    if prefill_library_free:
        g = max((r for r in prefill_library_free if r["mode"] == "dense"), key=lambda r: r["us"])
        roofline_prefill_tall = {"bound": "mfma", "achieved": g["tflops"], "peak": MFMA_F16_PEAK_TFLOPS,
                                 "unit": "TFLOP/s", "frac": g["frac"], "traffic": None, "shape": g["shape"],
                                 "M": g["M"], "kernel": g["kernel"],
                                 "measured": "eager allocation-free calls (x repack + kernel), rotated weights"}
    prefill_min_gap = rot.min_gap
    del pools, rot
    torch.cuda.empty_cache()

    # ---------------- Llama-3-70B shapes, adversarial grading (thresholds -1:
    # every token exceeds every threshold, so every plane is read); M <= 64 as GB/s, M = 4096 as TFLOP/s
    big = None
    big_min_gap = None
    if not args.no_70b:
        big = []
        for i, (name, K, N) in enumerate(SHAPES_70B):
            w, s = synth_weight(torch, K, N, 2000 + i, dev)
            base = (prepare_weight(w, BITS), s)
            del w
            brot = ColdRotation({name: make_pool(base, base[0].numel() * 4 + s.numel() * 2, multiple=1)})
            touched = K * N + (K // GS) * N * 2
            for M in M_70B:
                x = synth_x(torch, M, K, 299 + i, dev)
                t = [-1.0] * 4
                n_it = min(len(brot.pools[name]), max(4, math.ceil((1 << 30) / touched)))
                with torch.cuda.stream(stream):
                    for _ in range(2):
                        run_product(x, *brot.take(name, touched), None, BITS, GS, N // 4, t, "union")
                    torch.cuda.synchronize()
                    g = torch.cuda.CUDAGraph()
                    brot.record()
                    with torch.cuda.graph(g, stream=stream):
                        for _ in range(n_it):
                            run_product(x, *brot.take(name, touched), None, BITS, GS, N // 4, t, "union")
                    brot.replay(brot.stop())
                    g.replay()
                    torch.cuda.synchronize()
                    e0.record(stream)
                    for _ in range(3):
                        g.replay()
                    e1.record(stream)
                e1.synchronize()
                us = e0.elapsed_time(e1) * 1e3 / (3 * n_it)
                rec = {"shape": name, "K": K, "N": N, "M": M, "us": round(us, 2)}
                if M <= 64:
                    b = decode_bytes(np.full(K, BITS // 2), K, N, M)
                    rec.update(bytes=b, gbs=round(b / (us * 1e-6) / 1e9, 1), frac=round(b / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4))
                    log(f"70B {name:8s} M={M:5d} {us:9.1f} us {rec['gbs']:8.1f} GB/s ({100 * rec['frac']:.1f}% HBM)")
                else:
                    tf = 2.0 * M * K * N / (us * 1e-6) / 1e12
                    rec.update(tflops=round(tf, 1), frac=round(tf / MFMA_F16_PEAK_TFLOPS, 4))
                    log(f"70B {name:8s} M={M:5d} {us:9.1f} us {tf:7.1f} TFLOP/s")
                big.append(rec)
                del g, x
            gap = brot.min_gap
            big_min_gap = gap if big_min_gap is None or (gap is not None and gap < big_min_gap) else big_min_gap
            del brot, base, s
            torch.cuda.empty_cache()

    # ---------------- BASELINE configs[3] stand-in: the linears of a Llama-3-8B decode step at batch 32
    model_step = None if args.no_model_step else llama8b_decode_step(torch, dev, stream)

    # ---------------- CPU baseline: the reference's pure-PyTorch math on the host cores, over the
    # whole decode sweep (graded union math), plus its dense dispatch (S9) at 16 rows
    cpu = None
    if not args.no_cpu_baseline:
        from oracle import cpu_reference
        cores = len(os.sched_getaffinity(0))
        torch.set_num_threads(cores)
        w_host = {}
        for i, (name, K, N) in enumerate(SHAPES):
            w, s = synth_weight(torch, K, N, 1000 + i, dev)
            w_host[name] = (prepare_weight(w, BITS).cpu(), s.cpu())
            del w
        xs = [(c, c["x"].cpu()) for c in cases]

        def sweep():
            for c, xc in xs:
                pc, sc = w_host[c["shape"]]
                cpu_reference.graded(xc, pc, sc, c["t"], GS, BITS)

        def dense16():
            for c, xc in xs:
                if c["M"] == 16:
                    pc, sc = w_host[c["shape"]]
                    cpu_reference.dense_prefill(xc, pc, sc, GS, BITS)

        def median_time(fn, runs=5):
            fn()  # warm-up
            ts = []
            for _ in range(runs):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
            return float(np.median(ts))

        t_sweep = median_time(sweep)
        t_dense = median_time(dense16)
        dense_bytes = sum(c["K"] * c["N"] + (c["K"] // GS) * c["N"] * 2 + c["M"] * (c["K"] + c["N"]) * 2
                          for c in cases if c["M"] == 16)
        cpu = {"value": round(step_bytes / t_sweep / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
               "sample": "the whole decode sweep (16 products) in the reference's graded union math (masked fp32 "
                         "weights + matmul, torch CPU eager), median of 5 after 1 warm-up",
               "ms_per_step": round(t_sweep * 1e3, 1),
               "dense_s9_m16": {"value": round(dense_bytes / t_dense / 1e9, 3), "unit": "GB/s",
                                "sample": "the reference's dense dispatch for more than one row (unpack, sign "
                                          "extend, postshuffle, x.dtype scale, matmul) on the four shapes at "
                                          "M=16, all planes, median of 5 after 1 warm-up",
                                "ms": round(t_dense * 1e3, 1)},
               "cpu": _cpu_model()}
        log(f"cpu baseline {cpu['value']} GB/s on {cores} cores ({t_sweep * 1e3:.0f} ms per step); dense S9 "
            f"M=16 {cpu['dense_s9_m16']['value']} GB/s")

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "fp16", "data": "synthetic",
        "config": {"workload": "decode sweep (BASELINE configs[1]): Llama-3-8B qkv/o_proj/gate_up/down x "
                               "M=1,4,16,64, union grading t=[0,P50,P80,P95], max_bits 8, group 128",
                   "weight_copies": copies_per_shape,
                   "min_bytes_between_rereads": {"decode": decode_min_gap, "prefill": prefill_min_gap,
                                                 "llama70b": big_min_gap},
                   "frac_of_hbm_roofline": round(value / HBM_PEAK_GBS, 4)},
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": cpu,
        "cases": [{k: (round(v, 3) if isinstance(v, float) else v) for k, v in c.items()
                   if k not in ("x", "t", "touched")} for c in cases],
        "prefill": prefill,
        "prefill_graded": prefill_graded,
        "roofline_prefill": roofline_prefill,
        "roofline_prefill_tall": roofline_prefill_tall,
        "prefill_library_free": prefill_library_free,
        "llama70b_adversarial": big,
        "llama8b_decode_step": model_step,
    }
    print(json.dumps(out), flush=True)
    return 0


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
