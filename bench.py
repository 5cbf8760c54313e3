#!/usr/bin/env python3
"""Benchmark of the MI355X ternary-E8 hot path; prints ONE JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--layers L]

Workload (the metric's headline): decode GEMV
y[M,N] = x[M,K] . Wq[N,K]^T on a stack of L (default 32) Llama-3-8B-shaped
decoder layers, each with seven E8-packed linears q 4096x4096, k/v 1024x4096,
o 4096x4096, gate/up 14336x4096, down 4096x14336 (ternary-E8 codes, group-32
fp16 scales, 1,744,830,464 bytes at L=32), at batch M in {1, 4, 16} with bf16
activations.  Weights are drawn N(0, 0.02) in fp32 on the GPU (seeded) and
encoded by this library's encoder; activations are bf16 N(0, 1).

One step = one GEMV over every linear of the stack at each M: one grouped launch
per M (the job table covers all 7 x L linears).  The stack is far larger than the
GPU's last-level (MALL) cache, so every step streams the weights from HBM.  The
same GEMVs issued as one launch per linear (replayed from a hipGraph) are timed
after the headline region and reported beside it.

value   = effective weight bandwidth: packed-code + scale bytes of the stack x 3
          passes / measured step time (GB/s), as the metric defines it.
warm-up = W untimed steps, then --settle-s (0.5) seconds of the same launches, untimed, so
          that the timed steps run at the GPU's steady clocks; every other leg likewise
          runs its own launches untimed for a fraction of that right before its timing.
roofline= HBM-bound: ALGORITHMIC bytes of the grouped GEMV launches in the timed
          region (codes + scales + x + y) / their summed durations (HIP events
          around each launch, on its stream), against 8 TB/s.

Also reported (not the headline): prefill GEMM TFLOP/s on the four shapes at
M in {512, 2048, 8192} and the backward dX of the same layers, encoder
throughput on one layer of fp16
weights with 0.1% +-8 sigma outliers, the 2-bit E8 and 1-bit Root E8 formats
(encoder, decode GEMV, prefill and backward dX per linear on an 8-layer stack), and the CPU
baseline: this
repo's torch restatement of the reference's portable decode-then-matmul path
(configs[0]) timed on the host cores.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "ojasx-open-source-cuda_amd")
for _p in (ROOT, PKG_DIR):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0
GS = 32

# (name, N, K) per decoder layer, Llama-3-8B
LAYER_SHAPES = [("q", 4096, 4096), ("k", 1024, 4096), ("v", 1024, 4096), ("o", 4096, 4096),
                ("gate", 14336, 4096), ("up", 14336, 4096), ("down", 4096, 14336)]
PREFILL_SHAPES = [("q_o", 4096, 4096), ("k_v", 1024, 4096), ("gate_up", 14336, 4096),
                  ("down", 4096, 14336)]
DECODE_M = (1, 4, 16)
PREFILL_M = (512, 2048, 8192)


def measured_traffic():
    """HBM bytes per grouped decode-GEMV launch (mean over M = 1, 4, 16) from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary, calibrated against a copy kernel of known
    size; None when the summary is absent."""
    path = os.path.join(ROOT, "profiles", "decode_gemv_traffic.md")
    try:
        text = open(path).read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        data = json.loads(block)
        return int(data["traffic_bytes_per_launch"]), data
    except (OSError, IndexError, KeyError, ValueError):
        return None, None


def weight_bytes(N: int, K: int) -> int:
    return N * K * 3 // 16 + (N * K // GS) * 2


# Seconds of untimed work before each timed region (--settle-s).
SETTLE_S = 0.5


def settle(torch, fn, seconds=None) -> None:
    """Runs `fn` (the leg's own launches) untimed for `seconds` of wall time right before a
    timed region.  From idle the GPU's clocks take a few hundred milliseconds of work to
    reach their steady state: the grouped M = 1 decode launch averaged 0.43 ms over 30
    launches from idle, 0.369 ms over 300 and 0.361 ms over 2000."""
    s = SETTLE_S if seconds is None else seconds
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < s:
        fn()
        torch.cuda.synchronize()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--layers", type=int, default=32)
    ap.add_argument("--prefill-m", type=str, default=",".join(map(str, PREFILL_M)))
    ap.add_argument("--prefill-time", type=float, default=0.15,
                    help="target seconds of timed work per prefill case")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="bounded CPU-baseline sample length")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-encode", action="store_true")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--e2e-layers", type=int, default=32)
    ap.add_argument("--encode-layers", type=int, default=32)
    ap.add_argument("--e8b-layers", type=int, default=8,
                    help="layers of the 2-bit and 1-bit E8 stacks (0: skip those legs)")
    ap.add_argument("--decode-m", type=str, default=",".join(map(str, DECODE_M)),
                    help="decode batch sizes of the headline step (profiling runs pick one)")
    ap.add_argument("--no-per-linear", action="store_true",
                    help="skip the per-linear hipGraph timing beside the headline")
    ap.add_argument("--settle-s", type=float, default=0.5,
                    help="seconds of each leg's own launches run untimed right before its "
                         "timed region, after the warm-up steps (0: none)")
    ap.add_argument("--e8b-grouped-layers", type=int, default=32,
                    help="layers of the grouped 2-bit and 1-bit decode legs (0: skip)")
    ap.add_argument("--gs-layers", type=int, default=8,
                    help="layers of the ternary group-size leg (group 32 against 64; 0: skip)")
    ap.add_argument("--launch-probe", action="store_true",
                    help="only measure the cost of a decode-sized launch (a one-workgroup GEMV "
                         "and a one-element torch kernel, eager and replayed from a hipGraph) "
                         "and exit")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="only run three device-to-device copies of this many MiB (the "
                         "known-size kernel that calibrates FETCH_SIZE / WRITE_SIZE) and exit")
    return ap.parse_args()


# --------------------------------------------------------------------------- setup

def build_stack(torch, ops, layers: int, dev):
    """Encode `layers` x 7 weight matrices on the GPU; returns list of dicts."""
    stack = []
    t0 = time.time()
    for layer in range(layers):
        for j, (name, N, K) in enumerate(LAYER_SHAPES):
            g = torch.Generator(device=dev).manual_seed(8200 + 7 * layer + j)
            w = torch.randn(N, K, generator=g, device=dev, dtype=torch.float32) * 0.02
            packed, scales = ops.encode(w, GS)
            del w
            stack.append(dict(layer=layer, name=name, N=N, K=K, packed=packed, scales=scales))
    torch.cuda.synchronize()
    log(f"encoded {len(stack)} linears ({sum(weight_bytes(s['N'], s['K']) for s in stack) / 1e9:.3f}"
        f" GB packed) in {time.time() - t0:.1f} s")
    return stack


def check_decode_outputs(torch, ops, stack, xs, ys, dev, Ms) -> float:
    """Max relative error of sampled GEMV outputs against a torch fp32 matmul of
    the decoded (bf16-rule) weights; a sanity check of what was timed."""
    worst = 0.0
    for M in Ms:
        for idx in (0, 4, 6):  # q, gate, down of layer 0
            s = stack[idx]
            w = ops.decode(s["packed"], s["scales"], s["N"] * s["K"], GS, torch.bfloat16)
            ref = xs[(M, s["K"])].float() @ w.view(s["N"], s["K"]).float().t()
            y = ys[(M, idx)].float()
            err = (y - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
            worst = max(worst, err)
    return worst


# --------------------------------------------------------------------------- decode GEMV

def _bench_per_linear(torch, N_, lib, stack, xs, ys, steps, Ms, wbytes):
    """The stack's GEMVs as one launch per linear, replayed from one hipGraph per M."""
    stream = torch.cuda.current_stream()

    def launch_all(M, stream_handle, name=None):
        for i, s in enumerate(stack):
            if name is not None and s["name"] != name:
                continue
            st = lib.ojx_e8t_gemm_fwd(xs[(M, s["K"])].data_ptr(), s["packed"].data_ptr(),
                                      s["scales"].data_ptr(), None, ys[(M, i)].data_ptr(), M,
                                      s["N"], s["K"], GS, N_.BF16, None, 0, stream_handle)
            N_.check(st, "gemm_fwd")

    for M in Ms:
        launch_all(M, stream.cuda_stream)
    torch.cuda.synchronize()
    graphs = {}
    cap_stream = torch.cuda.Stream()
    for M in Ms:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=cap_stream):
            launch_all(M, torch.cuda.current_stream().cuda_stream)
        graphs[M] = g
    for M in Ms:
        graphs[M].replay()
    torch.cuda.synchronize()
    per_linear = {}
    for M in Ms:
        settle(torch, graphs[M].replay, SETTLE_S / 2)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(steps):
            graphs[M].replay()
        b.record(stream)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / steps
        per_linear[str(M)] = dict(ms=round(ms, 4), weight_GBs=round(wbytes / ms / 1e6, 1),
                                  frac_hbm=round(wbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                                  launches=len(stack))
    # per shape: the stack's linears of one shape (one per layer, distinct weights), one
    # hipGraph per (M, shape); microseconds per launch
    for M in Ms:
        shapes = {}
        for name, N, K in LAYER_SHAPES:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=cap_stream):
                launch_all(M, torch.cuda.current_stream().cuda_stream, name)
            g.replay()
            torch.cuda.synchronize()
            settle(torch, g.replay, SETTLE_S / 5)
            n = sum(1 for s in stack if s["name"] == name)
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(steps):
                g.replay()
            b.record(stream)
            torch.cuda.synchronize()
            us = a.elapsed_time(b) * 1e3 / steps / n
            shapes[name] = dict(us=round(us, 2),
                                weight_GBs=round(weight_bytes(N, K) / us / 1e3, 1))
            del g
        per_linear[str(M)]["per_shape"] = shapes
    return per_linear


def bench_decode(torch, N_, stack, steps: int, warmup: int, dev, Ms=DECODE_M,
                 per_linear_too: bool = True):
    """Headline: one grouped launch per M over every linear of the stack.  Also timed
    (reported beside it): the same GEMVs as one launch per linear, replayed from a
    hipGraph per M."""
    from ojasx_amd.grouped import GroupedGemv, stack_jobs

    lib = N_.lib()
    xs, ys = {}, {}
    for M in Ms:
        for K in (4096, 14336):
            g = torch.Generator(device=dev).manual_seed(8300 + M + K)
            xs[(M, K)] = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
        for i, s in enumerate(stack):
            ys[(M, i)] = torch.empty(M, s["N"], dtype=torch.bfloat16, device=dev)

    plans = {}
    for M in Ms:
        xk = {K: xs[(M, K)] for K in (4096, 14336)}
        yl = [ys[(M, i)] for i in range(len(stack))]
        plans[M] = GroupedGemv(stack_jobs(stack, xk, yl), M, torch.bfloat16, dev,
                               keep=list(xk.values()) + yl)

    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        for M in Ms:
            plans[M]()
    torch.cuda.synchronize()
    settle(torch, lambda: [plans[M]() for M in Ms])

    # ---- timed region: exactly `steps` steps, synchronised on both sides
    ev = {M: [] for M in Ms}
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()  # barrier + sync (N=1: no other ranks)
    wall0 = time.perf_counter()
    t_start.record(stream)
    for _ in range(steps):
        for M in Ms:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            plans[M]()
            b.record(stream)
            ev[M].append((a, b))
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    total_ms = t_start.elapsed_time(t_end)

    wbytes = sum(weight_bytes(s["N"], s["K"]) for s in stack)
    per_m = {}
    alg_bytes_region = 0
    kernel_ms_region = 0.0
    for M in Ms:
        ms = sum(a.elapsed_time(b) for a, b in ev[M]) / steps
        act = sum(M * s["K"] * 2 + M * s["N"] * 2 for s in stack)
        per_m[str(M)] = dict(ms=round(ms, 4), weight_GBs=round(wbytes / ms / 1e6, 1),
                             frac_hbm=round(wbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                             grid=plans[M].grid)
        alg_bytes_region += (wbytes + act) * steps
        kernel_ms_region += ms * steps
    err = check_decode_outputs(torch, __import__("ojasx_amd").ops, stack, xs, ys, dev, Ms)

    per_linear = {}
    if per_linear_too:
        per_linear = _bench_per_linear(torch, N_, lib, stack, xs, ys, steps, Ms, wbytes)
        err = max(err, check_decode_outputs(torch, __import__("ojasx_amd").ops, stack, xs, ys,
                                            dev, Ms))
    return dict(total_ms=total_ms, wall_s=wall, wbytes=wbytes, per_m=per_m,
                per_linear=per_linear, alg_bytes=alg_bytes_region, kernel_ms=kernel_ms_region,
                launches=len(Ms) * steps, max_rel_err=err)


# --------------------------------------------------------------------------- prefill GEMM

def bench_prefill(torch, N_, stack, Ms, target_s: float, dev, backward: bool = False):
    """Prefill GEMM per shape and M; with backward=True the backward dX of the same layers
    (grad_x[M, K] = grad_y[M, N] . W[N, K], ojx_e8t_gemm_bwd_dx)."""
    from ojasx_amd import ops

    lib = N_.lib()
    by_name = {}
    for s in stack[:7]:
        by_name.setdefault((s["N"], s["K"]), s)
    results = {}
    tot_flop = 0.0
    tot_ms = 0.0
    worst = 0.0
    stream = torch.cuda.current_stream()
    for M in Ms:
        for name, N, K in PREFILL_SHAPES:
            s = by_name[(N, K)]
            g = torch.Generator(device=dev).manual_seed(8400 + M)
            ws = ops.workspace(ops.FMT_TERNARY, backward, M, N, K, GS, torch.bfloat16, dev)
            ws_p, ws_n = (0, 0) if ws is None else (ws.data_ptr(), ws.numel())
            if backward:
                x = torch.randn(M, N, generator=g, device=dev).to(torch.bfloat16)
                y = torch.empty(M, K, dtype=torch.bfloat16, device=dev)

                def run():
                    N_.check(lib.ojx_e8t_gemm_bwd_dx(x.data_ptr(), s["packed"].data_ptr(),
                                                     s["scales"].data_ptr(), y.data_ptr(), M, N,
                                                     K, GS, N_.BF16, ws_p, ws_n,
                                                     stream.cuda_stream),
                             "gemm_bwd_dx")
            else:
                x = torch.randn(M, K, generator=g, device=dev).to(torch.bfloat16)
                y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

                def run():
                    N_.check(lib.ojx_e8t_gemm_fwd(x.data_ptr(), s["packed"].data_ptr(),
                                                  s["scales"].data_ptr(), None, y.data_ptr(), M,
                                                  N, K, GS, N_.BF16, ws_p, ws_n,
                                                  stream.cuda_stream),
                             "gemm_fwd")

            run()
            torch.cuda.synchronize()
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            run()
            b.record(stream)
            torch.cuda.synchronize()
            one = max(a.elapsed_time(b), 1e-3)
            iters = max(1, min(200, int(target_s * 1e3 / one)))
            settle(torch, run, SETTLE_S / 5)
            a.record(stream)
            for _ in range(iters):
                run()
            b.record(stream)
            torch.cuda.synchronize()
            ms = a.elapsed_time(b) / iters
            flop = 2.0 * M * N * K
            tf = flop / ms / 1e9
            # output check of what was timed: every element against an fp32 matmul of the
            # decoded weights (the decoder is bit-exact with the oracle)
            wdq = ops.decode(s["packed"], s["scales"], N * K, GS, torch.bfloat16).view(N, K)
            ref = (x.float() @ wdq.float()) if backward else (x.float() @ wdq.float().t())
            err = ((y.float() - ref).abs().max() / ref.abs().max().clamp_min(1e-30)).item()
            worst = max(worst, err)
            del wdq, ref
            results[f"{name}_M{M}"] = dict(ms=round(ms, 4), TFLOPs=round(tf, 1),
                                           frac_mfma=round(tf / BF16_MFMA_PEAK_TFLOPS, 4),
                                           max_rel_err=float(f"{err:.3g}"))
            tot_flop += flop
            tot_ms += ms
            del x, y, ws
    agg = tot_flop / tot_ms / 1e9 if tot_ms > 0 else 0.0
    if worst > 1e-2:
        raise RuntimeError(f"prefill output check failed: max rel err {worst:.3g} > 1e-2")
    return dict(cases=results, TFLOPs=round(agg, 1),
                frac_mfma=round(agg / BF16_MFMA_PEAK_TFLOPS, 4), max_rel_err=worst)


# --------------------------------------------------------------------------- encoder

def bench_encode(torch, N_, dev, layers: int, reps: int = 3):
    """encode a `layers`-layer Llama-3-8B-shaped stack of fp16 N(0, 0.02) weights
    with 0.1% of entries set to +-8 sigma (seed 9000 + 7*layer + j), layer by layer: one
    encode launch per linear, the whole stack replayed from one hipGraph.  One layer of each
    shape (layer 0: 218 M weights) is checked bit for bit against the CPU oracle, whole, and
    the oracle's own encode rate on one q-shaped layer is reported beside it."""
    import numpy as np

    from oracle import oracle as O

    lib = N_.lib()
    t0 = time.time()
    items = []
    for layer in range(layers):
        for j, (name, N, K) in enumerate(LAYER_SHAPES):
            g = torch.Generator(device=dev).manual_seed(9000 + 7 * layer + j)
            w = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
            nout = w.numel() // 1000
            idx = torch.randperm(w.numel(), generator=g, device=dev)[:nout]
            sign = torch.where(torch.rand(nout, generator=g, device=dev) < 0.5, -1.0, 1.0)
            w.view(-1)[idx] = (0.16 * sign).half()
            del idx, sign
            packed = torch.empty(N * K * 3 // 16, dtype=torch.uint8, device=dev)
            scales = torch.empty(N * K // GS, dtype=torch.float16, device=dev)
            items.append((w, packed, scales, name, N, K))
    torch.cuda.synchronize()
    gen_s = time.time() - t0
    numel = sum(it[4] * it[5] for it in items)

    def launch_all(h):
        for w, pk, sc, _, _, _ in items:
            N_.check(lib.ojx_e8t_encode(w.data_ptr(), N_.F16, w.numel(), GS, pk.data_ptr(),
                                        sc.data_ptr(), h), "encode")

    stream = torch.cuda.current_stream()
    launch_all(stream.cuda_stream)
    torch.cuda.synchronize()
    cap = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        launch_all(torch.cuda.current_stream().cuda_stream)
    graph.replay()
    torch.cuda.synchronize()
    settle(torch, graph.replay)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps

    # bit-exactness: every linear of layer 0 (one per shape), whole, against the CPU oracle
    cores = max(1, min(len(os.sched_getaffinity(0)), 16))
    exact = True
    for w, pk, sc, name, N, K in items[:7]:
        ref_pk, ref_sc, _ = O.encode(w.float().cpu().numpy(), GS, cores)
        got_pk = pk.cpu().numpy()
        got_sc = sc.cpu().view(torch.int16).numpy().view(np.uint16)
        exact = exact and np.array_equal(got_pk, ref_pk) and np.array_equal(got_sc, ref_sc)
        del ref_pk, ref_sc, got_pk, got_sc

    # the CPU oracle's encode rate (host cores) on one q-shaped layer of the stack
    wq = items[0][0].float().cpu().numpy()
    O.encode(wq[:64], GS, cores)
    t1 = time.perf_counter()
    O.encode(wq, GS, cores)
    cpu_s = time.perf_counter() - t1
    del items
    torch.cuda.empty_cache()
    return dict(layers=layers, linears=7 * layers, weights=numel, ms=round(ms, 3),
                Gweights_s=round(numel / ms / 1e6, 1), GBs=round(numel * 2.25 / ms / 1e6, 1),
                frac_hbm=round(numel * 2.25 / ms / 1e6 / HBM_PEAK_GBS, 4),
                bytes_per_weight=2.25, bit_exact_sample=exact,
                sample="all of layer 0 (7 linears, 218 M weights) vs oracle/e8t_oracle.c",
                generate_s=round(gen_s, 1),
                cpu_oracle=dict(Gweights_s=round(wq.size / cpu_s / 1e9, 3), cores=cores,
                                sample="one 4096x4096 layer, oracle/e8t_oracle.c (OpenMP)"))


# --------------------------------------------------------------------------- 2-bit E8

E8B_GS = 32  # pack_model_e8's default group size (reference lattice.py:905)


def e8b_weight_bytes(N: int, K: int, gs: int = E8B_GS, per_byte: int = 4) -> int:
    return N * K // per_byte + N * K // gs * 2


# Low-bit formats of the leg below: C entry points, weights per code byte, CPU oracle encoder,
# GPU decoder (ops) name.
LOWBIT = {
    "2bit": dict(encode="ojx_e8_encode", gemm="ojx_e8_gemm_fwd", bwd="ojx_e8_gemm_bwd_dx",
                 per_byte=4, oracle="e8b_encode", decode="decode2"),
    "root": dict(encode="ojx_e8r_encode", gemm="ojx_e8r_gemm_fwd", bwd="ojx_e8r_gemm_bwd_dx",
                 per_byte=8, oracle="e8r_encode", decode="decode1"),
}


def bench_e8b(torch, N_, dev, layers: int, steps: int, Ms=(1, 4, 16), prefill_m: int = 512,
              check_rows: int = 32, fmt: str = "2bit"):
    """2-bit E8 (E8LatticePacker, the default bitrate of E8LatticeLinear/pack_model_e8), or
    with fmt "root" the 1-bit Root E8 (RootE8LatticePacker) in the same layout of work: a
    `layers`-layer Llama-3-8B-shaped stack of fp16 N(0, 0.02) weights (seed 9700 + 7*layer +
    j), group size 32.  Encoder: the stack's encode launches replayed from one hipGraph,
    layer 0 of each shape checked bit for bit against the CPU oracle on its first
    `check_rows` rows.  Decode: one ojx_e8_gemm_fwd launch per linear at each M, replayed
    from a hipGraph (the prefill launches with a caller-owned K-split workspace); outputs of
    layer 0 checked against an fp32 matmul of the decoded weights.
    Prefill: the same at M = `prefill_m`; backward: the backward dX launches (grad_x[M, K] =
    grad_y[M, N] . W) of the stack at M = `prefill_m`, checked the same way."""
    import numpy as np

    from oracle import oracle as O

    lib = N_.lib()
    F = LOWBIT[fmt]
    enc_fn, gemm_fn, per_byte = getattr(lib, F["encode"]), getattr(lib, F["gemm"]), F["per_byte"]
    bwd_fn = getattr(lib, F["bwd"])
    items = []
    for layer in range(layers):
        for j, (name, N, K) in enumerate(LAYER_SHAPES):
            g = torch.Generator(device=dev).manual_seed(9700 + 7 * layer + j)
            w = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
            packed = torch.empty(N * K // per_byte, dtype=torch.uint8, device=dev)
            scales = torch.empty(N * K // E8B_GS, dtype=torch.float16, device=dev)
            items.append(dict(w=w, packed=packed, scales=scales, name=name, N=N, K=K))
    numel = sum(it["N"] * it["K"] for it in items)
    wbytes = sum(e8b_weight_bytes(it["N"], it["K"], per_byte=per_byte) for it in items)
    stream = torch.cuda.current_stream()

    def replay_ms(launch_all, reps):
        launch_all(stream.cuda_stream)
        torch.cuda.synchronize()
        cap = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            launch_all(torch.cuda.current_stream().cuda_stream)
        graph.replay()
        torch.cuda.synchronize()
        settle(torch, graph.replay, SETTLE_S / 2)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    def encode_all(h):
        for it in items:
            N_.check(enc_fn(it["w"].data_ptr(), N_.F16, it["w"].numel(), E8B_GS,
                            it["packed"].data_ptr(), it["scales"].data_ptr(), h), "encode")

    enc_ms = replay_ms(encode_all, 3)
    exact = True
    for it in items[:7]:
        rows, K = min(check_rows, it["N"]), it["K"]
        ref_pk, ref_sc, _ = getattr(O, F["oracle"])(it["w"][:rows].float().cpu().numpy(), E8B_GS)
        got_pk = it["packed"][: rows * K // per_byte].cpu().numpy()
        got_sc = it["scales"][: rows * K // E8B_GS].cpu().view(torch.int16).numpy().view(np.uint16)
        exact = exact and np.array_equal(got_pk, ref_pk) and np.array_equal(got_sc, ref_sc)
    for it in items:
        del it["w"]
    torch.cuda.empty_cache()

    def gemm_leg(M, bwd=False):
        # forward: x[M, K] -> y[M, N]; backward dX: grad_y[M, N] -> grad_x[M, K]
        xin = (lambda it: it["N"]) if bwd else (lambda it: it["K"])
        xout = (lambda it: it["K"]) if bwd else (lambda it: it["N"])
        xs = {n: torch.randn(M, n, generator=torch.Generator(device=dev).manual_seed(9800 + M + n),
                             device=dev).to(torch.bfloat16) for n in {xin(it) for it in items[:7]}}
        ys = [torch.empty(M, xout(it), dtype=torch.bfloat16, device=dev) for it in items]
        # one workspace, as large as the largest launch needs, shared by the stream's launches
        from ojasx_amd import ops as ops_
        fmt_code = ops_.FMT_E8 if fmt == "2bit" else ops_.FMT_ROOT
        wss = [ops_.workspace(fmt_code, bwd, M, it["N"], it["K"], E8B_GS, torch.bfloat16, dev)
               for it in items[:7]]
        ws = max((w for w in wss if w is not None), key=lambda w: w.numel(), default=None)
        ws_p, ws_n = (0, 0) if ws is None else (ws.data_ptr(), ws.numel())

        def launch_all(h):
            for it, y in zip(items, ys):
                if bwd:
                    N_.check(bwd_fn(xs[it["N"]].data_ptr(), it["packed"].data_ptr(),
                                    it["scales"].data_ptr(), y.data_ptr(), M, it["N"], it["K"],
                                    E8B_GS, N_.BF16, ws_p, ws_n, h), "gemm_bwd_dx")
                else:
                    N_.check(gemm_fn(xs[it["K"]].data_ptr(), it["packed"].data_ptr(),
                                     it["scales"].data_ptr(), None, y.data_ptr(), M, it["N"],
                                     it["K"], E8B_GS, N_.BF16, ws_p, ws_n, h), "gemm")

        ms = replay_ms(launch_all, steps)
        worst = 0.0
        from ojasx_amd import ops
        for idx in (0, 4, 6):  # q, gate, down of layer 0
            it = items[idx]
            wd = getattr(ops, F["decode"])(it["packed"], it["scales"], it["N"] * it["K"], E8B_GS,
                                           torch.bfloat16).view(it["N"], it["K"]).float()
            ref = (xs[it["N"]].float() @ wd) if bwd else (xs[it["K"]].float() @ wd.t().contiguous())
            err = (ys[idx].float() - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
            worst = max(worst, err)
        return ms, worst

    decode, worst = {}, 0.0
    for M in Ms:
        ms, err = gemm_leg(M)
        worst = max(worst, err)
        decode[str(M)] = dict(ms=round(ms, 4), weight_GBs=round(wbytes / ms / 1e6, 1),
                              frac_hbm=round(wbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                              launches=len(items))
    ms, err = gemm_leg(prefill_m)
    worst = max(worst, err)
    flops = 2.0 * prefill_m * numel
    prefill = dict(M=prefill_m, ms=round(ms, 3), TFLOPs=round(flops / ms / 1e9, 1),
                   frac_mfma=round(flops / ms / 1e9 / BF16_MFMA_PEAK_TFLOPS, 4))
    ms, err = gemm_leg(prefill_m, bwd=True)
    worst = max(worst, err)
    backward = dict(M=prefill_m, ms=round(ms, 3), TFLOPs=round(flops / ms / 1e9, 1),
                    frac_mfma=round(flops / ms / 1e9 / BF16_MFMA_PEAK_TFLOPS, 4))
    del items
    torch.cuda.empty_cache()
    return dict(layers=layers, linears=7 * layers, group_size=E8B_GS, weights=numel,
                stack_weight_bytes=wbytes,
                encode=dict(ms=round(enc_ms, 3), Gweights_s=round(numel / enc_ms / 1e6, 1),
                            bit_exact_sample=exact,
                            sample=f"first {check_rows} rows of layer 0 of each shape vs "
                                   "oracle/e8t_oracle.c"),
                decode_per_linear=decode, prefill_per_linear=prefill,
                backward_dx_per_linear=backward, max_rel_err=worst)


# --------------------------------------------------------------------------- end-to-end decoder

E2E = dict(layers=32, hidden=4096, heads=32, kv_heads=8, head_dim=128, ffn=14336, vocab=128256,
           batch=4, prompt=512, gen=128, lora_rank=8, lora_alpha=16.0, rope_theta=500000.0,
           eps=1e-5)


class E8Decoder:
    """random-init Llama-3-8B-shaped decoder, every linear (and lm_head)
    ternary-E8 packed (group 32), rank-8 bf16 LoRA on q/v, RMSNorm and RoPE in bf16.
    Attention (not part of the E8 path) is computed in fp32 with a pre-transposed K
    cache; decode steps run the E8 linears as grouped GEMVs (fused q/k/v and gate/up).
    The adapters are added inside the E8 kernels' epilogue (u = scaling * x @ A by
    ojx_lora_down, u @ B before the output is rounded), in prefill and decode alike."""

    def __init__(self, torch, dev, cfg, layers, seed=9500):
        import ojasx_amd
        from ojasx_amd.grouped import GroupedGemv

        self.t, self.dev, self.c = torch, dev, cfg
        self.L = layers
        H, F_, V = cfg["hidden"], cfg["ffn"], cfg["vocab"]
        kvd = cfg["kv_heads"] * cfg["head_dim"]
        bf = torch.bfloat16
        g = torch.Generator(device=dev).manual_seed(seed)

        def lin(n_out, n_in, rank=0):
            m = ojasx_amd.E8LatticeLinear(n_in, n_out, bias=False, rank=rank,
                                          lora_alpha=cfg["lora_alpha"], group_size=32,
                                          bitrate=1.5, device=dev, dtype=bf)
            w = torch.randn(n_out, n_in, generator=g, device=dev) * 0.02
            pk, sc = ojasx_amd.ops.encode(w, 32)
            del w
            m.packed_weight.copy_(pk)
            m.block_scales.copy_(sc)
            if rank:
                with torch.no_grad():
                    m.lora_A.copy_((torch.randn(n_in, rank, generator=g, device=dev) * 0.02).to(bf))
                    m.lora_B.copy_((torch.randn(rank, n_out, generator=g, device=dev) * 0.02).to(bf))
            m.requires_grad_(False)
            return m

        self.emb = (torch.randn(V, H, generator=g, device=dev) * 0.02).to(bf)
        self.layers = []
        for _ in range(layers):
            self.layers.append(dict(
                q=lin(H, H, cfg["lora_rank"]), k=lin(kvd, H), v=lin(kvd, H, cfg["lora_rank"]),
                o=lin(H, H), gate=lin(F_, H), up=lin(F_, H), down=lin(H, F_),
                n1=torch.ones(H, dtype=bf, device=dev), n2=torch.ones(H, dtype=bf, device=dev)))
        self.norm = torch.ones(H, dtype=bf, device=dev)
        self.lm_head = lin(V, H)
        B = cfg["batch"]
        for ly in self.layers:  # decode-time grouped launches (planned once for M = batch)
            ly["qkv_g"] = GroupedGemv.fused([ly["q"], ly["k"], ly["v"]], B, bf)
            ly["gu_g"] = GroupedGemv.fused([ly["gate"], ly["up"]], B, bf)
        hd = cfg["head_dim"]
        Lmax = cfg["prompt"] + cfg["gen"]
        inv = 1.0 / (cfg["rope_theta"] ** (torch.arange(0, hd, 2, device=dev).float() / hd))
        ang = torch.arange(Lmax, device=dev).float()[:, None] * inv[None, :]
        self.cos, self.sin = ang.cos(), ang.sin()  # [Lmax, hd/2] fp32
        self.Lmax = Lmax
        self.kt = [torch.zeros(B, cfg["kv_heads"], hd, Lmax, device=dev) for _ in range(layers)]
        self.vc = [torch.zeros(B, cfg["kv_heads"], Lmax, hd, device=dev) for _ in range(layers)]

    def rms(self, x, w):
        t = self.t
        xf = x.float()
        y = xf * t.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.c["eps"])
        return y.to(x.dtype) * w

    def rope(self, x, cos, sin):
        # x [..., heads, hd] (rotate-half form); cos/sin broadcast over heads
        h = x.shape[-1] // 2
        xf = x.float()
        x1, x2 = xf[..., :h], xf[..., h:]
        return self.t.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1)

    # ---- prefill: M = batch * prompt rows through the prefill MFMA GEMM
    def prefill(self, ids, e8_events=None):
        t, c = self.t, self.c
        B, S = ids.shape
        nh, nkv, hd = c["heads"], c["kv_heads"], c["head_dim"]
        x = self.emb[ids]  # [B, S, H]
        cos, sin = self.cos[:S][None, :, None, :], self.sin[:S][None, :, None, :]
        causal = t.full((S, S), float("-inf"), device=self.dev).triu(1)

        def e8(m, h):
            if e8_events is None:
                return m(h)
            a = t.cuda.Event(enable_timing=True)
            b = t.cuda.Event(enable_timing=True)
            a.record()
            y = m(h)
            b.record()
            e8_events.append((a, b))
            return y

        for li, ly in enumerate(self.layers):
            h = self.rms(x, ly["n1"])
            q = e8(ly["q"], h).view(B, S, nh, hd)
            k = e8(ly["k"], h).view(B, S, nkv, hd)
            v = e8(ly["v"], h).view(B, S, nkv, hd)
            q = self.rope(q, cos, sin).permute(0, 2, 1, 3)          # [B, nh, S, hd] fp32
            k = self.rope(k, cos, sin).permute(0, 2, 1, 3)          # [B, nkv, S, hd]
            vf = v.float().permute(0, 2, 1, 3)                       # [B, nkv, S, hd]
            self.kt[li][:, :, :, :S] = k.transpose(-1, -2)
            self.vc[li][:, :, :S, :] = vf
            qg = q.reshape(B, nkv, (nh // nkv) * S, hd)               # heads grouped per kv head
            sc = t.matmul(qg, self.kt[li][:, :, :, :S].contiguous()) / math.sqrt(hd)
            sc = sc.view(B, nkv, nh // nkv, S, S) + causal
            o = t.matmul(sc.softmax(-1).view(B, nkv, (nh // nkv) * S, S), vf)
            o = o.view(B, nh, S, hd).permute(0, 2, 1, 3).reshape(B, S, nh * hd).to(x.dtype)
            x = x + e8(ly["o"], o)
            h2 = self.rms(x, ly["n2"])
            a = t.nn.functional.silu(e8(ly["gate"], h2)) * e8(ly["up"], h2)
            x = x + e8(ly["down"], a)
        hl = self.rms(x[:, -1, :], self.norm)
        return e8(self.lm_head, hl).argmax(-1)

    # ---- the E8 launches of one decode step alone, on static inputs: fused q/k/v (with the
    # q/v adapters' down-projection), o, fused gate/up, down, lm_head.  The residual adds,
    # norms and activations between them are not E8 work (decode_step times everything).
    def decode_step_e8_only(self, x, a):
        for ly in self.layers:
            ly["qkv_g"](x)
            ly["gu_g"](x)
            ly["o"].forward_fused(x)
            ly["down"].forward_fused(a)
        return self.lm_head.forward_fused(x)

    # ---- one decode step (M = batch) on static buffers; graph-capturable.  The caller
    # keeps pos < Lmax (the RoPE tables and the KV cache hold Lmax positions).
    def decode_step(self, ids, pos):
        t, c = self.t, self.c
        B = ids.shape[0]
        nh, nkv, hd, H = c["heads"], c["kv_heads"], c["head_dim"], c["hidden"]
        kvd = nkv * hd
        x = self.emb[ids]  # [B, H]
        cos = self.cos.index_select(0, pos)[:, None, :]  # [1, 1, hd/2]
        sin = self.sin.index_select(0, pos)[:, None, :]
        ar = t.arange(self.Lmax, device=self.dev)
        mask = t.where(ar <= pos, 0.0, float("-inf"))  # [Lmax]
        for li, ly in enumerate(self.layers):
            h = self.rms(x, ly["n1"])
            qkv = ly["qkv_g"](h)
            q = qkv[:, :H]  # the q/v adapters are fused into the grouped launch
            k = qkv[:, H:H + kvd]
            v = qkv[:, H + kvd:]
            q = self.rope(q.view(B, nh, hd), cos, sin)            # fp32 [B, nh, hd]
            k = self.rope(k.view(B, nkv, hd), cos, sin)
            self.kt[li].index_copy_(3, pos, k.unsqueeze(-1))
            self.vc[li].index_copy_(2, pos, v.float().view(B, nkv, 1, hd))
            qg = q.view(B, nkv, nh // nkv, hd)
            sc = t.matmul(qg, self.kt[li]) / math.sqrt(hd) + mask  # [B, nkv, g, Lmax]
            o = t.matmul(sc.softmax(-1), self.vc[li]).reshape(B, H).to(x.dtype)
            x = x + ly["o"].forward_fused(o)
            h2 = self.rms(x, ly["n2"])
            gu = ly["gu_g"](h2)
            a = t.nn.functional.silu(gu[:, : c["ffn"]]) * gu[:, c["ffn"]:]
            x = x + ly["down"].forward_fused(a)
        logits = self.lm_head.forward_fused(self.rms(x, self.norm))
        nxt = logits.argmax(-1)
        ids.copy_(nxt)
        pos.add_(1)
        return nxt


def bench_e8b_grouped(torch, dev, layers: int, steps: int, warmup: int, Ms=(1, 4, 16),
                      gs: int = 32, bitrate: float = 2.0) -> dict:
    """2-bit E8 (the reference's default bitrate, lattice.py:735, 906) or, with bitrate 1.0,
    1-bit Root E8 (lattice.py:426-533) decode over a `layers`-layer Llama-3-8B-shaped stack of
    fp16 N(0, 0.02) weights (seed 9700 + 7*layer + j, group size `gs`): one grouped launch
    (ojx_e8_gemv_grouped / ojx_e8r_gemv_grouped, device job table) per M over every linear,
    timed with HIP events as the ternary headline; outputs of layer 0's q, gate and down
    checked against an fp32 matmul of the decoded weights."""
    from ojasx_amd import ops
    from ojasx_amd.grouped import GroupedGemv, stack_jobs

    encode = ops.encode2 if bitrate == 2.0 else ops.encode1
    decode = ops.decode2 if bitrate == 2.0 else ops.decode1
    stack = []
    for layer in range(layers):
        for j, (name, N, K) in enumerate(LAYER_SHAPES):
            g = torch.Generator(device=dev).manual_seed(9700 + 7 * layer + j)
            w = (torch.randn(N, K, generator=g, device=dev) * 0.02).half()
            packed, scales = encode(w, gs)
            del w
            stack.append(dict(name=name, N=N, K=K, packed=packed, scales=scales))
    torch.cuda.synchronize()
    wbytes = sum(s["packed"].numel() + 2 * s["scales"].numel() for s in stack)
    plans, xs, ys = {}, {}, {}
    for M in Ms:
        xk = {K: torch.randn(M, K, generator=torch.Generator(device=dev).manual_seed(8300 + M + K),
                             device=dev).to(torch.bfloat16) for K in (4096, 14336)}
        yl = [torch.empty(M, s["N"], dtype=torch.bfloat16, device=dev) for s in stack]
        xs[M], ys[M] = xk, yl
        plans[M] = GroupedGemv(stack_jobs(stack, xk, yl), M, torch.bfloat16, dev,
                               keep=list(xk.values()) + yl, bitrate=bitrate, group_size=gs)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        for M in Ms:
            plans[M]()
    torch.cuda.synchronize()
    settle(torch, lambda: [plans[M]() for M in Ms])
    ev = {M: [] for M in Ms}
    for _ in range(steps):
        for M in Ms:
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            plans[M]()
            b.record(stream)
            ev[M].append((a, b))
    torch.cuda.synchronize()
    per_m, worst = {}, 0.0
    for M in Ms:
        ms = sum(a.elapsed_time(b) for a, b in ev[M]) / steps
        per_m[str(M)] = dict(ms=round(ms, 4), weight_GBs=round(wbytes / ms / 1e6, 1),
                             frac_hbm=round(wbytes / ms / 1e6 / HBM_PEAK_GBS, 4),
                             grid=plans[M].grid)
        for idx in (0, 4, 6):
            s = stack[idx]
            wd = decode(s["packed"], s["scales"], s["N"] * s["K"], gs,
                        torch.bfloat16).view(s["N"], s["K"]).float()
            ref = xs[M][s["K"]].float() @ wd.t()
            err = (ys[M][idx].float() - ref).abs().max().item() / max(ref.abs().max().item(),
                                                                      1e-30)
            worst = max(worst, err)
    return dict(layers=layers, linears=len(stack), group_size=gs, stack_weight_bytes=wbytes,
                per_M=per_m, max_rel_err=worst)


def bench_ternary_gs(torch, N_, dev, layers: int, steps: int, gs_list=(32, 16, 64),
                     Ms=(1, 4, 16), prefill_m: int = 2048) -> dict:
    """Ternary E8 at the reference's other group sizes: one `layers`-layer Llama-3-8B-shaped
    stack of fp32 N(0, 0.02) weights (seed 9900 + 7*layer + j) encoded at each group size
    in `gs_list` (E8LatticeLinear's default group size 8 becomes 16 at bitrate 1.5,
    lattice.py:752, 793; the reference's published decoder run uses ternary group 64,
    reports/apple_m5_1b_to_27b_gpu_benchmark.json:23-24), timed as per-linear
    ojx_e8t_gemm_fwd launches replayed from a hipGraph at the decode M, the prefill forward
    and the backward dX at M = `prefill_m`; outputs of layer 0's q, gate and down checked
    against an fp32 matmul of the decoded weights."""
    from ojasx_amd import ops

    lib = N_.lib()
    stream = torch.cuda.current_stream()
    ws_items = {}
    for layer in range(layers):
        for j, (name, N, K) in enumerate(LAYER_SHAPES):
            g = torch.Generator(device=dev).manual_seed(9900 + 7 * layer + j)
            w = torch.randn(N, K, generator=g, device=dev) * 0.02
            for gs in gs_list:
                packed, scales = ops.encode(w, gs)
                ws_items.setdefault(gs, []).append(dict(packed=packed, scales=scales, name=name,
                                                        N=N, K=K))
            del w
    torch.cuda.synchronize()

    def replay_ms(launch_all, reps):
        launch_all(stream.cuda_stream)
        torch.cuda.synchronize()
        cap = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            launch_all(torch.cuda.current_stream().cuda_stream)
        graph.replay()
        torch.cuda.synchronize()
        settle(torch, graph.replay, SETTLE_S / 2)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            graph.replay()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps

    def leg(items, gs, M, bwd=False):
        xin = (lambda it: it["N"]) if bwd else (lambda it: it["K"])
        xout = (lambda it: it["K"]) if bwd else (lambda it: it["N"])
        xs = {n: torch.randn(M, n, generator=torch.Generator(device=dev).manual_seed(9800 + M + n),
                             device=dev).to(torch.bfloat16) for n in {xin(it) for it in items[:7]}}
        ys = [torch.empty(M, xout(it), dtype=torch.bfloat16, device=dev) for it in items]
        wss = [ops.workspace(ops.FMT_TERNARY, bwd, M, it["N"], it["K"], gs, torch.bfloat16, dev)
               for it in items[:7]]
        ws = max((w for w in wss if w is not None), key=lambda w: w.numel(), default=None)
        ws_p, ws_n = (0, 0) if ws is None else (ws.data_ptr(), ws.numel())

        def launch_all(h):
            for it, y in zip(items, ys):
                if bwd:
                    N_.check(lib.ojx_e8t_gemm_bwd_dx(xs[it["N"]].data_ptr(), it["packed"].data_ptr(),
                                                     it["scales"].data_ptr(), y.data_ptr(), M,
                                                     it["N"], it["K"], gs, N_.BF16, ws_p, ws_n, h),
                             "gemm_bwd_dx")
                else:
                    N_.check(lib.ojx_e8t_gemm_fwd(xs[it["K"]].data_ptr(), it["packed"].data_ptr(),
                                                  it["scales"].data_ptr(), None, y.data_ptr(), M,
                                                  it["N"], it["K"], gs, N_.BF16, ws_p, ws_n, h),
                             "gemm_fwd")

        ms = replay_ms(launch_all, steps)
        worst = 0.0
        for idx in (0, 4, 6):
            it = items[idx]
            wd = ops.decode(it["packed"], it["scales"], it["N"] * it["K"], gs,
                            torch.bfloat16).view(it["N"], it["K"]).float()
            ref = (xs[it["N"]].float() @ wd) if bwd else (xs[it["K"]].float() @ wd.t())
            err = (ys[idx].float() - ref).abs().max().item() / max(ref.abs().max().item(), 1e-30)
            worst = max(worst, err)
        return ms, worst

    out = {"layers": layers, "linears": 7 * layers, "prefill_M": prefill_m}
    worst = 0.0
    numel = sum(it["N"] * it["K"] for it in ws_items[gs_list[0]])
    for gs in gs_list:
        items = ws_items[gs]
        wbytes = sum(it["packed"].numel() + 2 * it["scales"].numel() for it in items)
        res = {"stack_weight_bytes": wbytes, "decode_per_linear": {}}
        for M in Ms:
            ms, err = leg(items, gs, M)
            worst = max(worst, err)
            res["decode_per_linear"][str(M)] = dict(ms=round(ms, 4),
                                                    weight_GBs=round(wbytes / ms / 1e6, 1))
        for key, bwd in (("prefill", False), ("backward_dx", True)):
            ms, err = leg(items, gs, prefill_m, bwd)
            worst = max(worst, err)
            flops = 2.0 * prefill_m * numel
            res[key] = dict(ms=round(ms, 3), TFLOPs=round(flops / ms / 1e9, 1),
                            frac_mfma=round(flops / ms / 1e9 / BF16_MFMA_PEAK_TFLOPS, 4))
        out["gs" + str(gs)] = res
        log(f"ternary gs {gs}: decode M=1 {res['decode_per_linear'][str(Ms[0])]['ms']} ms, "
            f"prefill {res['prefill']['TFLOPs']} TFLOP/s")
    out["max_rel_err"] = worst
    return out


def bench_e2e(torch, dev, layers: int):
    """batch 4, 512 random prompt tokens, 128 greedy steps.  Decode steps are
    replayed from one captured hipGraph; the E8 linears of a decode step are also timed
    alone (a second graph holding only them, on the same buffers)."""
    c = E2E
    t0 = time.time()
    model = E8Decoder(torch, dev, c, layers)
    torch.cuda.synchronize()
    build_s = time.time() - t0
    g = torch.Generator(device=dev).manual_seed(9501)
    B, S, G = c["batch"], c["prompt"], c["gen"]
    prompt = torch.randint(0, c["vocab"], (B, S), generator=g, device=dev)
    stream = torch.cuda.current_stream()

    # warm-up prefill (also first token), then the timed prefill
    model.prefill(prompt)
    torch.cuda.synchronize()
    settle(torch, lambda: model.prefill(prompt), SETTLE_S / 2)
    ev = []
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    first = model.prefill(prompt, e8_events=ev)
    b.record(stream)
    torch.cuda.synchronize()
    prefill_ms = a.elapsed_time(b)
    prefill_e8_ms = sum(x.elapsed_time(y) for x, y in ev)

    if S + G > model.Lmax:
        raise RuntimeError("prompt + generated tokens exceed the KV cache")
    ids = first.clone()
    pos = torch.full((1,), S, dtype=torch.long, device=dev)
    # eager reference of the first 4 decode steps (for the graph check)
    eager = []
    for _ in range(4):
        eager.append(model.decode_step(ids, pos).clone())
    torch.cuda.synchronize()

    cap = torch.cuda.Stream()
    ids.copy_(first)
    pos.fill_(S)
    with torch.cuda.stream(cap):  # warm-up on the capture stream
        model.decode_step(ids, pos)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    ids.copy_(first)
    pos.fill_(S)
    with torch.cuda.graph(graph, stream=cap):
        model.decode_step(ids, pos)
    torch.cuda.synchronize()

    # graph replays must reproduce the eager tokens (the KV cache rows are rewritten)
    ids.copy_(first)
    pos.fill_(S)
    graph_tokens = []
    for _ in range(4):
        graph.replay()
        graph_tokens.append(ids.clone())
    torch.cuda.synchronize()
    match = all(bool((x == y).all()) for x, y in zip(eager, graph_tokens))

    def replay_all():  # G replays from the first decode position (KV rows S .. S+G-1)
        ids.copy_(first)
        pos.fill_(S)
        for _ in range(G):
            graph.replay()

    settle(torch, replay_all)
    ids.copy_(first)
    pos.fill_(S)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(G):
        graph.replay()
    b.record(stream)
    torch.cuda.synchronize()
    decode_ms = a.elapsed_time(b)

    # the E8 linears of one decode step, alone, on static [batch, hidden] / [batch, ffn] inputs
    xin = (torch.randn(B, c["hidden"], generator=g, device=dev) * 0.5).to(torch.bfloat16)
    ain = (torch.randn(B, c["ffn"], generator=g, device=dev) * 0.5).to(torch.bfloat16)
    with torch.cuda.stream(cap):
        model.decode_step_e8_only(xin, ain)
    torch.cuda.synchronize()
    g_e8 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g_e8, stream=cap):
        model.decode_step_e8_only(xin, ain)
    torch.cuda.synchronize()
    settle(torch, g_e8.replay, SETTLE_S / 2)
    a.record(stream)
    for _ in range(G):
        g_e8.replay()
    b.record(stream)
    torch.cuda.synchronize()
    decode_e8_ms = a.elapsed_time(b)
    wbytes = sum(weight_bytes(m.out_features, m.in_features) for ly in model.layers
                 for m in (ly["q"], ly["k"], ly["v"], ly["o"], ly["gate"], ly["up"], ly["down"]))
    wbytes += weight_bytes(model.lm_head.out_features, model.lm_head.in_features)
    return dict(
        layers=layers, batch=B, prompt=S, generated=G, build_s=round(build_s, 1),
        prefill_ms=round(prefill_ms, 2), prefill_tokens_s=round(B * S / prefill_ms * 1e3, 1),
        prefill_e8_linear_ms=round(prefill_e8_ms, 2),
        decode_ms=round(decode_ms, 2), decode_tokens_s=round(B * G / decode_ms * 1e3, 1),
        decode_ms_per_step=round(decode_ms / G, 3),
        decode_e8_linear_ms=round(decode_e8_ms, 2),
        decode_e8_weight_GBs=round(wbytes * G / decode_e8_ms / 1e6, 1),
        total_tokens_s=round(B * (S + G) / (prefill_ms + decode_ms) * 1e3, 1),
        graph_replay_matches_eager=match,
        lm_head="E8-packed (128256 x 4096)", attention="fp32 math, pre-transposed K cache")


# --------------------------------------------------------------------------- CPU baseline

def cpu_baseline(seconds: float):
    """The reference's Linux CPU path (unpack into the workspace, then F.linear), restated in
    oracle/portable.py, timed on the host cores:
      * one 4096x4096 layer at M = 1 in fp32 for about `seconds` (the `value`);
      * configs[1]/[2] CPU side: the same path in fp32 on each of the four Llama-3-8B shapes
        at M in {1, 4, 16} (median of 3 calls after one warm-up);
      * configs[3] CPU side: the C oracle encoder (OpenMP) on one layer of each shape."""
    import platform

    import numpy as np
    import torch

    from oracle import oracle as O
    from oracle import portable

    cores = len(os.sched_getaffinity(0))
    cores = max(1, min(cores, 16))  # the GPU box's CPU share
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(8101)
    w = torch.randn(4096, 4096, generator=g) * 0.02
    x = torch.randn(1, 4096, generator=torch.Generator().manual_seed(8102))
    packed, s16, _ = O.encode(w.numpy(), GS)
    packed_t = torch.from_numpy(packed)
    scales_t = torch.from_numpy(s16.view(np.float16).copy())
    portable.linear(x, packed_t, scales_t, None, 4096, 4096)
    n = 0
    t0 = time.perf_counter()
    while True:
        portable.linear(x, packed_t, scales_t, None, 4096, 4096)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / n
    wb = weight_bytes(4096, 4096)

    shapes, encoder = {}, {}
    for name, N, K in (("q_o", 4096, 4096), ("k_v", 1024, 4096), ("gate_up", 14336, 4096),
                       ("down", 4096, 14336)):
        gw = torch.Generator().manual_seed(8110 + N + K)
        wl = (torch.randn(N, K, generator=gw) * 0.02).numpy()
        t1 = time.perf_counter()
        pk, sc, _ = O.encode(wl, GS, nthreads=cores)
        enc_s = time.perf_counter() - t1
        encoder[name] = dict(weights_per_s=round(N * K / enc_s / 1e9, 4), unit="G weights/s",
                             seconds=round(enc_s, 3))
        del wl
        pk_t, sc_t = torch.from_numpy(pk), torch.from_numpy(sc.view(np.float16).copy())
        for M in (1, 4, 16):
            xs = torch.randn(M, K, generator=gw)
            portable.linear(xs, pk_t, sc_t, None, N, K)
            ts = []
            for _ in range(3):
                t1 = time.perf_counter()
                portable.linear(xs, pk_t, sc_t, None, N, K)
                ts.append(time.perf_counter() - t1)
            med = sorted(ts)[1]
            shapes[f"{name}_M{M}"] = dict(ms=round(med * 1e3, 3),
                                          weight_GBs=round(weight_bytes(N, K) / med / 1e9, 3))
    portable._WS.clear()  # the fp32 workspace of the largest shape (235 MB)

    cpu_model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return dict(value=round(wb / per / 1e9, 3), unit="GB/s", cores=cores, kind="port",
                sample=(f"configs[0]: 4096x4096 ternary-E8 layer (seed 8101), x[1,4096] fp32 "
                        f"(seed 8102); unpack(use_workspace)+F.linear restated in "
                        f"oracle/portable.py; {n} calls in {el:.1f} s = {per * 1e3:.2f} ms/call; "
                        f"{cpu_model}"),
                cpu_model=cpu_model, per_shape_fp32=shapes, oracle_encoder=encoder)


# --------------------------------------------------------------------------- main

def launch_probe(torch, N_, ops, dev, launches: int = 224, reps: int = 20) -> dict:
    """Cost of one decode-sized launch: microseconds per launch of (a) this library's GEMV on
    a 16 x 1024 layer at M = 1 (one workgroup, 3 KB of codes) and (b) torch's elementwise add
    on one element, each issued `launches` times back to back, eagerly and from a hipGraph
    (the way the per-linear decode stack is replayed)."""
    lib = N_.lib()
    g = torch.Generator(device=dev).manual_seed(7)
    w = torch.randn(16, 1024, generator=g, device=dev) * 0.02
    packed, scales = ops.encode(w, GS)
    x = torch.randn(1, 1024, generator=g, device=dev).to(torch.bfloat16)
    y = torch.empty(1, 16, dtype=torch.bfloat16, device=dev)
    a = torch.ones(1, device=dev)

    def gemv(stream_handle):
        for _ in range(launches):
            N_.check(lib.ojx_e8t_gemm_fwd(x.data_ptr(), packed.data_ptr(), scales.data_ptr(),
                                          None, y.data_ptr(), 1, 16, 1024, GS, N_.BF16, None, 0,
                                          stream_handle), "gemm_fwd")

    def add(stream_handle):
        for _ in range(launches):
            a.add_(1.0)

    out = {"launches": launches, "reps": reps}
    for name, fn in (("gemv_16x1024_M1", gemv), ("torch_add_1elem", add)):
        fn(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        cap = torch.cuda.Stream()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=cap):
            fn(torch.cuda.current_stream().cuda_stream)
        res = {}
        for mode in ("eager", "graph"):
            run = (lambda: graph.replay()) if mode == "graph" else \
                (lambda: fn(torch.cuda.current_stream().cuda_stream))
            for _ in range(3):
                run()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                run()
            e1.record()
            torch.cuda.synchronize()
            res[mode + "_us_per_launch"] = round(e0.elapsed_time(e1) * 1e3 / (reps * launches), 3)
        out[name] = res
        log(f"launch probe {name}: {res}")
    err = (y.float() - (x.float() @ ops.decode(packed, scales, 16 * 1024, GS,
                                              torch.bfloat16).view(16, 1024).float().t())).abs()
    out["gemv_max_abs_err"] = float(err.max())
    return out


def main() -> int:
    args = parse_args()
    global SETTLE_S
    SETTLE_S = max(0.0, args.settle_s)
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures one GPU only (the E8 path is benchmarked on a "
              "single MI355X; multi-GPU sharding is a design note, not a measured path). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    import ojasx_amd
    from ojasx_amd import _native as N_
    from ojasx_amd import ops

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.copy_probe_mib > 0:
        # reads n bytes and writes n bytes per launch: torch's elementwise negation
        n = args.copy_probe_mib << 20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": n, "copy_probe_bytes_written": n,
                          "launches": 3, "kernel": "torch.neg (elementwise) fp32"}), flush=True)
        return 0
    if args.launch_probe:
        print(json.dumps(launch_probe(torch, N_, ops, dev)), flush=True)
        return 0
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} {getattr(props, 'gcnArchName', '')} CUs={props.multi_processor_count}")

    stack = build_stack(torch, ops, args.layers, dev)
    log("decode GEMV timing")
    decode_mlist = tuple(int(m) for m in args.decode_m.split(",") if m)
    dec = bench_decode(torch, N_, stack, args.steps, args.warmup, dev, decode_mlist,
                       per_linear_too=not args.no_per_linear)
    ms_per_step = dec["total_ms"] / args.steps
    value = dec["wbytes"] * len(decode_mlist) / ms_per_step / 1e6  # GB/s
    achieved = dec["alg_bytes"] / dec["kernel_ms"] / 1e6
    log(f"decode: {ms_per_step:.3f} ms/step, {value:.1f} GB/s weights, "
        f"rel err {dec['max_rel_err']:.2e}")

    result = {
        "metric": "E8 GEMV effective GB/s (% HBM peak) + prefill TFLOP/s (% MFMA), 8B shapes",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_s": SETTLE_S,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (f"decode GEMV over a {args.layers}-layer Llama-3-8B-shaped ternary-E8 "
                         "stack (q/o 4096x4096, k/v 1024x4096, gate/up 14336x4096, down "
                         "4096x14336; group-32 fp16 scales), batch M in {1,4,16}, bf16 "
                         "activations, fp32 accumulation; one grouped GEMV launch per M "
                         "covering every linear of the stack (per-linear launches from a "
                         "hipGraph are reported under decode.per_linear)"),
            "layers": args.layers,
            "decode_M": list(decode_mlist),
            "group_size": GS,
            "stack_weight_bytes": dec["wbytes"],
            "parallelism": "single GPU",
        },
        "decode": dict(per_M=dec["per_m"], per_linear=dec["per_linear"],
                       max_rel_err=dec["max_rel_err"], launches_per_step=len(decode_mlist)),
        "roofline": {
            "bound": "hbm",
            "kernel": "ojx e8t decode GEMV",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic()[0],
            "traffic_note": ("HBM bytes per launch (mean over the M = 1, 4, 16 launches) from "
                             "rocprofv3 FETCH_SIZE/WRITE_SIZE scaled by a copy-kernel "
                             "calibration: profiles/decode_gemv_traffic.md; algorithmic bytes "
                             "per launch (mean) = " + str(int(dec["alg_bytes"] / dec["launches"]))),
        },
    }

    if not args.no_prefill:
        Ms = [int(m) for m in args.prefill_m.split(",") if m]
        log(f"prefill timing M={Ms}")
        result["prefill"] = bench_prefill(torch, N_, stack, Ms, args.prefill_time, dev)
        log(f"prefill: {result['prefill']['TFLOPs']} TFLOP/s")
        log(f"backward dX timing M={Ms}")
        result["backward_dx"] = bench_prefill(torch, N_, stack, Ms, args.prefill_time, dev,
                                              backward=True)
        log(f"backward dX: {result['backward_dx']['TFLOPs']} TFLOP/s")
    if not args.no_encode:
        del stack
        torch.cuda.empty_cache()
        log(f"encode timing ({args.encode_layers}-layer stack)")
        result["encode"] = bench_encode(torch, N_, dev, args.encode_layers)
        log(f"encode: {result['encode']['Gweights_s']} Gweights/s, "
            f"bit-exact sample {result['encode']['bit_exact_sample']}")
    if args.e8b_layers > 0:
        torch.cuda.empty_cache()
        log(f"2-bit E8 ({args.e8b_layers}-layer stack)")
        result["e8_2bit"] = bench_e8b(torch, N_, dev, args.e8b_layers, args.steps)
        log(f"2-bit: decode M=1 {result['e8_2bit']['decode_per_linear']['1']['weight_GBs']} GB/s, "
            f"encode {result['e8_2bit']['encode']['Gweights_s']} Gweights/s")
        torch.cuda.empty_cache()
        log(f"1-bit Root E8 ({args.e8b_layers}-layer stack)")
        result["e8_1bit"] = bench_e8b(torch, N_, dev, args.e8b_layers, args.steps, fmt="root")
        log(f"1-bit: decode M=16 {result['e8_1bit']['decode_per_linear']['16']['weight_GBs']} GB/s")
    if args.e8b_grouped_layers > 0:
        torch.cuda.empty_cache()
        log(f"2-bit E8 grouped decode ({args.e8b_grouped_layers}-layer stack)")
        result["e8_2bit_grouped"] = bench_e8b_grouped(torch, dev, args.e8b_grouped_layers,
                                                      args.steps, args.warmup)
        log(f"2-bit grouped: {result['e8_2bit_grouped']['per_M']}")
        torch.cuda.empty_cache()
        log(f"1-bit Root E8 grouped decode ({args.e8b_grouped_layers}-layer stack)")
        result["e8_1bit_grouped"] = bench_e8b_grouped(torch, dev, args.e8b_grouped_layers,
                                                      args.steps, args.warmup, bitrate=1.0)
        log(f"1-bit grouped: {result['e8_1bit_grouped']['per_M']}")
    if args.gs_layers > 0:
        torch.cuda.empty_cache()
        log(f"ternary group sizes 32 / 16 / 64 ({args.gs_layers}-layer stack)")
        result["ternary_gs"] = bench_ternary_gs(torch, N_, dev, args.gs_layers, args.steps)
    if not args.no_e2e:
        torch.cuda.empty_cache()
        log(f"end-to-end decoder ({args.e2e_layers} layers)")
        result["e2e"] = bench_e2e(torch, dev, args.e2e_layers)
        log(f"e2e: decode {result['e2e']['decode_tokens_s']} tok/s, prefill "
            f"{result['e2e']['prefill_tokens_s']} tok/s")
    if not args.no_cpu_baseline:
        log(f"cpu baseline ({args.cpu_seconds:.0f} s sample)")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    else:
        result["cpu_baseline"] = None
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
