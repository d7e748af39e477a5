"""Benchmark of the quantized-matmul hot path on one MI355X.

Default workload (one "step"): the Q4_K x Q8_K decode GEMV shapes at batch 1 --
4096->4096, 4096->12288 and 12288->4096 -- each launch reading its own copy of the weights
(copies rotate over >= 768 MB so the 256 MB Infinity Cache never serves a repeat).  The
step is captured once in a HIP graph and replayed; HIP events on the replay stream time
the K steps.  `value` is algorithmic bytes (weights + Q8_K activation + f32 output) per
second over the whole step.  Extra fields: the Q6_K 4096->151936 output head, and the
per-shape kernel averages.

roofline: the Q4_K GEMV kernel (all three shapes): algorithmic bytes per launch over the
average launch duration measured with events; peak = 8 TB/s HBM.
cpu_baseline: the CPU oracle's GEMV (C restatement of the reference's matvec_any row-chunk
path, scalar, pthreads over all host cores) on the same three shapes.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--copy-probe MB]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "jero-engine_amd"), os.path.join(ROOT, "oracle")]

HBM_PEAK_GBS = 8000.0
SHAPES = [(4096, 4096), (4096, 12288), (12288, 4096)]  # (n_in, n_out), Q4_K
HEAD = (4096, 151936)  # Q6_K output head
ROTATE_BYTES = 768e6


def synth_weights(torch, J, quant, n_in, n_out, copies, dev, seed):
    """Random-init quantized weights of the given shape (uniform payload bytes, f16 scale
    fields at the magnitudes N(0, 0.02) weights quantize to), `copies` distinct buffers."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    rb = J.row_bytes(quant, n_in)
    nbytes = rb * n_out
    buf = torch.randint(0, 256, (copies, nbytes), dtype=torch.uint8, device=dev, generator=g)
    blk = 144 if quant == J.Q4_K else 210
    v = buf.view(copies, -1, blk)
    nb = v.shape[1]
    if quant == J.Q4_K:
        d = (torch.rand(copies, nb, device=dev, generator=g) * 3e-4 + 1e-4).half().view(torch.uint8)
        m = (torch.rand(copies, nb, device=dev, generator=g) * 1.5e-3 + 5e-4).half().view(torch.uint8)
        v[:, :, 0:2] = d.view(copies, nb, 2)
        v[:, :, 2:4] = m.view(copies, nb, 2)
    else:
        d = (torch.rand(copies, nb, device=dev, generator=g) * 2e-4 + 1e-4).half().view(torch.uint8)
        v[:, :, 208:210] = d.view(copies, nb, 2)
        sc = torch.randint(-64, 64, (copies, nb, 16), dtype=torch.int8, device=dev, generator=g)
        v[:, :, 192:208] = sc.view(torch.uint8)
    return buf


def time_graph(torch, fn, steps, warmup, stream):
    """Captures `fn` (one step) `steps` times in a graph; returns (seconds per step)."""
    with torch.cuda.stream(stream):
        for _ in range(max(warmup, 1)):
            fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            for _ in range(steps):
                fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):  # graph replays run on the current stream
        g.replay()  # warm replay
        stream.synchronize()
        s.record(stream)
        g.replay()
        e.record(stream)
    e.synchronize()
    return s.elapsed_time(e) / 1e3 / steps


def cpu_baseline(O, host_w, host_xq, budget_s=12.0):
    """Times the oracle's threaded GEMV on the same shapes; returns GB/s and the sample."""
    threads = len(os.sched_getaffinity(0))
    done, t0, nbytes = 0, time.perf_counter(), 0
    per_step = sum(w.size for w in host_w) + sum(x.size for x in host_xq) + 4 * sum(n for _, n in SHAPES)
    while True:
        for (n_in, n_out), w, xq in zip(SHAPES, host_w, host_xq):
            O.matvec(O.Q4_K, w, n_in, n_out, xq, threads=threads)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s or done >= 2000:
            break
    return per_step * done / el / 1e9, threads, done, el


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=float, default=0.0,
                    help="also run one device copy of this many MB (PMC byte-counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import jero_hip as J
    J.init(0)
    dev = torch.device("cuda", 0)
    stream = torch.cuda.Stream()

    if args.copy_probe > 0:
        n = int(args.copy_probe * 1e6) // 4
        a = torch.ones(n, dtype=torch.float32, device=dev)
        b = torch.empty_like(a)
        b.copy_(a)
        torch.cuda.synchronize()
        del a, b

    # ---- Q4_K decode shapes
    bufs, xqs, ys, views, algo = [], [], [], [], []
    for i, (n_in, n_out) in enumerate(SHAPES):
        nbytes = J.row_bytes(J.Q4_K, n_in) * n_out
        copies = max(2, int(np.ceil(ROTATE_BYTES / nbytes)))
        buf = synth_weights(torch, J, J.Q4_K, n_in, n_out, copies, dev, 1000 + i)
        bufs.append(buf)
        views.append([J.TensorView(f"w{i}", J.Q4_K, [n_in, n_out], buf[c]) for c in range(copies)])
        x = torch.randn(n_in, generator=torch.Generator(device=dev).manual_seed(7 + i), device=dev)
        xqs.append(J.quantize_act(J.Q8_K, x))
        ys.append(torch.empty(n_out, dtype=torch.float32, device=dev))
        algo.append(nbytes + J.row_bytes(J.Q8_K, n_in) + 4 * n_out)
    torch.cuda.synchronize()

    counter = [0]

    def step():
        c = counter[0]
        for i in range(len(SHAPES)):
            vv = views[i]
            J.matvec(vv[c % len(vv)], xqs[i], ys[i], stream=stream)
        counter[0] += 1

    t_step = time_graph(torch, step, args.steps, args.warmup, stream)
    step_bytes = sum(algo)
    value = step_bytes / t_step / 1e9

    # per-shape kernel averages (same method, one shape per graph)
    per_shape = {}
    for i, (n_in, n_out) in enumerate(SHAPES):
        cnt = [0]

        def one(i=i, cnt=cnt):
            vv = views[i]
            J.matvec(vv[cnt[0] % len(vv)], xqs[i], ys[i], stream=stream)
            cnt[0] += 1

        t = time_graph(torch, one, args.steps, args.warmup, stream)
        per_shape[f"{n_in}x{n_out}"] = {"us": round(t * 1e6, 3), "GB_s": round(algo[i] / t / 1e9, 1),
                                        "bytes": algo[i]}
    gemv_launch_us = t_step * 1e6 / len(SHAPES)
    achieved = (step_bytes / len(SHAPES)) / (gemv_launch_us * 1e-6) / 1e9

    # ---- Q6_K head (extra)
    head = {}
    n_in, n_out = HEAD
    hbytes = J.row_bytes(J.Q6_K, n_in) * n_out
    hbuf = synth_weights(torch, J, J.Q6_K, n_in, n_out, 2, dev, 2000)
    hv = [J.repack(J.TensorView("output.weight", J.Q6_K, [n_in, n_out], hbuf[c])) for c in range(2)]
    del hbuf
    hx = J.quantize_act(J.Q8_K, torch.randn(n_in, device=dev))
    hy = torch.empty(n_out, dtype=torch.float32, device=dev)
    hc = [0]

    def head_step():
        J.matvec(hv[hc[0] % 2], hx, hy, stream=stream)
        hc[0] += 1

    th = time_graph(torch, head_step, max(10, args.steps // 10), 2, stream)
    h_algo = hbytes + J.row_bytes(J.Q8_K, n_in) + 4 * n_out
    head = {"shape": "Q6_K 4096x151936 (planar device layout)", "us": round(th * 1e6, 2), "GB_s": round(h_algo / th / 1e9, 1),
            "frac_hbm": round(h_algo / th / 1e9 / HBM_PEAK_GBS, 4)}
    del hv

    # ---- CPU baseline: the oracle's GEMV on the same three shapes
    cpu = None
    if not args.no_cpu:
        import pyoracle as O
        host_w = [bufs[i][0].cpu().numpy() for i in range(len(SHAPES))]
        host_xq = [xqs[i].cpu().numpy() for i in range(len(SHAPES))]
        gbs, threads, reps, el = cpu_baseline(O, host_w, host_xq)
        cpu = {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"{reps} passes over the three Q4_K shapes (66.2 MB of weights, full size), "
                         f"{el:.1f} s, C restatement of matvec_any row chunks, scalar, pthreads"}

    out = {
        "metric": "Q4_K GEMV GB/s (% HBM peak); decode tok/s, 8B-shape Q4_K_M, 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: random-init Q4_K weights (uniform payload, N(0,0.02)-scale fields), N(0,1) activations",
        "config": {"workload": "Q4_K x Q8_K decode GEMV, batch 1: 4096->4096, 4096->12288, 12288->4096",
                   "rotated_weight_bytes": int(ROTATE_BYTES), "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
        "per_shape": per_shape,
        "q6k_head": head,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
