"""Benchmark of the quantized-matmul hot path on one MI355X.

Default workload (one "step"): the Q4_K x Q8_K decode GEMV shapes at batch 1 --
4096->4096, 4096->12288 and 12288->4096 -- each launch reading its own copy of the weights
(copies rotate over >= 768 MB so the 256 MB Infinity Cache never serves a repeat).  The
weights are GGUF Q4_K tensors re-laid out once at load into the planar Q4_K_R device layout
(jero_hip_repack, the layout the decode step runs on; same bytes); per_shape_gguf times the
same GEMV straight on the GGUF layout.  The
step is captured once in a HIP graph and replayed; HIP events on the replay stream time
the K steps.  `value` is algorithmic bytes (weights + Q8_K activation + f32 output) per
second over the whole step.  Extra fields: the Q6_K 4096->151936 output head, the per-shape
kernel averages, the pure-read ceiling of each shape (one launch that reads the same rotated
weight bytes and nothing else, jero_hip_read_probe) with the GEMV's ratio to it, and the Q8_0 x Q8_0
4096x4096 GEMV with its own ceiling and CPU line.

roofline: the Q4_K GEMV kernel (all three shapes): algorithmic bytes per launch over the
average launch duration measured with events; peak = 8 TB/s HBM.
cpu_baseline: the CPU oracle's GEMV (C restatement of the reference's matvec_any row-chunk
path, scalar, pthreads over all host cores) on the same three shapes.

Second part ("decode"): the full batch-1 decode step of a random-init Qwen3-8B-shaped model
in Q4_K_M (36 layers, hidden 4096, 32/8 heads of 128, FFN 12288, vocab 151936; Q6_K head and
Q6_K attn_v/ffn_down on 18 layers), f16 KV ring of 4096 slots pre-filled with N(0,1) values,
greedy next token.  One step is captured in a HIP graph; each replay decodes the next token
(the token and position advance on the device).  Reported as tokens/s and as fractions of the
weight-only (4.671 GB/token) and weights+KV (+0.604 GB) HBM rooflines, next to the oracle's
C decode step timed on the host cores.

Third and fourth parts: the Q4_K x Q8_K prefill GEMM (M=512, K=4096, N=14336) on int8 MFMA, as
TOP/s and fractions of the int8 peak, next to the oracle's per-token GEMV; and the Qwen3-MoE expert
layer (H=2048, 128 experts, FFN 768, top-8) at 1 and 64 tokens, as GB/s over the routed experts.

Fifth part ("forward_model"): the int8 ForwardModel matrix bench (prompt "hello world", vocab
256, n_ctx 64: 53 greedy tokens) through jero_hip_forward_model_evaluate, as prefill ms and decode
tokens/s, next to the oracle's scalar C evaluate of the same run (and whether its tokens agree).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode] [--no-gemm]
                       [--no-moe] [--no-forward] [--copy-probe MB]
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
QWEN3_8B = dict(hidden=4096, ffn=12288, n_layers=36, vocab=151936, nq=32, nkv=8, hd=128, eps=1e-6, theta=1e6)
KV_CAP = 4096


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


def q8_0_weights(torch, n_in, n_out, copies, dev, seed):
    """Q8_0 weights quantized from N(0, 0.02) floats (32-element blocks: f16 d = max|x|/127, int8
    round-to-nearest of x/d); 4 distinct matrices, their bytes repeated over `copies` buffers."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    mats = []
    for _ in range(min(4, copies)):
        x = (0.02 * torch.randn(n_out, n_in // 32, 32, generator=g, device=dev)).float()
        d = (x.abs().amax(dim=2, keepdim=True) / 127.0).half()
        q = torch.where(d.float() > 0, torch.round(x / d.float()), torch.zeros_like(x)).clamp(-127, 127)
        blk = torch.cat([d.view(torch.uint8).view(n_out, n_in // 32, 2),
                         q.to(torch.int8).view(torch.uint8)], dim=2)
        mats.append(blk.reshape(-1))
        del x, d, q
    return [mats[c % len(mats)].clone() for c in range(copies)]


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


def time_graph_dist(torch, fn, chunk, reps, stream):
    """Per-step time distribution: one graph of `chunk` steps (chunk covers every rotated weight
    copy, so no replay re-reads what the previous one left in the Infinity Cache), replayed `reps`
    times with events around each replay; returns the p10 / p50 / p90 of the per-step mean (us)."""
    import numpy as np
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        fn()
        stream.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for _ in range(chunk):
                fn()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    with torch.cuda.stream(stream):
        g.replay()  # warm replay
        ev[0].record(stream)
        for r in range(reps):
            g.replay()
            ev[r + 1].record(stream)
    ev[-1].synchronize()
    t = np.array([ev[r].elapsed_time(ev[r + 1]) * 1e3 / chunk for r in range(reps)])
    return {"p10_us": round(float(np.percentile(t, 10)), 3), "p50_us": round(float(np.median(t)), 3),
            "p90_us": round(float(np.percentile(t, 90)), 3), "replays": reps, "steps_per_replay": chunk}


def q6k_layers(n):
    """llama.cpp's Q4_K_M rule: Q6_K attn_v / ffn_down on these layers."""
    return [i for i in range(n) if i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2]


def decode_tensors(spec):
    """(name, quant, n_in, n_out) of the Q4_K_M Qwen3 model."""
    H, F, L, V = spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"]
    Q, KV, hd = spec["nq"] * spec["hd"], spec["nkv"] * spec["hd"], spec["hd"]
    hi = set(q6k_layers(L))
    out = [("token_embd.weight", 12, H, V), ("output.weight", 14, H, V), ("output_norm.weight", 0, H, 1)]
    for i in range(L):
        p = f"blk.{i}."
        out += [(p + "attn_norm.weight", 0, H, 1), (p + "ffn_norm.weight", 0, H, 1),
                (p + "attn_q_norm.weight", 0, hd, 1), (p + "attn_k_norm.weight", 0, hd, 1),
                (p + "attn_q.weight", 12, H, Q), (p + "attn_k.weight", 12, H, KV),
                (p + "attn_v.weight", 14 if i in hi else 12, H, KV), (p + "attn_output.weight", 12, Q, H),
                (p + "ffn_gate.weight", 12, H, F), (p + "ffn_up.weight", 12, H, F),
                (p + "ffn_down.weight", 14 if i in hi else 12, F, H)]
    return out


def bench_decode(torch, J, dev, stream, steps, warmup, keep_host):
    """Builds the model on the device, times graph-replayed decode steps; optionally returns
    host copies of every tensor and of the KV rings for the CPU baseline."""
    spec = QWEN3_8B
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], KV_CAP, J.KV_F16, True)
    host = {}
    weight_bytes = 0
    g = torch.Generator(device=dev)
    g.manual_seed(4242)
    for i, (name, quant, n_in, n_out) in enumerate(decode_tensors(spec)):
        if quant == 0:
            t = (1.0 + 0.1 * torch.randn(n_in, generator=g, device=dev)).float()
        else:
            t = synth_weights(torch, J, quant, n_in, n_out, 1, dev, 5000 + i)[0]
            if name != "token_embd.weight":
                weight_bytes += t.numel()
        m.set_tensor(name, quant, t, n_in, n_out)
        if keep_host:
            host[name] = (quant, t.cpu().numpy())
        del t
    m.finalize()
    kvd = spec["nkv"] * spec["hd"]
    host_kv = None
    if keep_host:
        import numpy as np
        host_kv = np.empty((spec["n_layers"], 2, KV_CAP, kvd), np.float32)
    for L in range(spec["n_layers"]):
        k = torch.randn(KV_CAP, kvd, generator=g, device=dev).half()
        v = torch.randn(KV_CAP, kvd, generator=g, device=dev).half()
        m.write_kv(L, k, v)
        if keep_host:
            host_kv[L, 0] = k.float().cpu().numpy()
            host_kv[L, 1] = v.float().cpu().numpy()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        m.set_position(1, KV_CAP - 1, stream=stream)
        for _ in range(max(1, warmup)):
            m.decode_step(stream=stream)
    stream.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            m.decode_step(stream=stream)
        graph.replay()
        stream.synchronize()
        s0, e0 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record(stream)
        for _ in range(steps):
            graph.replay()
        e0.record(stream)
    e0.synchronize()
    t_tok = s0.elapsed_time(e0) / 1e3 / steps
    tok, pos = m.read_token_pos()
    # prefill (extra): a 512-token prompt from position 0 through jero_hip_model_prefill, every
    # projection a GEMM over the 512 rows; one warm call allocates the row buffers and builds the
    # int8 planes of the Q6_K tensors
    import numpy as np
    n_pf = 512
    prompt = np.random.default_rng(5).integers(0, spec["vocab"], n_pf).tolist()
    with torch.cuda.stream(stream):
        m.prefill(prompt, 0, stream=stream)
        stream.synchronize()
        s1, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s1.record(stream)
        for _ in range(3):
            m.prefill(prompt, 0, stream=stream)
        e1.record(stream)
    e1.synchronize()
    t_pf = s1.elapsed_time(e1) / 1e3 / 3
    kv_bytes = spec["n_layers"] * 2 * KV_CAP * kvd * 2
    res = {"workload": "Qwen3-8B-shape Q4_K_M batch-1 greedy decode, 36 layers, f16 KV ring 4096 slots full",
           "tok_s": round(1.0 / t_tok, 1), "ms_per_token": round(t_tok * 1e3, 4), "steps": steps,
           "weight_bytes_per_token": weight_bytes, "kv_bytes_per_token": kv_bytes,
           "frac_weight_roofline": round(weight_bytes / t_tok / 1e9 / HBM_PEAK_GBS, 4),
           "frac_weights_kv_roofline": round((weight_bytes + kv_bytes) / t_tok / 1e9 / HBM_PEAK_GBS, 4),
           "last_token": tok, "position": pos, "graph": "one decode step captured, replayed per token",
           "prefill": {"tokens": n_pf, "ms": round(t_pf * 1e3, 3), "tok_s": round(n_pf / t_pf, 1),
                       "what": "jero_hip_model_prefill of a 512-token prompt from position 0 (GEMMs over the "
                               "token rows, causal attention), eager, events around 3 calls"}}
    m.close()
    return res, host, host_kv


INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
GEMM_SHAPE = (512, 4096, 14336)  # (tokens M, n_in K, n_out N), Q4_K weights


def bench_gemm(torch, J, dev, stream, steps, keep_host):
    """Prefill GEMM: Y[512, 14336] = X[512, 4096] (Q8_K) . W (Q4_K), int8 MFMA.  The weights are
    re-laid out once at load into the GEMM's fragment order (jero_hip_repack_gemm: Q4_K_G, the
    quants regrouped and the scales unpacked, 160 bytes per 256-block against 144, as the model's
    prefill holds them); the kernel over the GGUF bytes is timed too
    (`gguf`).  Weights rotate over 4 copies.  `mfma_issue_frac`: the MFMA work the kernel issues
    (two int8 planes of 2MNK ops each, plus the f16 mins product of 2MN*16 per block) over the
    time at peak."""
    M, K, N = GEMM_SHAPE
    copies = 4
    buf = synth_weights(torch, J, J.Q4_K, K, N, copies, dev, 3000)
    views = [J.TensorView("ffn_up", J.Q4_K, [K, N], buf[c]) for c in range(copies)]
    laid = [J.repack_gemm(v) for v in views]
    g = torch.Generator(device=dev)
    g.manual_seed(3001)
    x = torch.randn(M, K, generator=g, device=dev)
    xq = J.quantize_act(J.Q8_K, x)
    y = torch.empty(M, N, device=dev)
    ops = 2.0 * M * N * K
    issued = 2 * ops / (INT8_PEAK_TOPS * 1e12) + 2.0 * M * N * 16 * (K // 256) / (F16_PEAK_TFLOPS * 1e12)

    def timed(vs):
        cnt = [0]

        def one():
            J.gemm(vs[cnt[0] % copies], xq, M, y, stream=stream)
            cnt[0] += 1

        return time_graph(torch, one, steps, 3, stream)

    t = timed(laid)
    tg = timed(views)
    res = {"workload": f"Q4_K x Q8_K prefill GEMM M={M} K={K} N={N}, int8 MFMA, weights in the GEMM layout "
                       f"(Q4_K_G: the quants in MFMA fragment order, scales unpacked, repacked once at load)",
           "us": round(t * 1e6, 2), "tops": round(ops / t / 1e12, 1), "unit": "TOP/s", "peak": INT8_PEAK_TOPS,
           "frac_int8_peak": round(ops / t / 1e12 / INT8_PEAK_TOPS, 4),
           "mfma_issue_frac": round(issued / t, 4), "tokens_per_s": round(M / t, 1),
           "gguf": {"what": "the same GEMM over the GGUF Q4_K bytes (no repack)", "us": round(tg * 1e6, 2),
                    "tops": round(ops / tg / 1e12, 1), "frac_int8_peak": round(ops / tg / 1e12 / INT8_PEAK_TOPS, 4)}}
    host = None
    if keep_host:
        host = (buf[0].cpu().numpy(), xq.cpu().numpy())
    del buf, views, laid
    return res, host


def cpu_gemm_baseline(O, host, budget_s=8.0):
    """The oracle's GEMM (prefill = one matvec_any per token, C restatement, scalar, pthreads over
    all host cores) on the same weights, a bounded number of token rows."""
    M, K, N = GEMM_SHAPE
    w, xq = host
    threads = len(os.sched_getaffinity(0))
    rb = len(xq) // M
    t0 = time.perf_counter()
    rows = 0
    while time.perf_counter() - t0 < budget_s and rows < M:
        O.matvec(12, w, K, N, xq[rows * rb:(rows + 1) * rb], threads=threads)
        rows += 1
    el = time.perf_counter() - t0
    return rows / el, threads, rows, el


MOE = dict(hidden=2048, experts=128, ffn=768, top_k=8)


def bench_moe(torch, J, dev, stream, steps):
    """Qwen3-MoE expert layer: H=2048, 128 experts of FFN 768 (gate/up Q4_K, down Q6_K, repacked
    at load time), router logits N(0,1), top-8; T=1 (decode) and T=64.  Two weight copies and 8
    logit sets rotate, so the experts read differ between launches.  Algorithmic bytes: the
    distinct routed experts' weights (3.06 MB each) + activations."""
    H, E, F, k = MOE["hidden"], MOE["experts"], MOE["ffn"], MOE["top_k"]
    copies = 2
    gate = synth_weights(torch, J, J.Q4_K, H, E * F, copies, dev, 3100)
    up = synth_weights(torch, J, J.Q4_K, H, E * F, copies, dev, 3101)
    down = synth_weights(torch, J, J.Q6_K, F, E * H, copies, dev, 3102)
    # the expert tensors in the load-time device layouts (Q4_K_T / Q6_K_T: 16-row tiles)
    gv = [J.repack(J.TensorView("ffn_gate_exps", J.Q4_K, [H, F, E], gate[c])) for c in range(copies)]
    uv = [J.repack(J.TensorView("ffn_up_exps", J.Q4_K, [H, F, E], up[c])) for c in range(copies)]
    dv = [J.repack(J.TensorView("ffn_down_exps", J.Q6_K, [F, H, E], down[c])) for c in range(copies)]
    per_expert = (J.row_bytes(J.Q4_K, H) * F * 2 + J.row_bytes(J.Q6_K, F) * H)
    g = torch.Generator(device=dev)
    g.manual_seed(3103)
    out = {}
    for T in (1, 64):
        x = torch.randn(T, H, generator=g, device=dev)
        logits = [torch.randn(T, E, generator=g, device=dev) for _ in range(8)]
        y = torch.empty(T, H, device=dev)
        ws = torch.empty(J.lib().jero_hip_moe_workspace_bytes(T, E, k, H, F), dtype=torch.uint8, device=dev)
        cnt = [0]
        sels = []

        def one():
            c = cnt[0]
            sel, _ = J.dispatch_qwen3_moe_ffn(y, x, logits[c % 8], k, gv[c % copies], uv[c % copies],
                                             dv[c % copies], workspace=ws, stream=stream)
            if len(sels) < 8:
                sels.append(sel)
            cnt[0] += 1

        t = time_graph(torch, one, steps, 1, stream)
        distinct = sum(len(set(s.cpu().numpy().reshape(-1).tolist())) for s in sels[:8]) / len(sels[:8])
        algo = distinct * per_expert + T * H * 4 * 2 + T * E * 4
        out[f"T{T}"] = {"us": round(t * 1e6, 2), "distinct_experts": round(distinct, 1),
                        "bytes": int(algo), "GB_s": round(algo / t / 1e9, 1),
                        "frac_hbm": round(algo / t / 1e9 / HBM_PEAK_GBS, 4)}
    out["workload"] = "Qwen3-MoE expert layer H=2048, E=128, F=768, top-8, gate/up Q4_K, down Q6_K"
    out["weight_layout"] = "Q4_K_T / Q6_K_T (16-row tiles; load-time repack of the GGUF expert tensors)"
    del gate, up, down, gv, uv, dv
    return out


def bench_q8_0(torch, J, dev, stream, steps, warmup, keep_host):
    """Q8_0 x Q8_0 GEMV 4096x4096, batch 1 (weights N(0,0.02) quantized to Q8_0, activation N(0,1)
    quantized to the 32-element Q8 activation blocks), copies rotating over >= 768 MB; with the
    pure-read ceiling over the same buffers."""
    n_in = n_out = 4096
    nbytes = J.row_bytes(J.Q8_0, n_in) * n_out
    copies = max(2, int(-(-ROTATE_BYTES // nbytes)))
    bufs = q8_0_weights(torch, n_in, n_out, copies, dev, 4000)
    views = [J.TensorView("w", J.Q8_0, [n_in, n_out], b) for b in bufs]
    x = torch.randn(n_in, generator=torch.Generator(device=dev).manual_seed(4001), device=dev)
    xq = J.quantize_act(J.ACT_Q8, x)
    y = torch.empty(n_out, dtype=torch.float32, device=dev)
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    cnt = [0]

    def one():
        J.matvec(views[cnt[0] % copies], xq, y, stream=stream)
        cnt[0] += 1

    def probe():
        J.read_probe(bufs[cnt[0] % copies], sink, stream=stream)
        cnt[0] += 1

    t = time_graph(torch, one, steps, warmup, stream)
    tc = time_graph(torch, probe, steps, warmup, stream)
    algo = nbytes + J.row_bytes(J.ACT_Q8, n_in) + 4 * n_out
    res = {"workload": "Q8_0 x Q8_0 GEMV 4096x4096, batch 1", "us": round(t * 1e6, 3),
           "GB_s": round(algo / t / 1e9, 1), "bytes": algo, "frac_hbm": round(algo / t / 1e9 / HBM_PEAK_GBS, 4),
           "read_ceiling_us": round(tc * 1e6, 3), "gemv_over_ceiling": round(tc / t, 4)}
    host = (bufs[0].cpu().numpy(), xq.cpu().numpy()) if keep_host else None
    del bufs, views
    return res, host


def cpu_q8_0_baseline(O, host, budget_s=5.0):
    """The oracle's Q8_0 GEMV (matvec_any row chunks, scalar, pthreads over all host cores)."""
    w, xq = host
    threads = len(os.sched_getaffinity(0))
    done, t0 = 0, time.perf_counter()
    while True:
        O.matvec(O.Q8_0, w, 4096, 4096, xq, threads=threads)
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return (w.size + xq.size + 4 * 4096) * done / el / 1e9, threads, done, el


def cpu_decode_baseline(O, host, host_kv, budget_s=10.0):
    """The oracle's decode step (execute_token_standard_with_hidden restated in C, scalar,
    pthreads over all host cores) on the same weights and KV values (widened to f32)."""
    spec = QWEN3_8B
    threads = len(os.sched_getaffinity(0))
    om = O.DecodeModel(spec, host, KV_CAP)
    done, t0, tok = 0, time.perf_counter(), 1
    pos = KV_CAP - 1
    while True:
        logits = om.step(host_kv, tok, pos, threads=threads)
        tok = int(logits.argmax())
        pos += 1
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return done / el, threads, done, el


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
        if el >= budget_s:
            break
    return per_step * done / el / 1e9, threads, done, el


def fnv1a(text):
    """The matrix bench's model seed: FNV-1a of the prompt text (src/bin/jero-diag/bench.rs:1142-1147)."""
    h = 0xCBF29CE484222325
    for b in text.encode():
        h = ((h ^ b) * 0x100000001B3) & ((1 << 64) - 1)
    return h


FWD_PROMPT_TEXT, FWD_VOCAB, FWD_CTX = "hello world", 256, 64
FWD_LAYER_MACS = 4 * (4 * 512 * 512 + 2 * 512 * 1024)  # ForwardModel::layer_macs_per_token


def bench_forward_model(J, reps):
    """The int8 ForwardModel's matrix bench (src/bin/jero-diag/bench.rs:1125-1148 -> evaluate): prompt
    "hello world" as byte tokens, vocab 256, n_ctx 64, so 11 prompt tokens and 53 generated."""
    import numpy as np
    prompt = list(FWD_PROMPT_TEXT.encode())
    max_tokens = min(128, FWD_CTX - len(prompt))
    m = J.ForwardModel(fnv1a(FWD_PROMPT_TEXT), FWD_VOCAB, FWD_CTX)
    toks, _ = m.evaluate(prompt, max_tokens, timing=True)  # warm-up
    pre, dec, wall = [], [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        t, (p_ms, d_ms) = m.evaluate(prompt, max_tokens, timing=True)
        wall.append(time.perf_counter() - t0)
        assert t == toks, "ForwardModel evaluate is not deterministic"
        pre.append(p_ms)
        dec.append(d_ms)
    m.close()
    steps = max_tokens - 1
    d_ms = float(np.median(dec))
    macs = FWD_LAYER_MACS + FWD_VOCAB * 512
    return {
        "workload": "ForwardModel (4 layers, dim 512, FFN 1024, vocab 256), prompt 'hello world' (11 byte tokens), "
                    f"{max_tokens} greedy tokens, n_ctx {FWD_CTX}",
        "reps": reps,
        "prefill_ms": round(float(np.median(pre)), 4),
        "decode_ms": round(d_ms, 4),
        "decode_tok_s": round(steps / (d_ms * 1e-3), 1),
        "decode_us_per_token": round(d_ms * 1e3 / steps, 2),
        "decode_gmac_s": round(macs * steps / (d_ms * 1e-3) / 1e9, 2),
        "evaluate_wall_ms": round(float(np.median(wall)) * 1e3, 3),
        "tokens": toks,
    }, (prompt, max_tokens)


def cpu_forward_baseline(O, prompt, max_tokens, budget_s=3.0):
    """The oracle's ForwardModel evaluate (scalar C restatement, one thread) on the same workload."""
    f = O.ForwardModel(fnv1a(FWD_PROMPT_TEXT), FWD_VOCAB, FWD_CTX, threads=1)
    reps, toks, t0 = 0, None, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or reps == 0:
        toks = f.evaluate(prompt, max_tokens)
        reps += 1
    el = time.perf_counter() - t0
    return reps * max_tokens / el, reps, el, toks


def measured_traffic():
    """HBM bytes per Q4_K GEMV launch (mean of the three shapes) from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes, each scaled by the counter's reading for a 512 MB copy; None if
    the summary is absent."""
    path = os.path.join(ROOT, "profiles", "gemv_q4k_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)["q4k_gemv_traffic_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-gemm", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--no-forward", action="store_true")
    ap.add_argument("--decode-steps", type=int, default=50)
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

    # ---- Q4_K decode shapes: the GGUF tensors re-laid out once at load (Q4_K -> Q4_K_R, the
    # layout the decode step runs on); the GGUF-layout kernel is timed too (per_shape_gguf)
    bufs, xqs, ys, views, raw_views, algo = [], [], [], [], [], []
    for i, (n_in, n_out) in enumerate(SHAPES):
        nbytes = J.row_bytes(J.Q4_K, n_in) * n_out
        copies = max(2, int(np.ceil(ROTATE_BYTES / nbytes)))
        buf = synth_weights(torch, J, J.Q4_K, n_in, n_out, copies, dev, 1000 + i)
        bufs.append(buf)
        raw_views.append([J.TensorView(f"w{i}", J.Q4_K, [n_in, n_out], buf[c]) for c in range(copies)])
        views.append([J.repack(v) for v in raw_views[-1]])
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
    max_copies = max(len(v) for v in views)
    step_dist = time_graph_dist(torch, step, max_copies, 21, stream)

    # per-shape kernel averages (same method, one shape per graph), planar and GGUF layouts
    per_shape, per_shape_gguf = {}, {}
    for table, vlist in ((per_shape, views), (per_shape_gguf, raw_views)):
        for i, (n_in, n_out) in enumerate(SHAPES):
            cnt = [0]

            def one(i=i, cnt=cnt, vlist=vlist):
                vv = vlist[i]
                J.matvec(vv[cnt[0] % len(vv)], xqs[i], ys[i], stream=stream)
                cnt[0] += 1

            t = time_graph(torch, one, args.steps, args.warmup, stream)
            table[f"{n_in}x{n_out}"] = {"us": round(t * 1e6, 3), "GB_s": round(algo[i] / t / 1e9, 1),
                                        "bytes": algo[i],
                                        "dist": time_graph_dist(torch, one, len(vlist[i]), 21, stream)}
    # pure-read ceiling: one launch per shape reading the same rotated buffers and nothing else
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    ceiling = {}
    for i, (n_in, n_out) in enumerate(SHAPES):
        cnt = [0]

        def probe(i=i, cnt=cnt):
            vv = views[i]
            J.read_probe(vv[cnt[0] % len(vv)].data, sink, stream=stream)
            cnt[0] += 1

        tc = time_graph(torch, probe, args.steps, args.warmup, stream)
        key = f"{n_in}x{n_out}"
        per_shape[key]["read_ceiling_us"] = round(tc * 1e6, 3)
        per_shape[key]["gemv_over_ceiling"] = round(tc * 1e6 / per_shape[key]["us"], 4)
        ceiling[key] = tc
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

    # ---- Q8_0 4096x4096 (the reference's CPU-runnable case; extra)
    q8_0, q8host = bench_q8_0(torch, J, dev, stream, args.steps, args.warmup, not args.no_cpu)
    torch.cuda.empty_cache()

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

    if q8host is not None:
        import pyoracle as O
        gbs, threads, reps, el = cpu_q8_0_baseline(O, q8host)
        q8_0["cpu_baseline"] = {"value": round(gbs, 2), "unit": "GB/s", "cores": threads, "kind": "port",
                                "sample": f"{reps} full GEMVs, {el:.1f} s, C restatement of matvec_any row chunks"}

    # ---- prefill GEMM (extra)
    gemm = None
    if not args.no_gemm:
        gemm, ghost = bench_gemm(torch, J, dev, stream, max(10, args.steps // 10), not args.no_cpu)
        torch.cuda.empty_cache()
        if ghost is not None:
            import pyoracle as O
            tps, threads, rows, el = cpu_gemm_baseline(O, ghost)
            gemm["cpu_baseline"] = {"value": round(tps, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
                                    "sample": f"{rows} of the 512 token rows (matvec_any per token), {el:.1f} s"}

    # ---- routed experts (extra)
    moe = None
    if not args.no_moe:
        moe = bench_moe(torch, J, dev, stream, max(20, args.steps // 5))
        torch.cuda.empty_cache()

    # ---- int8 ForwardModel matrix bench (extra)
    fwd = None
    if not args.no_forward:
        fwd, (fprompt, fmax) = bench_forward_model(J, 20)
        if not args.no_cpu:
            import pyoracle as O
            tps, reps, el, ctoks = cpu_forward_baseline(O, fprompt, fmax)
            fwd["cpu_baseline"] = {"value": round(tps, 1), "unit": "generated tok/s (prefill included)", "cores": 1,
                                   "kind": "port", "tokens_equal": ctoks == fwd["tokens"],
                                   "sample": f"{reps} full evaluate runs, {el:.1f} s, scalar C restatement"}
            fwd["evaluate_tok_s"] = round(fmax / (fwd["evaluate_wall_ms"] * 1e-3), 1)

    # ---- full decode step (extra)
    decode = None
    if not args.no_decode:
        del bufs, views
        torch.cuda.empty_cache()
        decode, host, host_kv = bench_decode(torch, J, dev, stream, args.decode_steps, 3, not args.no_cpu)
        if not args.no_cpu:
            import pyoracle as O
            tps, threads, reps, el = cpu_decode_baseline(O, host, host_kv)
            decode["cpu_baseline"] = {"value": round(tps, 3), "unit": "tok/s", "cores": threads, "kind": "port",
                                      "sample": f"{reps} greedy steps of the same model from position {KV_CAP - 1}, "
                                                f"{el:.1f} s, f32 KV ring"}
            del host, host_kv

    out = {
        "metric": "Q4_K GEMV GB/s (% HBM peak); decode tok/s, 8B-shape Q4_K_M, 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(t_step * 1e3, 5),
        "step_dist": step_dist,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: random-init Q4_K weights (uniform payload, N(0,0.02)-scale fields), N(0,1) activations",
        "config": {"workload": "Q4_K x Q8_K decode GEMV, batch 1: 4096->4096, 4096->12288, 12288->4096",
                   "weight_layout": "Q4_K_R (GGUF Q4_K bytes re-laid out once at load by jero_hip_repack)",
                   "rotated_weight_bytes": int(ROTATE_BYTES), "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic()},
        "cpu_baseline": cpu,
        "per_shape": per_shape,
        "per_shape_gguf": per_shape_gguf,
        "read_ceiling": {"what": "one launch per shape that only reads the same rotated weight bytes "
                                 "(jero_hip_read_probe); per_shape[...].gemv_over_ceiling = ceiling / GEMV time",
                         "step_us": round(sum(ceiling.values()) * 1e6, 3),
                         "gemv_step_over_ceiling": round(sum(ceiling.values()) / t_step, 4)},
        "q8_0_4096": q8_0,
        "q6k_head": head,
        "prefill_gemm": gemm,
        "moe": moe,
        "decode": decode,
        "forward_model": fwd,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
