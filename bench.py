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

Sixth part ("moe_decode"): the same decode step for a random-init Qwen3-30B-A3B-shaped model
(48 layers, hidden 2048, 32/4 heads of 128, 128 experts of FFN 768, top-8, vocab 151936; Q4_K_M),
as tokens/s and fractions of the HBM roofline over the bytes one token reads (attention, router,
the 8 routed experts of every layer, head; + the KV ring), next to the oracle's step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-decode] [--no-gemm]
                       [--no-moe] [--no-forward] [--no-dense-decode] [--no-moe-layer] [--copy-probe MB]
(--no-decode and --no-moe each also skip moe_decode)
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
PF_REPS = 15


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


def time_graph(torch, fn, steps, warmup, stream, span=1):
    """Captures `fn` (one step) max(steps, span) times in a graph and times one replay after a
    warm one; returns seconds per step.  `span` is the number of steps after which the rotated
    weight copies repeat, so a graph of at least that many steps never replays a copy that the
    previous replay left in the Infinity Cache."""
    n = max(steps, span)
    with torch.cuda.stream(stream):
        for _ in range(max(warmup, 1)):
            fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(g, stream=stream):
            for _ in range(n):
                fn()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):  # graph replays run on the current stream
        g.replay()  # warm replay
        stream.synchronize()
        s.record(stream)
        g.replay()
        e.record(stream)
    e.synchronize()
    return s.elapsed_time(e) / 1e3 / n


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
    # int8 planes of the Q6_K tensors.  The prompt sits in pinned host memory (its 2 KB upload is
    # an asynchronous copy inside each call); events around each of PF_REPS back-to-back calls
    import numpy as np
    n_pf = 512
    prompt = torch.tensor(np.random.default_rng(5).integers(0, spec["vocab"], n_pf), dtype=torch.int32).pin_memory()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(PF_REPS + 1)]
    host_s = []
    with torch.cuda.stream(stream):
        m.prefill(prompt, 0, stream=stream)
        stream.synchronize()
        ev[0].record(stream)
        for r in range(PF_REPS):
            h0 = time.perf_counter()
            m.prefill(prompt, 0, stream=stream)
            host_s.append(time.perf_counter() - h0)
            ev[r + 1].record(stream)
    ev[-1].synchronize()
    pf = np.array([ev[r].elapsed_time(ev[r + 1]) for r in range(PF_REPS)])  # ms per call
    t_pf = float(np.median(pf)) * 1e-3
    kv_bytes = spec["n_layers"] * 2 * KV_CAP * kvd * 2
    res = {"workload": "Qwen3-8B-shape Q4_K_M batch-1 greedy decode, 36 layers, f16 KV ring 4096 slots full",
           "tok_s": round(1.0 / t_tok, 1), "ms_per_token": round(t_tok * 1e3, 4), "steps": steps,
           "weight_bytes_per_token": weight_bytes, "kv_bytes_per_token": kv_bytes,
           "frac_weight_roofline": round(weight_bytes / t_tok / 1e9 / HBM_PEAK_GBS, 4),
           "frac_weights_kv_roofline": round((weight_bytes + kv_bytes) / t_tok / 1e9 / HBM_PEAK_GBS, 4),
           "last_token": tok, "position": pos, "graph": "one decode step captured, replayed per token",
           "prefill": {"tokens": n_pf, "ms": round(t_pf * 1e3, 3), "tok_s": round(n_pf / t_pf, 1),
                       "ms_p10": round(float(np.percentile(pf, 10)), 3), "ms_p90": round(float(np.percentile(pf, 90)), 3),
                       "ms_min": round(float(pf.min()), 3), "ms_max": round(float(pf.max()), 3), "calls": PF_REPS,
                       "host_enqueue_ms": round(float(np.median(host_s)) * 1e3, 3),
                       "what": "jero_hip_model_prefill of a 512-token prompt from position 0 (GEMMs over the "
                               "token rows, causal attention), eager, prompt in pinned host memory; median of "
                               "per-call events over back-to-back calls (ms); host_enqueue_ms: the host's time "
                               "to enqueue one call"}}
    m.close()
    return res, host, host_kv


QWEN3_30B_A3B = dict(hidden=2048, ffn=6144, n_layers=48, vocab=151936, nq=32, nkv=4, hd=128, eps=1e-6, theta=1e6)
QWEN3_30B_A3B_MOE = (128, 8, 768, False)  # (experts, top_k, expert FFN, shared expert)


def moe_decode_tensors(spec, moe):
    """(name, quant, dims) of the Q4_K_M Qwen3-MoE model: the Qwen3 attention of decode_tensors,
    an F32 router [hidden, E] and stacked experts per layer (gate / up Q4_K [hidden, F, E], down
    [F, hidden, E] Q6_K on the Q4_K_M rule's layers, else Q4_K)."""
    E, _, F, _ = moe
    H, L = spec["hidden"], spec["n_layers"]
    hi = set(q6k_layers(L))
    out = []
    for name, quant, n_in, n_out in decode_tensors(spec):
        if ".ffn_gate." in name or ".ffn_up." in name or ".ffn_down." in name:
            continue
        out.append((name, quant, (n_in, n_out) if n_out > 1 else (n_in,)))
    for i in range(L):
        p = f"blk.{i}."
        out += [(p + "ffn_gate_inp.weight", 0, (H, E)), (p + "ffn_gate_exps.weight", 12, (H, F, E)),
                (p + "ffn_up_exps.weight", 12, (H, F, E)), (p + "ffn_down_exps.weight", 14 if i in hi else 12, (F, H, E))]
    return out


def bench_moe_decode(torch, J, dev, stream, steps, warmup, keep_host):
    """The batch-1 decode step of a random-init Qwen3-30B-A3B-shaped model (48 layers, hidden 2048,
    32/4 heads of 128, 128 experts of FFN 768, top-8, vocab 151936) in Q4_K_M, f16 KV ring of 4096
    slots pre-filled, greedy next token; one step captured in a HIP graph, each replay the next
    token.  Algorithmic bytes per token: every attention / router / norm weight, the 8 routed
    experts of every layer, the head, and the KV ring."""
    import numpy as np
    spec, moe = QWEN3_30B_A3B, QWEN3_30B_A3B_MOE
    E, k, F, _ = moe
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], KV_CAP, J.KV_F16, True, moe=moe)
    host = {}
    dense_bytes, expert_bytes, total = 0, 0, 0
    g = torch.Generator(device=dev)
    g.manual_seed(4343)
    for i, (name, quant, dims) in enumerate(moe_decode_tensors(spec, moe)):
        n_in, n_out = dims[0], int(np.prod(dims[1:]))
        if quant == 0:
            t = (1.0 + 0.1 * torch.randn(n_in * n_out, generator=g, device=dev)).float() if n_out == 1 else \
                (0.02 * torch.randn(n_in * n_out, generator=g, device=dev)).float()
            nbytes = 4 * n_in * n_out
        else:
            t = synth_weights(torch, J, quant, n_in, n_out, 1, dev, 7000 + i)[0]
            nbytes = t.numel()
        total += nbytes
        if "_exps." in name:
            expert_bytes += nbytes // E * k  # the k routed experts of the layer
        elif name != "token_embd.weight":
            dense_bytes += nbytes
        m.set_tensor(name, quant, t, n_in, n_out)
        if keep_host:
            host[name] = (quant, t.cpu().numpy(), list(dims))
        del t
    m.finalize()
    kvd = spec["nkv"] * spec["hd"]
    host_kv = np.empty((spec["n_layers"], 2, KV_CAP, kvd), np.float32) if keep_host else None
    for L in range(spec["n_layers"]):
        kk = torch.randn(KV_CAP, kvd, generator=g, device=dev).half()
        vv = torch.randn(KV_CAP, kvd, generator=g, device=dev).half()
        m.write_kv(L, kk, vv)
        if keep_host:
            host_kv[L, 0] = kk.float().cpu().numpy()
            host_kv[L, 1] = vv.float().cpu().numpy()
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
    # prefill (extra): a 512-token prompt from position 0, every layer's experts as GEMMs over the
    # tokens each expert was routed (jero_hip_model_prefill's batched MoE pass); timed as the dense
    # model's prefill is
    n_pf = 512
    prompt = torch.tensor(np.random.default_rng(6).integers(0, spec["vocab"], n_pf), dtype=torch.int32).pin_memory()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(PF_REPS + 1)]
    with torch.cuda.stream(stream):
        m.prefill(prompt, 0, stream=stream)
        stream.synchronize()
        ev[0].record(stream)
        for r in range(PF_REPS):
            m.prefill(prompt, 0, stream=stream)
            ev[r + 1].record(stream)
    ev[-1].synchronize()
    pf = np.array([ev[r].elapsed_time(ev[r + 1]) for r in range(PF_REPS)])
    t_pf = float(np.median(pf)) * 1e-3
    m.close()
    kv_bytes = spec["n_layers"] * 2 * KV_CAP * kvd * 2
    wb = dense_bytes + expert_bytes
    res = {"workload": "Qwen3-30B-A3B-shape Q4_K_M batch-1 greedy decode, 48 layers, 128 experts top-8, "
                       "f16 KV ring 4096 slots full",
           "tok_s": round(1.0 / t_tok, 1), "ms_per_token": round(t_tok * 1e3, 4), "steps": steps,
           "model_bytes": total, "weight_bytes_per_token": wb, "kv_bytes_per_token": kv_bytes,
           "frac_weight_roofline": round(wb / t_tok / 1e9 / HBM_PEAK_GBS, 4),
           "frac_weights_kv_roofline": round((wb + kv_bytes) / t_tok / 1e9 / HBM_PEAK_GBS, 4),
           "last_token": tok, "position": pos, "graph": "one decode step captured, replayed per token",
           "prefill": {"tokens": n_pf, "ms": round(t_pf * 1e3, 3), "tok_s": round(n_pf / t_pf, 1),
                       "ms_p10": round(float(np.percentile(pf, 10)), 3), "ms_p90": round(float(np.percentile(pf, 90)), 3),
                       "calls": PF_REPS,
                       "what": "jero_hip_model_prefill of a 512-token prompt from position 0 (attention and "
                               "projections over the token rows, each layer's experts as GEMMs over the tokens "
                               "routed to them), eager, prompt in pinned host memory; median of per-call events"}}
    return res, host, host_kv


def cpu_moe_decode_baseline(O, host, host_kv, budget_s=10.0):
    """The oracle's Qwen3-MoE decode step (the C attention sublayer and head, moe_layer's GEMVs;
    pthreads over all host cores) on the same weights and KV values (widened to f32)."""
    spec, moe = QWEN3_30B_A3B, QWEN3_30B_A3B_MOE
    threads = len(os.sched_getaffinity(0))
    om = O.DecodeModel(spec, {n: (q, a) for n, (q, a, _) in host.items()}, KV_CAP)
    done, t0, tok = 0, time.perf_counter(), 1
    pos = KV_CAP - 1
    while True:
        logits = om.moe_step(host_kv, tok, pos, moe, host, threads=threads)
        tok = int(logits.argmax())
        pos += 1
        done += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    return done / el, threads, done, el


INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
GEMM_SHAPE = (512, 4096, 14336)  # (tokens M, n_in K, n_out N), Q4_K weights
GEMM_ROTATE_BYTES = 512 * 10 ** 6


def bench_gemm(torch, J, dev, stream, steps, keep_host):
    """Prefill GEMM: Y[512, 14336] = X[512, 4096] (Q8_K) . W (Q4_K), int8 MFMA.  The weights are
    re-laid out once at load into the GEMM's fragment order (jero_hip_repack_gemm: Q4_K_G, the
    quants regrouped and the scales unpacked, 160 bytes per 256-block against 144, as the model's
    prefill holds them); the kernel over the GGUF bytes is timed too
    (`gguf`).  Weights rotate over copies of >= 512 MB in all (14 of 36.7 MB in the GGUF layout,
    40.8 MB in the GEMM layout), every graph spanning all of them.  `mfma_issue_frac`: the MFMA work the kernel issues
    (two int8 planes of 2MNK ops each, plus the f16 mins product of 2MN*16 per block) over the
    time at peak."""
    M, K, N = GEMM_SHAPE
    nbytes = J.row_bytes(J.Q4_K, K) * N
    copies = -(-GEMM_ROTATE_BYTES // nbytes)
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

        return time_graph(torch, one, steps, 3, stream, span=copies)

    t = timed(laid)
    tg = timed(views)
    laid_bytes = sum(v.nbytes() for v in laid)
    res = {"workload": f"Q4_K x Q8_K prefill GEMM M={M} K={K} N={N}, int8 MFMA, weights in the GEMM layout "
                       f"(Q4_K_G: the quants in MFMA fragment order, scales unpacked, repacked once at load)",
           "us": round(t * 1e6, 2), "tops": round(ops / t / 1e12, 1), "unit": "TOP/s", "peak": INT8_PEAK_TOPS,
           "frac_int8_peak": round(ops / t / 1e12 / INT8_PEAK_TOPS, 4),
           "mfma_issue_frac": round(issued / t, 4), "tokens_per_s": round(M / t, 1),
           "rotation_bytes": laid_bytes, "graph_launches": max(steps, copies),
           "gguf": {"what": "the same GEMM over the GGUF Q4_K bytes (no repack)", "us": round(tg * 1e6, 2),
                    "tops": round(ops / tg / 1e12, 1), "frac_int8_peak": round(ops / tg / 1e12 / INT8_PEAK_TOPS, 4),
                    "rotation_bytes": copies * nbytes}}
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
    at load time), top-8; T=1 (decode) and T=64.  Two weight copies (392 MB of experts each).
    T=1: router logits N(0,1) with +16 on 8 experts of a random permutation, 16 logit sets that
    route the token to each of the 128 experts once, so 32 calls (16 sets x 2 copies) read all
    784 MB of expert bytes once and no call re-reads what an earlier one left in the Infinity
    Cache.  T=64: 8 sets of N(0,1) logits (each call routes to ~126 of the 128 experts), copies
    alternating.  Every graph spans 32 calls.  Algorithmic bytes: the distinct routed experts'
    weights (3.06 MB each) + activations."""
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
    sets = E // k  # T=1 logit sets: each expert the top-8 of exactly one
    span = sets * copies
    for T in (1, 64):
        x = torch.randn(T, H, generator=g, device=dev)
        if T == 1:
            perm = torch.randperm(E, generator=g, device=dev)
            logits = []
            for i in range(sets):
                lg = torch.randn(T, E, generator=g, device=dev)
                lg[:, perm[i * k:(i + 1) * k]] += 16.0
                logits.append(lg)
        else:
            logits = [torch.randn(T, E, generator=g, device=dev) for _ in range(8)]
        y = torch.empty(T, H, device=dev)
        ws = torch.empty(J.lib().jero_hip_moe_workspace_bytes(T, E, k, H, F), dtype=torch.uint8, device=dev)
        cnt = [0]
        sels = []

        def one():
            c = cnt[0]
            # T=1: all 16 sets on one copy, then on the other; T=64: copies alternate
            cp = (c // sets) % copies if T == 1 else c % copies
            sel, _ = J.dispatch_qwen3_moe_ffn(y, x, logits[c % len(logits)], k, gv[cp], uv[cp], dv[cp],
                                             workspace=ws, stream=stream)
            if len(sels) < span:
                sels.append((cp, sel))
            cnt[0] += 1

        t = time_graph(torch, one, steps, 1, stream, span=span)
        per_call = [set(s.cpu().numpy().reshape(-1).tolist()) for _, s in sels]
        distinct = sum(len(u) for u in per_call) / len(per_call)
        rotation = sum(len(set().union(*[u for (cp, _), u in zip(sels, per_call) if cp == c]))
                       for c in range(copies)) * per_expert
        algo = distinct * per_expert + T * H * 4 * 2 + T * E * 4
        out[f"T{T}"] = {"us": round(t * 1e6, 2), "distinct_experts": round(distinct, 1),
                        "bytes": int(algo), "GB_s": round(algo / t / 1e9, 1),
                        "frac_hbm": round(algo / t / 1e9 / HBM_PEAK_GBS, 4),
                        "rotation_bytes": int(rotation), "graph_launches": max(steps, span)}
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

    t = time_graph(torch, one, steps, warmup, stream, span=copies)
    tc = time_graph(torch, probe, steps, warmup, stream, span=copies)
    algo = nbytes + J.row_bytes(J.ACT_Q8, n_in) + 4 * n_out
    res = {"workload": "Q8_0 x Q8_0 GEMV 4096x4096, batch 1", "us": round(t * 1e6, 3),
           "GB_s": round(algo / t / 1e9, 1), "bytes": algo, "frac_hbm": round(algo / t / 1e9 / HBM_PEAK_GBS, 4),
           "read_ceiling_us": round(tc * 1e6, 3), "gemv_over_ceiling": round(tc / t, 4),
           "rotation_bytes": copies * nbytes}
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
    """The oracle's ForwardModel evaluate (scalar C restatement) on the same workload, every
    projection, attention and head split over a persistent pool of all host cores (the
    reference's WorkerPool under its Spin profile)."""
    threads = len(os.sched_getaffinity(0))
    f = O.ForwardModel(fnv1a(FWD_PROMPT_TEXT), FWD_VOCAB, FWD_CTX, threads=threads)
    reps, toks, t0 = 0, None, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or reps == 0:
        toks = f.evaluate(prompt, max_tokens)
        reps += 1
    el = time.perf_counter() - t0
    f.close()
    return reps * max_tokens / el, reps, el, toks, threads


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


def kernel_short_name(name):
    """`void ns::kern<T, 4>(args...)` -> `ns::kern<T, 4>` (the name up to its argument list)."""
    name = name.strip()
    if name.startswith("_Z"):  # a mangled name (some counter rows carry one)
        import subprocess
        try:
            name = subprocess.run(["c++filt", name], capture_output=True, text=True, check=True).stdout.strip()
        except (OSError, subprocess.CalledProcessError):
            return name
    name = name.replace("(anonymous namespace)", "{anon}")
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i]
    return name


def read_profile_csv(dirs, suffix):
    """Rows of every rocprofv3 `*<suffix>` CSV file under `dirs` (recursive)."""
    import csv
    import glob
    rows = []
    for d in dirs:
        for path in sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True)):
            with open(path, newline="") as f:
                rows += list(csv.DictReader(f))
    return rows


def summarize_profiles(dirs, match, step_end, last, out, until=None):
    """Markdown summary of rocprofv3 CSV output (--output-format csv) under `dirs`: per (kernel,
    grid) launch counts and mean / median duration from *_kernel_trace.csv; per (kernel, grid)
    counter means per dispatch (and per wave for SQ_INSTS_* given SQ_WAVES) from
    *_counter_collection.csv; with `step_end`, the wall time and kernel-time sum of the last
    `last` steps, a step being the dispatches after one `step_end` kernel up to the next; with
    `until`, only the dispatches before the first kernel whose name contains it."""
    import numpy as np
    w = out.write
    trace = [r for r in read_profile_csv(dirs, "_kernel_trace.csv") if match in r["Kernel_Name"]]
    if until:
        trace.sort(key=lambda r: int(r["Start_Timestamp"]))
        cut = next((i for i, r in enumerate(trace) if until in r["Kernel_Name"]), len(trace))
        trace = trace[:cut]
    if trace:
        groups = {}
        for r in trace:
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            groups.setdefault((kernel_short_name(r["Kernel_Name"]), grid), []).append(dur)
        w("| kernel | grid | launches | mean ns | median ns | min ns | total us |\n|---|---|---|---|---|---|---|\n")
        for (k, grid), d in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
            a = np.array(d, np.float64)
            w(f"| `{k}` | {grid} | {len(d)} | {a.mean():.0f} | {np.median(a):.0f} | {a.min():.0f} | "
              f"{a.sum() / 1e3:.1f} |\n")
        if step_end:
            ev = sorted(trace, key=lambda r: int(r["Start_Timestamp"]))
            ends = [i for i, r in enumerate(ev) if step_end in r["Kernel_Name"]]
            walls, sums, counts = [], [], []
            for a, b in zip(ends[:-1], ends[1:]):
                step = ev[a + 1:b + 1]
                walls.append(int(step[-1]["End_Timestamp"]) - int(step[0]["Start_Timestamp"]))
                sums.append(sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in step))
                counts.append(len(step))
            walls, sums, counts = walls[-last:], sums[-last:], counts[-last:]
            if walls:
                w(f"\nLast {len(walls)} steps ending in `{step_end}` ({counts[-1]} kernels per step): wall "
                  f"mean {np.mean(walls) / 1e3:.1f} us (min {min(walls) / 1e3:.1f}, max {max(walls) / 1e3:.1f}); "
                  f"kernel-time sum mean {np.mean(sums) / 1e3:.1f} us\n")
                per = {}
                for a, b in list(zip(ends[:-1], ends[1:]))[-len(walls):]:
                    for r in ev[a + 1:b + 1]:
                        grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
                        p = per.setdefault((kernel_short_name(r["Kernel_Name"]), grid), [0, 0])
                        p[0] += 1
                        p[1] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
                n = len(walls)
                w("\n| kernel (per step) | grid | launches | us per step | mean us |\n|---|---|---|---|---|\n")
                for (k, grid), (c, d) in sorted(per.items(), key=lambda kv: -kv[1][1]):
                    w(f"| `{k}` | {grid} | {c / n:.0f} | {d / n / 1e3:.1f} | {d / c / 1e3:.2f} |\n")
    pmc = [r for r in read_profile_csv(dirs, "_counter_collection.csv") if match in r["Kernel_Name"]]
    if pmc:
        vals = {}
        for r in pmc:
            key = (kernel_short_name(r["Kernel_Name"]), int(r["Grid_Size"]))
            vals.setdefault(key, {}).setdefault(r["Counter_Name"], {}).setdefault(r["Dispatch_Id"], 0.0)
            vals[key][r["Counter_Name"]][r["Dispatch_Id"]] += float(r["Counter_Value"])
        names = sorted({c for v in vals.values() for c in v})
        w("\n| kernel | grid | dispatches | " + " | ".join(names) + " |\n|---|---|---|" + "---|" * len(names) + "\n")
        for (k, grid), cs in sorted(vals.items()):
            disp = max(len(d) for d in cs.values())
            means = {c: float(np.mean(list(d.values()))) for c, d in cs.items()}
            waves = means.get("SQ_WAVES")
            cells = []
            for c in names:
                if c not in means:
                    cells.append("")
                elif c.startswith("SQ_INSTS_") and waves:
                    cells.append(f"{means[c] / waves:.1f}/wave")
                else:
                    cells.append(f"{means[c]:.4g}")
            w(f"| `{k}` | {grid} | {disp} | " + " | ".join(cells) + " |\n")


def traffic_summary(fetch_dirs, write_dirs, match, copy_bytes):
    """HBM bytes per dispatch from a FETCH_SIZE pass and a WRITE_SIZE pass (KiB per dispatch),
    each scaled by what the counter reads for the torch copy of `copy_bytes` bytes in the same
    run (--copy-probe): {(kernel, grid): (fetch KiB, write KiB, bytes)} and the two factors."""
    import numpy as np

    def means(dirs, counter):
        out, copy = {}, []
        for r in read_profile_csv(dirs, "_counter_collection.csv"):
            if r["Counter_Name"] != counter:
                continue
            v = float(r["Counter_Value"])
            if "copyBuffer" in r["Kernel_Name"] and v * 1024 > 0.4 * copy_bytes:
                copy.append(v)
            elif match in r["Kernel_Name"]:
                out.setdefault((kernel_short_name(r["Kernel_Name"]), int(r["Grid_Size"])), []).append(v)
        return {k: float(np.mean(v)) for k, v in out.items()}, (float(np.mean(copy)) if copy else None)

    fetch, fcopy = means(fetch_dirs, "FETCH_SIZE")
    write, wcopy = means(write_dirs, "WRITE_SIZE")
    if not fcopy or not wcopy:
        raise SystemExit("traffic: no copy-probe dispatch in the counter passes (run bench.py with --copy-probe)")
    ff, wf = copy_bytes / (fcopy * 1024), copy_bytes / (wcopy * 1024)
    res = {k: (fetch[k], write.get(k, 0.0), fetch[k] * 1024 * ff + write.get(k, 0.0) * 1024 * wf) for k in fetch}
    return res, ff, wf


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
    ap.add_argument("--no-dense-decode", action="store_true", help="skip the Qwen3-8B decode (keep moe_decode)")
    ap.add_argument("--no-moe-layer", action="store_true", help="skip the MoE layer part (keep moe_decode)")
    ap.add_argument("--decode-steps", type=int, default=50)
    ap.add_argument("--copy-probe", type=float, default=0.0,
                    help="also run one device copy of this many MB (PMC byte-counter calibration)")
    ap.add_argument("--summarize", nargs="+", metavar="DIR",
                    help="print a markdown summary of rocprofv3 CSV output under DIR(s) and exit (no GPU)")
    ap.add_argument("--match", default="jero", help="--summarize: kernels whose name contains this")
    ap.add_argument("--step-end", default=None, help="--summarize: kernel that ends one step (per-step wall times)")
    ap.add_argument("--last", type=int, default=16, help="--summarize: steps to average with --step-end")
    ap.add_argument("--until", default=None, help="--summarize: only dispatches before the first kernel named so")
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="print HBM bytes per dispatch from a FETCH_SIZE and a WRITE_SIZE pass run with "
                         "--copy-probe MB (give the same MB) and exit (no GPU)")
    args = ap.parse_args()
    if args.summarize:
        summarize_profiles(args.summarize, args.match, args.step_end, args.last, sys.stdout, args.until)
        return
    if args.traffic:
        res, ff, wf = traffic_summary([args.traffic[0]], [args.traffic[1]], args.match, args.copy_probe * 1e6)
        print(f"copy probe factors: fetch {ff:.4f}, write {wf:.4f}")
        print("| kernel | grid | FETCH_SIZE KiB | WRITE_SIZE KiB | bytes |\n|---|---|---|---|---|")
        for (k, grid), (fk, wk, b) in sorted(res.items()):
            print(f"| `{k}` | {grid} | {fk:.1f} | {wk:.1f} | {b:.0f} |")
        return
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
    bufs, xqs, ys, views, raw_views, algo, wbytes = [], [], [], [], [], [], []
    for i, (n_in, n_out) in enumerate(SHAPES):
        nbytes = J.row_bytes(J.Q4_K, n_in) * n_out
        wbytes.append(nbytes)
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

    max_copies = max(len(v) for v in views)
    t_step = time_graph(torch, step, args.steps, args.warmup, stream, span=max_copies)
    step_bytes = sum(algo)
    value = step_bytes / t_step / 1e9
    step_dist = time_graph_dist(torch, step, max_copies, 21, stream)
    rotation = {f"{n_in}x{n_out}": len(views[i]) * wbytes[i] for i, (n_in, n_out) in enumerate(SHAPES)}

    # per-shape kernel averages (same method, one shape per graph), planar and GGUF layouts
    per_shape, per_shape_gguf = {}, {}
    for table, vlist in ((per_shape, views), (per_shape_gguf, raw_views)):
        for i, (n_in, n_out) in enumerate(SHAPES):
            cnt = [0]

            def one(i=i, cnt=cnt, vlist=vlist):
                vv = vlist[i]
                J.matvec(vv[cnt[0] % len(vv)], xqs[i], ys[i], stream=stream)
                cnt[0] += 1

            nc = len(vlist[i])
            t = time_graph(torch, one, args.steps, args.warmup, stream, span=nc)
            table[f"{n_in}x{n_out}"] = {"us": round(t * 1e6, 3), "GB_s": round(algo[i] / t / 1e9, 1),
                                        "bytes": algo[i], "rotation_bytes": nc * wbytes[i],
                                        "graph_launches": max(args.steps, nc),
                                        "dist": time_graph_dist(torch, one, nc, 21, stream)}
    # pure-read ceiling: one launch per shape reading the same rotated buffers and nothing else
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    ceiling = {}
    for i, (n_in, n_out) in enumerate(SHAPES):
        cnt = [0]

        def probe(i=i, cnt=cnt):
            vv = views[i]
            J.read_probe(vv[cnt[0] % len(vv)].data, sink, stream=stream)
            cnt[0] += 1

        tc = time_graph(torch, probe, args.steps, args.warmup, stream, span=len(views[i]))
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
            "frac_hbm": round(h_algo / th / 1e9 / HBM_PEAK_GBS, 4), "rotation_bytes": 2 * hbytes}
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
    if not args.no_moe and not args.no_moe_layer:
        moe = bench_moe(torch, J, dev, stream, max(20, args.steps // 5))
        torch.cuda.empty_cache()

    # ---- int8 ForwardModel matrix bench (extra)
    fwd = None
    if not args.no_forward:
        fwd, (fprompt, fmax) = bench_forward_model(J, 20)
        if not args.no_cpu:
            import pyoracle as O
            tps, reps, el, ctoks, fthreads = cpu_forward_baseline(O, fprompt, fmax)
            fwd["cpu_baseline"] = {"value": round(tps, 1), "unit": "generated tok/s (prefill included)",
                                   "cores": fthreads, "kind": "port", "tokens_equal": ctoks == fwd["tokens"],
                                   "sample": f"{reps} full evaluate runs, {el:.1f} s, scalar C restatement, "
                                             f"persistent spin pool of {fthreads} threads"}
            fwd["evaluate_tok_s"] = round(fmax / (fwd["evaluate_wall_ms"] * 1e-3), 1)

    # ---- full decode step (extra)
    decode = None
    del bufs, views
    torch.cuda.empty_cache()
    if not args.no_decode and not args.no_dense_decode:
        decode, host, host_kv = bench_decode(torch, J, dev, stream, args.decode_steps, 3, not args.no_cpu)
        if not args.no_cpu:
            import pyoracle as O
            tps, threads, reps, el = cpu_decode_baseline(O, host, host_kv)
            decode["cpu_baseline"] = {"value": round(tps, 3), "unit": "tok/s", "cores": threads, "kind": "port",
                                      "sample": f"{reps} greedy steps of the same model from position {KV_CAP - 1}, "
                                                f"{el:.1f} s, f32 KV ring"}
            del host, host_kv

    # ---- Qwen3-MoE decode step (extra)
    moe_decode = None
    if not args.no_decode and not args.no_moe:
        torch.cuda.empty_cache()
        moe_decode, mhost, mkv = bench_moe_decode(torch, J, dev, stream, args.decode_steps, 3, not args.no_cpu)
        torch.cuda.empty_cache()
        if not args.no_cpu:
            import pyoracle as O
            tps, threads, reps, el = cpu_moe_decode_baseline(O, mhost, mkv)
            moe_decode["cpu_baseline"] = {"value": round(tps, 3), "unit": "tok/s", "cores": threads, "kind": "port",
                                          "sample": f"{reps} greedy steps of the same model from position "
                                                    f"{KV_CAP - 1}, {el:.1f} s, f32 KV ring"}
            del mhost, mkv

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
                   "rotation_bytes": rotation,
                   "graph_steps": max(args.steps, max_copies), "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4)},
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
        "moe_decode": moe_decode,
        "forward_model": fwd,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
