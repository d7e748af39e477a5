"""The device decode step against the oracle and against the reference's golden fixture.

Golden llama Q8_0 fixture: first-token logits within 1e-4 and the greedy ids, as the
reference's own certification (tests/architecture_certification_gate.rs:305).

Random Qwen3-shaped models against the oracle, every step traced (decode_parity.run_traced):
  * teacher-forced, layer by layer: the device's activation blocks bit-exact, every GEMV within
    1e-5, attention within 1e-3, RMSNorm / QK-norm / RoPE / SwiGLU at f32
    precision, each stage recomputed by the oracle from the device's own input to it;
  * free-running (device and oracle each from their own state): the int8 flips between the two
    runs are counted at every quantization point and each must be a +-1 flip whose two
    pre-rounding values differ by less than half a quantum; a step without flips must match the
    oracle's logits within 1e-3, a step with flips within 2e-2 at cosine >= 0.9999 (the
    reference's certification floor, src/certification.rs:240-318).
Why flips happen at all: activations are re-quantized to int8 before every GEMV, and the device
(f32, its own summation order) and the oracle (f64 accumulation) round an element lying within
~1e-6 of a rounding boundary to neighbouring int8 values; one flip moves the hidden state by
~1e-4 and the logits by up to ~1e-2 on that step.
"""
import numpy as np
import pytest
import torch

import decode_parity as DP
import golden_llama as GL
import jero_hip as J
import model_spec as MS
import pyoracle as O

pytestmark = pytest.mark.gpu


def make_gpu_model(spec, tensors, cap, kv_dtype, qk_norm):
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], cap, kv_dtype, qk_norm)
    for name, (quant, arr, n_in, n_out) in tensors.items():
        if not qk_norm and "_q_norm" in name or not qk_norm and "_k_norm" in name:
            continue
        m.set_tensor(name, quant, arr, n_in, n_out)
    m.finalize()
    return m


def test_golden_llama_on_device(dev):
    """The reference's golden fixture through the device decode path (Q8_0 x ACT_Q8 GEMVs)."""
    print("golden llama on device", flush=True)
    g = GL.golden()
    s = dict(GL.SPEC)
    tensors = {}
    shapes = {n: shp for n, _, shp in GL.tensor_specs()}
    for name, (quant, arr) in GL.build().items():
        shp = shapes[name]
        tensors[name] = (quant, arr, shp[0], shp[1] if len(shp) > 1 else 1)
    m = make_gpu_model(s, tensors, 128, J.KV_F32, False)
    check_golden(m, g, s, dev)


def test_golden_llama_from_gguf_file(dev, tmp_path):
    """The same golden model read from the GGUF v3 file the reference's test builds
    (architecture_certification_gate.rs:82-176): hyperparameters from its metadata, tensors
    from the mapped file."""
    print("golden llama from gguf", flush=True)
    path = tmp_path / "llama_authentic_q8_0.gguf"
    path.write_bytes(GL.gguf_file_bytes())
    m = J.DecodeModel.from_gguf(str(path), 128, J.KV_F32)
    assert (m.cfg.hidden, m.cfg.n_layers, m.cfg.head_dim, m.cfg.qk_norm) == (128, 2, 32, 0)
    check_golden(m, GL.golden(), GL.SPEC, dev)


def check_golden(m, g, s, dev):
    logits = torch.empty(s["vocab"], dtype=torch.float32, device=dev)
    for pos, tok in enumerate(g["prompt_token_ids"]):
        m.set_position(tok, pos)
        m.decode_step()
    torch.cuda.synchronize()
    m.read_logits(logits)
    first = logits.cpu().numpy()
    for e in g["first_token_top_k"]:
        assert abs(first[e["token_id"]] - e["logit"]) <= 1e-4, (e, first[e["token_id"]])
    greedy = [m.read_token_pos()[0]]
    for _ in range(len(g["greedy_token_ids"]) - 1):
        m.decode_step()
        torch.cuda.synchronize()
        greedy.append(m.read_token_pos()[0])
    assert greedy == g["greedy_token_ids"]
    assert m.read_token_pos()[1] == len(g["prompt_token_ids"]) + len(g["greedy_token_ids"]) - 1


def test_golden_llama_traced_against_oracle(dev):
    """The golden llama (Q8_0 weights, ACT_Q8 activations, no QK-norm) decoded with the trace on:
    the same layer-by-layer checks as the Qwen3 models, over the prompt and four more steps."""
    print("golden llama traced", flush=True)
    s = dict(GL.SPEC)
    tensors = {}
    shapes = {n: shp for n, _, shp in GL.tensor_specs()}
    for name, (quant, arr) in GL.build().items():
        shp = shapes[name]
        tensors[name] = (quant, arr, shp[0], shp[1] if len(shp) > 1 else 1)
    spec = dict(hidden=s["hidden"], ffn=s["ffn"], n_layers=s["n_layers"], vocab=s["vocab"], nq=s["nq"], nkv=s["nkv"],
                hd=s["hd"], eps=s["eps"], theta=s["theta"])
    m = make_gpu_model(spec, tensors, 128, J.KV_F32, False)
    om = O.DecodeModel(spec, MS.oracle_tensors(tensors), 128)
    kv = om.new_kv()
    DP.run_traced(m, om, tensors, spec, kv, 128, 0, 8, False, dev, 1, qk_norm=False)
    m.close()


def write_model_gguf(path, arch, spec, tensors, extra_kvs=()):
    """A GGUF v3 file holding `tensors` ({name: (quant, bytes, n_in, n_out)}) and the spec's
    hyperparameters under {arch}.* keys (plus extra_kvs)."""
    import gguf_writer as W
    kvs = [(f"{arch}.block_count", W.U32, spec["n_layers"]), (f"{arch}.embedding_length", W.U32, spec["hidden"]),
           (f"{arch}.feed_forward_length", W.U32, spec["ffn"]), (f"{arch}.attention.head_count", W.U32, spec["nq"]),
           (f"{arch}.attention.head_count_kv", W.U32, spec["nkv"]),
           (f"{arch}.attention.key_length", W.U32, spec["hd"]), (f"{arch}.rope.freq_base", W.F32, spec["theta"]),
           (f"{arch}.attention.layer_norm_rms_epsilon", W.F32, spec["eps"])] + list(extra_kvs)
    ts = [(n, q, (n_in, n_out) if n_out > 1 else (n_in,), W.as_bytes(a)) for n, (q, a, n_in, n_out) in tensors.items()]
    path.write_bytes(W.gguf_bytes(arch, kvs, ts))


def test_qwen3_from_gguf_matches_set_tensor(dev, tmp_path):
    """Q4_K_M-mix Qwen3-shaped model (tied output: no output.weight in the file) from a GGUF file
    against the same tensors given one by one: logits bit-equal over several steps."""
    print("qwen3 from gguf", flush=True)
    spec = dict(QWEN_SMALL)
    t = MS.build(spec, seed=11)
    tied = dict(t)
    tied["output.weight"] = t["token_embd.weight"]
    path = tmp_path / "qwen3.gguf"
    write_model_gguf(path, "qwen3", spec, {k: v for k, v in t.items() if k != "output.weight"})
    a = make_gpu_model(spec, tied, 64, J.KV_F16, True)
    b = J.DecodeModel.from_gguf(str(path), 64, J.KV_F16)
    assert b.cfg.qk_norm == 1 and b.cfg.vocab == spec["vocab"] and b.cfg.ffn == spec["ffn"]
    la = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    lb = torch.empty_like(la)
    for m in (a, b):
        m.set_position(17, 0)
    for step in range(6):
        a.decode_step()
        b.decode_step()
        torch.cuda.synchronize()
        a.read_logits(la)
        b.read_logits(lb)
        assert torch.equal(la, lb), step
        assert a.read_token_pos() == b.read_token_pos()


def test_gguf_upload_registers_once(dev, tmp_path):
    """gguf_upload copies a tensor's mapped bytes to HBM once; later calls return that address."""
    print("gguf upload", flush=True)
    path = tmp_path / "g.gguf"
    path.write_bytes(GL.gguf_file_bytes())
    with J.GGUFFile(str(path)) as g:
        for name in ("blk.1.attn_q.weight", "output_norm.weight"):
            host = g.tensor_bytes(name)
            d0 = g.upload(name)
            assert g.upload(name) == d0
            back = np.zeros_like(host)
            J._memcpy(back.ctypes.data, d0, host.nbytes)
            np.testing.assert_array_equal(back, host)


def test_gguf_tensor_view_repacks_on_device(dev, tmp_path):
    """GGUF tensors to device views in the kernels' layouts: a stacked Q4_K expert tensor to
    16-row tiles, a 2-D Q6_K matrix to the planar layout, byte-equal to repacking the same bytes
    given directly."""
    import gguf_writer as W
    import qdata
    print("gguf tensor_view repack", flush=True)
    n_in, rows, E = 512, 32, 3
    exps = qdata.rand_weights(J.Q4_K, rows * E, n_in, 5)
    head = qdata.rand_weights(J.Q6_K, 40, n_in, 6)
    path = tmp_path / "e.gguf"
    path.write_bytes(W.gguf_bytes("qwen3moe", [], [("blk.0.ffn_gate_exps.weight", J.Q4_K, (n_in, rows, E), exps.tobytes()),
                                                   ("output.weight", J.Q6_K, (n_in, 40), head.tobytes())]))
    with J.GGUFFile(str(path)) as g:
        for name, arr, shape, want in (("blk.0.ffn_gate_exps.weight", exps, [n_in, rows, E], J.Q4_K_T),
                                       ("output.weight", head, [n_in, 40], J.Q6_K_R)):
            v = g.tensor_view(name, dev, repack_layout=True)
            assert v.quant == want and v.shape == shape
            raw = g.tensor_view(name, dev)
            assert raw.quant in (J.Q4_K, J.Q6_K)
            assert torch.equal(raw.data.cpu(), torch.from_numpy(np.ascontiguousarray(arr).view(np.uint8).reshape(-1)))
            ref = J.repack(J.TensorView(name, raw.quant, shape, raw.data.clone()))
            torch.cuda.synchronize()
            assert ref.quant == want and torch.equal(v.data, ref.data)


QWEN_SMALL = dict(hidden=512, ffn=1024, n_layers=4, vocab=1000, nq=8, nkv=2, hd=64, eps=1e-6, theta=1e6)


@pytest.mark.parametrize("kv_name,cap,prefill,steps", [("f32", 300, 40, 12), ("f16", 300, 290, 24), ("f16", 128, 0, 12),
                                                       ("f32", 128, 100, 40)])
def test_decode_matches_oracle(dev, kv_name, cap, prefill, steps):
    """Prefilled cache (f16-exact values), then decode steps; the second case wraps the ring."""
    print(f"decode kv={kv_name} cap={cap} prefill={prefill}", flush=True)
    spec = QWEN_SMALL
    t = MS.build(spec, seed=3)
    kv_dtype = J.KV_F32 if kv_name == "f32" else J.KV_F16
    m = make_gpu_model(spec, t, cap, kv_dtype, True)
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = prefill_kv(m, om, spec, cap, prefill, 7, dev, kv_dtype == J.KV_F16)
    DP.run_traced(m, om, t, spec, kv, cap, prefill, steps, kv_dtype == J.KV_F16, dev, 17)


def prefill_kv(m, om, spec, cap, prefill, seed, dev, kv_f16=True):
    """Both rings (device and oracle) pre-filled with the same N(0, 1) values, f16-exact, for
    positions [0, prefill)."""
    kv = om.new_kv()
    kvd = spec["nkv"] * spec["hd"]
    rng = np.random.default_rng(seed)
    for L in range(spec["n_layers"]):
        k = rng.standard_normal((cap, kvd)).astype(np.float16)
        v = rng.standard_normal((cap, kvd)).astype(np.float16)
        k[prefill:] = 0
        v[prefill:] = 0
        kv[L, 0] = k.astype(np.float32)
        kv[L, 1] = v.astype(np.float32)
        tdt = torch.float16 if kv_f16 else torch.float32
        m.write_kv(L, torch.from_numpy(k).to(tdt).to(dev), torch.from_numpy(v).to(tdt).to(dev))
    return kv


QWEN3_8B = dict(hidden=4096, ffn=12288, n_layers=36, vocab=151936, nq=32, nkv=8, hd=128, eps=1e-6, theta=1e6)


def test_decode_qwen3_8b_layer_shape(dev):
    """Two layers of the Qwen3-8B shape (hidden 4096, 32/8 heads of 128, FFN 12288, vocab
    151936), Q4_K_M mix, f16 cache of 4096 slots pre-filled to 4094, then decode."""
    print("decode qwen3-8b layer shape", flush=True)
    spec = dict(QWEN3_8B, n_layers=2)
    cap, prefill = 4096, 4094
    t = MS.build(spec, seed=8)
    m = make_gpu_model(spec, t, cap, J.KV_F16, True)
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = prefill_kv(m, om, spec, cap, prefill, 9, dev)
    DP.run_traced(m, om, t, spec, kv, cap, prefill, 2, True, dev, 1234)
    m.close()


def test_decode_qwen3_8b_full_depth(dev):
    """The benchmark's decode model at its full depth: a random-init Qwen3-8B-shaped model in
    Q4_K_M (36 layers; Q6_K head, Q6_K attn_v / ffn_down on 18 layers), f16 KV ring of 4096
    slots pre-filled with N(0, 1) values to position 4094, three greedy steps (the last one at
    position 4096 wraps the ring), every layer of every step checked teacher-forced and the
    free-running flips accounted for."""
    import time
    print("decode qwen3-8b full depth: building weights on the device", flush=True)
    t0 = time.time()
    spec = dict(QWEN3_8B)
    cap, prefill = 4096, 4094
    t, on_dev = MS.build_device(spec, dev, seed=40)
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], cap, J.KV_F16, True)
    for name, (quant, arr, n_in, n_out) in t.items():
        m.set_tensor(name, quant, on_dev.get(name, arr), n_in, n_out)
    del on_dev
    m.finalize()
    torch.cuda.empty_cache()
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = prefill_kv(m, om, spec, cap, prefill, 41, dev)
    print(f"  model ready in {time.time() - t0:.0f} s", flush=True)
    res = DP.run_traced(m, om, t, spec, kv, cap, prefill, 3, True, dev, 4321)
    print(f"  flips per step {[r[0] for r in res]}", flush=True)
    m.close()


def test_decode_graph_replay_matches_eager(dev):
    """One captured step replayed for consecutive tokens equals eager steps bit for bit."""
    print("decode graph replay", flush=True)
    spec = dict(QWEN_SMALL, n_layers=2)
    t = MS.build(spec, seed=5)
    cap = 256
    a = make_gpu_model(spec, t, cap, J.KV_F16, True)
    b = make_gpu_model(spec, t, cap, J.KV_F16, True)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        a.set_position(5, 0, stream=s)
        b.set_position(5, 0, stream=s)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        a.decode_step(stream=s)  # warm (position 0)
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            a.decode_step(stream=s)
    b.decode_step()
    torch.cuda.synchronize()
    la = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    lb = torch.empty_like(la)
    for i in range(6):
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        b.decode_step()
        torch.cuda.synchronize()
        a.read_logits(la)
        b.read_logits(lb)
        assert torch.equal(la, lb), i
        assert a.read_token_pos() == b.read_token_pos()
        _ = torch.randn(1000, device=dev).sum().item()  # unrelated eager work between replays


def test_decode_untraced_matches_traced(dev):
    """Decode steps without a trace (the path bench.py replays as a graph, itself equal to eager
    steps above) give the same logits and tokens, bit for bit, as traced steps, which the parity
    tests hold to the oracle."""
    print("decode untraced vs traced", flush=True)
    spec = dict(QWEN_SMALL, n_layers=2)
    t = MS.build(spec, seed=6)
    cap = 256
    a = make_gpu_model(spec, t, cap, J.KV_F16, True)
    b = make_gpu_model(spec, t, cap, J.KV_F16, True)
    _, _, _, total = a.trace_layout()
    buf = torch.zeros(total, dtype=torch.uint8, device=dev)
    a.set_trace(buf)
    a.set_position(7, 0)
    b.set_position(7, 0)
    la = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    lb = torch.empty_like(la)
    for i in range(4):
        a.decode_step()
        b.decode_step()
        torch.cuda.synchronize()
        a.read_logits(la)
        b.read_logits(lb)
        assert torch.equal(la, lb), i
        assert a.read_token_pos() == b.read_token_pos(), i
    a.set_trace(None)
    a.close()
    b.close()


def test_decode_untraced_matches_traced_8b_layer_shape(dev):
    """The same at the timed layer shape: two layers of the Qwen3-8B shape (the fused Q|K|V,
    the Q|K + Q6_K V launch, gate|up SwiGLU, both down formats, the LM head over 151936 rows),
    f16 ring of 4096 slots filled to 4094, three steps (the last one wraps the ring)."""
    print("decode untraced vs traced, qwen3-8b layer shape", flush=True)
    spec = dict(QWEN3_8B, n_layers=2)
    cap = 4096
    t = MS.build(spec, seed=66)
    a = make_gpu_model(spec, t, cap, J.KV_F16, True)
    b = make_gpu_model(spec, t, cap, J.KV_F16, True)
    kvd = spec["nkv"] * spec["hd"]
    rng = np.random.default_rng(67)
    for L in range(spec["n_layers"]):
        k = torch.from_numpy(rng.standard_normal((cap, kvd)).astype(np.float16)).to(dev)
        v = torch.from_numpy(rng.standard_normal((cap, kvd)).astype(np.float16)).to(dev)
        a.write_kv(L, k, v)
        b.write_kv(L, k, v)
    _, _, _, total = a.trace_layout()
    buf = torch.zeros(total, dtype=torch.uint8, device=dev)
    a.set_trace(buf)
    a.set_position(11, 4094)
    b.set_position(11, 4094)
    la = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    lb = torch.empty_like(la)
    for i in range(3):
        a.decode_step()
        b.decode_step()
        torch.cuda.synchronize()
        a.read_logits(la)
        b.read_logits(lb)
        assert torch.equal(la, lb), i
        assert a.read_token_pos() == b.read_token_pos(), i
    a.set_trace(None)
    a.close()
    b.close()


def test_model_errors(dev):
    m = J.DecodeModel(512, 1024, 1, 100, 8, 2, 64, 1e-6, 1e6, 64)
    with pytest.raises(J.K3Error) as ei:
        m.set_tensor("blk.0.attn_q.weight", J.Q4_K, np.zeros(10, np.uint8), 512, 512)
    assert ei.value.variant == "TensorBoundsError"
    with pytest.raises(J.K3Error) as ei:
        m.set_tensor("blk.7.attn_q.weight", J.Q4_K, np.zeros(512 * 2 * 144, np.uint8), 512, 512)
    assert ei.value.variant == "CapabilityMismatch"
    with pytest.raises(J.K3Error) as ei:
        m.decode_step()  # before finalize
    assert ei.value.variant == "InvalidArgument"
    with pytest.raises(J.K3Error) as ei:  # a format the step cannot read
        m.set_tensor("blk.0.attn_norm.weight", 15, np.zeros(292, np.uint8), 256, 1)
    assert ei.value.variant == "CapabilityMismatch"
    with pytest.raises(J.K3Error) as ei:  # hidden not a multiple of 32
        J.DecodeModel(500, 1024, 1, 100, 4, 2, 64, 1e-6, 1e6, 64)
    assert ei.value.variant == "TensorBoundsError"
    with pytest.raises(J.K3Error) as ei:
        m.set_position(-2, 0)
    assert ei.value.variant == "TensorBoundsError"
    # every tensor absent is a model too (the reference's defaults throughout): it decodes
    m.finalize()
    assert m.logits_len() == 100
    m.set_position(7, 0)
    m.decode_step()
    m.status()
    assert m.read_token_pos()[1] == 1
    with pytest.raises(J.K3Error) as ei:
        J.DecodeModel(512, 1024, 1, 100, 8, 3, 64, 1e-6, 1e6, 64)
    assert ei.value.variant == "TensorBoundsError"


@pytest.mark.parametrize("mix,spec", [
    ("q8_0", dict(hidden=5120, ffn=13824, n_layers=2, vocab=1000, nq=40, nkv=8, hd=128, eps=1e-6, theta=1e6)),
    ("q4_k_m", dict(hidden=512, ffn=20480, n_layers=2, vocab=700, nq=8, nkv=2, hd=64, eps=1e-6, theta=1e6))])
def test_decode_long_rows(dev, mix, spec):
    """Projections whose rows are longer than the register-resident decode GEMV takes: a Q8_0
    model at hidden 5120 / FFN 13824 (every Q8_0 matrix is longer than 4096 elements: the Q|K|V
    store, SwiGLU, residual and LM-head argmax epilogues all run the long-row kernel), and a Q4_K_M
    model whose ffn_down rows hold 20480 elements; every layer checked as the other models are."""
    print(f"decode long rows {mix}", flush=True)
    t, on_dev = MS.build_device(spec, dev, seed=77, mix=mix)
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], 256, J.KV_F16, True)
    for name, (quant, arr, n_in, n_out) in t.items():
        m.set_tensor(name, quant, on_dev.get(name, arr), n_in, n_out)
    m.finalize()
    om = O.DecodeModel(spec, MS.oracle_tensors(t), 256)
    kv = prefill_kv(m, om, spec, 256, 100, 78, dev)
    DP.run_traced(m, om, t, spec, kv, 256, 100, 3, True, dev, 11)
    m.close()


def test_deterministic_projection_fallback(dev):
    """project_or_deterministic_slice (src/gemma.rs:841-860) in the decode step: projections left
    out, and one passed with the wrong element count (ignored, as the reference ignores it), take
    the fallback slice with the Qwen3 call sites' scales; the present ones run unfused.  Device
    logits against the oracle's over three greedy steps, within 1e-3."""
    from qdata import rand_weights
    spec = dict(hidden=512, ffn=1024, n_layers=2, vocab=300, nq=8, nkv=2, hd=64, eps=1e-6, theta=1e6)
    H, KV = spec["hidden"], spec["nkv"] * spec["hd"]
    print("decode with absent projections", flush=True)
    t = MS.build(spec, seed=21)
    absent = ["blk.0.attn_q.weight", "blk.0.attn_v.weight", "blk.0.ffn_up.weight", "blk.1.attn_output.weight",
              "blk.1.ffn_gate.weight", "blk.1.ffn_down.weight"]
    dev_t = {k: v for k, v in t.items() if k not in absent and k != "blk.1.attn_k.weight"}
    dev_t["blk.1.attn_k.weight"] = (J.Q4_K, rand_weights(J.Q4_K, 2 * KV, H, 77), H, 2 * KV)  # wrong count
    m = make_gpu_model(spec, dev_t, 64, J.KV_F32, True)
    host = {k: v for k, v in MS.oracle_tensors(t).items() if k not in absent and k != "blk.1.attn_k.weight"}
    om = O.DecodeModel(spec, host, 64)
    kv = om.new_kv()
    lg = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    tok = 5
    m.set_position(tok, 0)
    for pos in range(3):
        m.decode_step()
        torch.cuda.synchronize()
        m.read_logits(lg)
        ref = om.step(kv, tok, pos, threads=4)
        got = lg.cpu().numpy()
        err = DP.rel(got, ref)
        print(f"pos {pos}: rel err {err:.2e}", flush=True)
        assert err <= 1e-3, (pos, err)
        tok = int(O.argmax(ref))
        assert m.read_token_pos() == (tok, pos + 1)
    m.close()
