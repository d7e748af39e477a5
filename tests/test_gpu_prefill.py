"""GPU parity of the batched prefill (jero_hip_model_prefill): the prompt's tokens through each
layer at once as GEMMs over the token rows, causal attention over the ring, against the oracle's
token loop (run_prefill_with_hidden, src/qwen_deepseek.rs:2217-2316).  Prefill writes each
token's trace in the decode step's layout, so every prompt token is held to the decode bars
(decode_parity.run_prefill_traced): every layer teacher-forced, each token's hidden state and the
last token's logits within 1e-3 end to end with tie flips accounted.  Decode steps then continue
from the prefilled ring (decode_parity.run_traced)."""
import numpy as np
import pytest
import torch

import decode_parity as DP
import jero_hip as J
import model_spec as MS
import pyoracle as O
from test_gpu_decode import make_gpu_model, prefill_kv

pytestmark = pytest.mark.gpu

SMALL = dict(hidden=512, ffn=1024, n_layers=3, vocab=1000, nq=8, nkv=2, hd=64, eps=1e-6, theta=1e6)


@pytest.mark.parametrize("mix,kv_name,qk_norm,cap,pos0,n", [
    ("q4_k_m", "f16", True, 400, 0, 17),       # Q4_K_R rows through the int8-MFMA GEMM, Q6_K rows per token
    ("q4_k_m", "f32", True, 400, 37, 300),     # a prompt longer than one attention batch, after a filled ring
    ("q4_k_m", "f16", True, 400, 37, 300),     # the same on the f16 ring (the batched MFMA attention kernel)
    ("q8_0", "f16", False, 128, 5, 40),         # Q8_0 rows (GEMV per row), no QK-norm
    ("q4_k_m", "f16", True, 64, 0, 1)])         # a one-token prompt
def test_prefill_matches_oracle(dev, mix, kv_name, qk_norm, cap, pos0, n):
    print(f"prefill mix={mix} kv={kv_name} qk_norm={qk_norm} cap={cap} pos0={pos0} n={n}", flush=True)
    spec = SMALL
    t = MS.build(spec, seed=11, mix=mix)
    kv_f16 = kv_name == "f16"
    m = make_gpu_model(spec, t, cap, J.KV_F16 if kv_f16 else J.KV_F32, qk_norm)
    host = MS.oracle_tensors(t)
    if not qk_norm:
        host = {k: v for k, v in host.items() if "_q_norm" not in k and "_k_norm" not in k}
    om = O.DecodeModel(spec, host, cap)
    kv = prefill_kv(m, om, spec, cap, pos0, 13, dev, kv_f16)
    rng = np.random.default_rng(pos0 + n)
    tokens = rng.integers(0, spec["vocab"], size=n).tolist()
    gtok, _ = DP.run_prefill_traced(m, om, t, spec, kv, cap, pos0, tokens, kv_f16, dev, qk_norm)
    if pos0 + n + 2 <= cap:  # decoding continues from the ring the prefill wrote
        DP.run_traced(m, om, t, spec, kv, cap, pos0 + n, 2, kv_f16, dev, gtok, qk_norm)
    m.close()


@pytest.mark.parametrize("nq,nkv,hd", [(16, 2, 64), (4, 4, 64), (4, 2, 128), (12, 4, 64), (6, 2, 128)])
def test_prefill_group_sizes(dev, nq, nkv, hd):
    """The flash attention kernel gives each column set 16 / group tokens: groups of 8, 1, 2 and 3
    (15 of the 16 columns used; the group's rows fill no whole 256-block, so the output projection
    quantizes the f32 rows), head_dim 64 and 128, f16 ring, 40 prompt tokens after 37 filled
    slots (crossing a 64-slot run)."""
    print(f"prefill nq={nq} nkv={nkv} hd={hd}", flush=True)
    spec = dict(SMALL, nq=nq, nkv=nkv, hd=hd, n_layers=2)
    cap, pos0, n = 128, 37, 40
    t = MS.build(spec, seed=29)
    m = make_gpu_model(spec, t, cap, J.KV_F16, True)
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = prefill_kv(m, om, spec, cap, pos0, 31, dev, True)
    tokens = np.random.default_rng(nq * 10 + nkv).integers(0, spec["vocab"], size=n).tolist()
    gtok, _ = DP.run_prefill_traced(m, om, t, spec, kv, cap, pos0, tokens, True, dev, True)
    DP.run_traced(m, om, t, spec, kv, cap, pos0 + n, 2, True, dev, gtok, True)
    m.close()


@pytest.mark.parametrize("kv_name,n", [("f16", 300), ("f16", 17), ("f32", 300)])
def test_prefill_untraced_matches_traced(dev, kv_name, n):
    """The prefill without a trace -- the path bench.py times: attention writes only Wo's Q8_K
    rows, no normalised rows are stored, a split V projection's two K halves are added by the
    QK-norm / RoPE step -- leaves the same KV rings, logits and next token, bit for bit, as the
    traced prefill that the other tests hold to the oracle (layer 0 of the mix has a Q6_K attn_v,
    projected apart and split in K)."""
    print(f"prefill untraced vs traced kv={kv_name} n={n}", flush=True)
    spec = SMALL
    cap = 400
    t = MS.build(spec, seed=11)
    kv_dtype, es = (J.KV_F16, 2) if kv_name == "f16" else (J.KV_F32, 4)
    tokens = np.random.default_rng(n).integers(0, spec["vocab"], size=n).tolist()
    ring_bytes = cap * spec["nkv"] * spec["hd"] * es
    outs = []
    for traced in (True, False):
        m = make_gpu_model(spec, t, cap, kv_dtype, True)
        if traced:
            _, _, _, total = m.trace_layout()
            buf = torch.zeros(n * total, dtype=torch.uint8, device=dev)
            m.set_trace(buf)
        m.prefill(tokens, 0)
        m.status()
        if traced:
            m.set_trace(None)
        logits = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
        m.read_logits(logits)
        rings = []
        for layer in range(spec["n_layers"]):
            for ptr in m.kv_ptrs(layer):
                r = torch.empty(ring_bytes, dtype=torch.uint8, device=dev)
                J._memcpy(r.data_ptr(), ptr, ring_bytes)
                rings.append(r.cpu().numpy())
        outs.append((logits.cpu().numpy(), rings, m.read_token_pos()))
        m.close()
    (la, ra, ta), (lb, rb, tb) = outs
    assert ta == tb == (ta[0], n)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    for x, y in zip(ra, rb):
        assert np.array_equal(x, y)


def test_prefill_matches_decode_steps_8b_layer_shape(dev):
    """Two layers of the Qwen3-8B shape, f16 ring: a 24-token prompt after 4000 filled slots."""
    spec = dict(hidden=4096, ffn=12288, n_layers=2, vocab=151936, nq=32, nkv=8, hd=128, eps=1e-6, theta=1e6)
    cap, pos0, n = 4096, 4000, 24
    print("prefill qwen3-8b layer shape", flush=True)
    t = MS.build(spec, seed=19)
    m = make_gpu_model(spec, t, cap, J.KV_F16, True)
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = prefill_kv(m, om, spec, cap, pos0, 23, dev)
    tokens = np.random.default_rng(3).integers(0, spec["vocab"], size=n).tolist()
    DP.run_prefill_traced(m, om, t, spec, kv, cap, pos0, tokens, True, dev)
    m.close()


QWEN3_8B_2L = dict(hidden=4096, ffn=12288, n_layers=2, vocab=151936, nq=32, nkv=8, hd=128, eps=1e-6, theta=1e6)


@pytest.mark.timeout(900)
def test_prefill_8b_layer_shape_512_tokens(dev):
    """The prefill bench.py times -- a 512-token prompt from position 0 into an f16 ring of 4096
    slots -- on two layers of the Qwen3-8B shape: at 512 rows the Q|K (320 workgroups) and
    gate|up (1536) GEMMs run unsplit with the workgroup-to-tile remap, Wo and ffn_down split K, the
    Q6_K attn_v of layer 0 runs on the second stream, and the flash attention kernel covers 512
    queries.  Every one of the 512 prompt tokens is held to the decode bars (every layer
    teacher-forced, its hidden state within 1e-3 end to end, the last token's logits within 1e-3)."""
    spec = QWEN3_8B_2L
    cap, pos0, n = 4096, 0, 512
    print("prefill qwen3-8b layer shape, 512 tokens from position 0", flush=True)
    t = MS.build(spec, seed=51)
    m = make_gpu_model(spec, t, cap, J.KV_F16, True)
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = prefill_kv(m, om, spec, cap, pos0, 53, dev)
    tokens = np.random.default_rng(57).integers(0, spec["vocab"], size=n).tolist()
    gtok, res = DP.run_prefill_traced(m, om, t, spec, kv, cap, pos0, tokens, True, dev)
    print(f"  tie flips over the prompt {sum(r[0] for r in res)}, worst error {max(r[1] for r in res):.2e}",
          flush=True)
    DP.run_traced(m, om, t, spec, kv, cap, pos0 + n, 1, True, dev, gtok)
    m.close()


@pytest.mark.timeout(600)
def test_prefill_untraced_matches_traced_8b_layer_shape(dev):
    """The untraced prefill (the timed path) equals the traced one bit for bit at the timed size:
    two layers of the 8B shape, 512 tokens from position 0, f16 ring of 4096 slots (rings,
    logits, next token)."""
    print("prefill untraced vs traced, qwen3-8b layer shape, 512 tokens", flush=True)
    spec = QWEN3_8B_2L
    cap, n = 4096, 512
    t = MS.build(spec, seed=61)
    tokens = np.random.default_rng(62).integers(0, spec["vocab"], size=n).tolist()
    ring_bytes = cap * spec["nkv"] * spec["hd"] * 2
    outs = []
    for traced in (True, False):
        m = make_gpu_model(spec, t, cap, J.KV_F16, True)
        buf = None
        if traced:
            _, _, _, total = m.trace_layout()
            buf = torch.zeros(n * total, dtype=torch.uint8, device=dev)
            m.set_trace(buf)
        m.prefill(tokens, 0)
        m.status()
        if traced:
            m.set_trace(None)
            del buf
        logits = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
        m.read_logits(logits)
        rings = []
        for layer in range(spec["n_layers"]):
            for ptr in m.kv_ptrs(layer):
                r = torch.empty(ring_bytes, dtype=torch.uint8, device=dev)
                J._memcpy(r.data_ptr(), ptr, ring_bytes)
                rings.append(r.cpu().numpy())
        outs.append((logits.cpu().numpy(), rings, m.read_token_pos()))
        m.close()
        torch.cuda.empty_cache()
    (la, ra, ta), (lb, rb, tb) = outs
    assert ta == tb == (ta[0], n)
    assert np.array_equal(la.view(np.uint32), lb.view(np.uint32))
    for x, y in zip(ra, rb):
        assert np.array_equal(x, y)


def test_prefill_errors(dev):
    spec = SMALL
    t = MS.build(spec, seed=2)
    m = make_gpu_model(spec, t, 32, J.KV_F16, True)
    with pytest.raises(J.K3Error) as ei:
        m.prefill(list(range(20)), 13)  # positions 13 .. 32 past the 32-slot ring
    assert ei.value.variant == "ContextLengthExceeded"
    with pytest.raises(J.K3Error) as ei:  # a token id beyond the vocabulary embeds (embed_token); a negative one is no id
        m.prefill([1, 2, -1], 0)
    assert ei.value.variant == "TensorBoundsError"
    with pytest.raises(J.K3Error) as ei:
        m.prefill([], 0)
    assert ei.value.variant == "TensorBoundsError"
    m.close()
