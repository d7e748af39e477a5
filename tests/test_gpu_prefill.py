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


@pytest.mark.parametrize("nq,nkv,hd", [(16, 2, 64), (4, 4, 64), (4, 2, 128)])
def test_prefill_group_sizes(dev, nq, nkv, hd):
    """The batched attention kernel gives each wave 16 / group tokens: groups of 8, 1 and 2 (head_dim
    64 and 128), f16 ring, 40 prompt tokens after 37 filled slots (crossing a 64-slot split)."""
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


def test_prefill_errors(dev):
    spec = SMALL
    t = MS.build(spec, seed=2)
    m = make_gpu_model(spec, t, 32, J.KV_F16, True)
    with pytest.raises(J.K3Error) as ei:
        m.prefill(list(range(20)), 13)  # positions 13 .. 32 past the 32-slot ring
    assert ei.value.variant == "ContextLengthExceeded"
    with pytest.raises(J.K3Error) as ei:
        m.prefill([1, 2, spec["vocab"]], 0)
    assert ei.value.variant == "TensorBoundsError"
    with pytest.raises(J.K3Error) as ei:
        m.prefill([], 0)
    assert ei.value.variant == "TensorBoundsError"
    m.close()
