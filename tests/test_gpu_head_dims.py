"""GPU parity of the decode step and the batched prefill at head dims and group sizes outside the
head_dim-built attention kernels (32 / 64 / 128, at most 8 q heads per kv head): the generic split
kernel and its merge, fused with QK-norm, RoPE and the ring append in the decode step, and the
prefill's QK-norm / RoPE rows at head_dim up to 256.  The recipes take any even head_dim
(even_head_dim, src/qwen_deepseek.rs:58-65).  Every layer teacher-forced against the oracle at the
decode bars (decode_parity.run_traced / run_prefill_traced)."""
import numpy as np
import pytest

import decode_parity as DP
import jero_hip as J
import model_spec as MS
import pyoracle as O
from test_gpu_decode import make_gpu_model, prefill_kv

pytestmark = pytest.mark.gpu

BASE = dict(hidden=512, ffn=1024, n_layers=2, vocab=1000, eps=1e-6, theta=1e6)


@pytest.mark.parametrize("nq,nkv,hd,kv_name", [
    (8, 2, 96, "f16"),    # head_dim 96, group 4
    (16, 4, 80, "f32"),   # head_dim 80 (40 RoPE pairs), f32 ring
    (4, 2, 256, "f16"),   # head_dim 256 (two RoPE pairs per lane in the prefill rows)
    (16, 1, 64, "f16"),   # group 16 at head_dim 64
    (24, 2, 64, "f32"),   # group 12, f32 ring
])
def test_decode_and_prefill_head_dims(dev, nq, nkv, hd, kv_name):
    print(f"head dims nq={nq} nkv={nkv} hd={hd} kv={kv_name}", flush=True)
    spec = dict(BASE, nq=nq, nkv=nkv, hd=hd)
    kv_f16 = kv_name == "f16"
    cap, pos0, n = 160, 37, 40
    t = MS.build(spec, seed=hd + nq)
    m = make_gpu_model(spec, t, cap, J.KV_F16 if kv_f16 else J.KV_F32, True)
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = prefill_kv(m, om, spec, cap, pos0, hd + 1, dev, kv_f16)
    tokens = np.random.default_rng(hd).integers(0, spec["vocab"], size=n).tolist()
    gtok, _ = DP.run_prefill_traced(m, om, t, spec, kv, cap, pos0, tokens, kv_f16, dev, True)
    DP.run_traced(m, om, t, spec, kv, cap, pos0 + n, 3, kv_f16, dev, gtok, True)
    m.close()
