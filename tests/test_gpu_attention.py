"""GPU parity of decode attention against the oracle (gqa_causal_attention_f32 semantics).

Bar: |out - ref| <= 1e-3 * max(|ref|, rms(ref)) per element (the attention tolerance of the
north-star spec); f16 K/V are compared with the oracle run on the same f16 values widened.
"""
import numpy as np
import pytest
import torch

import jero_hip as J
import pyoracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def rel_err(y, ref):
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.sqrt(np.mean(ref ** 2))), 1e-30)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref) / np.maximum(np.abs(ref), scale)))


CASES = [  # nq, nkv, hd, seq
    (32, 8, 128, 1), (32, 8, 128, 7), (32, 8, 128, 128), (32, 8, 128, 129), (32, 8, 128, 1000),
    (32, 8, 128, 4096), (4, 2, 32, 4), (4, 2, 32, 300), (8, 8, 64, 257), (16, 2, 64, 64), (8, 1, 128, 513),
]


# head_dim outside {32, 64, 128} or more than 8 q heads per kv head: the generic kernels
GENERIC_CASES = [
    (4, 4, 48, 4), (8, 2, 80, 300), (12, 4, 96, 129), (16, 1, 256, 700), (32, 2, 32, 65), (64, 2, 128, 257),
    (6, 3, 2, 70), (10, 5, 160, 64), (8, 8, 192, 4096), (3, 1, 256, 1), (48, 4, 64, 1000),
]


@pytest.mark.parametrize("kv", ["f32", "f16"])
@pytest.mark.parametrize("nq,nkv,hd,seq", CASES + GENERIC_CASES)
def test_gqa_attention_parity(dev, kv, nq, nkv, hd, seq):
    print(f"attention kv={kv} nq={nq} nkv={nkv} hd={hd} seq={seq}", flush=True)
    rng = np.random.default_rng(nq * 1000 + seq + hd)
    q = rng.standard_normal(nq * hd).astype(np.float32)
    k = rng.standard_normal((seq, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((seq, nkv * hd)).astype(np.float32)
    if kv == "f16":
        k = k.astype(np.float16)
        v = v.astype(np.float16)
    scale = 1.0 / np.sqrt(hd)
    out = torch.empty(nq * hd, dtype=torch.float32, device=dev)
    J.gqa_causal_attention_f32(out, torch.from_numpy(q).to(dev), torch.from_numpy(k).to(dev),
                               torch.from_numpy(v).to(dev), nq, nkv, hd, seq, scale)
    torch.cuda.synchronize()
    ref = O.gqa_attention(q, k.astype(np.float32), v.astype(np.float32), nq, nkv, hd, seq, scale)
    assert rel_err(out.cpu().numpy(), ref) < TOL


def test_attention_shape_errors(dev):
    z = torch.zeros(1024, dtype=torch.float32, device=dev)
    with pytest.raises(J.K3Error) as ei:
        J.gqa_causal_attention_f32(z, z, z, z, 6, 4, 32, 4, 1.0)
    assert ei.value.variant == "TensorBoundsError"
    with pytest.raises(J.K3Error) as ei:  # odd head_dim (even_head_dim never gives one)
        J.gqa_causal_attention_f32(z, z, z, z, 4, 4, 47, 4, 1.0)
    assert ei.value.variant == "CapabilityMismatch"
    with pytest.raises(J.K3Error) as ei:  # above 256
        J.gqa_causal_attention_f32(z, z, z, z, 1, 1, 258, 1, 1.0)
    assert ei.value.variant == "CapabilityMismatch"
