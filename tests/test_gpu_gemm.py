"""GPU parity of the prefill GEMM (Q4_K x Q8_K on int8 MFMA, other formats row by row) and of
the exact int8 GEMM.

Bar: GEMM rows within 1e-5 relative (|y - ref| / max(|ref|, rms(ref))) of the oracle's GEMV of
the same quantized activation row (the reference's prefill is one matvec_any per token); the
int8 GEMM bit-exact against an int64 numpy product and the oracle's jo_gemm_i8.
"""
import numpy as np
import pytest
import torch

import jero_hip as J
import pyoracle as O
from qdata import rand_act, rand_weights

pytestmark = pytest.mark.gpu

REL_TOL = 1e-5


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rel_err(y, ref):
    ref = np.asarray(ref, np.float64)
    y = np.asarray(y, np.float64)
    out = 0.0
    for r in range(ref.shape[0]):
        scale = max(float(np.sqrt(np.mean(ref[r] ** 2))), 1e-30)
        out = max(out, float(np.max(np.abs(y[r] - ref[r]) / np.maximum(np.abs(ref[r]), scale))))
    return out


def run_gemm(dev, quant, m, k, n, seed):
    w = rand_weights(quant, n, k, seed)
    x = rand_act(k, seed + 1, m=m)
    xq = J.quantize_act(J.act_format(quant), to_dev(x, dev))
    view = J.TensorView("w", quant, [k, n], to_dev(w, dev))
    y = torch.full((m, n), float("nan"), device=dev)
    J.gemm(view, xq, m, y)
    torch.cuda.synchronize()
    return w, xq.cpu().numpy(), y.cpu().numpy(), view


@pytest.mark.parametrize("m,k,n", [(1, 256, 128), (37, 512, 256), (128, 1024, 384), (200, 4096, 128),
                                   (130, 256, 640), (257, 2048, 256)])
def test_gemm_q4k_mfma_matches_oracle(dev, m, k, n):
    print(f"gemm q4_k m={m} k={k} n={n}", flush=True)
    w, xq, y, _ = run_gemm(dev, J.Q4_K, m, k, n, 5000 + m + k + n)
    ref = O.gemm(J.Q4_K, w, k, n, xq, m, threads=8)
    assert np.all(np.isfinite(y))
    assert rel_err(y, ref) < REL_TOL


def test_gemm_q4k_extreme_scales_and_zero_rows(dev):
    """Sub-block scales and mins at 63 and 0, nibbles at 15, zero activation rows."""
    m, k, n = 64, 1024, 128
    w = rand_weights(J.Q4_K, n, k, 77).reshape(n * (k // 256), 144)
    w[0::3, 4:16] = 0xFF          # every 6-bit scale and min at 63
    w[1::3, 4:16] = 0x00          # all zero: rows reduce to 0 * ... - 0
    w[0::5, 16:] = 0xFF           # nibbles at 15
    w = w.reshape(-1)
    x = rand_act(k, 78, m=m)
    x[3] = 0.0
    x[5, :256] = 1e-30            # tiny block next to normal ones
    xq = J.quantize_act(J.Q8_K, to_dev(x, dev))
    view = J.TensorView("w", J.Q4_K, [k, n], to_dev(w, dev))
    y = torch.empty((m, n), device=dev)
    J.gemm(view, xq, m, y)
    ref = O.gemm(J.Q4_K, w, k, n, xq.cpu().numpy(), m, threads=8)
    y = y.cpu().numpy()
    assert np.all(y[3] == 0.0)
    assert rel_err(y, ref) < REL_TOL


def test_gemm_q4k_prefill_shape_rows_equal_gemv(dev):
    """M=512 tokens, K=4096, N=14336: every row equals the GPU GEMV of that token (itself
    bit-exact in its partials against the oracle), and a sample of rows matches the oracle."""
    m, k, n = 512, 4096, 14336
    w, xq, y, view = run_gemm(dev, J.Q4_K, m, k, n, 9100)
    assert np.all(np.isfinite(y))
    rb = J.row_bytes(J.Q8_K, k)
    xqd = to_dev(xq, dev)
    g = torch.empty((m, n), device=dev)
    for r in range(m):
        J.matvec(view, xqd[r * rb:(r + 1) * rb], g[r])
    assert rel_err(y, g.cpu().numpy()) < REL_TOL
    rows = [0, 1, 127, 128, 255, 300, 511]
    ref = np.stack([O.matvec(J.Q4_K, w, k, n, xq[r * rb:(r + 1) * rb], threads=8) for r in rows])
    assert rel_err(y[rows], ref) < REL_TOL


@pytest.mark.parametrize("m,k,n", [(8, 256, 64), (37, 512, 96), (128, 1024, 384), (200, 4096, 130),
                                   (513, 12288, 256)])
def test_gemm_q6k_planes_matches_oracle(dev, m, k, n):
    """Q6_K from 8 rows: the int8-MFMA kernel over the tensor's hi / lo planes (w = sc (q6 - 32)
    = 128 hi + lo), on GGUF bytes and on the Q6_K_R device layout."""
    print(f"gemm q6_k m={m} k={k} n={n}", flush=True)
    w, xq, y, view = run_gemm(dev, J.Q6_K, m, k, n, 7000 + m + k + n)
    ref = O.gemm(J.Q6_K, w, k, n, xq, m, threads=8)
    assert np.all(np.isfinite(y))
    assert rel_err(y, ref) < REL_TOL
    yr = torch.full((m, n), float("nan"), device=dev)
    J.gemm(J.repack(view), to_dev(xq, dev), m, yr)
    torch.cuda.synchronize()
    assert np.array_equal(yr.cpu().numpy(), y)


def test_gemm_q6k_planes_extremes(dev):
    """Sub-block scales at -128 and 127 with q6 at 0 and 63 (w = 4096 and 3937: the planes' hi
    at its top), zero and tiny activation rows."""
    m, k, n = 40, 1024, 128
    w = rand_weights(J.Q6_K, n, k, 81).reshape(n * (k // 256), 210)
    w[0::4, 192:208] = np.uint8(0x80)   # every scale -128
    w[1::4, 192:208] = np.uint8(0x7F)   # every scale 127
    w[0::8, :192] = 0x00                # q6 = 0
    w[1::8, :192] = 0xFF                # q6 = 63
    w = w.reshape(-1)
    x = rand_act(k, 82, m=m)
    x[3] = 0.0
    x[7, :256] = 1e-30
    xq = J.quantize_act(J.Q8_K, to_dev(x, dev))
    view = J.TensorView("w", J.Q6_K, [k, n], to_dev(w, dev))
    y = torch.empty((m, n), device=dev)
    J.gemm(view, xq, m, y)
    ref = O.gemm(J.Q6_K, w, k, n, xq.cpu().numpy(), m, threads=8)
    y = y.cpu().numpy()
    assert np.all(y[3] == 0.0)
    assert rel_err(y, ref) < REL_TOL


@pytest.mark.parametrize("quant,m,k,n", [(J.Q8_0, 5, 512, 96), (J.Q4_0, 3, 256, 40), (J.Q6_K, 4, 512, 64),
                                         (J.Q4_K, 3, 256, 100)])
def test_gemm_row_path_formats(dev, quant, m, k, n):
    """Formats and shapes outside the MFMA kernel run one GEMV per row."""
    w, xq, y, _ = run_gemm(dev, quant, m, k, n, 6100 + quant)
    ref = O.gemm(quant, w, k, n, xq, m, threads=8)
    assert rel_err(y, ref) < REL_TOL


def test_gemm_errors(dev):
    w = to_dev(rand_weights(J.Q4_K, 128, 256, 1), dev)
    view = J.TensorView("w", J.Q4_K, [256, 128], w)
    xq = J.quantize_act(J.Q8_K, to_dev(rand_act(256, 2, m=2), dev))
    y = torch.empty((2, 128), device=dev)
    with pytest.raises(J.K3Error) as e:
        J.gemm(view, xq, 0, y)
    assert e.value.variant == "TensorBoundsError"
    bad = J.TensorView("w", J.Q4_K, [256, 129], w)
    with pytest.raises(J.K3Error) as e:
        J.gemm(bad, xq, 2, y)
    assert e.value.variant == "TensorBoundsError"


@pytest.mark.parametrize("m,k,n", [(512, 512, 512), (1024, 512, 512), (512, 1024, 512), (37, 80, 45),
                                   (130, 4096, 260), (5, 33, 7), (1, 16, 1)])
def test_gemm_i8_bit_exact(dev, m, k, n):
    print(f"gemm_i8 m={m} k={k} n={n}", flush=True)
    rng = np.random.default_rng(m * 7 + k * 3 + n)
    x = rng.integers(-128, 128, size=(m, k), dtype=np.int64).astype(np.int8)
    w = rng.integers(-128, 128, size=(n, k), dtype=np.int64).astype(np.int8)
    out = J.gemm_i8(to_dev(x, dev), to_dev(w, dev)).cpu().numpy()
    ref = x.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(out.astype(np.int64), ref)
    if m * n * k <= 1 << 24:
        assert np.array_equal(out, O.gemm_i8(x, w))


def test_gemm_i8_extremes(dev):
    """All -128 x -128 over k = 8192 (the largest magnitude sums) and alternating signs."""
    m, k, n = 64, 8192, 128
    x = np.full((m, k), -128, np.int8)
    w = np.full((n, k), -128, np.int8)
    w[1::2] = 127
    out = J.gemm_i8(to_dev(x, dev), to_dev(w, dev)).cpu().numpy()
    ref = x.astype(np.int64) @ w.astype(np.int64).T
    assert np.array_equal(out.astype(np.int64), ref)


def test_gemm_i8_errors(dev):
    x = torch.zeros((4, 200000), dtype=torch.int8, device=dev)
    with pytest.raises(J.K3Error) as e:
        J.gemm_i8(x, x)
    assert e.value.variant == "CapabilityMismatch"
    with pytest.raises(J.K3Error) as e:
        J.gemm_i8(x[:, :16], torch.zeros((3, 8), dtype=torch.int8, device=dev))
    assert e.value.variant == "TensorBoundsError"
