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


def layout_numpy(quant, w, k, n):
    """The records of jero_hip_repack_gemm restated in numpy from the GGUF bytes (the layouts its
    header documents), rows padded to a multiple of 32 with zeros.  Q4_K_G: per (32-row tile,
    block) the qs bytes 32 i + 16 h .. + 16 of row r at lane (r, h) of pair i, then per half h and
    row: d, dmin, the 8 unpacked 6-bit scales, the mins of sub-blocks 4 h .. 4 h + 3.  Q6_K_P: w = sc (q6 - 32) = 128 hi + lo, the planes at lane (r, h) of K step s
    (elements 32 s + 16 h .. + 16), then d as f32."""
    nb = k // 256
    tiles = (n + 31) // 32
    if quant == J.Q4_K:
        blk = np.zeros((tiles * 32, nb, 144), np.uint8)
        blk[:n] = w.reshape(n, nb, 144)
        out = np.zeros((tiles, nb, 5120), np.uint8)
        for t in range(tiles):
            for b in range(nb):
                rows = blk[32 * t:32 * t + 32, b]
                for i in range(4):
                    for h in range(2):
                        lanes = rows[:, 16 + 32 * i + 16 * h:16 + 32 * i + 16 * h + 16]  # [32 rows][16]
                        o = (i * 64 + 32 * h) * 16
                        out[t, b, o:o + 512] = lanes.reshape(-1)
                hdr = np.zeros((32, 2, 16), np.uint8)
                for r in range(32):
                    x = rows[r]
                    sc8 = x[4:16].astype(np.int64)
                    sc = [sc8[j] & 63 if j < 4 else (sc8[j + 4] & 15) | ((sc8[j - 4] >> 6) << 4) for j in range(8)]
                    mn = [sc8[j + 4] & 63 if j < 4 else (sc8[j + 4] >> 4) | ((sc8[j] >> 6) << 4) for j in range(8)]
                    for h in range(2):
                        hdr[r, h, :4] = x[:4]
                        hdr[r, h, 4:12] = sc
                        hdr[r, h, 12:16] = mn[4 * h:4 * h + 4]
                out[t, b, 4096:] = hdr.transpose(1, 0, 2).reshape(-1)  # [half][row][16]
        return out.reshape(-1)
    blk = w.reshape(n, nb, 210)
    wint = np.zeros((tiles * 32, nb, 256), np.int64)
    d = np.zeros((tiles * 32, nb), np.float32)
    for r in range(n):
        for b in range(nb):
            x = blk[r, b]
            ql, qh, scales = x[:128].astype(np.int64), x[128:192].astype(np.int64), x[192:208].view(np.int8)
            d[r, b] = x[208:210].view(np.float16)[0]
            for e in range(256):
                hn, rem = e // 128, e % 128
                kq, l = rem // 32, rem % 32
                lo4 = (ql[64 * hn + l + 32 * (kq & 1)] >> (4 * (kq >> 1))) & 15
                h2 = (qh[32 * hn + l] >> (2 * kq)) & 3
                wint[r, b, e] = int(scales[8 * hn + l // 16 + 2 * kq]) * ((lo4 | (h2 << 4)) - 32)
    hi = (wint + 64) >> 7
    lo = wint - 128 * hi
    out = np.zeros((tiles, nb, 16512), np.uint8)
    for t in range(tiles):
        for b in range(nb):
            for s_ in range(8):
                for p, plane in enumerate((hi, lo)):
                    for h in range(2):
                        e0 = 32 * s_ + 16 * h
                        frag = np.ascontiguousarray(plane[32 * t:32 * t + 32, b, e0:e0 + 16]).astype(np.int8).view(np.uint8)
                        o = ((2 * s_ + p) * 64 + 32 * h) * 16
                        out[t, b, o:o + 512] = frag.reshape(-1)
            out[t, b, 16384:] = np.ascontiguousarray(d[32 * t:32 * t + 32, b]).view(np.uint8)
    return out.reshape(-1)


@pytest.mark.parametrize("quant", [J.Q4_K, J.Q6_K])
def test_gemm_layout_bytes(dev, quant):
    """The GEMM layouts of GGUF bytes and of the _R device layouts equal a numpy restatement of
    the documented records byte for byte (rows past n_out zero)."""
    k, n = 512, 40
    w = rand_weights(quant, n, k, 8800 + quant)
    view = J.TensorView("w", quant, [k, n], to_dev(w, dev))
    ref = layout_numpy(quant, w, k, n)
    for v in (view, J.repack(view)):
        p = J.repack_gemm(v)
        assert p.quant == (J.Q4_K_G if quant == J.Q4_K else J.Q6_K_P)
        assert np.array_equal(p.data.cpu().numpy(), ref)


@pytest.mark.parametrize("quant", [J.Q4_K, J.Q6_K])
@pytest.mark.parametrize("m,k,n", [(8, 256, 64), (37, 512, 96), (128, 1024, 384), (200, 4096, 130),
                                   (513, 2048, 256), (257, 512, 8224)])
def test_gemm_laid_matches_oracle(dev, quant, m, k, n):
    """jero_hip_gemm over the GEMM layouts (Q4_K_G / Q6_K_P) against the oracle: ragged token
    tiles, n_out past the last 32-row tile, one block (no K split), the two-way K split of small
    grids and the unsplit grid (257 x 8224: 325 tiles of 64 x 128).  The layouts of the _R tensors give the
    same bits."""
    print(f"gemm laid quant={quant} m={m} k={k} n={n}", flush=True)
    w = rand_weights(quant, n, k, 7300 + quant + m + n)
    x = rand_act(k, 7301 + m, m=m)
    xq = J.quantize_act(J.Q8_K, to_dev(x, dev))
    view = J.TensorView("w", quant, [k, n], to_dev(w, dev))
    y = torch.full((m, n), float("nan"), device=dev)
    J.gemm(J.repack_gemm(view), xq, m, y)
    yr = torch.full((m, n), float("nan"), device=dev)
    J.gemm(J.repack_gemm(J.repack(view)), xq, m, yr)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert np.array_equal(yr.cpu().numpy(), y)
    ref = O.gemm(quant, w, k, n, xq.cpu().numpy(), m, threads=8)
    assert np.all(np.isfinite(y))
    assert rel_err(y, ref) < REL_TOL


@pytest.mark.parametrize("quant,m,k,n", [
    (J.Q4_K, 512, 4096, 14336),   # the timed prefill GEMM: 8 x 112 tiles, 896 workgroups, unsplit
    (J.Q4_K, 512, 4096, 24576),   # the 8B prefill's gate|up: 1536 workgroups
    (J.Q4_K, 512, 4096, 5120),    # Q|K of the Q6_K-attn_v layers: 320 workgroups
    (J.Q4_K, 512, 4096, 4096),    # Wo: 256 tiles, K split in two
    (J.Q4_K, 512, 12288, 4096),   # Q4_K ffn_down, K split
    (J.Q6_K, 512, 4096, 14336),   # the timed shape over Q6_K_P
    (J.Q6_K, 512, 12288, 4096),   # Q6_K ffn_down, K split
    (J.Q6_K, 512, 4096, 1024)])   # Q6_K attn_v, K split
def test_gemm_laid_prefill_shapes(dev, quant, m, k, n):
    """jero_hip_gemm over the GEMM layouts at the sizes bench.py and the 8B prefill run (the
    grids whose workgroup-to-tile remap and K split the small cases above do not reach): every
    row equals the GPU GEMV of that token row (bit-exact in its int32 partials against the
    oracle) within 1e-5, and 8 rows spread over the token tiles match the oracle within 1e-5."""
    print(f"gemm laid prefill shape quant={quant} m={m} k={k} n={n}", flush=True)
    w = rand_weights(quant, n, k, 9300 + quant + n + k)
    x = rand_act(k, 9301 + n + k, m=m)
    xqd = J.quantize_act(J.Q8_K, to_dev(x, dev))
    view = J.TensorView("w", quant, [k, n], to_dev(w, dev))
    y = torch.full((m, n), float("nan"), device=dev)
    J.gemm(J.repack_gemm(view), xqd, m, y)
    rb = J.row_bytes(J.Q8_K, k)
    g = torch.full((m, n), float("nan"), device=dev)
    for r in range(m):
        J.matvec(view, xqd[r * rb:(r + 1) * rb], g[r])
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    assert np.all(np.isfinite(y))
    assert rel_err(y, g.cpu().numpy()) < REL_TOL
    xq = xqd.cpu().numpy()
    rows = [0, 63, 64, 200, 255, 256, 383, 511]
    ref = np.stack([O.matvec(quant, w, k, n, xq[r * rb:(r + 1) * rb], threads=8) for r in rows])
    assert rel_err(y[rows], ref) < REL_TOL


def test_gemm_laid_q4k_extremes(dev):
    """Q4_K_G at the top of the expanded planes (scale 63 = 8 * 7 + 7, nibble 15: 105 each),
    zero scales and mins, zero and tiny activation rows."""
    m, k, n = 64, 1024, 128
    w = rand_weights(J.Q4_K, n, k, 77).reshape(n * (k // 256), 144)
    w[0::3, 4:16] = 0xFF
    w[1::3, 4:16] = 0x00
    w[0::5, 16:] = 0xFF
    w = w.reshape(-1)
    x = rand_act(k, 78, m=m)
    x[3] = 0.0
    x[5, :256] = 1e-30
    xq = J.quantize_act(J.Q8_K, to_dev(x, dev))
    view = J.TensorView("w", J.Q4_K, [k, n], to_dev(w, dev))
    y = torch.empty((m, n), device=dev)
    J.gemm(J.repack_gemm(view), xq, m, y)
    ref = O.gemm(J.Q4_K, w, k, n, xq.cpu().numpy(), m, threads=8)
    y = y.cpu().numpy()
    assert np.all(y[3] == 0.0)
    assert rel_err(y, ref) < REL_TOL


def test_gemm_layout_errors(dev):
    w = to_dev(rand_weights(J.Q4_K, 64, 256, 3), dev)
    assert J.gemm_layout_bytes(J.Q4_K, 256, 64) == 2 * 5120
    assert J.gemm_layout_bytes(J.Q6_K, 512, 33) == 2 * 2 * 16512
    assert J.gemm_layout_bytes(J.Q8_0, 256, 64) == 0 and J.gemm_layout_bytes(J.Q4_K, 100, 64) == 0
    with pytest.raises(J.K3Error) as e:
        J.repack_gemm(J.TensorView("w", J.Q8_0, [256, 64], w))
    assert e.value.variant == "CapabilityMismatch"
    p = J.repack_gemm(J.TensorView("w", J.Q4_K, [256, 64], w))
    xq = J.quantize_act(J.Q8_K, to_dev(rand_act(256, 4, m=2), dev))
    y = torch.empty((2, 64), device=dev)
    short = J.TensorView("w", J.Q4_K_G, [256, 64], p.data[:-16])
    with pytest.raises(J.K3Error) as e:
        J.gemm(short, xq, 2, y)
    assert e.value.variant == "TensorBoundsError"
    with pytest.raises(J.K3Error) as e:
        J.matvec(p, xq[:J.row_bytes(J.Q8_K, 256)], y[0])
    assert e.value.variant == "CapabilityMismatch"


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
