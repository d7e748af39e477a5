"""GPU parity of the Q8 activation quantizers and the GEMV family against the oracle.

Bar: activation bytes and int32 partial sums bit-exact; f32 outputs within 1e-5 relative
to the oracle's f64 result, relative meaning |y - y_ref| / max(|y_ref|, rms(y_ref)).
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
    scale = max(float(np.sqrt(np.mean(ref ** 2))), 1e-30)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref) / np.maximum(np.abs(ref), scale)))


@pytest.mark.parametrize("act,k,m", [(J.ACT_Q8, 32, 1), (J.ACT_Q8, 4096, 1), (J.ACT_Q8, 4096, 7),
                                     (J.Q8_K, 256, 1), (J.Q8_K, 4096, 1), (J.Q8_K, 12288, 1),
                                     (J.Q8_K, 4096, 512)])
def test_quantize_act_bit_exact(dev, act, k, m):
    print(f"quantize act={act} k={k} m={m}", flush=True)
    x = rand_act(k, 100 + k + m, m=m)
    x[0, :32] = 0.0                      # zero block (ACT_Q8) / partly zero (Q8_K)
    if act == J.Q8_K and m > 1:
        x[1, :256] = 0.0                 # all-zero Q8_K block
        x[1, 256 + 5], x[1, 256 + 9] = -3.0, 3.0  # tie of opposite signs: first one wins
    xd = to_dev(x, dev)
    q = J.quantize_act(act, xd)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(q.cpu().numpy(), O.quantize_act(act, x))


SHAPES = [  # (quant, n_in, n_out)
    (J.Q4_K, 4096, 4096), (J.Q4_K, 4096, 12288), (J.Q4_K, 12288, 4096), (J.Q4_K, 2048, 768),
    (J.Q4_K, 256, 77), (J.Q4_K, 768, 33), (J.Q4_K, 32768, 5),
    (J.Q6_K, 4096, 4096), (J.Q6_K, 768, 2048), (J.Q6_K, 12288, 100), (J.Q6_K, 256, 9), (J.Q6_K, 1280, 3),
    (J.Q8_0, 4096, 4096), (J.Q8_0, 128, 16), (J.Q8_0, 96, 5), (J.Q8_0, 16384, 7),
    (J.Q4_0, 4096, 1000), (J.Q4_0, 160, 3),
]


@pytest.mark.parametrize("quant,n_in,n_out", SHAPES)
def test_matvec_parity(dev, quant, n_in, n_out):
    print(f"matvec quant={quant} n_in={n_in} n_out={n_out}", flush=True)
    w = rand_weights(quant, n_out, n_in, quant * 1000 + n_in + n_out, full_range=True)
    act = J.act_format(quant)
    x = rand_act(n_in, n_in + n_out)
    xq = O.quantize_act(act, x)
    W = J.TensorView("w", quant, [n_in, n_out], to_dev(w, dev))
    y = torch.empty(n_out, dtype=torch.float32, device=dev)
    pp = O.lib().jo_partials_per_row(quant, n_in)
    part = torch.empty((n_out, pp), dtype=torch.int32, device=dev)
    J.matvec_partials(W, to_dev(xq, dev), y, part)
    y2 = torch.empty_like(y)
    J.matvec(W, to_dev(xq, dev), y2)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(part.cpu().numpy(), O.partials(quant, w, n_in, n_out, xq))
    ref = O.matvec_f64(quant, w, n_in, n_out, xq)
    assert rel_err(y.cpu().numpy(), ref) < REL_TOL
    # the partials instantiation and the plain one reduce in the same order
    assert torch.equal(y, y2)


@pytest.mark.parametrize("quant", [J.Q4_K, J.Q6_K, J.Q8_0, J.Q4_0])
def test_vec_dot_f32_input_equals_quantize_then_matvec(dev, quant):
    print(f"vec_dot quant={quant}", flush=True)
    n_in, n_out = 4096, 300
    w = rand_weights(quant, n_out, n_in, 7 + quant)
    x = rand_act(n_in, 8 + quant)
    W = J.TensorView("w", quant, [n_in, n_out], to_dev(w, dev))
    xd = to_dev(x, dev)
    y = torch.empty(n_out, dtype=torch.float32, device=dev)
    {J.Q4_K: J.vec_dot_q4_k_m, J.Q6_K: J.vec_dot_q6_k, J.Q8_0: J.vec_dot_q8_0, J.Q4_0: J.vec_dot_q4_0}[quant](y, W, xd)
    ws = torch.empty(J.row_bytes(J.act_format(quant), n_in), dtype=torch.uint8, device=dev)
    y2 = torch.empty_like(y)
    J.matvec_any(y2, W, xd, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    ref = O.vec_dot(quant, w, n_in, n_out, x)
    assert rel_err(y.cpu().numpy(), ref) < REL_TOL


def test_row_slices_are_bitwise_identical(dev):
    """Partition invariance: any row slice reproduces the full GEMV bit for bit
    (tests/wave1_engine_regression_test.rs:1286-1295)."""
    n_in, n_out = 4096, 12288
    w = rand_weights(J.Q4_K, n_out, n_in, 77)
    W = J.TensorView("w", J.Q4_K, [n_in, n_out], to_dev(w, dev))
    xq = to_dev(O.quantize_act(J.Q8_K, rand_act(n_in, 78)), dev)
    y = torch.empty(n_out, dtype=torch.float32, device=dev)
    J.matvec(W, xq, y)
    for start, cnt in [(0, 16), (5, 2048), (4096, 1), (12000, 288)]:
        ys = torch.empty(cnt, dtype=torch.float32, device=dev)
        J.matvec(W.slice_rows(start, cnt), xq, ys)
        torch.cuda.synchronize()
        assert torch.equal(ys, y[start:start + cnt])


def test_wrong_quant_and_empty_raise(dev):
    W = J.TensorView("blk.0.attn_q.weight", J.Q6_K, [256, 4],
                     torch.zeros(4 * 210, dtype=torch.uint8, device=dev))
    x = torch.zeros(256, dtype=torch.float32, device=dev)
    with pytest.raises(J.K3Error) as ei:
        J.vec_dot_q4_k_m(torch.empty(4, device=dev), W, x)
    assert ei.value.variant == "CapabilityMismatch"
    with pytest.raises(J.K3Error) as ei:
        J.matvec_any(torch.empty(0, device=dev), W, x)
    assert ei.value.variant == "TensorBoundsError"


def test_dequantize_rows_matches_oracle(dev):
    for quant, k in [(J.Q4_K, 512), (J.Q6_K, 768), (J.Q8_0, 96), (J.Q4_0, 64)]:
        print(f"dequant quant={quant}", flush=True)
        w = rand_weights(quant, 6, k, 300 + quant)
        W = J.TensorView("w", quant, [k, 6], to_dev(w, dev))
        out = torch.empty((3, k), dtype=torch.float32, device=dev)
        J.dequantize_rows(W, 2, 3, out)
        torch.cuda.synchronize()
        ref = O.dequantize(quant, w, 6, k)[2:5]
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("n_in,n_out", [(4096, 4096), (768, 2048), (12288, 300), (1280, 7), (4096, 151936)])
def test_q6_k_repacked_layout_is_bitwise_identical(dev, n_in, n_out):
    """The planar Q6_K_R layout computes exactly what the raw GGUF Q6_K path computes."""
    print(f"q6k_r n_in={n_in} n_out={n_out}", flush=True)
    w = rand_weights(J.Q6_K, n_out, n_in, 500 + n_in + n_out, full_range=True)
    W = J.TensorView("output.weight", J.Q6_K, [n_in, n_out], to_dev(w, dev))
    Wr = J.repack(W)
    assert Wr.quant == J.Q6_K_R and Wr.nbytes() == W.nbytes()
    x = rand_act(n_in, 501)
    xq = to_dev(O.quantize_act(J.Q8_K, x), dev)
    y, yr = (torch.empty(n_out, dtype=torch.float32, device=dev) for _ in range(2))
    J.matvec(W, xq, y)
    J.matvec(Wr, xq, yr)
    if n_out <= 4096:
        pp = n_in // 16
        part = torch.empty((n_out, pp), dtype=torch.int32, device=dev)
        J.matvec_partials(Wr, xq, torch.empty_like(yr), part)
    torch.cuda.synchronize()
    assert torch.equal(y, yr)
    if n_out <= 4096:
        np.testing.assert_array_equal(part.cpu().numpy(), O.partials(J.Q6_K, w, n_in, n_out, O.quantize_act(J.Q8_K, x)))
        ref = O.matvec_f64(J.Q6_K, w, n_in, n_out, O.quantize_act(J.Q8_K, x))
        assert rel_err(yr.cpu().numpy(), ref) < REL_TOL


@pytest.mark.parametrize("n_in,n_out", [(4096, 4096), (4096, 12288), (12288, 4096), (768, 2048), (2304, 7),
                                        (256, 1)])
def test_q4_k_repacked_layout_is_bitwise_identical(dev, n_in, n_out):
    """The planar Q4_K_R layout computes exactly what the raw GGUF Q4_K path computes."""
    print(f"q4k_r n_in={n_in} n_out={n_out}", flush=True)
    w = rand_weights(J.Q4_K, n_out, n_in, 700 + n_in + n_out, full_range=True)
    W = J.TensorView("blk.0.ffn_up.weight", J.Q4_K, [n_in, n_out], to_dev(w, dev))
    Wr = J.repack(W)
    assert Wr.quant == J.Q4_K_R and Wr.nbytes() == W.nbytes()
    x = rand_act(n_in, 701)
    xq = to_dev(O.quantize_act(J.Q8_K, x), dev)
    y, yr = (torch.empty(n_out, dtype=torch.float32, device=dev) for _ in range(2))
    J.matvec(W, xq, y)
    J.matvec(Wr, xq, yr)
    if n_out <= 4096:
        pp = n_in // 32
        part = torch.empty((n_out, pp), dtype=torch.int32, device=dev)
        J.matvec_partials(Wr, xq, torch.empty_like(yr), part)
    torch.cuda.synchronize()
    assert torch.equal(y, yr)
    if n_out <= 4096:
        np.testing.assert_array_equal(part.cpu().numpy(), O.partials(J.Q4_K, w, n_in, n_out, O.quantize_act(J.Q8_K, x)))
        ref = O.matvec_f64(J.Q4_K, w, n_in, n_out, O.quantize_act(J.Q8_K, x))
        assert rel_err(yr.cpu().numpy(), ref) < REL_TOL


def tile_q4k(w, n_rows, nb):
    """Q4_K_T pieces from GGUF Q4_K bytes: per (16-row tile, block) q [4][2][16 rows][16] | h [16 rows][16]."""
    t = n_rows // 16
    blk = w.reshape(t, 16, nb, 144)
    q = blk[..., 16:].reshape(t, 16, nb, 4, 2, 16).transpose(0, 2, 3, 4, 1, 5).reshape(t, nb, 2048)
    h = blk[..., :16].transpose(0, 2, 1, 3).reshape(t, nb, 256)
    return np.concatenate([q, h], axis=2).reshape(-1)


def tile_q6k(w, n_rows, nb):
    """Q6_K_T pieces: ql [4 units][2 halves][16 rows][16] | qh [4][16 rows][16] | sc [16 rows][4][4] | d [16 rows]."""
    t = n_rows // 16
    blk = w.reshape(t, 16, nb, 210)
    ql = blk[..., :128].reshape(t, 16, nb, 2, 2, 2, 16).transpose(0, 2, 3, 5, 4, 1, 6).reshape(t, nb, 2048)
    qh = blk[..., 128:192].reshape(t, 16, nb, 2, 2, 16).transpose(0, 2, 3, 4, 1, 5).reshape(t, nb, 1024)
    sc = blk[..., 192:208].reshape(t, 16, nb, 2, 4, 2).transpose(0, 2, 1, 3, 5, 4).reshape(t, nb, 256)
    d = blk[..., 208:].transpose(0, 2, 1, 3).reshape(t, nb, 32)
    return np.concatenate([ql, qh, sc, d], axis=2).reshape(-1)


@pytest.mark.parametrize("quant", [J.Q4_K, J.Q6_K])
def test_repack_experts_tiled_layout(dev, quant):
    """jero_hip_repack_experts writes the 16-row tiled pieces, byte for byte."""
    print(f"repack experts quant={quant}", flush=True)
    n_in, rows, experts = 768, 48, 3
    w = rand_weights(quant, rows * experts, n_in, 900 + quant, full_range=True)
    W = J.TensorView("blk.0.ffn_gate_exps.weight", quant, [n_in, rows, experts], to_dev(w, dev))
    Wt = J.repack(W)
    torch.cuda.synchronize()
    assert Wt.quant == (J.Q4_K_T if quant == J.Q4_K else J.Q6_K_T) and Wt.nbytes() == W.nbytes()
    tile = tile_q4k if quant == J.Q4_K else tile_q6k
    np.testing.assert_array_equal(Wt.data.cpu().numpy(), tile(np.frombuffer(w.tobytes(), np.uint8), rows * experts,
                                                              n_in // 256))
    with pytest.raises(J.K3Error) as ei:  # rows per expert not a multiple of 16
        J.repack(J.TensorView("e", quant, [n_in, 24, 2], W.data), experts=True)
    assert ei.value.variant == "CapabilityMismatch"


def test_repack_rejects_other_formats(dev):
    W = J.TensorView("w", J.Q8_0, [256, 4], torch.zeros(4 * 8 * 34, dtype=torch.uint8, device=dev))
    with pytest.raises(J.K3Error) as ei:
        J.repack(W)
    assert ei.value.variant == "CapabilityMismatch"


@pytest.mark.parametrize("quant", [0, 1, 30])
@pytest.mark.parametrize("n_in,n_out", [(2048, 128), (4096, 4096), (1000, 77), (130, 3), (65536, 40)])
def test_float_weights_matvec(dev, quant, n_in, n_out):
    """matvec_f32 / vec_dot_f16 / vec_dot_bf16 (src/gemma.rs:72-74,140-189): the Qwen3-MoE router
    shape (F32 ffn_gate_inp 2048 x 128), a square matrix, rows that are not 16-byte aligned, tiny
    rows and a 65536-long row, against the oracle within 1e-5."""
    from qdata import rand_float_weights
    print(f"float matvec quant={quant} {n_in}x{n_out}", flush=True)
    w = rand_float_weights(quant, n_out, n_in, 17)
    x = rand_act(n_in, 18)
    W = J.TensorView("blk.0.ffn_gate_inp.weight", quant, [n_in, n_out], torch.from_numpy(w).to(dev))
    y = torch.empty(n_out, dtype=torch.float32, device=dev)
    J.matvec_any(y, W, torch.from_numpy(x).to(dev))
    y2 = torch.empty_like(y)
    J.vec_dot_noalloc(y2, W, torch.from_numpy(x).to(dev))
    torch.cuda.synchronize()
    ref = O.vec_dot(quant, w, n_in, n_out, x, threads=8)
    got = y.cpu().numpy()
    scale = max(np.sqrt(np.mean(ref.astype(np.float64) ** 2)), 1e-30)
    err = np.max(np.abs(got - ref) / np.maximum(np.abs(ref), scale))
    assert err <= 1e-5, err
    assert torch.equal(y, y2)


def test_float_weights_kat_and_gemm(dev):
    """dot_product_f32([2], [3]) = 6 (src/lib.rs:380-387) on the device, F32 rows through
    jero_hip_gemm for several token rows (the router of a batch), each row equal to its matvec,
    and F32 weights rejected where integer partial sums are asked for."""
    from qdata import rand_float_weights
    W = J.TensorView("w", J.F32, [1, 1], torch.tensor([2.0], device=dev).view(torch.uint8))
    y = torch.empty(1, dtype=torch.float32, device=dev)
    J.matvec_f32(y, W, torch.tensor([3.0], device=dev))
    assert y.item() == 6.0
    w = rand_float_weights(J.F32, 128, 2048, 19)
    x = rand_act(2048, 20, m=5)
    Wt = J.TensorView("router", J.F32, [2048, 128], torch.from_numpy(w).to(dev))
    xt = torch.from_numpy(x).to(dev)
    Y = torch.empty((5, 128), dtype=torch.float32, device=dev)
    J.gemm(Wt, xt, 5, Y)
    for r in range(5):
        yr = torch.empty(128, dtype=torch.float32, device=dev)
        J.matvec_any(yr, Wt, xt[r].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(Y[r], yr), r
    with pytest.raises(J.K3Error) as ei:
        J.matvec_partials(Wt, xt[0], torch.empty(128, device=dev), torch.empty(128, dtype=torch.int32, device=dev))
    assert ei.value.variant == "CapabilityMismatch"


@pytest.mark.parametrize("quant,n_in,n_out", [(8, 28672, 512), (2, 20480, 300), (12, 65536, 200), (14, 40960, 130),
                                              (112, 49152, 96), (114, 36864, 64)])
def test_long_rows(dev, quant, n_in, n_out):
    """Rows longer than the register-resident activation (the reference's vec_dot_* has no
    row-length limit, src/gemma.rs:66-138): Q8_0 at 28672 (a 70B-class ffn_down), Q4_0, Q4_K,
    Q6_K and the planar layouts, with the int32 partial sums bit-exact on the first case."""
    print(f"long rows quant={quant} {n_in}x{n_out}", flush=True)
    base = {112: J.Q4_K, 114: J.Q6_K}.get(quant, quant)
    w = rand_weights(base, n_out, n_in, 71)
    x = rand_act(n_in, 72)
    xq = J.quantize_act(J.act_format(base), torch.from_numpy(x).to(dev))
    W = J.TensorView("long", base, [n_in, n_out], torch.from_numpy(w).to(dev))
    if quant != base:
        W = J.repack(W)
        assert W.quant == quant
    y = torch.empty(n_out, dtype=torch.float32, device=dev)
    J.matvec(W, xq, y)
    torch.cuda.synchronize()
    ref = O.matvec(base, w, n_in, n_out, xq.cpu().numpy(), threads=8)
    scale = max(np.sqrt(np.mean(ref.astype(np.float64) ** 2)), 1e-30)
    err = np.max(np.abs(y.cpu().numpy() - ref) / np.maximum(np.abs(ref), scale))
    assert err <= 1e-5, err
    if quant == 8:
        pp = O.partials(base, w, n_in, n_out, xq.cpu().numpy())
        part = torch.empty(pp.shape, dtype=torch.int32, device=dev)
        y2 = torch.empty_like(y)
        J.matvec_partials(W, xq, y2, part)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(part.cpu().numpy(), pp)
        assert torch.equal(y, y2)


@pytest.mark.parametrize("nbytes", [16, 8192, 8192 + 48, 9458240])
def test_read_probe_reads_and_leaves_sink(dev, nbytes):
    """The bandwidth probe runs over any 16-byte multiple (partial last workgroup included) and
    writes nothing for data whose wave XOR is not its sentinel."""
    buf = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.full((256,), 7, dtype=torch.int32, device=dev)
    J.read_probe(buf, sink)
    torch.cuda.synchronize()
    assert bool((sink == 7).all())
