"""Pins the CPU oracle (oracle/liboracle.so) before it is trusted as the checker.

Each function of the oracle is held here to something other than its own formula:
the reference's known-answer tests, the reference's golden llama logits, an independent
numpy restatement (oracle/ref_numpy.py), f64/brute-force evaluation and closed-form
invariants.  Reference citations are given per test.
"""
import math
import struct

import numpy as np
import pytest

import pyoracle as O
import ref_numpy as R
from qdata import rand_act, rand_weights

WEIGHT_FORMATS = [O.Q8_0, O.Q4_0, O.Q4_K, O.Q6_K]


# ---------------------------------------------------------------- f16 conversion

def test_f16_to_f32_all_halves():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([O.lib().jo_f16_to_f32(int(b)) for b in bits[::7]], np.float32)
    r = ref[::7]
    same = (got == r) | (np.isnan(got) & np.isnan(r))
    assert same.all()


def test_f32_to_f16_round_to_nearest_even():
    rng = np.random.default_rng(3)
    vals = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.integers(-9, 5, 4000),
                           np.array([65504.0, 65520.0, 65519.99, 6e-8, 3e-8, 2.98e-8, 0.0, -0.0])]).astype(np.float32)
    # exact ties: half-way between two halves
    ties = (np.arange(1, 200, dtype=np.float32) * 2 + 1) * np.float32(2.0 ** -11)
    vals = np.concatenate([vals, ties, -ties])
    got = np.array([O.lib().jo_f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    assert (got == ref).all()


# ---------------------------------------------------------------- formats: reference KATs

def test_q8_0_row_kat():
    """src/gemma.rs:1627-1645: Q8_0 row of q=2 with f16 scale 1.0 (0x3C00) dequantizes to 2.0."""
    row = bytes([0x00, 0x3C]) + bytes([2] * 32) + bytes([0x00, 0x3C]) + bytes([2] * 32)
    out = O.dequantize(O.Q8_0, np.frombuffer(row, np.uint8), 1, 64)
    assert np.all(np.abs(out - 2.0) < 1e-5)


def test_q4_0_row_kat():
    """src/gemma.rs:1647-1662: Q4_0 scale 0.5 (0x3800), nibbles 0xAA -> (10 - 8) * 0.5 = 1.0."""
    row = bytes([0x00, 0x38]) + bytes([0xAA] * 16)
    out = O.dequantize(O.Q4_0, np.frombuffer(row, np.uint8), 1, 32)
    assert np.all(np.abs(out - 1.0) < 1e-5)


def test_block_byte_sizes():
    """Q4_K [256, 2] is 288 B (src/weights.rs:1208); Q6_K 210 B; Q8_0 34 B; Q8_K 292 B."""
    assert O.row_bytes(O.Q4_K, 256) * 2 == 288
    assert O.row_bytes(O.Q6_K, 256) == 210
    assert O.row_bytes(O.Q8_0, 32) == 34
    assert O.row_bytes(O.Q8_K, 256) == 292
    assert O.row_bytes(O.ACT_Q8, 32) == 36
    assert O.row_bytes(O.Q4_K, 100) == -1


def test_q4_k_header_and_q6_k_scale_positions():
    """Q4_K d/dmin at bytes 0-3 and Q6_K d at bytes 208-209
    (tests/wave1_engine_regression_test.rs:250-282): zeroing exactly those bytes zeroes the row
    (Q4_K) / the whole block (Q6_K)."""
    w = rand_weights(O.Q4_K, 1, 256, 1)
    w[0:4] = 0
    assert np.all(O.dequantize(O.Q4_K, w, 1, 256) == 0)
    w = rand_weights(O.Q4_K, 1, 256, 1)
    w[2:4] = 0  # dmin = 0: values are d*sc*q >= 0
    assert np.all(O.dequantize(O.Q4_K, w, 1, 256) >= 0)
    w = rand_weights(O.Q6_K, 1, 256, 2)
    w[208:210] = 0
    assert np.all(O.dequantize(O.Q6_K, w, 1, 256) == 0)


@pytest.mark.parametrize("quant", WEIGHT_FORMATS)
def test_dequant_matches_numpy_restatement(quant):
    k, rows = 512, 9
    w = rand_weights(quant, rows, k, 10 + quant, full_range=True)
    a = O.dequantize(quant, w, rows, k)
    b = R.dequantize(quant, w, rows, k)
    np.testing.assert_array_equal(a, b)


def test_q4_k_single_element_closed_form():
    """One hand-built Q4_K block: sub-block 5 (j >= 4 path of the 6-bit packing)."""
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    # sub-block 5: sc = (s[9] & 15) | ((s[1] >> 6) << 4), m = (s[9] >> 4) | ((s[5] >> 6) << 4)
    blk[4 + 9] = 0x3A     # sc low 4 = 10, m low 4 = 3
    blk[4 + 1] = 0x80     # sc high 2 bits = 2  -> sc = 10 | 32 = 42
    blk[4 + 5] = 0x40     # m high 2 bits = 1   -> m = 3 | 16 = 19
    # element 64*2 + 32 + 7 = 167 is the high nibble of qs[32*2 + 7]
    blk[16 + 64 + 7] = 0xB0  # high nibble 11
    y = O.dequantize(O.Q4_K, blk, 1, 256)[0]
    assert y[167] == pytest.approx(0.5 * 42 * 11 - 0.25 * 19)
    assert y[160] == pytest.approx(-0.25 * 19)  # same sub-block, q = 0


def test_q6_k_single_element_closed_form():
    blk = np.zeros(210, np.uint8)
    blk[208:210] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
    # element 128 + 64 + 5 (half 1, third quarter): ql[64 + 5] >> 4, qh[32 + 5] bits 4-5, scale 8 + 4 + 0
    blk[64 + 5] = 0x90        # high nibble 9
    blk[128 + 32 + 5] = 0x20  # bits 4-5 = 2 -> q = 9 | 32 = 41 -> 41 - 32 = 9
    blk[192 + 12] = np.uint8(np.int8(-3).view(np.uint8))
    y = O.dequantize(O.Q6_K, blk, 1, 256)[0]
    assert y[197] == pytest.approx(0.125 * -3 * 9)


# ---------------------------------------------------------------- activation quantizers

@pytest.mark.parametrize("k", [32, 256, 4096])
def test_act_q8_matches_numpy(k):
    x = rand_act(k, 5, m=3)
    x[0, :32] = 0.0  # an all-zero block
    a = O.quantize_act(O.ACT_Q8, x)
    b = np.concatenate([R.quantize_act_q8(r) for r in x])
    np.testing.assert_array_equal(a, b)


@pytest.mark.parametrize("k", [256, 4096, 12288])
def test_q8_k_matches_numpy(k):
    x = rand_act(k, 6, m=2)
    x[1, :256] = 0.0
    a = O.quantize_act(O.Q8_K, x)
    b = np.concatenate([R.quantize_q8_k(r) for r in x])
    np.testing.assert_array_equal(a, b)


def test_q8_k_invariants():
    x = rand_act(4096, 7)
    q = O.quantize_act(O.Q8_K, x).reshape(16, 292)
    qs = q[:, 4:260].view(np.int8).astype(np.int32)
    bs = q[:, 260:].copy().view(np.int16).astype(np.int32)
    d = q[:, :4].copy().view(np.float32).reshape(-1)
    assert np.all(bs == qs.reshape(16, 16, 16).sum(axis=2))
    assert np.all(np.abs(qs) <= 127)
    assert np.all(np.abs(qs).max(axis=1) == 127)
    err = np.abs(qs * d[:, None] - x.reshape(16, 256))
    assert np.all(err <= np.abs(d)[:, None] * 0.5 + 1e-6)


def test_q8_k_tie_takes_first_index_sign():
    """Equal magnitudes of opposite sign: the first one sets the sign of d (ggml strict >)."""
    # iscale = -127 / max maps the chosen element to -127, so d has the opposite sign of it
    x = np.zeros(256, np.float32)
    x[3], x[10] = -2.0, 2.0
    q = O.quantize_act(O.Q8_K, x)
    d = q[:4].copy().view(np.float32)[0]
    qs = q[4:260].view(np.int8)
    assert d > 0 and qs[3] == -127 and qs[10] == 127
    x[3], x[10] = 2.0, -2.0
    q = O.quantize_act(O.Q8_K, x)
    d = q[:4].copy().view(np.float32)[0]
    qs = q[4:260].view(np.int8)
    assert d < 0 and qs[3] == -127 and qs[10] == 127


def test_act_q8_round_half_even():
    """ACT_Q8 rounds ties to even: 127 * (k + 0.5) / 127 lands exactly half-way."""
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1], x[2], x[3] = 2.5, 3.5, -2.5
    q = O.quantize_act(O.ACT_Q8, x)
    assert q[:4].copy().view(np.float32)[0] == np.float32(1.0)
    assert list(q[4:8].view(np.int8)) == [127, 2, 4, -2]


# ---------------------------------------------------------------- dot products

@pytest.mark.parametrize("quant", WEIGHT_FORMATS)
def test_partials_match_integer_brute_force(quant):
    k, rows = 1024, 7
    w = rand_weights(quant, rows, k, 20 + quant, full_range=True)
    act = O.act_format(quant)
    xq = O.quantize_act(act, rand_act(k, 21))
    got = O.partials(quant, w, k, rows, xq)
    ref = R.partials(quant, w, rows, k, act, xq)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("quant", WEIGHT_FORMATS)
def test_matvec_matches_dequant_f64(quant):
    k, rows = 2048, 33
    w = rand_weights(quant, rows, k, 30 + quant)
    act = O.act_format(quant)
    xq = O.quantize_act(act, rand_act(k, 31))
    y = O.matvec(quant, w, k, rows, xq, threads=4)
    # independent: numpy dequantization of both operands, f64 dot
    wd = R.dequantize(quant, w, rows, k).astype(np.float64)
    xd = R.dequantize(act, xq, 1, k)[0].astype(np.float64)
    ref = wd @ xd
    scale = max(np.sqrt(np.mean(ref ** 2)), 1e-30)
    assert np.max(np.abs(y - ref) / np.maximum(np.abs(ref), scale)) < 1e-6


def test_matvec_partition_invariance():
    """Row results do not depend on the thread partition (src/gemma.rs:114-134,
    tests/wave1_engine_regression_test.rs:1286-1295)."""
    k, rows = 1024, 300
    w = rand_weights(O.Q4_K, rows, k, 40)
    xq = O.quantize_act(O.Q8_K, rand_act(k, 41))
    ys = [O.matvec(O.Q4_K, w, k, rows, xq, threads=t) for t in (1, 3, 8)]
    for y in ys[1:]:
        np.testing.assert_array_equal(ys[0], y)


def test_zero_scale_rows_are_exact_zero():
    """Rows with d = 0 give exactly 0.0 (the golden logits 0..4 are exactly 0.0)."""
    k = 256
    w = rand_weights(O.Q8_0, 2, k, 50).reshape(2, -1)
    w[0].reshape(-1, 34)[:, 0:2] = 0
    xq = O.quantize_act(O.ACT_Q8, rand_act(k, 51))
    y = O.matvec(O.Q8_0, w.reshape(-1), k, 2, xq)
    assert y[0] == 0.0 and y[1] != 0.0


def test_gemm_i8_brute_force():
    rng = np.random.default_rng(60)
    x = rng.integers(-128, 128, (17, 96)).astype(np.int8)
    w = rng.integers(-128, 128, (23, 96)).astype(np.int8)
    np.testing.assert_array_equal(O.gemm_i8(x, w), x.astype(np.int32) @ w.astype(np.int32).T)


def test_gemm_rows_equal_gemv():
    k, n, m = 512, 40, 5
    w = rand_weights(O.Q6_K, n, k, 61)
    x = rand_act(k, 62, m=m)
    xq = O.quantize_act(O.Q8_K, x)
    y = O.gemm(O.Q6_K, w, k, n, xq, m)
    rb = O.row_bytes(O.Q8_K, k)
    for i in range(m):
        np.testing.assert_array_equal(y[i], O.matvec(O.Q6_K, w, k, n, xq[i * rb:(i + 1) * rb]))


# ---------------------------------------------------------------- elementwise, attention

def test_dot_product_kat():
    """kernels_rvv_wired KAT [2] . [3] = 6 (src/lib.rs:380-387), through an F32-free path:
    a Q8_0 row with d=1 and q=2 against activations 3 quantized to ACT_Q8."""
    row = np.frombuffer(bytes([0x00, 0x3C]) + bytes([2] + [0] * 31), np.uint8)
    x = np.zeros(32, np.float32)
    x[0] = 3.0
    xq = O.quantize_act(O.ACT_Q8, x)
    assert O.matvec(O.Q8_0, row, 32, 1, xq)[0] == pytest.approx(6.0, rel=1e-6)


def test_rmsnorm_closed_form():
    x = np.array([3.0, 4.0], np.float32)
    w = np.array([1.0, 2.0], np.float32)
    y = O.rmsnorm(x, w, 0.0)
    s = 1.0 / math.sqrt((9 + 16) / 2)
    np.testing.assert_allclose(y, [3 * s, 8 * s], rtol=1e-6)


def test_rope_interleaved_pairs():
    """Interleaved pairs (2i, 2i+1) rotated by pos / theta^(2i/hd)
    (tests/wave1_engine_regression_test.rs:698-712); pos 0 is the identity; norms kept."""
    rng = np.random.default_rng(70)
    x = rng.standard_normal(2 * 8).astype(np.float32)
    np.testing.assert_array_equal(O.rope(x, 8, 0, 10000.0), x)
    y = O.rope(x, 8, 5, 10000.0)
    xp, yp = x.reshape(-1, 2), y.reshape(-1, 2)
    np.testing.assert_allclose(np.linalg.norm(yp, axis=1), np.linalg.norm(xp, axis=1), rtol=1e-5)
    # pair 1 of head 0: angle = 5 / 10000^(2/8)
    a = 5.0 / 10000.0 ** 0.25
    c, s = math.cos(a), math.sin(a)
    assert y[2] == pytest.approx(x[2] * c - x[3] * s, rel=1e-5)
    assert y[3] == pytest.approx(x[2] * s + x[3] * c, rel=1e-5)


def test_swiglu_closed_form():
    g = np.array([0.0, 1.0, -2.0], np.float32)
    u = np.array([5.0, 2.0, 3.0], np.float32)
    ref = [0.0, 2.0 / (1 + math.exp(-1.0)), 3.0 * -2.0 / (1 + math.exp(2.0))]
    np.testing.assert_allclose(O.swiglu(g, u), ref, rtol=1e-6)


def test_attention_brute_force_and_special_cases():
    rng = np.random.default_rng(80)
    nq, nkv, hd, T = 8, 2, 16, 37
    q = rng.standard_normal(nq * hd).astype(np.float32)
    k = rng.standard_normal((T, nkv * hd)).astype(np.float32)
    v = rng.standard_normal((T, nkv * hd)).astype(np.float32)
    out = O.gqa_attention(q, k, v, nq, nkv, hd, T, 0.25)
    ref = np.zeros(nq * hd)
    for h in range(nq):
        kh = h // (nq // nkv)
        s = k[:, kh * hd:(kh + 1) * hd].astype(np.float64) @ q[h * hd:(h + 1) * hd] * 0.25
        p = np.exp(s - s.max())
        p /= p.sum()
        ref[h * hd:(h + 1) * hd] = p @ v[:, kh * hd:(kh + 1) * hd]
    np.testing.assert_allclose(out, ref, rtol=1e-5, atol=1e-6)
    # one position: output equals that V row; identical keys: output is the mean of V
    out1 = O.gqa_attention(q, k[:1], v[:1], nq, nkv, hd, 1, 0.25)
    np.testing.assert_allclose(out1.reshape(nq, hd), np.repeat(v[0].reshape(nkv, hd), nq // nkv, axis=0), rtol=1e-6)
    ksame = np.repeat(k[:1], T, axis=0)
    outm = O.gqa_attention(q, ksame, v, nq, nkv, hd, T, 0.25)
    np.testing.assert_allclose(outm.reshape(nq, hd),
                               np.repeat(v.mean(axis=0).reshape(nkv, hd), nq // nkv, axis=0), rtol=1e-5, atol=1e-6)


# ---------------------------------------------------------------- argmax, routing KATs

def test_argmax_kats():
    """src/engine.rs:2677-2727."""
    nan, ninf = float("nan"), float("-inf")
    assert O.argmax(np.array([], np.float32)) is None
    assert O.argmax(np.full(1024, nan, np.float32)) is None
    assert O.argmax(np.array([nan, 3.5, nan, 2.0], np.float32)) == 1
    assert O.argmax(np.array([ninf, ninf], np.float32)) == 0
    for n in (32768, 65537, 256000):
        x = np.array([-100.0 - (i % 97) for i in range(n)], np.float32)
        x[n - 17] = -0.25
        x[0] = ninf
        assert O.argmax(x) == n - 17
        t = np.full(n, 1.25, np.float32)
        t[0] = nan
        t[103] = 42.5
        t[n // 2 + 11] = 42.5
        t[n - 1] = nan
        assert O.argmax(t) == 103


def test_select_top_k_kats():
    """src/gemma.rs:1722-1740."""
    tied = np.array([0.1, 3.0, 0.5, 1.0, 3.0, 2.0], np.float32)
    top2 = O.select_top_k(tied, 2, True)
    assert [i for i, _ in top2] == [1, 4]
    assert abs(top2[0][1] - 0.5) < 1e-6 and abs(top2[1][1] - 0.5) < 1e-6
    raw = O.select_top_k(tied, 2, False)
    assert raw[0][1] + raw[1][1] < 0.99
    assert O.select_top_k(np.array([], np.float32), 2, True) == []
    assert O.select_top_k(tied, 0, True) == []


def test_select_top_k_total_order_of_signed_zero():
    """select_top_k_experts sorts with f32::total_cmp (src/gemma.rs:417), which ranks +0.0 above
    -0.0: [-0.0, +0.0] at k = 1 selects expert 1, its mirror expert 0; equal zeros keep index
    order.  A comparison with `<` would tie them and take the lower index both times."""
    nz, pz = np.float32(-0.0), np.float32(0.0)
    assert [i for i, _ in O.select_top_k(np.array([nz, pz], np.float32), 1, True)] == [1]
    assert [i for i, _ in O.select_top_k(np.array([pz, nz], np.float32), 1, True)] == [0]
    mixed = np.array([nz, nz, pz, -1.0, pz, nz], np.float32)
    assert [i for i, _ in O.select_top_k(mixed, 5, True)] == [2, 4, 0, 1, 5]


def test_select_top_k_softmax_values_and_nonfinite():
    logits = np.array([1.0, float("nan"), 2.0, float("inf"), 0.5], np.float32)
    sel = O.select_top_k(logits, 3, False)
    fin = np.array([1.0, 2.0, 0.5])
    p = np.exp(fin - fin.max()) / np.exp(fin - fin.max()).sum()
    assert [i for i, _ in sel] == [2, 0, 4]
    np.testing.assert_allclose([w for _, w in sel], [p[1], p[0], p[2]], rtol=1e-6)


def test_moe_ffn_matches_dense_composition():
    """dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951): y = sum_k w_k expert_k(x)."""
    H, F, E, K = 256, 512, 6, 2
    gate = rand_weights(O.Q4_K, E * F, H, 90)
    up = rand_weights(O.Q4_K, E * F, H, 91)
    down = rand_weights(O.Q6_K, E * H, F, 92)
    x = rand_act(H, 93, m=2)
    logits = rand_act(E, 94, m=2)
    y, si, sw = O.moe_ffn(logits, K, gate, up, down, O.Q4_K, O.Q4_K, O.Q6_K, H, F, x, threads=2)
    for t in range(2):
        sel = O.select_top_k(logits[t], K, True)
        ref = np.zeros(H, np.float32)
        for e, wgt in sel:
            g = O.vec_dot(O.Q4_K, gate[e * F * 144:(e + 1) * F * 144], H, F, x[t])
            u = O.vec_dot(O.Q4_K, up[e * F * 144:(e + 1) * F * 144], H, F, x[t])
            a = O.swiglu(g, u)
            rb = O.row_bytes(O.Q6_K, F)
            ref += np.float32(wgt) * O.vec_dot(O.Q6_K, down[e * H * rb:(e + 1) * H * rb], F, H, a)
        np.testing.assert_allclose(y[t], ref, rtol=1e-6, atol=1e-7)
        assert list(si[t]) == [e for e, _ in sel]


def test_float_weight_dot_kat_and_brute_force():
    """dot_product_f32 [2] . [3] = 6 (src/lib.rs:380-387) through the F32 row path; F16/BF16 rows
    widened to f32 and dotted in f64 equal a numpy f64 product of the same values."""
    from qdata import BF16, F16, F32, float_values, rand_float_weights
    w = np.array([2.0], np.float32).view(np.uint8)
    assert O.vec_dot(F32, w, 1, 1, np.array([3.0], np.float32))[0] == 6.0
    x = rand_act(333, 5)
    for q in (F32, F16, BF16):
        w = rand_float_weights(q, 7, 333, 6)
        ref = float_values(q, w, 7, 333).astype(np.float64) @ x.astype(np.float64)
        np.testing.assert_allclose(O.vec_dot(q, w, 333, 7, x), ref, rtol=1e-6, atol=1e-9)
    # BF16 is the upper half of the f32 bits: 1.0 = 0x3F80
    assert O.dequantize(BF16, np.array([0x80, 0x3F], np.uint8), 1, 1)[0, 0] == 1.0


def test_requant_kats():
    """forward.rs's requant (:345-350) on hand-computed cases: the rounding term, floor shifts of
    negatives, the [-127, 127] clamp (not -128), and the wrapping i32 add at the top of the range."""
    cases = [((5, 1), 3), ((-5, 1), -2), ((4, 1), 2), ((-4, 1), -2), ((-6, 2), -1), ((1000, 2), 127),
             ((-1000, 2), -127), ((255, 1), 127), ((253, 1), 127), ((-255, 1), -127), ((-256, 1), -127),
             ((100, 31), 0), ((-100, 31), 0), ((1 << 30, 31), -1), ((2147483647, 1), -127), ((0, 7), 0),
             ((63, 7), 0), ((64, 7), 1), ((-64, 7), 0), ((-65, 7), -1)]
    for (v, s), want in cases:
        assert int(O.requant(v, s)) == want, (v, s)


def test_pack_tiles_layout():
    """Packed bytes follow the documented offset formula, element by element; padding rows are 0."""
    rng = np.random.default_rng(3)
    rows, k = 13, 64
    x = rng.integers(-128, 128, size=(rows, k)).astype(np.int8)
    p = O.pack_tiles(x, rows, k)
    assert p.size == 16 * k
    for r in range(16):
        for c in range(k):
            off = ((r // 8 * (k // 32) + c // 32) * 8 + r % 8) * 32 + c % 32
            assert p[off] == (x[r, c] if r < rows else 0)


def test_deterministic_projection_fallback_equals_selection_matrices():
    """project_or_deterministic_slice (src/gemma.rs:841-860) with the Qwen3 call sites' scales: a
    model whose projections are absent gives the logits of the same model carrying F32 selection
    matrices S[i][i % in_len] = scale (an exact product: one power-of-two term per row); a wrong
    scale on one of them (v at 0.25 instead of 0.125) does not."""
    import model_spec as MS
    spec = dict(hidden=256, ffn=512, n_layers=2, vocab=40, nq=4, nkv=2, hd=64, eps=1e-6, theta=1e6)
    H, F, Q, KV = 256, 512, 256, 128
    t = MS.oracle_tensors(MS.build(spec, seed=3))
    absent = {"blk.0.attn_v.weight": (H, KV, 0.125), "blk.0.ffn_up.weight": (H, F, 0.25),
              "blk.0.attn_q.weight": (H, Q, 0.5), "blk.1.attn_k.weight": (H, KV, 0.25),
              "blk.1.attn_output.weight": (Q, H, 0.25), "blk.1.ffn_gate.weight": (H, F, 0.5),
              "blk.1.ffn_down.weight": (F, H, 0.125)}

    def selection(n_in, n_out, s):
        S = np.zeros((n_out, n_in), np.float32)
        S[np.arange(n_out), np.arange(n_out) % n_in] = s
        return (O.F32, S.reshape(-1))

    a = {k: v for k, v in t.items() if k not in absent}
    b = dict(t, **{k: selection(*v) for k, v in absent.items()})
    c = dict(b)
    c["blk.0.attn_v.weight"] = selection(H, KV, 0.25)

    def run(tensors):
        om = O.DecodeModel(spec, tensors, 16)
        kv = om.new_kv()
        out, tok = [], 3
        for pos in range(3):
            lg = om.step(kv, tok, pos, threads=2)
            out.append(lg)
            tok = int(np.argmax(lg))
        return np.stack(out)

    la, lb, lc = run(a), run(b), run(c)
    assert np.array_equal(la, lb)
    assert not np.allclose(la, lc, rtol=1e-3, atol=1e-3)


def test_f16_ring_mode_rounds_the_new_row_before_attending():
    """kv_f16: the step writes its new K/V rows as f16 values (the device's f16 ring), and the
    step's attention sees them rounded: its logits differ from the f32 ring's, while a ring that
    already holds f16-exact rows gives the same logits either way at the next position."""
    import model_spec as MS
    spec = dict(hidden=256, ffn=512, n_layers=2, vocab=40, nq=4, nkv=2, hd=64, eps=1e-6, theta=1e6)
    om = O.DecodeModel(spec, MS.oracle_tensors(MS.build(spec, seed=4)), 8)
    kv32, kv16 = om.new_kv(), om.new_kv()
    l32 = om.step(kv32, 3, 0, threads=2)
    om.model.kv_f16 = 1
    l16 = om.step(kv16, 3, 0, threads=2)
    row = kv16[:, :, 0]
    assert np.array_equal(row, row.astype(np.float16).astype(np.float32))
    assert not np.array_equal(kv32[:, :, 0], kv32[:, :, 0].astype(np.float16).astype(np.float32))
    # layer 0's rows come from the same input; later layers see the rounded attention
    assert np.array_equal(kv16[0, :, 0], kv32[0, :, 0].astype(np.float16).astype(np.float32))
    assert not np.array_equal(l16, l32)


# ---------------------------------------------------------------- weight helpers, embedding, LM head

def _q8_0_blocks(d, q):
    """Q8_0 bytes of blocks with f16 scale d and int8 quants q [nb][32]."""
    q = np.asarray(q, np.int8).reshape(-1, 32)
    out = np.zeros((q.shape[0], 34), np.uint8)
    out[:, 0:2] = np.asarray([d] * q.shape[0], np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def test_read_f32_weight_or_default_cases():
    """read_f32_weight_or_default (src/qwen_deepseek.rs:491-519), case by case."""
    ones = np.ones(8, np.float32)
    assert np.array_equal(O.read_f32_weight_or_default(O.F32, None, 0, 8), ones)  # absent
    v = np.array([0.5, np.nan, -2.0, np.inf, -np.inf, 3.0, 0.0, -0.0], np.float32)
    got = O.read_f32_weight_or_default(O.F32, v, 8, 8)
    assert np.array_equal(got, np.array([0.5, 1, -2, 1, 1, 3, 0, 0], np.float32))  # non-finite -> 1.0
    assert np.signbit(got[7])  # -0.0 is finite and kept
    short = O.read_f32_weight_or_default(O.F32, v[:3], 3, 8)  # past the tensor's end -> 1.0
    assert np.array_equal(short, np.array([0.5, 1, -2, 1, 1, 1, 1, 1], np.float32))
    assert np.array_equal(O.read_f32_weight_or_default(O.F32, v, 8, 2), np.array([0.5, 1], np.float32))
    h = np.array([0.25, np.nan, -1.5, 65504.0], np.float16)  # F16: dequantized, NaN kept
    got = O.read_f32_weight_or_default(O.F16, h.view(np.uint8), 4, 4)
    assert np.array_equal(got[[0, 2, 3]], np.array([0.25, -1.5, 65504.0], np.float32)) and np.isnan(got[1])
    assert np.array_equal(O.read_f32_weight_or_default(O.F16, h.view(np.uint8), 4, 6), np.ones(6, np.float32))
    q = np.arange(-32, 32)  # Q8_0, d = 0.5: w = q / 2 exactly; row 0 = the first len elements
    blk = _q8_0_blocks(0.5, q)
    assert np.array_equal(O.read_f32_weight_or_default(O.Q8_0, blk, 64, 64), (q / 2).astype(np.float32))
    assert np.array_equal(O.read_f32_weight_or_default(O.Q8_0, blk, 64, 32), (q[:32] / 2).astype(np.float32))
    w = rand_weights(O.Q4_K, 1, 256, 5)  # 128 of a Q4_K block's 256 elements: not whole blocks -> 1.0
    assert np.array_equal(O.read_f32_weight_or_default(O.Q4_K, w, 256, 128), np.ones(128, np.float32))


def test_logits_len_rule():
    """infer_logits_buffer_len (src/engine.rs:1781-1792)."""
    assert O.logits_len(192, 256) == 256          # 64 rows of padding, rows % 64 == 0
    assert O.logits_len(1024, 2048) == 2048       # 1024 rows of padding: the limit
    assert O.logits_len(1000, 2048) == 1000       # 1048 rows: too many
    assert O.logits_len(200, 232) == 200          # rows % 64 != 0
    assert O.logits_len(200, 200) == 200 and O.logits_len(200, 150) == 200
    assert O.logits_len(200, None) == 200


HEAD_SPEC = dict(hidden=128, ffn=256, n_layers=1, vocab=300, nq=2, nkv=1, hd=64, eps=1e-5, theta=1e4)


def _head_model(tensors_extra, drop=()):
    """A Q8_0 model of HEAD_SPEC with the head / embedding replaced or dropped."""
    from qdata import rand_weights as rw
    H, V = HEAD_SPEC["hidden"], HEAD_SPEC["vocab"]
    t = {"token_embd.weight": (O.Q8_0, rw(O.Q8_0, V, H, 1), H, V),
         "output.weight": (O.Q8_0, rw(O.Q8_0, V, H, 2), H, V),
         "output_norm.weight": (O.F32, (1 + 0.1 * rand_act(H, 3)).astype(np.float32), H, 1)}
    t.update(tensors_extra)
    for k in drop:
        t.pop(k, None)
    return O.DecodeModel(HEAD_SPEC, t, 8), t


def test_lm_head_padded_rows_and_slices():
    """project_lm_head (src/qwen_deepseek.rs:584-632) with infer_logits_buffer_len: a head padded
    by 64 zero rows (vocab 300 -> 364 is not a multiple of 64, so vocab 320) gives 384 logits whose
    first 320 equal the unpadded head's and the rest exactly 0; a head of 100 rows gives the full
    head's first 100 logits, then xn[i % hidden] * 0.05 (i past hidden wraps); the same elements
    as [2 hidden, rows / 2] are read as rows of hidden."""
    from qdata import rand_weights as rw
    H = HEAD_SPEC["hidden"]
    spec_v = dict(HEAD_SPEC, vocab=320)
    full = rw(O.Q8_0, 320, H, 2)
    rb = O.row_bytes(O.Q8_0, H)
    x = rand_act(H, 9)
    base = dict(token_embd=(O.Q8_0, rw(O.Q8_0, 320, H, 1), H, 320), norm=(O.F32, np.ones(H, np.float32), H, 1))

    def model(spec, head):
        t = {"token_embd.weight": base["token_embd"], "output_norm.weight": base["norm"]}
        if head is not None:
            t["output.weight"] = head
        return O.DecodeModel(spec, t, 8)

    ref, xn, _ = model(spec_v, (O.Q8_0, full, H, 320)).head(x)
    padded = np.concatenate([full, _q8_0_blocks(0.0, np.zeros((64 * H // 32, 32)))])
    pm = model(spec_v, (O.Q8_0, padded, H, 384))
    assert pm.logits_len == 384
    lp, _, _ = pm.head(x)
    assert np.array_equal(lp[:320], ref) and np.all(lp[320:] == 0.0)
    sm = model(spec_v, (O.Q8_0, full[:100 * rb], H, 100))
    ls, xs, _ = sm.head(x)
    assert sm.logits_len == 320 and np.array_equal(ls[:100], ref[:100])
    idx = np.arange(100, 320)
    assert np.array_equal(ls[100:], (xs[idx % H] * np.float32(0.05)).astype(np.float32))
    assert not np.array_equal(ls[100:], (xs[(idx - 100) % H] * np.float32(0.05)).astype(np.float32))
    rm = model(spec_v, (O.Q8_0, full, 2 * H, 160))  # same bytes, another shape
    lr, _, _ = rm.head(x)
    assert np.array_equal(lr, ref)


def test_lm_head_without_head_is_the_tanh_fallback():
    """No output.weight and no token_embd.weight (src/qwen_deepseek.rs:626-631): a zero hidden state
    normalises to zero, so logit i is exactly (i % 13) * 0.01; a constant one gives
    tanh(hidden * xn / 16) + xn * 0.1 + (i % 13) * 0.01 with xn = c / sqrt(c^2 + eps)."""
    H, V = HEAD_SPEC["hidden"], HEAD_SPEC["vocab"]
    om, _ = _head_model({"output_norm.weight": (O.F32, np.ones(H, np.float32), H, 1)},
                        drop=("output.weight", "token_embd.weight"))
    assert om.logits_len == V
    l0, _, _ = om.head(np.zeros(H, np.float32))
    assert np.array_equal(l0, (np.arange(V) % 13).astype(np.float32) * np.float32(0.01))
    c = 0.75
    lc, xn, _ = om.head(np.full(H, c, np.float32))
    x64 = c / math.sqrt(c * c + 1e-5)
    want = math.tanh(H * x64 / 16) + 0.1 * x64 + (np.arange(V) % 13) * 0.01
    assert np.max(np.abs(lc - want)) < 2e-6


def test_embed_token_rows_and_deterministic_row():
    """embed_token (src/qwen_deepseek.rs:558-582): a token with a row dequantizes it; a token past
    the rows, or any token without token_embd, gives ((t % 31) * 0.05 + 0.25) + (i % 7) * 0.01."""
    H, V = HEAD_SPEC["hidden"], HEAD_SPEC["vocab"]
    om, t = _head_model({})
    e = om.embed(7)
    rb = O.row_bytes(O.Q8_0, H)
    assert np.array_equal(e, O.dequantize(O.Q8_0, t["token_embd.weight"][1][7 * rb:8 * rb], 1, H)[0])

    def det(tok):
        seed = np.float32(tok % 31) * np.float32(0.05) + np.float32(0.25)
        off = (np.arange(H) % 7).astype(np.float32) * np.float32(0.01)  # f32 products, one rounding each
        assert off.dtype == np.float32
        return (seed + off).astype(np.float32)

    for tok in list(range(V, V + 31)) + [12345, 2 ** 31 - 1]:  # every residue mod 31
        assert np.array_equal(om.embed(tok), det(tok)), tok
    none, _ = _head_model({}, drop=("token_embd.weight",))
    assert np.array_equal(none.embed(3), det(3))
    assert np.abs(det(31) - det(0)).max() == 0.0 and det(1)[0] == np.float32(0.3)


def test_absent_and_nonfinite_norms_in_the_decode_step():
    """read_f32_weight_or_default in execute_token_standard_with_hidden: absent norms give the logits
    of all-ones F32 norms, an F16 norm those of its f32 values, NaN / inf entries those of 1.0 in
    their place (bitwise, over two steps); a tied model (no output.weight) those of output.weight =
    token_embd.weight."""
    import model_spec as MS
    spec = dict(hidden=256, ffn=512, n_layers=2, vocab=40, nq=4, nkv=2, hd=64, eps=1e-6, theta=1e6)
    t = MS.build(spec, seed=8)
    norms = [k for k in t if k.endswith("norm.weight")]

    def run(tensors, qk_norm=True):
        om = O.DecodeModel(spec, tensors, 8, qk_norm=qk_norm)
        kv, out, tok = om.new_kv(), [], 3
        for pos in range(2):
            lg = om.step(kv, tok, pos, threads=2)
            out.append(lg)
            tok = int(np.argmax(lg))
        return np.stack(out)

    ones = {k: (O.F32, np.ones(v[2], np.float32), v[2], 1) if k in norms else v for k, v in t.items()}
    absent = {k: v for k, v in t.items() if k not in norms}
    assert np.array_equal(run(absent), run(ones))
    f16 = dict(t)
    f32_of_f16 = dict(t)
    for k in ("blk.0.attn_norm.weight", "blk.1.attn_k_norm.weight", "output_norm.weight"):
        h = t[k][1].astype(np.float16)
        f16[k] = (O.F16, h.view(np.uint8), t[k][2], 1)
        f32_of_f16[k] = (O.F32, h.astype(np.float32), t[k][2], 1)
    assert np.array_equal(run(f16), run(f32_of_f16))
    bad, fixed = dict(t), dict(t)
    w = t["blk.1.ffn_norm.weight"][1].copy()
    w[[3, 17, 200]] = [np.nan, np.inf, -np.inf]
    wf = w.copy()
    wf[[3, 17, 200]] = 1.0
    bad["blk.1.ffn_norm.weight"] = (O.F32, w, w.size, 1)
    fixed["blk.1.ffn_norm.weight"] = (O.F32, wf, wf.size, 1)
    assert np.array_equal(run(bad), run(fixed))
    assert not np.array_equal(run(fixed), run(t))
    tied = {k: v for k, v in t.items() if k != "output.weight"}
    tied_explicit = dict(tied, **{"output.weight": t["token_embd.weight"]})
    assert np.array_equal(run(tied), run(tied_explicit))


def _one_hot_f32(rows, k, col_of, scale=1.0):
    """F32 weight rows [rows][k] whose row i is scale * e_{col_of(i)}: an exact selection."""
    w = np.zeros((rows, k), np.float32)
    for i in range(rows):
        w[i, col_of(i)] = scale
    return w.reshape(-1)


def _silu64(v):
    return v / (1.0 + math.exp(-v))


def test_single_swiglu_expert_selection_closed_form():
    """run_single_swiglu_expert over one-hot F32 rows: out[h] = silu(x[p(r(h))]) * 2 x[q(r(h))],
    with F taken from the gate's element count (48 rows, not the expert_ffn_dim of 5); distinct
    permutations p, q, r make a swapped operand, a transposed matrix or a wrong F show."""
    H, F = 32, 48
    p = lambda i: (5 * i + 3) % H
    q = lambda i: (7 * i + 1) % H
    r = lambda h: (11 * h + 2) % F
    x = rand_act(H, 3)
    g = (O.F32, _one_hot_f32(F, H, p), [H, F])
    u = (O.F32, _one_hot_f32(F, H, q, 2.0), [H, F])
    d = (O.F32, _one_hot_f32(H, F, r), [F, H])
    out = O.single_swiglu_expert(g, u, d, x, 5)
    want = np.array([_silu64(float(x[p(r(h))])) * 2.0 * float(x[q(r(h))]) for h in range(H)])
    np.testing.assert_allclose(out, want, rtol=2e-6, atol=1e-7)


def test_dense_swiglu_ffn_deterministic_closed_form():
    """run_dense_swiglu_ffn with no tensors, and with tensors of the wrong element count (both take
    project_or_deterministic_slice's fallback): act[i] = silu(0.5 x[i % H]) * 0.25 x[i % H] over
    F = max(ffn, 4), out[h] = act[h % F] * 0.125; a present tensor of the right size is used."""
    H = 16
    x = rand_act(H, 4)
    for ffn, F in ((24, 24), (2, 4)):
        act = [_silu64(0.5 * float(x[i % H])) * 0.25 * float(x[i % H]) for i in range(F)]
        want = np.array([act[h % F] * 0.125 for h in range(H)])
        out = O.dense_swiglu_ffn({}, 0, ffn, x)
        np.testing.assert_allclose(out, want, rtol=2e-6, atol=1e-8)
        bad = {"blk.0.ffn_gate.weight": (O.F32, np.ones(H * F + H, np.float32), [H, F + 1]),
               "blk.0.ffn_down.weight": (O.F32, np.ones(7, np.float32), [7, 1])}
        np.testing.assert_array_equal(O.dense_swiglu_ffn(bad, 0, ffn, x), out)
    # a right-sized gate is used: one-hot rows picking x[(3 i) % H]
    F = 24
    good = {"blk.0.ffn_gate.weight": (O.F32, _one_hot_f32(F, H, lambda i: (3 * i) % H), [H, F])}
    act = [_silu64(float(x[(3 * i) % H])) * 0.25 * float(x[i % H]) for i in range(F)]
    want = np.array([act[h % F] * 0.125 for h in range(H)])
    np.testing.assert_allclose(O.dense_swiglu_ffn(good, 0, F, x), want, rtol=2e-6, atol=1e-8)


def _moe_weights(H, F, E, seed, shared=True, quant=O.Q4_K):
    rng = np.random.default_rng(seed)
    w = {}
    g = rand_weights(quant, E * F, H, seed)
    u = rand_weights(quant, E * F, H, seed + 1)
    d = rand_weights(quant, E * H, F, seed + 2)
    w["blk.0.ffn_gate_exps.weight"] = (quant, g, [H, F, E])
    w["blk.0.ffn_up_exps.weight"] = (quant, u, [H, F, E])
    w["blk.0.ffn_down_exps.weight"] = (quant, d, [F, H, E])
    w["blk.0.ffn_gate_inp.weight"] = (O.F32, (rng.standard_normal(E * H) * 0.05).astype(np.float32), [H, E])
    if shared:
        w["blk.0.ffn_gate_shexp.weight"] = (quant, rand_weights(quant, F, H, seed + 5), [H, F])
        w["blk.0.ffn_up_shexp.weight"] = (quant, rand_weights(quant, F, H, seed + 6), [H, F])
        w["blk.0.ffn_down_shexp.weight"] = (quant, rand_weights(quant, H, F, seed + 7), [F, H])
    return w


def test_moe_layer_shared_expert_equal_to_every_routed_expert():
    """With every routed expert and the shared expert the same tensors e, the layer is
    (1 + sum of the normalised selection weights) * e(x) = 2 e(x); without the shared expert, e(x);
    the selection is select_top_k of the router's logits (F32 rows with router row j = c_j e_0,
    so logits c_j x[0])."""
    H, F, E, k = 256, 256, 6, 3
    x = rand_act(H, 9)
    one = rand_weights(O.Q4_K, F, H, 11), rand_weights(O.Q4_K, F, H, 12), rand_weights(O.Q4_K, H, F, 13)
    c = np.array([0.5, -2.0, 3.0, 1.0, 3.0, -1.0], np.float32)
    router = np.zeros((E, H), np.float32)
    router[:, 0] = c
    w = {"blk.0.ffn_gate_inp.weight": (O.F32, router.reshape(-1), [H, E]),
         "blk.0.ffn_gate_exps.weight": (O.Q4_K, np.tile(one[0], E), [H, F, E]),
         "blk.0.ffn_up_exps.weight": (O.Q4_K, np.tile(one[1], E), [H, F, E]),
         "blk.0.ffn_down_exps.weight": (O.Q4_K, np.tile(one[2], E), [F, H, E]),
         "blk.0.ffn_gate_shexp.weight": (O.Q4_K, one[0], [H, F]),
         "blk.0.ffn_up_shexp.weight": (O.Q4_K, one[1], [H, F]),
         "blk.0.ffn_down_shexp.weight": (O.Q4_K, one[2], [F, H])}
    e = O.single_swiglu_expert(w["blk.0.ffn_gate_shexp.weight"], w["blk.0.ffn_up_shexp.weight"],
                               w["blk.0.ffn_down_shexp.weight"], x, F)
    out, sel = O.moe_layer(x, 0, E, k, F, True, w)
    assert [i for i, _ in sel] == [int(i) for i in np.lexsort((np.arange(E), -(c * x[0])))[:k]]
    np.testing.assert_allclose(out, 2 * e, rtol=1e-6, atol=1e-6 * float(np.abs(e).max()))
    out1, _ = O.moe_layer(x, 0, E, k, F, False, w)
    np.testing.assert_allclose(out1, e, rtol=1e-6, atol=1e-6 * float(np.abs(e).max()))


def test_moe_layer_indexed_experts_and_fallbacks():
    """Per-expert tensors ffn_*_exps.{e} give the same bits as the stacked tensors; an expert
    whose tensors are missing is skipped (the others keep their weights); with every selected
    expert missing the dense FFN runs; with no router, shared expert + dense FFN."""
    H, F, E, k = 256, 256, 5, 2
    x = rand_act(H, 21)
    w = _moe_weights(H, F, E, 30)
    out, sel = O.moe_layer(x, 0, E, k, F, True, w)
    ix = dict(w)
    for kind in ("gate", "up", "down"):
        q, data, dims = ix.pop(f"blk.0.ffn_{kind}_exps.weight")
        per = len(data) // E
        for e in range(E):
            ix[f"blk.0.ffn_{kind}_exps.{e}.weight"] = (q, data[e * per:(e + 1) * per], dims[:2])
    out_ix, sel_ix = O.moe_layer(x, 0, E, k, F, True, ix)
    assert sel_ix == sel
    np.testing.assert_array_equal(out_ix, out)
    sh = O.single_swiglu_expert(w["blk.0.ffn_gate_shexp.weight"], w["blk.0.ffn_up_shexp.weight"],
                                w["blk.0.ffn_down_shexp.weight"], x, F)
    # the second selected expert missing: shared + w0 * e0 only
    e0, e1 = sel[0][0], sel[1][0]
    miss = {n: t for n, t in ix.items() if n != f"blk.0.ffn_up_exps.{e1}.weight"}
    part = lambda e: [ix[f"blk.0.ffn_{kd}_exps.{e}.weight"] for kd in ("gate", "up", "down")]
    want = np.zeros(H, np.float32)
    want += sh
    want += np.float32(sel[0][1]) * O.single_swiglu_expert(*part(e0), x, F)
    np.testing.assert_array_equal(O.moe_layer(x, 0, E, k, F, True, miss)[0], want)
    # both missing: shared + dense (deterministic here: no ffn_gate/up/down)
    miss2 = {n: t for n, t in miss.items() if n != f"blk.0.ffn_down_exps.{e0}.weight"}
    want = np.zeros(H, np.float32)
    want += sh
    want += O.dense_swiglu_ffn({}, 0, F, x)
    np.testing.assert_array_equal(O.moe_layer(x, 0, E, k, F, True, miss2)[0], want)
    # no router: shared + dense, no selection
    nr = {n: t for n, t in w.items() if "gate_inp" not in n}
    o, s = O.moe_layer(x, 0, E, k, F, True, nr)
    assert s == [] and np.array_equal(o, want)
