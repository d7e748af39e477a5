"""The layer-by-layer parity checks (decode_parity) run on the CPU against the oracle's own trace:
a faithful trace passes, and each planted mistake -- a flipped activation byte, QK-norm applied
after RoPE, a 1e-4 error in a projection, an attention output from the wrong positions, a
flip of more than one quantum -- is caught."""
import numpy as np
import pytest

import decode_parity as DP
import model_spec as MS
import pyoracle as O

SPEC = dict(hidden=512, ffn=768, n_layers=2, vocab=300, nq=8, nkv=2, hd=64, eps=1e-6, theta=1e6)
CAP, POS = 40, 33


def oracle_trace(seed=5):
    t = MS.build(SPEC, seed=seed)
    om = O.DecodeModel(SPEC, MS.oracle_tensors(t), CAP)
    kv = om.new_kv()
    rng = np.random.default_rng(seed)
    kv[:, :, :POS] = rng.standard_normal(kv[:, :, :POS].shape).astype(np.float16).astype(np.float32)
    x = om.embed(17)
    layers = []
    for L in range(SPEC["n_layers"]):
        x_in = x.copy()
        x, tr = om.layer(kv, L, x, POS, threads=4)
        tr["x_in"] = x_in
        layers.append(tr)
    logits, xn, q8 = om.head(x, threads=4)
    return t, om, kv, layers, dict(x_final=x, xn_head=xn, q8_head=q8), logits


def check_all(t, kv, layers, head, logits):
    errs = []
    for L, D in enumerate(layers):
        x_next = layers[L + 1]["x_in"] if L + 1 < len(layers) else head["x_final"]
        errs.append(DP.check_layer(t, SPEC, D, L, POS, x_next, kv[L, 0], kv[L, 1], False, True, threads=4))
    DP.check_head(t, SPEC, head, logits, O.argmax(logits), threads=4)
    return errs


def test_faithful_trace_passes():
    t, om, kv, layers, head, logits = oracle_trace()
    errs = check_all(t, kv, layers, head, logits)
    for e in errs:
        assert e["gemv"] <= 1e-6 and e["attn"] <= 1e-6 and e["norm"] <= 1e-6, e


def test_planted_activation_byte_is_caught():
    t, om, kv, layers, head, logits = oracle_trace()
    q8 = layers[1]["q8_ffn"]
    q8[4 + 100] = np.uint8((int(q8[4 + 100]) + 1) & 0xFF)
    with pytest.raises(AssertionError, match="gate\\|up input"):
        check_all(t, kv, layers, head, logits)


def test_planted_norm_after_rope_is_caught():
    """QK-norm applied after RoPE instead of before (:1039-1071): RMSNorm does not commute with
    the rotation once the norm weights differ within a pair."""
    t, om, kv, layers, head, logits = oracle_trace()
    D = layers[0]
    hd, nq = SPEC["hd"], SPEC["nq"]
    Q = nq * hd
    q = O.rope(D["qkv"][:Q], hd, POS, SPEC["theta"])
    qn = t["blk.0.attn_q_norm.weight"][1]
    D["q_rope"] = np.concatenate([O.rmsnorm(q[h * hd:(h + 1) * hd], qn, SPEC["eps"]) for h in range(nq)])
    with pytest.raises(AssertionError):
        check_all(t, kv, layers, head, logits)


def test_planted_projection_error_is_caught():
    t, om, kv, layers, head, logits = oracle_trace()
    layers[1]["gu"][:SPEC["ffn"]] *= np.float32(1 + 1e-4)
    with pytest.raises(AssertionError):
        check_all(t, kv, layers, head, logits)


def test_planted_attention_window_is_caught():
    """Attention over one position too few (the oldest slot dropped)."""
    t, om, kv, layers, head, logits = oracle_trace()
    D = layers[0]
    kr, vr = kv[0, 0, 1:POS + 1], kv[0, 1, 1:POS + 1]
    D["attn"] = O.gqa_attention(D["q_rope"], kr, vr, SPEC["nq"], SPEC["nkv"], SPEC["hd"], POS,
                                1.0 / np.sqrt(np.float32(SPEC["hd"])))
    with pytest.raises(AssertionError):
        check_all(t, kv, layers, head, logits)


def test_adopting_step_on_a_faithful_trace():
    """The oracle's own trace as the 'device': no flips, and the adopting step reproduces the
    oracle's logits bit for bit."""
    t, om, kv0, layers, head, logits = oracle_trace()
    # rebuild the pre-step rings: the trace run wrote slot POS
    t2, om2, kv, layers2, head2, logits2 = oracle_trace()
    kv[:, :, POS] = 0
    ref, st, f16 = DP.oracle_step_adopting(t, SPEC, kv, POS, om.embed(17), layers, head, True, threads=4)
    assert st.flips == 0 and st.pre_diff == 0.0
    np.testing.assert_array_equal(ref, logits)


def test_tie_flips_accounting():
    """tie_flips: equal vectors have no flips; two f32 values a few ulps either side of a rounding
    boundary give one accounted flip; a vector off by a tenth of a quantum, or an int8 off by two,
    is rejected."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal(512).astype(np.float32)
    x[0] = 3.0  # block max: fixes the scale
    q = O.quantize_act(DP.Q8_K, x)
    assert DP.tie_flips("same", DP.Q8_K, 512, x, q, x, q)[0] == 0
    d = np.frombuffer(q[:4].tobytes(), np.float32)[0]
    y = x.copy()
    y[7] = np.float32((np.floor(x[7] / d) + 0.5) * d)  # on a boundary
    up, dn = y.copy(), y.copy()
    for _ in range(3):
        up[7] = np.nextafter(up[7], np.float32(np.inf))
        dn[7] = np.nextafter(dn[7], np.float32(-np.inf))
    qu, qd = O.quantize_act(DP.Q8_K, up), O.quantize_act(DP.Q8_K, dn)
    n, tie, pre = DP.tie_flips("tie", DP.Q8_K, 512, up, qu, dn, qd)
    assert n == 1 and tie < 1e-4 and pre < 1e-4
    # the reconstruction is the quantizer's own arithmetic: its rounding gives the stored int8s
    for v, qq in ((up, qu), (dn, qd)):
        pr = DP.pre_rounding(DP.Q8_K, v.reshape(-1, 256))
        want = np.minimum(np.rint(pr), 127).astype(np.int64)
        got = qq.reshape(-1, 292)[:, 4:260].view(np.int8).astype(np.int64)
        np.testing.assert_array_equal(got, want)
    xa = x.reshape(-1, 32)
    qa = O.quantize_act(DP.ACT_Q8, x).reshape(-1, 36)[:, 4:].view(np.int8).astype(np.int64)
    np.testing.assert_array_equal(qa, np.rint(DP.pre_rounding(DP.ACT_Q8, xa)).astype(np.int64))
    j = int(np.argmin(np.abs(x[:256])))  # far from the block maximum
    off = x.copy()
    off[j] = np.float32(x[j] + 0.1 * abs(d))
    with pytest.raises(AssertionError, match="pre-rounding"):
        DP.tie_flips("off", DP.Q8_K, 512, x, q, off, O.quantize_act(DP.Q8_K, off))
    q2 = q.copy()
    q2[4 + j] = np.uint8((int(q[4 + j]) + 2) & 0xFF)
    with pytest.raises(AssertionError, match="more than one"):
        DP.tie_flips("two", DP.Q8_K, 512, x, q, x, q2)
    q1 = q.copy()
    q1[4 + j] = np.uint8((int(q[4 + j]) + 1) & 0xFF)
    with pytest.raises(AssertionError, match="no rounding boundary"):
        DP.tie_flips("one", DP.Q8_K, 512, x, q, x, q1)


def test_rope_table_check():
    """check_rope_table accepts the f64 table of the f32 angles at any position and rejects a table
    built with the exponent i/hd instead of 2i/hd, or one position off."""
    hd, theta = SPEC["hd"], SPEC["theta"]
    i = np.arange(hd // 2, dtype=np.float32)

    def table(pos, expo):
        a = (np.float32(pos) / np.power(np.float32(theta), expo, dtype=np.float32)).astype(np.float64)
        return np.stack([np.cos(a), np.sin(a)], axis=1).reshape(-1).astype(np.float32)

    good_expo = (np.float32(2) * i) / np.float32(hd)
    for pos in (0, 1, 291, 4095, 100000):
        DP.check_rope_table(SPEC, pos, table(pos, good_expo))
    with pytest.raises(AssertionError):
        DP.check_rope_table(SPEC, 291, table(291, i / np.float32(hd)))
    with pytest.raises(AssertionError):
        DP.check_rope_table(SPEC, 291, table(292, good_expo))


def test_f16_tie_flips():
    """Two f32 values an ulp either side of an f16 midpoint give one accounted flip; a flip between
    f32 values far apart (relative to the row) is rejected, and so is a device row that is not its
    own f32 row rounded to nearest."""
    lo = np.float16(1.0)
    hi = np.nextafter(lo, np.float16(2.0))
    mid = np.float32((np.float64(lo) + np.float64(hi)) / 2)
    x = np.array([0.5, mid, -3.0], np.float32)
    up, dn = x.copy(), x.copy()
    up[1] = np.nextafter(mid, np.float32(2.0))
    dn[1] = np.nextafter(mid, np.float32(0.0))
    dev = up.astype(np.float16).astype(np.float32)
    n, gap = DP.f16_tie_flips("row", dn, up, dev)
    assert n == 1 and gap < 1e-6
    far = x.copy()
    far[1] = np.float32(np.float64(lo) + 0.25 * (np.float64(hi) - np.float64(lo)))
    with pytest.raises(AssertionError, match="apart"):
        DP.f16_tie_flips("row", far, up, dev)
    tiny = np.array([1.0, -1e-9, 2.0], np.float32)  # -0 and +1 subnormal are far apart in bits
    tiny_dev = np.array([1.0, 2e-9, 2.0], np.float32)
    assert DP.f16_tie_flips("row", tiny, tiny_dev, tiny_dev.astype(np.float16).astype(np.float32))[0] >= 0
    with pytest.raises(AssertionError, match="rounded"):
        DP.f16_tie_flips("row", dn, dn, dev)
