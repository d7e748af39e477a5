"""Layer-by-layer parity of the device decode step against the oracle.

Teacher-forced checks (check_layer, check_head): every stage of a layer is recomputed by the
oracle from the device's own input to that stage, as the device's debug trace recorded it
(jero_hip_model_trace), and compared at the north-star bars:
  * activation blocks (Q8_K / ACT_Q8) bit-exact: the oracle quantizes the f32 values the device
    quantized;
  * GEMV outputs (Q|K|V, Wo, gate|up, down, LM head) within GEMV_TOL = 1e-5 of max(|ref|, rms(ref)),
    the oracle reading the device's activation bytes; residual adds are checked through the GEMV
    (x_out - x_in against the oracle's projection, allowing the f32 rounding of the add);
  * attention within ATTN_TOL = 1e-3, the oracle attending with the device's q over the device's
    ring as it stands after the step (the new slot holds the device's k and v, rounded to f16 in
    an f16 ring: the values the kernel attends to); that slot must equal the device's f32 k and
    v rounded to the ring's type;
  * RMSNorm (attention, FFN, head) within NORM_TOL of the oracle's f64-accumulated norm, SwiGLU
    within SWIGLU_TOL (f32 against f64 arithmetic);
  * RoPE in two parts: the step's table of (cos, sin) must hold the f32 angles pos / theta^(2i/hd)
    to within two ulps of the angle (theta^(2i/hd) is an f32 powf, whose last bit differs
    between math libraries; at position 4095 one ulp of the angle is 4.9e-4 rad), and QK-norm +
    the rotation by that table within ROPE_TOL.

End to end with tie accounting (oracle_step_adopting): the oracle runs the whole step from its
own state (its own hidden state, K/V rings and f64-accumulated arithmetic) and, at each
quantization point, quantizes its own f32 vector.  The two f32 vectors must agree to PRE_TOL =
0.05 quantum in every element's pre-rounding value x/d (measured: a few 1e-3 at most, f32 noise
amplified by SwiGLU products in the random-init models; an error of 1e-3 in a stage moves values
near a block maximum by 0.13 quantum).  An int8 that differs from the device's is a flip; it is
accounted for only as a tie: the two int8s differ by one and a .5 rounding boundary lies between
the two pre-rounding values.  The oracle then continues with the device's activation bytes, so
a tie flip does not propagate, and the step's logits must meet the north-star 1e-3 bar outright.  The
new K/V row stored in an f16 ring is a rounding point too: the two f32 rows must agree to
F16_TIE_REL of the row's rms in every element, and the f16 values that differ are the two
sides' nearest roundings of such close values (f16_tie_flips); the oracle then keeps the
device's row.
A real error of 1e-3 in any stage shows up as flips far from ties, or as a logit error.
Beside it the oracle's plain free-running step (no adoption) must match within 1e-3 until the
first tie flip; after one, its error (a single flip moves the logits of a small model by up to a
few 1e-2) and cosine are reported.
"""
import numpy as np

import pyoracle as O

ACT_Q8, Q8_K = 100, 15
GEMV_TOL = 1e-5
ATTN_TOL = 1e-3
NORM_TOL = 4e-6
ROPE_TOL = 1e-5
SWIGLU_TOL = 1e-6
PRE_TOL = 0.05  # quanta: how far apart the two pre-rounding values x/d of any element may be


def act_fmt(quant):
    return ACT_Q8 if quant in (2, 8) else Q8_K


def rel(got, ref):
    """max |got - ref| / max(|ref|, rms(ref)), elementwise."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.sqrt(np.mean(ref ** 2))), 1e-30)
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), scale)))


def rel_resid(x_out, x_in, g_ref):
    """Error of a residual add x_out = fl(x_in + g) against the oracle's projection g_ref: the
    f32 rounding of the add (<= 2^-24 |x_out|) is allowed on top of the GEMV error."""
    x_out = np.asarray(x_out, np.float64)
    g_ref = np.asarray(g_ref, np.float64)
    d = np.abs(x_out - np.asarray(x_in, np.float64) - g_ref) - 2.0 ** -24 * np.abs(x_out)
    scale = max(float(np.sqrt(np.mean(g_ref ** 2))), 1e-30)
    return float(np.max(np.maximum(d, 0.0) / np.maximum(np.abs(g_ref), scale)))


def q8_bytes(fmt, n, buf):
    return np.asarray(buf[:O.row_bytes(fmt, n)], np.uint8)


def check_q8(tag, fmt, x, dev_q8):
    """The device's activation blocks equal the oracle's quantization of the same f32 values."""
    ref = O.quantize_act(fmt, x)
    got = q8_bytes(fmt, x.size, dev_q8)
    if not np.array_equal(got, ref):
        bad = np.nonzero(got != ref)[0]
        raise AssertionError(f"{tag}: activation blocks differ at {bad.size} bytes (first {bad[:8].tolist()})")


def _w(t, name):
    q, arr, n_in, n_out = t[name]
    return q, arr, n_in, n_out


def _mv(t, name, xq, threads):
    q, arr, n_in, n_out = _w(t, name)
    return O.matvec(q, arr, n_in, n_out, xq, threads=threads)


def check_rope_table(spec, pos, rope_cs):
    """The device's RoPE table against the f32 angles pos / theta^(2i/hd) (interleaved pairs,
    tests/wave1_engine_regression_test.rs:698-712): each (cos, sin) within two ulps of its angle."""
    hd = spec["hd"]
    i = np.arange(hd // 2, dtype=np.float32)
    base = np.power(np.float32(spec["theta"]), (np.float32(2) * i) / np.float32(hd), dtype=np.float32)
    ang = (np.float32(pos) / base).astype(np.float32)
    tol = 2.0 * np.spacing(np.abs(ang)).astype(np.float64) + 2e-7
    c, s_ = rope_cs[0::2].astype(np.float64), rope_cs[1::2].astype(np.float64)
    a64 = ang.astype(np.float64)
    assert np.all(np.abs(c - np.cos(a64)) <= tol) and np.all(np.abs(s_ - np.sin(a64)) <= tol), \
        f"RoPE table at position {pos} is not pos / theta^(2i/hd)"


def rotate(x, hd, rope_cs):
    """Interleaved-pair rotation of each head of x by the table (f64)."""
    x = np.asarray(x, np.float64).reshape(-1, hd // 2, 2)
    c, s_ = rope_cs[0::2].astype(np.float64), rope_cs[1::2].astype(np.float64)
    out = np.empty_like(x)
    out[..., 0] = x[..., 0] * c - x[..., 1] * s_
    out[..., 1] = x[..., 0] * s_ + x[..., 1] * c
    return out.reshape(-1)


def check_layer(t, spec, D, L, pos, x_next, ring_k, ring_v, kv_f16, qk_norm=True, threads=16, rope_cs=None):
    """Teacher-forced checks of layer L from its device trace D; x_next is the device's input to
    the next layer (or its final hidden state).  ring_k / ring_v: the layer's rings after the step
    as f32 [capacity][n_kv*hd].  Returns the largest error of each kind; raises on a breach."""
    err = check_attn(t, spec, D, L, pos, ring_k, ring_v, kv_f16, qk_norm, threads, rope_cs, final=False)
    return check_layer_ffn(t, spec, D, L, x_next, err, threads)


def check_attn(t, spec, D, L, pos, ring_k, ring_v, kv_f16, qk_norm=True, threads=16, rope_cs=None, final=True):
    """The attention sublayer of check_layer (RMSNorm, Q|K|V, QK-norm and RoPE, the ring slot,
    attention, Wo + residual into the trace's x_mid); with final, raises on a breach here."""
    H = spec["hidden"]
    nq, nkv, hd = spec["nq"], spec["nkv"], spec["hd"]
    Q, KV = nq * hd, nkv * hd
    eps = spec["eps"]
    p = f"blk.{L}."
    err = {}
    # attention RMSNorm and the Q|K|V activation blocks
    xn = O.rmsnorm(D["x_in"], t[p + "attn_norm.weight"][1], eps)
    err["norm"] = rel(D["xn_attn"], xn)
    qq = t[p + "attn_q.weight"][0]
    check_q8(f"layer {L} q|k|v input", act_fmt(qq), D["xn_attn"], D["q8_attn"])
    xq = q8_bytes(act_fmt(qq), H, D["q8_attn"])
    xv = xq if act_fmt(t[p + "attn_v.weight"][0]) == act_fmt(qq) else O.quantize_act(
        act_fmt(t[p + "attn_v.weight"][0]), D["xn_attn"])
    ref_q = _mv(t, p + "attn_q.weight", xq, threads)
    ref_k = _mv(t, p + "attn_k.weight", xq, threads)
    ref_v = _mv(t, p + "attn_v.weight", xv, threads)
    qkv = D["qkv"]
    err["gemv"] = max(rel(qkv[:Q], ref_q), rel(qkv[Q:Q + KV], ref_k), rel(qkv[Q + KV:], ref_v))
    # QK-norm (if present) and RoPE from the device's projections
    q, k = qkv[:Q].copy(), qkv[Q:Q + KV].copy()
    if qk_norm:
        qn, kn = t[p + "attn_q_norm.weight"][1], t[p + "attn_k_norm.weight"][1]
        q = np.concatenate([O.rmsnorm(q[h * hd:(h + 1) * hd], qn, eps) for h in range(nq)])
        k = np.concatenate([O.rmsnorm(k[h * hd:(h + 1) * hd], kn, eps) for h in range(nkv)])
    if rope_cs is None:
        q = O.rope(q, hd, pos, spec["theta"])
        k = O.rope(k, hd, pos, spec["theta"])
    else:
        q, k = rotate(q, hd, rope_cs), rotate(k, hd, rope_cs)
    err["rope"] = max(rel(D["q_rope"], q), rel(D["k_rope"], k))
    # the ring slot holds the new k and v (rounded to the ring's type)
    cap = ring_k.shape[0]
    slot, active = pos % cap, min(pos + 1, cap)
    v_new = qkv[Q + KV:]
    rnd = (lambda a: a.astype(np.float16).astype(np.float32)) if kv_f16 else (lambda a: a.astype(np.float32))
    assert np.array_equal(ring_k[slot], rnd(D["k_rope"])), f"layer {L}: K ring slot {slot} is not the new k"
    assert np.array_equal(ring_v[slot], rnd(v_new)), f"layer {L}: V ring slot {slot} is not the new v"
    ref_attn = O.gqa_attention(D["q_rope"], ring_k[:active], ring_v[:active], nq, nkv, hd, active,
                               1.0 / np.sqrt(np.float32(hd)))
    err["attn"] = rel(D["attn"], ref_attn)
    # Wo + residual
    wq_ = t[p + "attn_output.weight"][0]
    check_q8(f"layer {L} wo input", act_fmt(wq_), D["attn"], D["q8_wo"])
    g = _mv(t, p + "attn_output.weight", q8_bytes(act_fmt(wq_), Q, D["q8_wo"]), threads)
    err["gemv"] = max(err["gemv"], rel_resid(D["x_mid"], D["x_in"], g))
    if final:
        assert err["norm"] <= NORM_TOL, (L, err)
        assert err["gemv"] <= GEMV_TOL, (L, err)
        assert err["rope"] <= ROPE_TOL, (L, err)
        assert err["attn"] <= ATTN_TOL, (L, err)
    return err


def check_layer_ffn(t, spec, D, L, x_next, err, threads=16):
    """The dense FFN sublayer of check_layer, its errors added to err (check_attn's)."""
    H, F = spec["hidden"], spec["ffn"]
    eps_ffn = max(spec["eps"], 1e-6)
    p = f"blk.{L}."
    # FFN RMSNorm, gate|up, SwiGLU
    xn = O.rmsnorm(D["x_mid"], t[p + "ffn_norm.weight"][1], eps_ffn)
    err["norm"] = max(err["norm"], rel(D["xn_ffn"], xn))
    gq = t[p + "ffn_gate.weight"][0]
    check_q8(f"layer {L} gate|up input", act_fmt(gq), D["xn_ffn"], D["q8_ffn"])
    xq = q8_bytes(act_fmt(gq), H, D["q8_ffn"])
    ref_g = _mv(t, p + "ffn_gate.weight", xq, threads)
    ref_u = _mv(t, p + "ffn_up.weight", xq, threads)
    err["gemv"] = max(err["gemv"], rel(D["gu"][:F], ref_g), rel(D["gu"][F:], ref_u))
    err["swiglu"] = rel(D["act"], O.swiglu(D["gu"][:F], D["gu"][F:]))
    # down + residual
    dq = t[p + "ffn_down.weight"][0]
    check_q8(f"layer {L} down input", act_fmt(dq), D["act"], D["q8_down"])
    g = _mv(t, p + "ffn_down.weight", q8_bytes(act_fmt(dq), F, D["q8_down"]), threads)
    err["gemv"] = max(err["gemv"], rel_resid(x_next, D["x_mid"], g))
    assert err["norm"] <= NORM_TOL, (L, err)
    assert err["gemv"] <= GEMV_TOL, (L, err)
    assert err["rope"] <= ROPE_TOL, (L, err)
    assert err["attn"] <= ATTN_TOL, (L, err)
    assert err["swiglu"] <= SWIGLU_TOL, (L, err)
    return err


def resolve_norms(t, spec, qk_norm=True):
    """t with every norm weight replaced by the f32 vector the reference reads for it
    (read_f32_weight_or_default through the oracle: absent -> ones, non-finite F32 values -> 1.0,
    other formats dequantized), so that the checks below can use t[name][1] as the weight."""
    H, hd = spec["hidden"], spec["hd"]
    out = dict(t)
    names = [("output_norm.weight", H)]
    for L in range(spec["n_layers"]):
        names += [(f"blk.{L}.attn_norm.weight", H), (f"blk.{L}.ffn_norm.weight", H)]
        if qk_norm:
            names += [(f"blk.{L}.attn_q_norm.weight", hd), (f"blk.{L}.attn_k_norm.weight", hd)]
    for name, n in names:
        if name in t:
            q, a = t[name][:2]
            dims = t[name][2:4] if len(t[name]) >= 4 else None
            v = O.read_f32_weight_or_default(q, a, O._elements(q, a, dims), n)
        else:
            v = O.read_f32_weight_or_default(O.F32, None, 0, n)
        out[name] = (O.F32, v, n, 1)
    return out


def head_spec(t, spec):
    """project_lm_head's head (src/qwen_deepseek.rs:584-632): (tensor name or None -- output.weight,
    else token_embd.weight --, its n_in, its rows, the rows its GEMV gives, logits_len)."""
    H, V = spec["hidden"], spec["vocab"]
    name = "output.weight" if "output.weight" in t else ("token_embd.weight" if "token_embd.weight" in t else None)
    if name is None:
        return None, 0, 0, 0, O.logits_len(V, None)
    n_in, rows = t[name][2], t[name][3]
    L = O.logits_len(V, rows)
    if n_in == H:
        return name, n_in, rows, min(L, rows), L
    if n_in * rows == L * H:
        return name, n_in, rows, L, L
    return None, n_in, rows, 0, L


def oracle_head_on(om, t, spec, x, hq, threads):
    """The oracle's project_lm_head from the hidden state x (jo_decode_head), with its head GEMV, if
    any, recomputed over the activation blocks hq (the device's, once accounted for) instead of
    the oracle's own; hq None keeps the oracle's (an f32-input head)."""
    ref, xn, _ = om.head(x, threads)
    name, _, _, target, _ = head_spec(t, spec)
    if name is not None and target > 0 and hq is not None:
        q, arr = t[name][:2]
        ref = ref.copy()
        ref[:target] = O.matvec(q, arr, spec["hidden"], target, hq, threads=threads)
    return ref, xn


def check_head(t, spec, Dh, logits, token, threads=16, om=None):
    """Final RMSNorm, LM-head activation blocks and GEMV, and the greedy token from the device's
    own logits.  With om (the oracle model), any head project_lm_head takes: the rows past the
    head (xn * 0.05), a head read as rows of hidden, the tanh fallback, an f32-input head."""
    H = spec["hidden"]
    if om is None:
        xn = O.rmsnorm(Dh["x_final"], t["output_norm.weight"][1], max(spec["eps"], 1e-6))
        err = {"norm": rel(Dh["xn_head"], xn)}
        oq = t["output.weight"][0]
        check_q8("head input", act_fmt(oq), Dh["xn_head"], Dh["q8_head"])
        ref = _mv(t, "output.weight", q8_bytes(act_fmt(oq), H, Dh["q8_head"]), threads)
    else:
        name, _, _, target, L = head_spec(t, spec)
        logits = logits[:L]
        quantized = name is not None and target > 0 and t[name][0] not in (O.F32, O.F16, O.BF16)
        hq = None
        if quantized:
            fq = act_fmt(t[name][0])
            check_q8("head input", fq, Dh["xn_head"], Dh["q8_head"])
            hq = q8_bytes(fq, H, Dh["q8_head"])
        ref, xn = oracle_head_on(om, t, spec, Dh["x_final"], hq, threads)
        err = {"norm": rel(Dh["xn_head"], xn)}
    err["gemv"] = rel(logits, ref)
    want = O.argmax(logits)
    assert token == (-1 if want is None else want), (token, want)
    assert err["norm"] <= NORM_TOL and err["gemv"] <= GEMV_TOL, err
    return err


def _blocks(fmt, n, q8):
    bs, be = (292, 256) if fmt == Q8_K else (36, 32)
    a = q8_bytes(fmt, n, q8).reshape(-1, bs)
    d = a[:, :4].copy().view(np.float32)[:, 0].astype(np.float64)
    q = a[:, 4:4 + be].view(np.int8).astype(np.int64)
    return d, q, be


def pre_rounding(fmt, x):
    """The values each quantizer rounds, computed as it does in f32 (blocks along the last axis):
    Q8_K iscale = -127 / max (the signed element of largest magnitude, first on ties) times x;
    ACT_Q8 x times 1 / (amax / 127).  All-zero blocks give zeros."""
    x = np.asarray(x, np.float32)
    a = np.abs(x)
    if fmt == Q8_K:
        idx = np.argmax(a, axis=1)
        mx = x[np.arange(x.shape[0]), idx]
        with np.errstate(divide="ignore", invalid="ignore"):
            iscale = np.where(mx != 0, np.float32(-127.0) / mx, np.float32(0)).astype(np.float32)
        return (iscale[:, None] * x).astype(np.float32)
    d = (a.max(axis=1) / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0)).astype(np.float32)
    return (x * inv[:, None]).astype(np.float32)


def tie_flips(tag, fmt, n, x_or, q_or, x_dev, q_dev):
    """Compares the oracle's activation blocks q_or (of its own f32 vector x_or) with the device's
    q_dev (of x_dev).  The two vectors must agree to PRE_TOL quanta in every element's pre-rounding
    value x/d (the block scales then agree to PRE_TOL/127), and every differing int8 must be a +-1
    crossing of a rounding boundary lying between the two pre-rounding values.  Returns (flips,
    largest distance of a flipped element's oracle value from its boundary, in quanta, largest
    pre-rounding difference over all elements)."""
    do, qo, be = _blocks(fmt, n, q_or)
    dd, qd, _ = _blocks(fmt, n, q_dev)
    live = (do != 0) | (dd != 0)
    sdiff = np.where(live, np.abs(do - dd) / np.maximum(np.maximum(np.abs(do), np.abs(dd)), 1e-30), 0.0)
    b = int(np.argmax(sdiff))
    assert sdiff[b] <= PRE_TOL / 127, (f"{tag}: block {b} scales {do[b]!r} (oracle) and {dd[b]!r} (device) "
                                       f"differ by {sdiff[b]:.2e}")
    po = pre_rounding(fmt, np.asarray(x_or, np.float32).reshape(-1, be)).astype(np.float64)
    pd = pre_rounding(fmt, np.asarray(x_dev, np.float32).reshape(-1, be)).astype(np.float64)
    diff = np.abs(po - pd)
    pre = float(diff.max())
    assert pre <= PRE_TOL, f"{tag}: pre-rounding values differ by {pre:.2e} quanta"
    flip = qo != qd
    n_flips = int(flip.sum())
    tie_dist = 0.0
    if n_flips:
        assert int(np.abs(qo - qd)[flip].max()) == 1, f"{tag}: an int8 differs by more than one"
        bound = np.floor(np.maximum(po, pd)[flip] - 0.5) + 0.5  # the boundary between them
        lo, hi = np.minimum(po, pd)[flip], np.maximum(po, pd)[flip]
        assert np.all((lo <= bound) & (bound <= hi)), f"{tag}: a flip with no rounding boundary between the values"
        tie_dist = float(np.max(np.abs(po[flip] - bound)))
    return n_flips, tie_dist, pre


F16_TIE_REL = 1e-5  # of the row's rms: how far apart the two f32 values of an f16 flip may be


def f16_tie_flips(tag, x_or, x_dev, dev_f16):
    """The oracle's f32 row x_or rounded to f16 against the device's f16 row dev_f16.  The device's
    row must be its own f32 row x_dev rounded to nearest even, and the two f32 rows must agree to
    F16_TIE_REL of the row's rms in every element; the f16 values that then differ are roundings
    of two such close values to the two sides of a midpoint.  Returns (flips, largest
    |x_or - x_dev| over the row's rms)."""
    x_dev = np.asarray(x_dev, np.float32)
    dev = np.asarray(dev_f16, np.float32).astype(np.float16)
    assert np.array_equal(dev, x_dev.astype(np.float16)), f"{tag}: device row is not its f32 row rounded to f16"
    rms = max(float(np.sqrt(np.mean(x_dev.astype(np.float64) ** 2))), 1e-30)
    gap = float(np.max(np.abs(np.asarray(x_or, np.float64) - x_dev.astype(np.float64)))) / rms
    assert gap <= F16_TIE_REL, f"{tag}: f32 rows {gap:.2e} of the rms apart"
    return int(np.sum(np.asarray(x_or, np.float32).astype(np.float16) != dev)), gap


class FlipStats:
    def __init__(self):
        self.flips, self.tie_dist, self.pre_diff = 0, 0.0, 0.0

    def add(self, r):
        self.flips += r[0]
        self.tie_dist = max(self.tie_dist, r[1])
        self.pre_diff = max(self.pre_diff, r[2])


def _adopt(stats, tag, fmt, n, x_or, dev_q8, dev_x):
    q_or = O.quantize_act(fmt, x_or)
    stats.add(tie_flips(tag, fmt, n, x_or, q_or, dev_x, dev_q8))
    return q8_bytes(fmt, n, dev_q8)


def oracle_step_adopting(t, spec, kv, pos, x, dev_layers, dev_head, qk_norm=True, threads=16, dev_rows=None,
                         om=None):
    """The step's layers (oracle_layers_adopting), then the head adopting the device's head input
    bytes the same way (om given: any head, oracle_head_on).  Returns (logits, FlipStats, f16 flips)."""
    x, st, f16_flips = oracle_layers_adopting(t, spec, kv, pos, x, dev_layers, dev_head, qk_norm, threads, dev_rows)
    eps_ffn = max(spec["eps"], 1e-6)
    xn = O.rmsnorm(x, t["output_norm.weight"][1], eps_ffn)
    if om is None:
        fh = act_fmt(t["output.weight"][0])
        hq = _adopt(st, "head input", fh, spec["hidden"], xn, dev_head["q8_head"], dev_head["xn_head"])
        return _mv(t, "output.weight", hq, threads), st, f16_flips
    name, _, _, target, _ = head_spec(t, spec)
    hq = None
    if name is not None and target > 0 and t[name][0] not in (O.F32, O.F16, O.BF16):
        hq = _adopt(st, "head input", act_fmt(t[name][0]), spec["hidden"], xn, dev_head["q8_head"], dev_head["xn_head"])
    return oracle_head_on(om, t, spec, x, hq, threads)[0], st, f16_flips


def oracle_layers_adopting(t, spec, kv, pos, x, dev_layers, dev_head, qk_norm=True, threads=16, dev_rows=None):
    """The oracle's decode step from hidden state x (the embedding row) and its f32 rings kv,
    adopting the device's activation bytes at each quantization point after tie_flips has
    accounted for every difference, and rotating by the device's RoPE table (check_rope_table
    has bounded its angles by two ulps; the oracle's own powf may differ in the last bit, which
    at position p moves the rotation by up to ~p * 2.4e-7).  dev_rows (f16 rings): per layer
    the device's new (k, v) ring rows; the oracle's own rows, rounded to f16, are accounted
    against them by f16_tie_flips and the device's rows are attended to.  Returns (logits,
    FlipStats, f16 flips) -- here the hidden state after the last layer in place of the logits."""
    H, F = spec["hidden"], spec["ffn"]
    nq, nkv, hd = spec["nq"], spec["nkv"], spec["hd"]
    Q, KV = nq * hd, nkv * hd
    eps, eps_ffn = spec["eps"], max(spec["eps"], 1e-6)
    cap = kv.shape[2]
    slot, active = pos % cap, min(pos + 1, cap)
    st = FlipStats()
    f16_flips = 0
    x = np.asarray(x, np.float32).copy()
    for L, D in enumerate(dev_layers):
        p = f"blk.{L}."
        xn = O.rmsnorm(x, t[p + "attn_norm.weight"][1], eps)
        fq = act_fmt(t[p + "attn_q.weight"][0])
        xq = _adopt(st, f"layer {L} q|k|v input", fq, H, xn, D["q8_attn"], D["xn_attn"])
        fv = act_fmt(t[p + "attn_v.weight"][0])
        xv = xq if fv == fq else O.quantize_act(fv, xn)
        q = _mv(t, p + "attn_q.weight", xq, threads)
        k = _mv(t, p + "attn_k.weight", xq, threads)
        v = _mv(t, p + "attn_v.weight", xv, threads)
        if qk_norm:
            qn, kn = t[p + "attn_q_norm.weight"][1], t[p + "attn_k_norm.weight"][1]
            q = np.concatenate([O.rmsnorm(q[h * hd:(h + 1) * hd], qn, eps) for h in range(nq)])
            k = np.concatenate([O.rmsnorm(k[h * hd:(h + 1) * hd], kn, eps) for h in range(nkv)])
        if "rope_cs" in dev_head:
            q = rotate(q, hd, dev_head["rope_cs"]).astype(np.float32)
            k = rotate(k, hd, dev_head["rope_cs"]).astype(np.float32)
        else:
            q = O.rope(q, hd, pos, spec["theta"])
            k = O.rope(k, hd, pos, spec["theta"])
        if dev_rows is not None:
            for w, (mine, dev32) in enumerate(((k, D["k_rope"]), (v, D["qkv"][Q + KV:]))):
                f16_flips += f16_tie_flips(f"layer {L} {'KV'[w]} row", mine, dev32, dev_rows[L][w])[0]
            k, v = dev_rows[L]
        kv[L, 0, slot], kv[L, 1, slot] = k, v
        att = O.gqa_attention(q, kv[L, 0, :active], kv[L, 1, :active], nq, nkv, hd, active,
                              1.0 / np.sqrt(np.float32(hd)))
        fo = act_fmt(t[p + "attn_output.weight"][0])
        aq = _adopt(st, f"layer {L} wo input", fo, Q, att, D["q8_wo"], D["attn"])
        x = (x + _mv(t, p + "attn_output.weight", aq, threads)).astype(np.float32)
        xn = O.rmsnorm(x, t[p + "ffn_norm.weight"][1], eps_ffn)
        fg = act_fmt(t[p + "ffn_gate.weight"][0])
        fq8 = _adopt(st, f"layer {L} gate|up input", fg, H, xn, D["q8_ffn"], D["xn_ffn"])
        a = O.swiglu(_mv(t, p + "ffn_gate.weight", fq8, threads), _mv(t, p + "ffn_up.weight", fq8, threads))
        fd = act_fmt(t[p + "ffn_down.weight"][0])
        dq8 = _adopt(st, f"layer {L} down input", fd, F, a, D["q8_down"], D["act"])
        x = (x + _mv(t, p + "ffn_down.weight", dq8, threads)).astype(np.float32)
    return x, st, f16_flips


def read_ring(m, L, cap, kvd, kv_f16):
    """Layer L's K and V rings of the device model as f32 [cap][kvd]."""
    import jero_hip as J
    dt = np.float16 if kv_f16 else np.float32
    out = []
    for ptr in m.kv_ptrs(L):
        a = np.empty((cap, kvd), dt)
        J._memcpy(a.ctypes.data, ptr, a.nbytes)
        out.append(a.astype(np.float32))
    return out


def cosine(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def run_traced(m, om, t, spec, kv, cap, pos0, steps, kv_f16, dev, tok, qk_norm=True, threads=16):
    """Decode `steps` tokens from position pos0 on the device with the trace on, and per step:
      1. teacher-forced checks of every layer and of the head (check_layer / check_head);
      2. end to end: the oracle's step from its own state (kv: its f32 rings, kept in step with
         the device's ring type) adopting the device's activation bytes only at accounted tie
         flips (oracle_step_adopting): logits within the north-star 1e-3;
      3. the plain free-running oracle (its own rings, no adoption): within 1e-3 as long as no
         tie flip has occurred (afterwards a flip's ~1e-2 effect propagates through the rings,
         and its error and cosine are reported only);
      4. the greedy token equal to the adopting oracle's whenever its top-2 gap exceeds 1e-2 of
         the rms.
    The oracle follows the device's tokens.  Returns per-step (tie flips, logits error with
    adoption, logits error and cosine of the plain free-running oracle)."""
    import torch
    t = resolve_norms(t, spec, qk_norm)
    L_n = spec["n_layers"]
    kvd = spec["nkv"] * spec["hd"]
    _, _, _, total = m.trace_layout()
    buf = torch.zeros(total, dtype=torch.uint8, device=dev)
    m.set_trace(buf)
    logits = torch.empty(m.logits_len(), dtype=torch.float32, device=dev)
    m.set_position(tok, pos0)
    kv_free = kv.copy()
    om.model.kv_f16 = 1 if kv_f16 else 0  # the plain oracle's rings hold what the device's hold
    flips_so_far = 0
    out = []
    try:
        for i in range(steps):
            pos = pos0 + i
            m.decode_step()
            m.status()
            m.read_logits(logits)
            got = logits.cpu().numpy()
            gtok, gpos = m.read_token_pos()
            assert gpos == pos + 1
            dl, dh = m.read_trace(buf)
            x0 = om.embed(tok)
            assert np.array_equal(dl[0]["x_in"], x0), "embedding row differs"
            check_rope_table(spec, pos, dh["rope_cs"])
            worst = {}
            dev_rows = []
            for L in range(L_n):
                rk, rv = read_ring(m, L, cap, kvd, kv_f16)
                dev_rows.append((rk[pos % cap].copy(), rv[pos % cap].copy()))
                x_next = dl[L + 1]["x_in"] if L + 1 < L_n else dh["x_final"]
                e = check_layer(t, spec, dl[L], L, pos, x_next, rk, rv, kv_f16, qk_norm, threads, dh["rope_cs"])
                for k_, v_ in e.items():
                    worst[k_] = max(worst.get(k_, 0.0), v_)
            eh = check_head(t, spec, dh, got, gtok, threads, om)
            worst["head_gemv"] = eh["gemv"]
            ref, st, f16_flips = oracle_step_adopting(t, spec, kv, pos, x0, dl, dh, qk_norm, threads,
                                                      dev_rows if kv_f16 else None, om)
            free = om.step(kv_free, tok, pos, threads=threads)
            err, cs = rel(got, ref), cosine(got, ref)
            ferr, fcs = rel(got, free), cosine(got, free)
            print(f"  pos {pos}: teacher-forced max errors " +
                  " ".join(f"{k_} {v_:.1e}" for k_, v_ in sorted(worst.items())) +
                  f" | end to end: {st.flips} int8 + {f16_flips} f16 tie flips (farthest {st.tie_dist:.1e} quanta "
                  f"from its boundary, largest pre-rounding difference {st.pre_diff:.1e}), logits rel err {err:.2e}"
                  f" | free-running oracle: rel err {ferr:.2e} cos {fcs:.8f}", flush=True)
            assert err <= 1e-3, (pos, err)
            flips_so_far += st.flips + f16_flips
            if flips_so_far == 0:  # no tie flip yet: the plain oracle has seen the same int8s
                assert ferr <= 1e-3, (pos, ferr)
            top2 = np.sort(ref.astype(np.float64))[-2:]
            scale = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
            if top2[1] - top2[0] > 1e-2 * scale:
                assert gtok == O.argmax(ref), (pos, gtok, O.argmax(ref))
            out.append((st.flips + f16_flips, err, ferr, fcs))
            tok = gtok
    finally:
        m.set_trace(None)
    return out


def run_prefill_traced(m, om, t, spec, kv, cap, pos0, tokens, kv_f16, dev, qk_norm=True, threads=16):
    """jero_hip_model_prefill of `tokens` from position pos0 with the trace on.  Prefill writes
    token i's trace in the decode step's layout, so every prompt token is held to the decode
    step's bars: teacher-forced checks of every layer (check_layer, attention over the ring up to
    its own position); end to end, the oracle's token loop (run_prefill_with_hidden) adopting the
    device's activation bytes only at accounted tie flips, each token's final hidden state within
    1e-3 and, on the last token, the head checks and the logits within 1e-3.  kv: the oracle's f32
    rings, advanced in step.  Returns (greedy token, per-token (tie flips, hidden/logits error))."""
    import torch
    t = resolve_norms(t, spec, qk_norm)
    L_n = spec["n_layers"]
    kvd = spec["nkv"] * spec["hd"]
    n = len(tokens)
    _, _, _, total = m.trace_layout()
    buf = torch.zeros(n * total, dtype=torch.uint8, device=dev)
    m.set_trace(buf)
    try:
        m.prefill(tokens, pos0)
        m.status()
    finally:
        m.set_trace(None)
    logits = torch.empty(m.logits_len(), dtype=torch.float32, device=dev)
    m.read_logits(logits)
    got = logits.cpu().numpy()
    gtok, gpos = m.read_token_pos()
    assert gpos == pos0 + n
    rings = [read_ring(m, L, cap, kvd, kv_f16) for L in range(L_n)]
    out = []
    for i, tok in enumerate(tokens):
        pos = pos0 + i
        dl, dh = m.read_trace(buf[i * total:(i + 1) * total])
        x0 = om.embed(tok)
        assert np.array_equal(dl[0]["x_in"], x0), ("embedding row differs", i)
        check_rope_table(spec, pos, dh["rope_cs"])
        dev_rows = []
        worst = {}
        for L in range(L_n):
            rk, rv = rings[L]
            dev_rows.append((rk[pos % cap].copy(), rv[pos % cap].copy()))
            x_next = dl[L + 1]["x_in"] if L + 1 < L_n else dh["x_final"]
            e = check_layer(t, spec, dl[L], L, pos, x_next, rk, rv, kv_f16, qk_norm, threads, dh["rope_cs"])
            for k_, v_ in e.items():
                worst[k_] = max(worst.get(k_, 0.0), v_)
        last = i == n - 1
        if last:
            eh = check_head(t, spec, dh, got, gtok, threads, om)
            worst["head_gemv"] = eh["gemv"]
            ref, st, f16_flips = oracle_step_adopting(t, spec, kv, pos, x0, dl, dh, qk_norm, threads,
                                                      dev_rows if kv_f16 else None, om)
            err = rel(got, ref)
        else:
            xo, st, f16_flips = oracle_layers_adopting(t, spec, kv, pos, x0, dl, dh, qk_norm, threads,
                                                       dev_rows if kv_f16 else None)
            err = rel(dh["x_final"], xo)
        print(f"  prefill token {i} (pos {pos}): teacher-forced max errors " +
              " ".join(f"{k_} {v_:.1e}" for k_, v_ in sorted(worst.items())) +
              f" | end to end: {st.flips} int8 + {f16_flips} f16 tie flips, "
              f"{'logits' if last else 'hidden state'} rel err {err:.2e}", flush=True)
        assert err <= 1e-3, (i, err)
        out.append((st.flips + f16_flips, err))
    ref_top = np.sort(ref.astype(np.float64))[-2:]
    if ref_top[1] - ref_top[0] > 1e-2 * np.sqrt(np.mean(ref.astype(np.float64) ** 2)):
        assert gtok == O.argmax(ref), (gtok, O.argmax(ref))
    return gtok, out
