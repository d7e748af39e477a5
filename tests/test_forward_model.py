"""Pins the oracle's restatement of the synthetic int8 ForwardModel (src/forward.rs:834-1075)
and checks the device entry points' argument errors (no GPU needed).

The reference's tests hold no golden tokens for ForwardModel, so each piece is held to something
other than its own formula: SplitMix64's published outputs, math.isqrt, closed forms of the
integer RMSNorm and attention, brute force in exact Python integers on small cases, and
invariants of the whole pass (a prompt's forward equals the same tokens fed one at a time; the
evaluate loop equals forward + sample; weights are deterministic in the seed).
"""
import ctypes as C
import math

import numpy as np
import pytest

import pyoracle as O

GOLDEN = 0x9E3779B97F4A7C15
MASK = (1 << 64) - 1


def fnv1a(text):
    """The matrix bench's model seed (src/bin/jero-diag/bench.rs:1142-1147)."""
    h = 0xCBF29CE484222325
    for b in text.encode():
        h = ((h ^ b) * 0x100000001B3) & MASK
    return h


# ---------------------------------------------------------------- splitmix, fill_small, isqrt

def test_splitmix_published_outputs():
    # SplitMix64 (Steele, Lea, Flood 2014; Vigna's splitmix64.c): the generator seeded with s
    # returns splitmix(s + k * golden) for k = 0, 1, ...  Published first outputs:
    assert O.splitmix(0) == 0xE220A8397B1DCDAF
    seq = [O.splitmix((1234567 + k * GOLDEN) & MASK) for k in range(5)]
    assert seq == [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
                   16408922859458223821]


def test_fill_small_range_uniformity_and_seed_dependence():
    a = O.fill_small(42, 1 << 16)
    assert a.min() == -8 and a.max() == 7
    counts = np.bincount(a.astype(np.int64) + 8, minlength=16)
    assert counts.min() > 0.9 * (1 << 12) and counts.max() < 1.1 * (1 << 12)
    # element i hashes seed ^ i * C alone: a prefix is the shorter fill
    assert (O.fill_small(42, 100) == a[:100]).all()
    assert (O.fill_small(43, 100) != a[:100]).any()
    # the low nibble of splitmix, recentred (checked on the published splitmix(0) output)
    assert int(O.fill_small(0, 1)[0]) == (0xE220A8397B1DCDAF & 0xF) - 8


def test_isqrt_is_floor_sqrt():
    for v in range(0, 70000):
        assert O.isqrt(v) == math.isqrt(v)
    rng = np.random.default_rng(1)
    for v in list(rng.integers(0, 1 << 63, 2000, dtype=np.int64)) + [MASK, MASK - 1, (1 << 32) ** 2 - 1, 1 << 62]:
        v = int(v) & MASK
        assert O.isqrt(v) == math.isqrt(v)


def test_device_integer_shortcuts_are_exact():
    """The device RMSNorm replaces isqrt's Newton loop and the per-element division by cheaper
    exact forms; both claims are checked here over their whole domain."""
    # floor(sqrt(v)) from any root within one of it, by one correction each way, over the mean
    # squares a row can have (v <= 128^2) and well beyond
    v = np.arange(0, 1 << 20, dtype=np.int64)
    root = np.array([math.isqrt(int(x)) for x in v], np.int64)
    for off in (-1, 0, 1):
        r = np.maximum(root + off, 0)
        r = np.where(r * r > v, r - 1, r)
        r = np.where((r + 1) * (r + 1) <= v, r + 1, r)
        assert (r == root).all(), off
    # |a| / d for |a| <= 6144 = 128 * 48 and 2 <= d <= 128: the high word of |a| * ceil(2^32 / d)
    a = np.arange(0, 6145, dtype=np.uint64)
    for d in range(2, 129):
        mul = np.uint64(0xFFFFFFFF // d + 1)
        assert ((a * mul) >> np.uint64(32) == a // np.uint64(d)).all(), d


# ---------------------------------------------------------------- rmsnorm

def test_rmsnorm_closed_forms():
    rows = []
    for v in (1, -1, 5, -77, 127, -128):
        rows.append(np.full(512, v, np.int8))                       # rms = |v|: y = sign(v) 48
        rows.append(np.tile(np.array([v, -v], np.int64), 256).clip(-128, 127).astype(np.int8))
    rows.append(np.zeros(512, np.int8))                              # rms = max(0, 1): y = 0
    x = np.stack(rows)
    y = O.fwd_rmsnorm(x)
    for r in range(len(rows) - 1):
        nz = x[r] != 0
        exp = np.sign(x[r][nz].astype(np.int64)) * 48
        assert (y[r][nz] == exp).all(), r
    assert (y[-1] == 0).all()


def test_rmsnorm_truncates_toward_zero():
    # half the row at a, half zero: ms = a^2 / 2, rms = isqrt(a^2 // 2); y = a * 48 / rms truncated
    for a in (100, -100, 37, -37, 3, -3):
        x = np.array([a] * 256 + [0] * 256, np.int8)
        rms = max(math.isqrt(a * a * 256 // 512), 1)
        q = abs(a) * 48 // rms
        exp = min(q, 127) * (1 if a > 0 else -1)
        assert int(O.fwd_rmsnorm(x)[0][0]) == exp
    # a = -100: 4800 / 70 = 68.57 -> -68 (floor division would give -69)
    assert int(O.fwd_rmsnorm(np.array([-100] * 256 + [0] * 256, np.int8))[0][0]) == -68


def test_rmsnorm_brute_force():
    rng = np.random.default_rng(5)
    x = rng.integers(-128, 128, (6, 512)).astype(np.int8)
    y = O.fwd_rmsnorm(x)
    for r in range(6):
        row = [int(v) for v in x[r]]
        rms = max(math.isqrt(sum(v * v for v in row) // 512), 1)
        exp = [max(-127, min(127, (1 if v >= 0 else -1) * (abs(v) * 48 // rms))) for v in row]  # truncation
        assert [int(v) for v in y[r]] == exp


# ---------------------------------------------------------------- attention

def _attention_brute(q, kc, vc, start_pos):
    out = []
    for r in range(q.shape[0]):
        pos = start_pos + r
        acc = [0] * 512
        tot = 0
        qr = [int(v) for v in q[r]]
        for t in range(pos + 1):
            s = sum(a * int(b) for a, b in zip(qr, kc[t]))
            w = min(max(s >> 10, 0), 127) + 1
            tot += w
            for i in range(512):
                acc[i] += w * int(vc[t][i])
        out.append([(1 if a >= 0 else -1) * (abs(a) // tot) for a in acc])  # truncation toward zero
    return np.array(out, np.int64)


def test_attention_closed_forms():
    rng = np.random.default_rng(7)
    v = rng.integers(-127, 128, (1, 512)).astype(np.int8)
    k = rng.integers(-127, 128, (1, 512)).astype(np.int8)
    q = rng.integers(-127, 128, (1, 512)).astype(np.int8)
    # one position: sum(w v) / w = v whatever the score
    assert (O.fwd_attention(q, k, v, 0) == v).all()
    # zero query: every weight is 1, the output is the truncated mean of the cached v rows
    vs = rng.integers(-127, 128, (5, 512)).astype(np.int8)
    ks = rng.integers(-127, 128, (5, 512)).astype(np.int8)
    got = O.fwd_attention(np.zeros((1, 512), np.int8), ks, vs, 4)[0].astype(np.int64)
    s = vs.astype(np.int64).sum(0)
    assert (got == np.trunc(s / 5).astype(np.int64)).all()
    # saturated score (q . k >= 128 * 1024) weighs 128 against 1
    k2 = np.zeros((2, 512), np.int8)
    k2[1, :] = 127
    q2 = np.full((1, 512), 127, np.int8)
    v2 = np.stack([np.full(512, -127, np.int8), np.full(512, 127, np.int8)])
    exp = int((-127 * 1 + 127 * 128) / 129)
    assert (O.fwd_attention(q2, k2, v2, 1) == exp).all()


def test_attention_brute_force_causal():
    rng = np.random.default_rng(9)
    kc = rng.integers(-40, 41, (7, 512)).astype(np.int8)
    vc = rng.integers(-127, 128, (7, 512)).astype(np.int8)
    q = rng.integers(-40, 41, (3, 512)).astype(np.int8)
    got = O.fwd_attention(q, kc, vc, 4)  # rows at positions 4, 5, 6
    assert (got.astype(np.int64) == _attention_brute(q, kc, vc, 4)).all()


# ---------------------------------------------------------------- the model

def test_weights_shapes_padding_and_seeds():
    f = O.ForwardModel(11, 5, 8)
    assert f.head_rows == 8
    head, sh = f.weight(-1)
    assert head.shape == (8, 512) and sh == 6
    assert (head[5:] == 0).all() and (head[:5].reshape(-1) == O.fill_small(O.splitmix(11 ^ 0xFFFF), 5 * 512)).all()
    for l in range(4):
        for j, (n, k) in enumerate([(512, 512)] * 4 + [(1024, 512), (512, 1024)]):
            w, sh = f.weight(l, j)
            assert w.shape == (n, k) and sh == (7 if j == 5 else 6)
            if l in (0, 3):
                assert (w.reshape(-1) == O.fill_small(O.splitmix(11 ^ (16 * l + j + 1)), n * k)).all()
    assert O.ForwardModel(0, 0, 4).head_rows == 8  # vocab.max(1) rows, padded


def test_embed_is_scaled_fill_small():
    e = O.fwd_embed(99, 7)
    assert (e == O.fill_small(99 ^ (7 * 0x9E3779B9), 512) * 8).all()
    assert set(np.unique(e) % 8) == {0}


def test_sample_first_maximum():
    assert O.fwd_sample(np.array([1, 5, 5, 2], np.int32), 4) == 1
    assert O.fwd_sample(np.array([1, 5, 5, 9], np.int32), 3) == 1  # only the first vocab logits
    assert O.fwd_sample(np.array([-3, -3], np.int32), 2) == 0
    assert O.fwd_sample(np.array([7], np.int32), 0) == 0


def test_prompt_forward_equals_token_by_token():
    prompt = [104, 101, 108, 108, 111, 32, 119]
    a = O.ForwardModel(fnv1a("hello world"), 256, 16)
    whole = a.forward(prompt, 0)
    b = O.ForwardModel(fnv1a("hello world"), 256, 16)
    for i, t in enumerate(prompt):
        last = b.forward([t], i)
    assert (whole == last).all()
    # and the cache state carries on identically
    assert (a.forward([3], len(prompt)) == b.forward([3], len(prompt))).all()
    # two chunks
    c = O.ForwardModel(fnv1a("hello world"), 256, 16)
    c.forward(prompt[:3], 0)
    assert (c.forward(prompt[3:], 3) == whole).all()


@pytest.mark.parametrize("threads", [2, 5, 16])
def test_pooled_threads_equal_one_thread(threads):
    """The persistent worker pool splits every projection, the attention rows and the head over
    `threads` ranges (more threads than rows of a 3-token prompt's attention included): prompt
    logits, decode logits and a 40-token evaluate equal the one-thread run's."""
    seed, prompt = fnv1a("hello world"), [104, 101, 108]
    one = O.ForwardModel(seed, 256, 64)
    many = O.ForwardModel(seed, 256, 64, threads=threads)
    assert (one.forward(prompt, 0) == many.forward(prompt, 0)).all()
    for i, t in enumerate([7, 255, 0]):
        assert (one.forward([t], 3 + i) == many.forward([t], 3 + i)).all()
    one.reset(), many.reset()
    assert one.evaluate(list(b"hello world"), 40) == many.evaluate(list(b"hello world"), 40)
    many.close()
    many.close()


def test_forward_rejects_wrong_start_and_capacity():
    f = O.ForwardModel(1, 16, 4)
    with pytest.raises(ValueError):
        f.forward([1], 1)
    f.forward([1, 2], 0)
    with pytest.raises(ValueError):
        f.forward([3, 4, 5], 2)


def test_evaluate_is_forward_then_greedy_loop():
    seed, vocab = fnv1a("hello world"), 256
    prompt = list(b"hello world")
    got = O.ForwardModel(seed, vocab, 64).evaluate(prompt, 10)
    f = O.ForwardModel(seed, vocab, 64)
    logits = f.forward(prompt, 0)
    toks = [O.fwd_sample(logits, vocab)]
    while len(toks) < 10:
        logits = f.forward([toks[-1]], len(prompt) + len(toks) - 1)
        toks.append(O.fwd_sample(logits, vocab))
    assert got == toks
    assert O.ForwardModel(seed, vocab, 64).evaluate(prompt, 0) == []
    with pytest.raises(ValueError):
        O.ForwardModel(seed, vocab, 64).evaluate([], 4)
    with pytest.raises(ValueError):
        O.ForwardModel(seed, vocab, 12).evaluate(prompt, 3)  # 11 + 2 positions > 12


def test_logits_exact_int32_magnitudes():
    """Logits are exact int32 sums: bounded by 512 * 127 * 8 and varied across the vocabulary."""
    f = O.ForwardModel(fnv1a("hello world"), 256, 16)
    l = f.forward(list(b"hello"), 0)
    assert l.dtype == np.int32 and np.abs(l).max() <= 512 * 127 * 8
    assert len(np.unique(l)) > 100


# ---------------------------------------------------------------- device entry points, no GPU needed

def test_forward_model_argument_errors():
    import jero_hip as J
    L = J.lib()
    BOUNDS, INVALID = 14, 21  # TensorBoundsError, InvalidArgument
    assert J.STATUS_NAMES[BOUNDS] == "TensorBoundsError" and J.STATUS_NAMES[INVALID] == "InvalidArgument"
    h = C.c_void_p()
    assert L.jero_hip_forward_model_create(C.c_uint64(1), -1, 64, C.byref(h)) == BOUNDS
    assert L.jero_hip_forward_model_create(C.c_uint64(1), 256, 0, C.byref(h)) == BOUNDS
    assert L.jero_hip_forward_model_create(C.c_uint64(1), 256, 1 << 23, C.byref(h)) == BOUNDS
    assert L.jero_hip_forward_model_create(C.c_uint64(1), 256, 64, None) == INVALID
    logits = C.c_void_p(16)
    toks = (C.c_uint32 * 2)(1, 2)
    assert L.jero_hip_forward_model_forward(None, toks, 2, 0, logits, None) == INVALID
    assert L.jero_hip_forward_model_evaluate(None, toks, 2, 4, toks, None, None) == INVALID
    assert L.jero_hip_forward_model_reset(None) == INVALID
    assert L.jero_hip_forward_model_head_rows(None) == -1
    assert L.jero_hip_forward_model_positions(None) == -1
    assert L.jero_hip_forward_model_destroy(None) == 0
