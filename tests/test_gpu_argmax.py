"""The device argmax (jero_hip_argmax, the LM-head epilogue's reduction) on the reference's own
known-answer cases for sample_greedy_argmax / argmax_f32
(test_sample_greedy_argmax_large_vocab_parity_ties_nan_and_inf, src/engine.rs:2677-2727), and
the decode step failing closed on all-NaN logits (test_engine_fails_closed_on_all_nan_logits,
src/engine.rs:2729; the engine's error at src/engine.rs:636-641)."""
import numpy as np
import pytest
import torch

import jero_hip as J
import model_spec as MS
import pyoracle as O

pytestmark = pytest.mark.gpu


def dev_argmax(dev, vals):
    x = torch.tensor(np.asarray(vals, np.float32), device=dev)
    return J.sample_greedy_argmax(x)


def test_argmax_reference_kats(dev):
    print("argmax kats", flush=True)
    nan, inf = float("nan"), float("inf")
    assert dev_argmax(dev, []) is None
    assert dev_argmax(dev, [nan] * 1024) is None
    assert dev_argmax(dev, [nan, 3.5, nan, 2.0]) == 1
    assert dev_argmax(dev, [-inf, -inf]) == 0
    for vocab_len in (32_768, 65_537, 256_000):
        all_neg = (-100.0 - (np.arange(vocab_len) % 97)).astype(np.float32)
        peak = vocab_len - 17
        all_neg[peak] = -0.25
        all_neg[0] = -inf
        assert dev_argmax(dev, all_neg) == peak, vocab_len
        ties = np.full(vocab_len, 1.25, np.float32)
        first_tie, second_tie = 103, vocab_len // 2 + 11
        ties[0] = nan
        ties[first_tie] = 42.5
        ties[second_tie] = 42.5
        ties[vocab_len - 1] = nan
        assert dev_argmax(dev, ties) == first_tie, vocab_len
        assert O.argmax(ties) == first_tie


def test_argmax_random_against_oracle(dev):
    """Random vectors with duplicated maxima and NaN runs at sizes around the partial chunking."""
    print("argmax random", flush=True)
    rng = np.random.default_rng(5)
    for n in (1, 63, 64, 1000, 8191, 8192, 8193, 151_936, 1 << 20, 9_000_001):
        x = rng.integers(-50, 50, size=n).astype(np.float32)  # many exact ties
        x[rng.integers(0, n, size=max(1, n // 7))] = np.nan
        assert dev_argmax(dev, x) == O.argmax(x), n


def test_decode_fails_closed_on_all_nan_logits(dev):
    """An LM head whose Q6_K scales are NaN gives all-NaN logits: the step stores token -1, keeps
    the position and reports CapabilityMismatch; replays stay closed until a new position is
    set, after which a sound model decodes again."""
    print("decode all-NaN logits", flush=True)
    spec = dict(hidden=256, ffn=512, n_layers=1, vocab=300, nq=4, nkv=2, hd=64, eps=1e-6, theta=1e6)
    t = MS.build(spec, seed=21)
    q, arr, n_in, n_out = t["output.weight"]
    bad = arr.copy().reshape(n_out, -1, 210)
    bad[:, :, 208:210] = np.frombuffer(np.float16(np.nan).tobytes(), np.uint8)
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], 32, J.KV_F16, True)
    for name, (qq, a, ni, no) in t.items():
        m.set_tensor(name, qq, bad.reshape(-1) if name == "output.weight" else a, ni, no)
    m.finalize()
    m.set_position(7, 3)
    m.status()
    m.decode_step()
    with pytest.raises(J.K3Error) as ei:
        m.status()
    assert ei.value.variant == "CapabilityMismatch" and "all-NaN" in str(ei.value)
    assert m.read_token_pos() == (-1, 3)
    m.decode_step()
    m.decode_step()
    assert m.read_token_pos() == (-1, 3)
    with pytest.raises(J.K3Error):
        m.status()
    m.set_position(7, 3)
    m.status()  # cleared
    m.close()
    good = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                         spec["hd"], spec["eps"], spec["theta"], 32, J.KV_F16, True)
    for name, (qq, a, ni, no) in t.items():
        good.set_tensor(name, qq, a, ni, no)
    good.finalize()
    good.set_position(7, 3)
    good.decode_step()
    good.status()
    tok, pos = good.read_token_pos()
    assert 0 <= tok < spec["vocab"] and pos == 4
    good.close()
