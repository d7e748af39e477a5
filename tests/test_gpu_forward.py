"""GPU parity of the synthetic int8 ForwardModel (src/forward.rs:834-1075) against the oracle.

Everything is integer arithmetic, so the bar is bit-exact: the generated weights byte for byte,
every head row's int32 logit after every forward call, and the generated token ids.  The calls
cover the matvec path (up to 64 token rows per call), the int8 MFMA path (longer prompts), chunked
prefills at start_pos > 0, vocabularies with padded head rows, token ids beyond the vocabulary,
attention past one LDS pass of cache positions, and the argument errors."""
import os

import numpy as np
import pytest
import torch

import jero_hip as J
import pyoracle as O

pytestmark = pytest.mark.gpu

MASK = (1 << 64) - 1


def fnv1a(text):
    """The matrix bench's model seed (src/bin/jero-diag/bench.rs:1142-1147)."""
    h = 0xCBF29CE484222325
    for b in text.encode():
        h = ((h ^ b) * 0x100000001B3) & MASK
    return h


SEED = fnv1a("hello world")
PROMPT = list(b"hello world")
THREADS = min(16, os.cpu_count() or 1)


def dev_bytes(ptr, n):
    t = torch.empty(n, dtype=torch.int8)
    J._memcpy(t.data_ptr(), ptr, n)
    return t.numpy()


def gpu_forward(g, tokens, start, dev):
    logits = torch.empty(g.head_rows, dtype=torch.int32, device=dev)
    g.forward(tokens, start, logits)
    torch.cuda.synchronize()
    return logits.cpu().numpy()


def test_weights_bit_exact(dev):
    g = J.ForwardModel(SEED, 256, 64)
    o = O.ForwardModel(SEED, 256, 64)
    for layer in [-1, 0, 1, 2, 3]:
        for which in range(6 if layer >= 0 else 1):
            ptr, n, k, sh = g.weight(layer, which)
            w, osh = o.weight(layer, which)
            assert (n, k) == w.shape and sh == osh
            assert np.array_equal(dev_bytes(ptr, n * k).reshape(n, k), w), (layer, which)
    g.close()


@pytest.mark.parametrize("vocab", [0, 1, 5, 256, 1000])
def test_prompt_then_decode_steps(dev, vocab):
    print(f"forward prompt + steps vocab={vocab}", flush=True)
    seed = SEED ^ vocab
    g = J.ForwardModel(seed, vocab, 64)
    o = O.ForwardModel(seed, vocab, 64, threads=THREADS)
    assert g.head_rows == o.head_rows
    lg = gpu_forward(g, PROMPT, 0, dev)
    lo = o.forward(PROMPT, 0)
    assert np.array_equal(lg, lo)
    tok = O.fwd_sample(lo, vocab)
    for i in range(12):
        pos = len(PROMPT) + i
        lg = gpu_forward(g, [tok], pos, dev)
        lo = o.forward([tok], pos)
        assert np.array_equal(lg, lo), f"step {i}"
        tok = O.fwd_sample(lo, vocab)
    assert g.positions == len(PROMPT) + 12
    g.close()


@pytest.mark.parametrize("chunks", [[64], [65], [3, 61, 1], [11, 100, 2], [130, 64]])
def test_chunked_prefill(dev, chunks):
    """Up to 64 rows per call the matvec kernel runs; longer calls the int8 MFMA GEMM."""
    print(f"forward chunks={chunks}", flush=True)
    rng = np.random.default_rng(sum(chunks))
    total = sum(chunks)
    toks = rng.integers(0, 1 << 32, total, dtype=np.uint64).astype(np.uint32)  # ids past the vocabulary
    toks[:3] = [0, 0xFFFFFFFF, 255]
    g = J.ForwardModel(SEED, 256, total + 1)
    o = O.ForwardModel(SEED, 256, total + 1, threads=THREADS)
    start = 0
    for c in chunks:
        part = toks[start:start + c]
        assert np.array_equal(gpu_forward(g, part, start, dev), o.forward(part, start)), f"chunk at {start}"
        start += c
    g.close()


def test_evaluate_matrix_bench_workload(dev):
    """The matrix bench's default run: prompt "hello world" as bytes, vocab 256, n_ctx 64, so
    53 generated tokens (src/bin/jero-diag/bench.rs:1125-1148)."""
    g = J.ForwardModel(SEED, 256, 64)
    toks, (pre_ms, dec_ms) = g.evaluate(PROMPT, 53, timing=True)
    assert toks == O.ForwardModel(SEED, 256, 64).evaluate(PROMPT, 53)
    assert pre_ms > 0 and dec_ms > 0
    assert g.positions == len(PROMPT) + 52
    # a second evaluate starts from an empty cache and repeats itself (the decode steps replay the
    # graph recorded by the first); another shape records a new one, and the first comes back
    assert g.evaluate(PROMPT, 53) == toks
    short = O.ForwardModel(SEED, 256, 64).evaluate(PROMPT[:5], 20)
    assert g.evaluate(PROMPT[:5], 20) == short
    assert g.evaluate(PROMPT[:5], 20) == short
    assert g.evaluate(PROMPT, 53) == toks
    assert g.evaluate(PROMPT, 1) == toks[:1]
    assert g.evaluate(PROMPT, 0) == [] and g.positions == len(PROMPT)
    g.close()


@pytest.mark.parametrize("seed,vocab,n,max_tokens", [(7, 1000, 40, 30), (123456789, 3, 1, 20), (0, 256, 80, 16)])
def test_evaluate_matches_oracle(dev, seed, vocab, n, max_tokens):
    print(f"evaluate seed={seed} vocab={vocab} n={n} max_tokens={max_tokens}", flush=True)
    prompt = np.random.default_rng(seed).integers(0, max(vocab, 1), n).tolist()
    g = J.ForwardModel(seed, vocab, n + max_tokens)
    o = O.ForwardModel(seed, vocab, n + max_tokens, threads=THREADS)
    assert g.evaluate(prompt, max_tokens) == o.evaluate(prompt, max_tokens)
    g.close()


def test_attention_past_one_lds_pass(dev):
    """Positions beyond 4096 take a second pass of the attention kernel's position loop."""
    n = 4150
    toks = (np.arange(n, dtype=np.uint32) * 2654435761) & 0xFFFF
    g = J.ForwardModel(SEED, 256, n + 4)
    o = O.ForwardModel(SEED, 256, n + 4, threads=THREADS)
    assert np.array_equal(gpu_forward(g, toks[:4000], 0, dev), o.forward(toks[:4000], 0))
    assert np.array_equal(gpu_forward(g, toks[4000:], 4000, dev), o.forward(toks[4000:], 4000))
    for i in range(3):
        assert np.array_equal(gpu_forward(g, [i], n + i, dev), o.forward([i], n + i)), i
    g.close()


def test_argument_errors(dev):
    g = J.ForwardModel(SEED, 256, 16)
    logits = torch.empty(g.head_rows, dtype=torch.int32, device=dev)
    with pytest.raises(J.K3Error) as e:
        g.forward([1], 3, logits)
    assert e.value.variant == "InvalidArgument"
    g.forward([1, 2, 3], 0, logits)
    with pytest.raises(J.K3Error) as e:
        g.forward(list(range(14)), 3, logits)
    assert e.value.variant == "ContextLengthExceeded"
    with pytest.raises(J.K3Error) as e:
        g.evaluate([], 4)
    assert e.value.variant == "CapabilityMismatch"
    with pytest.raises(J.K3Error) as e:
        g.evaluate(list(range(10)), 8)  # 10 + 7 positions > 16
    assert e.value.variant == "ContextLengthExceeded"
    g.reset()
    assert g.positions == 0
    g.forward([5], 0, logits)
    torch.cuda.synchronize()
    o = O.ForwardModel(SEED, 256, 16)
    assert np.array_equal(logits.cpu().numpy(), o.forward([5], 0))
    g.close()
