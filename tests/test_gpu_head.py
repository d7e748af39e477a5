"""GPU parity of the LM head, embedding and norm-weight branches of the decode step:
project_lm_head (src/qwen_deepseek.rs:584-632) with infer_logits_buffer_len (src/engine.rs:1781-1792),
embed_token (:558-582) and read_f32_weight_or_default (:491-519).

Each model decodes under decode_parity.run_traced: every layer teacher-forced against the oracle,
the head checked over whatever form it takes (rows past a short head, a padded head, a head read
as rows of hidden, an f32-input head, the tanh fallback), end to end within 1e-3 with tie flips
accounted, and the greedy token over all logits.  The oracle's versions of these branches are
pinned on the CPU (tests/test_oracle.py)."""
import numpy as np
import pytest
import torch

import decode_parity as DP
import jero_hip as J
import model_spec as MS
import pyoracle as O
from qdata import rand_float_weights, rand_weights
from test_gpu_decode import make_gpu_model, prefill_kv

pytestmark = pytest.mark.gpu

SPEC = dict(hidden=256, ffn=512, n_layers=2, vocab=320, nq=4, nkv=2, hd=64, eps=1e-6, theta=1e6)


def zero_rows(quant, rows, k):
    """rows x k weights of `quant` whose every value is 0 (zero scales)."""
    return np.zeros(rows * J.row_bytes(quant, k), np.uint8)


def run_model(dev, tensors, cap=64, prefill=20, steps=3, tok=5, qk_norm=True, want_len=None):
    spec = SPEC
    m = make_gpu_model(spec, tensors, cap, J.KV_F16, qk_norm)
    host = {k: v for k, v in tensors.items()}
    om = O.DecodeModel(spec, host, cap, qk_norm=qk_norm)
    assert m.logits_len() == om.logits_len
    if want_len is not None:
        assert m.logits_len() == want_len
    kv = prefill_kv(m, om, spec, cap, prefill, 13, dev)
    DP.run_traced(m, om, tensors, spec, kv, cap, prefill, steps, True, dev, tok, qk_norm)
    m.close()


def base_tensors(seed=31):
    return MS.build(SPEC, seed=seed)


def test_head_padded_rows(dev):
    """A Q6_K head of vocab + 64 rows (384, a multiple of 64): 384 logits, the padding rows zero."""
    print("head padded", flush=True)
    t = base_tensors()
    H = SPEC["hidden"]
    q, w, n_in, n_out = t["output.weight"]
    t["output.weight"] = (q, np.concatenate([w, zero_rows(q, 64, H)]), H, 384)
    run_model(dev, t, want_len=384)


@pytest.mark.parametrize("quant", [J.Q6_K, J.Q8_0, J.F16])
def test_head_short_rows(dev, quant):
    """A head of 100 rows for a vocabulary of 320: logits 100 .. 319 are xn[i % hidden] * 0.05
    (wrapping past hidden = 256); quantized heads run the GEMV over 100 rows then the slice, an F16
    head the f32-input GEMV."""
    print(f"head short quant={quant}", flush=True)
    t = base_tensors(33)
    H = SPEC["hidden"]
    w = rand_float_weights(quant, 100, H, 34) if quant == J.F16 else rand_weights(quant, 100, H, 34)
    t["output.weight"] = (quant, w, H, 100)
    run_model(dev, t, want_len=320)


@pytest.mark.parametrize("quant", [J.Q6_K, J.F32])
def test_head_read_as_rows_of_hidden(dev, quant):
    """A head given as [2 hidden, vocab / 2] (the same elements): read as vocab rows of hidden."""
    print(f"head reshaped quant={quant}", flush=True)
    t = base_tensors(35)
    H, V = SPEC["hidden"], SPEC["vocab"]
    w = rand_float_weights(quant, V, H, 36) if quant == J.F32 else rand_weights(quant, V, H, 36)
    t["output.weight"] = (quant, w, 2 * H, V // 2)
    run_model(dev, t, want_len=V)


def test_head_float_padded(dev):
    """An F16 head of 384 rows: an f32-input head over all logits."""
    print("head f16 padded", flush=True)
    t = base_tensors(37)
    H = SPEC["hidden"]
    t["output.weight"] = (J.F16, rand_float_weights(J.F16, 384, H, 38), H, 384)
    run_model(dev, t, want_len=384)


def test_head_tied_to_embedding(dev):
    """No output.weight: the head is token_embd.weight (ModelWeights' tied fallback); the logits
    equal those of output.weight = token_embd.weight, bit for bit."""
    print("head tied", flush=True)
    t = base_tensors(39)
    tied = {k: v for k, v in t.items() if k != "output.weight"}
    run_model(dev, tied)
    explicit = dict(tied, **{"output.weight": t["token_embd.weight"]})
    outs = []
    for tensors in (tied, explicit):
        m = make_gpu_model(SPEC, tensors, 64, J.KV_F16, True)
        m.set_position(9, 0)
        lg = torch.empty(m.logits_len(), dtype=torch.float32, device=dev)
        seq = []
        for _ in range(3):
            m.decode_step()
            m.status()
            m.read_logits(lg)
            seq.append(lg.cpu().numpy().copy())
        outs.append(np.stack(seq))
        m.close()
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_no_head_no_embedding(dev):
    """Neither output.weight nor token_embd.weight: every token embeds as the deterministic row
    and every logit is tanh(sum(xn) / 16) + xn[i % hidden] * 0.1 + (i % 13) * 0.01."""
    print("no head, no embedding", flush=True)
    t = {k: v for k, v in base_tensors(41).items() if k not in ("output.weight", "token_embd.weight")}
    run_model(dev, t, want_len=SPEC["vocab"])


def test_tokens_past_the_embedding_rows(dev):
    """token_embd.weight of 200 rows for a vocabulary of 320: tokens 200 and up embed as the
    deterministic row (a prompt token of 250 and of 2^31 - 1, then the greedy tokens)."""
    print("tokens past the embedding", flush=True)
    t = base_tensors(43)
    H = SPEC["hidden"]
    q, w, _, _ = t["token_embd.weight"]
    t["token_embd.weight"] = (q, w[:200 * J.row_bytes(q, H)], H, 200)
    run_model(dev, t, tok=250)
    run_model(dev, t, tok=2 ** 31 - 1, steps=1)


def test_norm_weights_as_read(dev):
    """read_f32_weight_or_default on the device: attention / FFN / QK / output norms absent (all
    ones), F16, Q8_0 (dequantized), F32 with NaN and inf entries (1.0 in their place) and an F32
    k-norm of 40 of its 64 values (1.0 past them)."""
    print("norm weights", flush=True)
    t = base_tensors(45)
    H, hd = SPEC["hidden"], SPEC["hd"]
    for name in ("blk.0.attn_norm.weight", "blk.1.attn_q_norm.weight", "output_norm.weight"):
        del t[name]
    h = t["blk.0.ffn_norm.weight"][1].astype(np.float16)
    t["blk.0.ffn_norm.weight"] = (J.F16, h.view(np.uint8), H, 1)
    rng = np.random.default_rng(46)
    q = np.zeros((H // 32, 34), np.uint8)
    q[:, 0:2] = np.full(H // 32, 0.01, np.float16).view(np.uint8).reshape(-1, 2)
    q[:, 2:] = rng.integers(60, 127, size=(H // 32, 32)).astype(np.int8).view(np.uint8)
    t["blk.1.attn_norm.weight"] = (J.Q8_0, q.reshape(-1), H, 1)
    w = t["blk.1.ffn_norm.weight"][1].copy()
    w[[1, 50, 255]] = [np.nan, np.inf, -np.inf]
    t["blk.1.ffn_norm.weight"] = (J.F32, w, H, 1)
    kn = t["blk.0.attn_k_norm.weight"][1][:40].copy()
    t["blk.0.attn_k_norm.weight"] = (J.F32, kn, 40, 1)
    run_model(dev, t)


def test_prefill_with_padded_and_short_heads(dev):
    """The batched prefill ends in the same head step: a padded Q6_K head and a short Q8_0 one,
    every prompt token held to the decode bars."""
    print("prefill padded / short heads", flush=True)
    H = SPEC["hidden"]
    for variant in ("padded", "short"):
        t = base_tensors(47)
        q, w, _, _ = t["output.weight"]
        if variant == "padded":
            t["output.weight"] = (q, np.concatenate([w, zero_rows(q, 64, H)]), H, 384)
        else:
            t["output.weight"] = (J.Q8_0, rand_weights(J.Q8_0, 100, H, 48), H, 100)
        cap, pos0, n = 64, 3, 20
        m = make_gpu_model(SPEC, t, cap, J.KV_F16, True)
        om = O.DecodeModel(SPEC, t, cap)
        kv = prefill_kv(m, om, SPEC, cap, pos0, 49, dev)
        tokens = np.random.default_rng(50).integers(0, SPEC["vocab"], size=n).tolist()
        DP.run_prefill_traced(m, om, t, SPEC, kv, cap, pos0, tokens, True, dev)
        m.close()


def test_padded_head_from_gguf(dev, tmp_path):
    """A GGUF whose {arch}.vocab_size is 320 and whose output.weight has 384 rows loads (the head
    rows are not held to the vocabulary) and decodes 384 logits."""
    from test_gpu_decode import write_model_gguf
    print("padded head from gguf", flush=True)
    t = base_tensors(51)
    H = SPEC["hidden"]
    q, w, _, _ = t["output.weight"]
    t["output.weight"] = (q, np.concatenate([w, zero_rows(q, 64, H)]), H, 384)
    path = tmp_path / "padded.gguf"
    import gguf_writer as W
    write_model_gguf(path, "qwen3", SPEC, t, extra_kvs=[("qwen3.vocab_size", W.U32, SPEC["vocab"])])
    m = J.DecodeModel.from_gguf(str(path), 64, J.KV_F16)
    assert m.cfg.vocab == SPEC["vocab"] and m.logits_len() == 384
    om = O.DecodeModel(SPEC, t, 64)
    kv = prefill_kv(m, om, SPEC, 64, 10, 52, dev)
    DP.run_traced(m, om, t, SPEC, kv, 64, 10, 2, True, dev, 7)
    m.close()
