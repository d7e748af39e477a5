"""The reference's golden llama Q8_0 model, rebuilt from its recipe.

Restates build_authentic_llama_q8_0_gguf / build_q8_0_matrix_bytes / f32_to_f16_bits of
tests/architecture_certification_gate.rs:39-176 (reference): 2 layers, hidden 128, ffn 256,
4 q / 2 kv heads of 32, vocab 16, RoPE base 5e5, eps 1e-5; Q8_0 payload
q = ((b*19 + k*7 + seed*13) % 121) - 60 with seed = tensor index + 1 (spec order), scale the
truncating f16 of 0.025, norms 0.85 + (e % 13) * 0.02, rows 0..4 of output.weight zeroed.
Expected outputs: tests/golden/llama_authentic_q8_0.json (copied from the reference's
tests/fixtures/golden_parity/llama_authentic_q8_0.json).
"""
import json
import os

import numpy as np

Q8_0, F32 = 8, 0
HERE = os.path.dirname(os.path.abspath(__file__))

SPEC = dict(hidden=128, ffn=256, nq=4, nkv=2, hd=32, vocab=16, n_layers=2, eps=1e-5, theta=500000.0)


def f32_to_f16_bits_trunc(val):
    """The test's own truncating f32->f16 (architecture_certification_gate.rs:39-54)."""
    bits = int(np.array([val], np.float32).view(np.uint32)[0])
    sign = (bits >> 16) & 0x8000
    exp = ((bits >> 23) & 0xFF) - 127 + 15
    mant = (bits >> 13) & 0x3FF
    if exp <= 0:
        return sign
    if exp >= 31:
        return sign | 0x7BFF
    return sign | (exp << 10) | mant


def q8_0_matrix(rows, cols, seed):
    blocks = rows * (cols // 32)
    out = np.zeros((blocks, 34), np.uint8)
    d = f32_to_f16_bits_trunc(0.025)
    out[:, 0] = d & 0xFF
    out[:, 1] = d >> 8
    b = np.arange(blocks)[:, None]
    k = np.arange(32)[None, :]
    out[:, 2:] = (((b * 19 + k * 7 + seed * 13) % 121) - 60).astype(np.int8).view(np.uint8)
    return out


def tensor_specs():
    h, f, nq, nkv, hd, v = 128, 256, 4, 2, 32, 16
    specs = [("token_embd.weight", Q8_0, (h, v))]
    for L in range(2):
        specs += [
            (f"blk.{L}.attn_norm.weight", F32, (h,)),
            (f"blk.{L}.attn_q.weight", Q8_0, (h, nq * hd)),
            (f"blk.{L}.attn_k.weight", Q8_0, (h, nkv * hd)),
            (f"blk.{L}.attn_v.weight", Q8_0, (h, nkv * hd)),
            (f"blk.{L}.attn_output.weight", Q8_0, (nq * hd, h)),
            (f"blk.{L}.ffn_norm.weight", F32, (h,)),
            (f"blk.{L}.ffn_gate.weight", Q8_0, (h, f)),
            (f"blk.{L}.ffn_up.weight", Q8_0, (h, f)),
            (f"blk.{L}.ffn_down.weight", Q8_0, (f, h)),
        ]
    specs += [("output_norm.weight", F32, (h,)), ("output.weight", Q8_0, (h, v))]
    assert len(specs) == 21
    return specs


def build():
    """{name: (quant, ndarray)}: Q8_0 tensors as flat uint8, norms as f32."""
    tensors = {}
    for idx, (name, quant, shape) in enumerate(tensor_specs()):
        if len(shape) == 1:
            tensors[name] = (F32, np.array([0.85 + (e % 13) * 0.02 for e in range(shape[0])], np.float32))
            continue
        cols, rows = shape
        payload = q8_0_matrix(rows, cols, idx + 1)
        if name == "output.weight":
            per_row = cols // 32
            z = f32_to_f16_bits_trunc(0.0)
            for r in range(5):
                payload[r * per_row:(r + 1) * per_row, 0] = z & 0xFF
                payload[r * per_row:(r + 1) * per_row, 1] = z >> 8
                payload[r * per_row:(r + 1) * per_row, 2:] = 0
        tensors[name] = (Q8_0, payload.reshape(-1))
    return tensors


def golden():
    with open(os.path.join(HERE, "golden", "llama_authentic_q8_0.json")) as f:
        return json.load(f)


def gguf_kvs():
    """The metadata of build_authentic_llama_q8_0_gguf (architecture_certification_gate.rs:90-106)."""
    from gguf_writer import U32, F32 as GF32
    return [("llama.block_count", U32, 2), ("llama.embedding_length", U32, 128),
            ("llama.feed_forward_length", U32, 256), ("llama.attention.head_count", U32, 4),
            ("llama.attention.head_count_kv", U32, 2), ("llama.attention.key_length", U32, 32),
            ("llama.rope.freq_base", GF32, 500000.0), ("llama.attention.layer_norm_rms_epsilon", GF32, 1.0e-5),
            ("llama.context_length", U32, 128), ("llama.vocab_size", U32, 16),
            ("tokenizer.ggml.eos_token_id", U32, 2)]


def gguf_file_bytes():
    """The golden model as the GGUF v3 file the reference's test builds (alignment 32)."""
    from gguf_writer import as_bytes, gguf_bytes
    t = build()
    return gguf_bytes("llama", gguf_kvs(), [(n, q, shp, as_bytes(t[n][1])) for n, q, shp in tensor_specs()])
