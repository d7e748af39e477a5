"""GGUF v3 reader (host code of libjero_hip.so; no GPU needed).

Parity anchors: the reference's golden llama file (tests/architecture_certification_gate.rs:82-176)
parsed back to the exact tensors and hyperparameters it was built from; tensor lookup with the
tied-embedding fallback of ModelWeights::tensor (src/weights.rs:1097-1144); hyperparameter
inference of GgufHyperparams::from_metadata (src/capability.rs:107-285); malformed files rejected
with TensorBoundsError rather than read out of bounds.
"""
import numpy as np
import pytest

import golden_llama as GL
import gguf_writer as W
import jero_hip as J


def open_bytes(tmp_path, data, name="m.gguf"):
    p = tmp_path / name
    p.write_bytes(data)
    return J.GGUFFile(str(p))


def test_golden_llama_file_round_trip(tmp_path):
    with open_bytes(tmp_path, GL.gguf_file_bytes()) as g:
        assert g.arch == "llama"
        specs = GL.tensor_specs()
        assert g.tensor_names() == [n for n, _, _ in specs]
        built = GL.build()
        for name, quant, shape in specs:
            t = g.tensor(name)
            assert t["quant"] == quant and t["n_dims"] == len(shape)
            assert t["dims"][:len(shape)] == list(shape)
            assert t["host"] % 32 == 0
            np.testing.assert_array_equal(g.tensor_bytes(name), np.frombuffer(W.as_bytes(built[name][1]), np.uint8))
        hp = g.hyperparams()
        s = GL.SPEC
        assert (hp["hidden"], hp["ffn"], hp["n_layers"], hp["vocab"]) == (s["hidden"], s["ffn"], s["n_layers"],
                                                                         s["vocab"])
        assert (hp["n_heads_q"], hp["n_heads_kv"], hp["head_dim"]) == (s["nq"], s["nkv"], s["hd"])
        assert hp["rms_eps"] == float(np.float32(1e-5)) and hp["rope_theta"] == 500000.0
        assert hp["qk_norm"] is False
        assert g.meta_int("tokenizer.ggml.eos_token_id") == 2
        assert g.meta_int("general.alignment") == 32


def test_tied_output_falls_back_to_embedding(tmp_path):
    emb = np.arange(2 * 34 * 3, dtype=np.uint8)
    norm = np.ones(64, np.float32)
    tensors = [("token_embd.weight", 8, (64, 3), emb.tobytes()), ("output_norm.weight", 0, (64,), W.as_bytes(norm))]
    with open_bytes(tmp_path, W.gguf_bytes("qwen3", [], tensors)) as g:
        np.testing.assert_array_equal(g.tensor_bytes("output.weight"), emb)
        assert g.tensor("output.weight")["dims"][:2] == [64, 3]
        with pytest.raises(J.K3Error) as e:
            g.tensor("blk.0.attn_q.weight")
        assert e.value.status == 14 and "blk.0.attn_q.weight" in str(e.value)
    # BitNet models keep separate heads: no fallback
    with open_bytes(tmp_path, W.gguf_bytes("bitnet-b1.58", [], tensors), "b.gguf") as g:
        with pytest.raises(J.K3Error) as e:
            g.tensor("output.weight")
        assert e.value.status == 14
    # architectures without a KV cache (architecture_requires_kv_cache, src/memory.rs:863-868)
    # get no tied head either; a name that only starts like one ("bert-like") does
    for i, arch in enumerate(("bert", "modernbert", "deberta-v3", "ttm", "ft-transformer", "tabpfn-v2")):
        with open_bytes(tmp_path, W.gguf_bytes(arch, [], tensors), f"e{i}.gguf") as g:
            with pytest.raises(J.K3Error) as e:
                g.tensor("output.weight")
            assert e.value.status == 14, arch
    with open_bytes(tmp_path, W.gguf_bytes("bert-like", [], tensors), "bl.gguf") as g:
        np.testing.assert_array_equal(g.tensor_bytes("output.weight"), emb)


def test_metadata_value_types(tmp_path):
    kvs = [("a.u8", W.U8, 250), ("a.i8", W.I8, -7), ("a.u16", W.U16, 65000), ("a.i16", W.I16, -300),
           ("a.u32", W.U32, 4000000000), ("a.i32", W.I32, -5), ("a.f32", W.F32, 0.5), ("a.bool", W.BOOL, True),
           ("a.str", W.STRING, "héllo"), ("a.arr", W.ARRAY, (W.U32, [1, 2, 3])),
           ("a.sarr", W.ARRAY, (W.STRING, ["x", "yz", ""])), ("a.u64", W.U64, 2 ** 40), ("a.i64", W.I64, -2 ** 40),
           ("a.f64", W.F64, 1e300), ("a.after", W.U32, 17)]
    t = [("token_embd.weight", 0, (32, 2), bytes(256))]
    with open_bytes(tmp_path, W.gguf_bytes("x", kvs, t)) as g:
        for k, ty, v in kvs:
            if ty in (W.STRING,):
                assert g.meta_str(k) == v
            elif ty == W.ARRAY:
                with pytest.raises(J.K3Error):
                    g.meta_int(k)
            elif ty in (W.F32, W.F64):
                assert g.meta_float(k) == v
                with pytest.raises(J.K3Error):
                    g.meta_int(k)
            else:
                assert g.meta_int(k) == int(v) and g.meta_float(k) == float(int(v))
        with pytest.raises(J.K3Error):
            g.meta_str("a.u32")
        with pytest.raises(J.K3Error):
            g.meta_int("missing.key")
        assert g.meta_int("missing.key", 9) == 9


def test_hyperparams_inferred_from_tensor_shapes(tmp_path):
    """No block_count / key_length / head_count_kv / vocab metadata: taken from the tensors."""
    h, nq, nkv, hd, ffn, vocab = 64, 4, 2, 16, 96, 5
    def q8(n_in, n_out):
        return (8, (n_in, n_out), bytes(n_out * (n_in // 32) * 34))
    def f32(n):
        return (0, (n,), bytes(4 * n))
    spec = {"token_embd.weight": q8(h, vocab), "output_norm.weight": f32(h)}
    for L in range(3):
        spec.update({f"blk.{L}.attn_norm.weight": f32(h), f"blk.{L}.attn_q.weight": q8(h, nq * hd),
                     f"blk.{L}.attn_k.weight": q8(h, nkv * hd), f"blk.{L}.attn_v.weight": q8(h, nkv * hd),
                     f"blk.{L}.attn_q_norm.weight": f32(hd), f"blk.{L}.attn_k_norm.weight": f32(hd),
                     f"blk.{L}.ffn_gate.weight": q8(h, ffn)})
    tensors = [(n, q, shp, b) for n, (q, shp, b) in spec.items()]
    kvs = [("qwen3.attention.head_count", W.U32, nq), ("qwen3.attention.head_count_kv", W.U32, nkv)]
    with open_bytes(tmp_path, W.gguf_bytes("qwen3", kvs, tensors)) as g:
        hp = g.hyperparams()
    assert (hp["hidden"], hp["n_layers"], hp["n_heads_kv"], hp["head_dim"], hp["ffn"], hp["vocab"]) == \
        (h, 3, nkv, hd, ffn, vocab)
    assert hp["qk_norm"] is True
    # without head_count_kv the reference takes head_count, and key_length = attn_k width / that
    with open_bytes(tmp_path, W.gguf_bytes("qwen3", kvs[:1], tensors), "nokv.gguf") as g:
        hp = g.hyperparams()
    assert (hp["n_heads_kv"], hp["head_dim"]) == (nq, nkv * hd // nq)


def test_custom_alignment_and_v2(tmp_path):
    a = np.arange(48, dtype=np.float32)
    b = np.arange(7, dtype=np.float32) * -1
    t = [("x", 0, (48,), W.as_bytes(a)), ("y", 0, (7,), W.as_bytes(b))]
    for align, version in ((64, 3), (256, 3), (32, 2)):
        with open_bytes(tmp_path, W.gguf_bytes("t", [], t, alignment=align, version=version), f"{align}.gguf") as g:
            assert g.tensor("y")["host"] % align == 0
            np.testing.assert_array_equal(g.tensor_bytes("x").view(np.float32), a)
            np.testing.assert_array_equal(g.tensor_bytes("y").view(np.float32), b)


def _status(tmp_path, data, name):
    with pytest.raises(J.K3Error) as e:
        open_bytes(tmp_path, data, name)
    return e.value.status


def test_malformed_files_are_rejected(tmp_path):
    good = GL.gguf_file_bytes()
    assert _status(tmp_path, b"GGUX" + good[4:], "magic.gguf") == 14
    assert _status(tmp_path, good[:4] + (4).to_bytes(4, "little") + good[8:], "v4.gguf") == 10
    # every truncation inside the header, and cuts into the data section
    head_end = good.index(b"output.weight") + 64
    cuts = list(range(0, head_end, 7)) + [len(good) - 1, len(good) - 34, head_end + 100]
    for c in cuts:
        if c == 0:
            continue
        assert _status(tmp_path, good[:c], f"cut{c}.gguf") == 14, c
    t = [("x", 0, (8,), bytes(32)), ("y", 0, (8,), bytes(32))]
    assert _status(tmp_path, W.gguf_bytes("t", [], t, offsets=[0, 16]), "misaligned.gguf") == 14
    assert _status(tmp_path, W.gguf_bytes("t", [], t, offsets=[0, 1 << 40]), "past.gguf") == 14
    assert _status(tmp_path, W.gguf_bytes("t", [], [("x", 0, (8,), bytes(32))] * 2), "dup.gguf") == 14
    assert _status(tmp_path, W.gguf_bytes("t", [], t, alignment=48), "align48.gguf") == 14
    huge = [("x", 8, (1 << 39, 1 << 39), bytes(34))]
    assert _status(tmp_path, W.gguf_bytes("t", [], huge), "huge.gguf") == 14
    assert _status(tmp_path, W.gguf_bytes("t", [], [("x", 0, (2 ** 64 - 32,), bytes(32))]), "neg.gguf") == 14
    with pytest.raises(J.K3Error):
        J.GGUFFile(str(tmp_path / "does-not-exist.gguf"))
    # strings must be well-formed UTF-8: a bad continuation, an overlong form, a surrogate
    for i, bad in enumerate((b"\xc3(", b"\xc0\xaf", b"\xed\xa0\x80")):
        name = b"blk." + bad + b".weight"
        data = W.gguf_bytes("t", [], [("x" * len(name), 0, (8,), bytes(32))]).replace(b"x" * len(name), name)
        assert _status(tmp_path, data, f"utf8{i}.gguf") == 14
    ok = W.gguf_bytes("t", [("t.s", W.STRING, "€ 𝄞 ü")], [("ß", 0, (8,), bytes(32))])
    with open_bytes(tmp_path, ok, "utf8ok.gguf") as g:
        assert g.tensor_names() == ["ß"] and g.meta_str("t.s") == "€ 𝄞 ü"


def test_unsupported_tensor_type_is_listed_but_not_fetched(tmp_path):
    t = [("q5_0", 6, (32, 2), bytes(44)), ("bf16", 30, (8, 2), bytes(32)), ("x", 0, (8,), bytes(32))]
    with open_bytes(tmp_path, W.gguf_bytes("t", [], t)) as g:
        assert g.tensor_names() == ["q5_0", "bf16", "x"]
        with pytest.raises(J.K3Error) as e:
            g.tensor("q5_0")
        assert e.value.status == 10
        bf = g.tensor("bf16")  # BF16 rows have a size (2 bytes per element)
        assert bf["quant"] == 30 and bf["nbytes"] == 32


def test_corrupted_headers_never_read_out_of_bounds(tmp_path):
    """Seeded byte corruptions of the golden file's header: each open either succeeds or raises
    K3Error; every tensor a successful open reports lies inside the file."""
    good = bytearray(GL.gguf_file_bytes())
    head_end = good.index(b"output.weight") + 40
    rng = np.random.default_rng(123)
    p = tmp_path / "fuzz.gguf"
    for case in range(400):
        bad = bytearray(good)
        for _ in range(int(rng.integers(1, 4))):
            bad[int(rng.integers(0, head_end))] = int(rng.integers(0, 256))
        p.write_bytes(bytes(bad))
        try:
            g = J.GGUFFile(str(p))
        except J.K3Error:
            continue
        with g:
            for name in g.tensor_names():
                try:
                    t = g.tensor(name)
                except J.K3Error:
                    continue
                b = g.tensor_bytes(name)
                assert b.size == t["nbytes"] and t["nbytes"] <= len(bad), (case, name)
