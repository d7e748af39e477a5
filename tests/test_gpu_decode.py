"""The device decode step against the oracle and against the reference's golden fixture.

Bars: golden llama Q8_0 first-token logits within 1e-4 of the fixture and its greedy ids;
random Qwen3-shaped models: logits within 1e-3 of max(|ref|, rms(ref)) at every step, greedy
token equal to the oracle's argmax whenever the oracle's top-2 gap exceeds that tolerance.
"""
import numpy as np
import pytest
import torch

import golden_llama as GL
import jero_hip as J
import model_spec as MS
import pyoracle as O

pytestmark = pytest.mark.gpu


def make_gpu_model(spec, tensors, cap, kv_dtype, qk_norm):
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], cap, kv_dtype, qk_norm)
    for name, (quant, arr, n_in, n_out) in tensors.items():
        if not qk_norm and "_q_norm" in name or not qk_norm and "_k_norm" in name:
            continue
        m.set_tensor(name, quant, arr, n_in, n_out)
    m.finalize()
    return m


def rel_err(y, ref):
    ref = np.asarray(ref, np.float64)
    scale = max(float(np.sqrt(np.mean(ref ** 2))), 1e-30)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref) / np.maximum(np.abs(ref), scale)))


def test_golden_llama_on_device(dev):
    """The reference's golden fixture through the device decode path (Q8_0 x ACT_Q8 GEMVs)."""
    print("golden llama on device", flush=True)
    g = GL.golden()
    s = dict(GL.SPEC)
    tensors = {}
    shapes = {n: shp for n, _, shp in GL.tensor_specs()}
    for name, (quant, arr) in GL.build().items():
        shp = shapes[name]
        tensors[name] = (quant, arr, shp[0], shp[1] if len(shp) > 1 else 1)
    m = make_gpu_model(s, tensors, 128, J.KV_F32, False)
    logits = torch.empty(s["vocab"], dtype=torch.float32, device=dev)
    for pos, tok in enumerate(g["prompt_token_ids"]):
        m.set_position(tok, pos)
        m.decode_step()
    torch.cuda.synchronize()
    m.read_logits(logits)
    first = logits.cpu().numpy()
    for e in g["first_token_top_k"]:
        assert abs(first[e["token_id"]] - e["logit"]) <= 1e-4, (e, first[e["token_id"]])
    greedy = [m.read_token_pos()[0]]
    for _ in range(len(g["greedy_token_ids"]) - 1):
        m.decode_step()
        torch.cuda.synchronize()
        greedy.append(m.read_token_pos()[0])
    assert greedy == g["greedy_token_ids"]
    assert m.read_token_pos()[1] == len(g["prompt_token_ids"]) + len(g["greedy_token_ids"]) - 1


QWEN_SMALL = dict(hidden=512, ffn=1024, n_layers=4, vocab=1000, nq=8, nkv=2, hd=64, eps=1e-6, theta=1e6)


@pytest.mark.parametrize("kv_name,cap,prefill,steps", [("f32", 300, 40, 3), ("f16", 300, 297, 5), ("f16", 128, 0, 3)])
def test_decode_matches_oracle(dev, kv_name, cap, prefill, steps):
    """Prefilled cache (f16-exact values), then decode steps; the second case wraps the ring."""
    print(f"decode kv={kv_name} cap={cap} prefill={prefill}", flush=True)
    spec = QWEN_SMALL
    t = MS.build(spec, seed=3)
    kv_dtype = J.KV_F32 if kv_name == "f32" else J.KV_F16
    m = make_gpu_model(spec, t, cap, kv_dtype, True)
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = om.new_kv()
    kvd = spec["nkv"] * spec["hd"]
    rng = np.random.default_rng(7)
    for L in range(spec["n_layers"]):
        k = rng.standard_normal((cap, kvd)).astype(np.float16)
        v = rng.standard_normal((cap, kvd)).astype(np.float16)
        k[prefill:] = 0
        v[prefill:] = 0
        kv[L, 0] = k.astype(np.float32)
        kv[L, 1] = v.astype(np.float32)
        tdt = torch.float16 if kv_dtype == J.KV_F16 else torch.float32
        m.write_kv(L, torch.from_numpy(k).to(tdt).to(dev), torch.from_numpy(v).to(tdt).to(dev))
    tok = 17
    logits = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    m.set_position(tok, prefill)
    for i in range(steps):
        pos = prefill + i
        m.decode_step()
        torch.cuda.synchronize()
        m.read_logits(logits)
        ref = om.step(kv, tok, pos, threads=8)
        got = logits.cpu().numpy()
        err = rel_err(got, ref)
        assert err < 1e-3, (pos, err)
        gtok, gpos = m.read_token_pos()
        assert gpos == pos + 1
        top2 = np.sort(ref)[-2:]
        scale = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
        if top2[1] - top2[0] > 1e-3 * max(abs(top2[1]), scale):
            assert gtok == int(np.argmax(ref))
        tok = gtok if gtok >= 0 else 0
        if gtok != int(np.argmax(ref)):  # keep the oracle on the device's token
            pass


def test_decode_graph_replay_matches_eager(dev):
    """One captured step replayed for consecutive tokens equals eager steps bit for bit."""
    print("decode graph replay", flush=True)
    spec = dict(QWEN_SMALL, n_layers=2)
    t = MS.build(spec, seed=5)
    cap = 256
    a = make_gpu_model(spec, t, cap, J.KV_F16, True)
    b = make_gpu_model(spec, t, cap, J.KV_F16, True)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        a.set_position(5, 0, stream=s)
        b.set_position(5, 0, stream=s)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        a.decode_step(stream=s)  # warm (position 0)
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            a.decode_step(stream=s)
    b.decode_step()
    torch.cuda.synchronize()
    la = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    lb = torch.empty_like(la)
    for i in range(6):
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        b.decode_step()
        torch.cuda.synchronize()
        a.read_logits(la)
        b.read_logits(lb)
        assert torch.equal(la, lb), i
        assert a.read_token_pos() == b.read_token_pos()
        _ = torch.randn(1000, device=dev).sum().item()  # unrelated eager work between replays


def test_model_errors(dev):
    m = J.DecodeModel(512, 1024, 1, 100, 8, 2, 64, 1e-6, 1e6, 64)
    with pytest.raises(J.K3Error) as ei:
        m.set_tensor("blk.0.attn_q.weight", J.Q4_K, np.zeros(10, np.uint8), 512, 512)
    assert ei.value.variant == "TensorBoundsError"
    with pytest.raises(J.K3Error) as ei:
        m.set_tensor("blk.7.attn_q.weight", J.Q4_K, np.zeros(512 * 2 * 144, np.uint8), 512, 512)
    assert ei.value.variant == "CapabilityMismatch"
    with pytest.raises(J.K3Error) as ei:
        m.finalize()
    assert ei.value.variant == "CapabilityMismatch" and "missing" in str(ei.value)
    with pytest.raises(J.K3Error) as ei:
        m.decode_step()
    assert ei.value.variant == "InvalidArgument"
    with pytest.raises(J.K3Error) as ei:
        J.DecodeModel(512, 1024, 1, 100, 8, 3, 64, 1e-6, 1e6, 64)
    assert ei.value.variant == "TensorBoundsError"
