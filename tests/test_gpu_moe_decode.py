"""Qwen3-MoE decode on the device: execute_token_standard_with_hidden with a MoE spec
(src/qwen_deepseek.rs:1239-1314), every layer's FFN dispatch_qwen3_moe_ffn (:847-951, called at
:1286-1300) -- jero_hip_model_set_moe -- against the oracle (pyoracle.DecodeModel.moe_step: the C
attention sublayer, then pyoracle.moe_layer, itself pinned in tests/test_oracle.py).

Per step, every layer teacher-forced from the device's own trace:
  * the attention sublayer from the device's layer input (the oracle's rings kept in step): the
    layer's mid state within 1e-3 (the attention bar; the dense decode tests hold its parts to
    their separate bars);
  * the FFN's normalised input at f32 precision, the router logits within 1e-5 (the GEMV bar)
    and the same top-k selection;
  * the FFN output (next layer input - mid state) against moe_layer on the device's normalised
    input within 1e-3 of max(|ref|, rms(ref)), the bar of tests/test_gpu_moe_layer.py (the two
    sides quantize the SwiGLU rows (Q8_K, or ACT_Q8 for Q8_0 / Q4_0 down experts) separately: a
    value within float error of a rounding boundary may round the other way);
end to end, the logits against the oracle's free-running step: cosine >= 0.9999 (the reference's
certification floor) and the greedy token equal when the top-2 gap exceeds 1e-2 of the rms.
The batched prefill (expert GEMMs over the prompt rows) writes every prompt token's trace in the
same layout: each token is held to the same bars, the last token's logits to the oracle's token
loop.  Also: a prefill that the batched pass does not take equals the decode steps it stands for,
bit for bit; a GGUF qwen3moe file loads to the same model; a captured step replays as eager
steps; the routing bias and incomplete expert sets are refused."""
import numpy as np
import pytest
import torch

import decode_parity as DP
import jero_hip as J
import model_spec as MS
import pyoracle as O

pytestmark = pytest.mark.gpu

TOL = 1e-3


def make(spec, moe, t, cap):
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], cap, J.KV_F16, True, moe=moe)
    for name, (quant, arr, n_in, n_out) in t.items():
        m.set_tensor(name, quant, arr, n_in, n_out)
    m.finalize()
    return m


def prefill_rings(m, om, spec, cap, prefill, seed, dev):
    kv = om.new_kv()
    kvd = spec["nkv"] * spec["hd"]
    rng = np.random.default_rng(seed)
    for L in range(spec["n_layers"]):
        k = rng.standard_normal((cap, kvd)).astype(np.float16)
        v = rng.standard_normal((cap, kvd)).astype(np.float16)
        k[prefill:] = 0
        v[prefill:] = 0
        kv[L, 0] = k.astype(np.float32)
        kv[L, 1] = v.astype(np.float32)
        m.write_kv(L, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev))
    return kv


def rel(got, ref):
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / max(np.sqrt(np.mean(ref ** 2)), 1e-30))


def cosine(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))


QWEN3_MOE = dict(hidden=2048, ffn=6144, n_layers=2, vocab=2000, nq=32, nkv=4, hd=128, eps=1e-6, theta=1e6)
SMALL = dict(hidden=1024, ffn=512, n_layers=2, vocab=1000, nq=16, nkv=4, hd=64, eps=1e-6, theta=1e6)

# name: (spec, moe (E, top_k, F, use_shared), router layers (None: all), capacity, prefill, steps,
# build_moe's formats)
CASES = {
    "qwen3_30b_a3b_layers": (QWEN3_MOE, (128, 8, 768, False), None, 512, 500, 3, {}),
    "shared_expert": (SMALL, (16, 4, 256, True), None, 128, 60, 4, {}),
    "layer_without_router": (SMALL, (16, 4, 256, False), {0}, 128, 60, 4, {}),
    "256_experts": (SMALL, (256, 8, 256, False), None, 128, 0, 4, {}),
    # routers the F32 router-norm kernel does not take (F16 values; Q8_0 through the quantized
    # activation and GEMV), and Q4_K down experts (the Q4_K_T down kernels)
    "f16_router_q4k_down": (SMALL, (32, 4, 256, False), None, 128, 30, 3, dict(router_quant=J.F16, down_quant=J.Q4_K)),
    "q8_0_router": (SMALL, (32, 4, 256, False), None, 128, 30, 3, dict(router_quant=J.Q8_0)),
    # experts in the 32-element formats (ACT_Q8 activations): Q8_0 gate / up, Q4_0 down; and the
    # Qwen3-30B-A3B layer shape with Q8_0 experts throughout
    "q8_0_gate_up_q4_0_down": (SMALL, (32, 4, 256, False), None, 128, 30, 3,
                               dict(gate_quant=J.Q8_0, down_quant=J.Q4_0)),
    "qwen3_30b_a3b_layers_q8_0": (QWEN3_MOE, (128, 8, 768, False), None, 256, 100, 2,
                                  dict(gate_quant=J.Q8_0, down_quant=J.Q8_0)),
}


def act_ties(act, fmt=DP.Q8_K):
    """Elements of an f32 row whose activation rounding lies within float error of a tie (|q|
    within 1e-3 of k + 0.5; Q8_K: ggml's rule, iscale = -127 / the block's first largest-magnitude
    value over 256 elements; ACT_Q8: 1 / d = 127 / amax over 32), and each element's block scale
    |d|: two correct computations of the row may round these apart."""
    n = 256 if fmt == DP.Q8_K else 32
    a = np.asarray(act, np.float64).reshape(-1, n)
    mx = a[np.arange(len(a)), np.argmax(np.abs(a), axis=1)]
    iscale = np.where(mx != 0, -127.0 / np.where(mx != 0, mx, 1.0), 0.0)
    y = np.abs(a * iscale[:, None])
    tie = (np.abs(y - np.floor(y) - 0.5) < 1e-3) & (mx != 0)[:, None]
    return tie.reshape(-1), np.repeat(np.abs(mx) / 127.0, n)


def flip_bound(xn, L, moe, w, sel):
    """Per output element, the largest change that rounding-tie flips of the SwiGLU rows can make
    to dispatch_qwen3_moe_ffn's output: sum over the selected experts e (weight w_e) and their
    tie elements f of |w_e| * d_f * |down_e[:, f]|."""
    E, k, F, shared = moe
    H = xn.size
    bound = np.zeros(H)
    for e, we in sel:
        parts = [O._expert_slice(w, f"blk.{L}.ffn_{kind}_exps.weight", f"blk.{L}.ffn_{kind}_exps.{e}.weight", e, E)
                 for kind in ("gate", "up", "down")]
        g, u, dn = parts
        Fe = O._n_el(g[2]) // H
        act = O.swiglu(O.vec_dot(g[0], g[1], H, Fe, xn), O.vec_dot(u[0], u[1], H, Fe, xn))
        tie, d = act_ties(act, DP.act_fmt(dn[0]))
        if tie.any():
            Dq = O.dequantize(dn[0], dn[1], H, Fe)
            bound += abs(we) * (np.abs(Dq[:, tie]).astype(np.float64) @ d[tie])
    return bound


def check_layers(m, dl, dh, t, w, spec, moe, pos, cap):
    """The teacher-forced checks of one token's trace, every layer from the device's own input to
    it: the attention sublayer as the dense decode tests check it (decode_parity.check_attn, on
    the device's rings), then the FFN's normalised input, the router logits and selection, and the
    MoE output against moe_layer within TOL of max(|ref|, rms(ref)) plus the reach of the SwiGLU
    rows' rounding ties; returns the worst errors."""
    E, k, F, shared = moe
    H = spec["hidden"]
    eps_ffn = max(spec["eps"], 1e-6)
    kvd = spec["nkv"] * spec["hd"]
    worst = dict(attn=0.0, gemv=0.0, xn=0.0, router=0.0, ffn=0.0, flips=0)
    DP.check_rope_table(spec, pos, dh["rope_cs"])
    for L in range(spec["n_layers"]):
        D = dl[L]
        x_next = dl[L + 1]["x_in"] if L + 1 < spec["n_layers"] else dh["x_final"]
        rk, rv = DP.read_ring(m, L, cap, kvd, True)
        ea = DP.check_attn(t, spec, D, L, pos, rk, rv, True, rope_cs=dh["rope_cs"])
        worst["attn"] = max(worst["attn"], ea["attn"])
        worst["gemv"] = max(worst["gemv"], ea["gemv"])
        nd = t[f"blk.{L}.ffn_norm.weight"][1]
        xn = O.rmsnorm(D["x_mid"], nd, eps_ffn)
        worst["xn"] = max(worst["xn"], rel(D["xn_ffn"], xn))
        assert worst["xn"] <= 1e-6, (L, pos, worst)
        xn_dev = np.ascontiguousarray(D["xn_ffn"], np.float32)
        router = w.get(f"blk.{L}.ffn_gate_inp.weight")
        if router is not None:
            lg = O.vec_dot(router[0], router[1], H, E, xn_dev)
            lg_dev = D["gu"][:E]
            worst["router"] = max(worst["router"], rel(lg_dev, lg))
            assert worst["router"] <= 1e-5, (L, pos, worst)
            assert [e for e, _ in O.select_top_k(lg_dev, k, True)] == \
                [e for e, _ in O.select_top_k(lg, k, True)], (L, pos)
        out_ref, sel = O.moe_layer(xn_dev, L, E, k, F, shared, w)
        out_dev = x_next.astype(np.float64) - D["x_mid"].astype(np.float64)
        scale = np.maximum(np.abs(out_ref.astype(np.float64)), np.sqrt(np.mean(out_ref.astype(np.float64) ** 2)))
        # x_next rounds x_mid + out: allow its half ulp on top of the bar
        err = np.abs(out_dev - out_ref) - 0.5 * np.spacing(np.abs(x_next)).astype(np.float64)
        if np.max(err / scale) > TOL and sel:
            err = err - flip_bound(xn_dev, L, moe, w, sel)
            worst["flips"] += 1
        worst["ffn"] = max(worst["ffn"], float(np.max(err / scale)))
        assert worst["ffn"] <= TOL, (L, pos, worst)
    return worst


def check_logits(got, free, gtok, pos):
    cs = cosine(got, free)
    assert cs >= 0.9999, (pos, cs)
    top2 = np.sort(free.astype(np.float64))[-2:]
    if top2[1] - top2[0] > 1e-2 * np.sqrt(np.mean(free.astype(np.float64) ** 2)):
        assert gtok == O.argmax(free), (pos, gtok, O.argmax(free))
    return cs


@pytest.mark.parametrize("case", sorted(CASES))
def test_moe_decode_matches_oracle(dev, case):
    spec, moe, routers, cap, prefill, steps, fmts = CASES[case]
    print(f"moe decode {case}", flush=True)
    t, w = MS.build_moe(spec, moe, seed=60 + sorted(CASES).index(case), router_layers=routers, **fmts)
    m = make(spec, moe, t, cap)
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = prefill_rings(m, om, spec, cap, prefill, 3, dev)
    kv_free = kv.copy()
    om.model.kv_f16 = 1
    _, _, _, total = m.trace_layout()
    buf = torch.zeros(total, dtype=torch.uint8, device=dev)
    m.set_trace(buf)
    logits = torch.empty(m.logits_len(), dtype=torch.float32, device=dev)
    tok = 29
    m.set_position(tok, prefill)
    for i in range(steps):
        pos = prefill + i
        m.decode_step()
        m.status()
        m.read_logits(logits)
        got = logits.cpu().numpy()
        gtok, gpos = m.read_token_pos()
        assert gpos == pos + 1
        dl, dh = m.read_trace(buf)
        worst = check_layers(m, dl, dh, t, w, spec, moe, pos, cap)
        free = om.moe_step(kv_free, tok, pos, moe, w)
        cs = check_logits(got, free, gtok, pos)
        print(f"  pos {pos}: teacher-forced max errors " + " ".join(f"{a} {b:.1e}" for a, b in worst.items()) +
              f" | free-running oracle: rel err {rel(got, free):.2e} cos {cs:.8f}", flush=True)
        tok = gtok
    m.set_trace(None)
    m.status()
    m.close()


# name: (spec, moe, capacity, filled slots before the prompt, prompt tokens); the batched pass
# (every layer routed over an F32 router, no shared expert): below 32 prompt tokens the experts
# take the GEMV passes, from 32 (256 (token, slot) pairs over 128 experts) the MFMA expert GEMMs
# in passes of 8 tokens, from 256 (16 per expert on average) in passes of 16
PREFILL_CASES = {
    # 1100 tokens at top-8: two routing chunks (8192 pairs each at most); sampled tokens checked
    "chunked_1100_tokens": (SMALL, (16, 8, 256, False), 1152, 8, 1100, [0, 1, 700, 1022, 1023, 1024, 1025, 1099]),
    "qwen3_30b_a3b_layers_288_tokens": (QWEN3_MOE, (128, 8, 768, False), 512, 16, 288),
    "qwen3_30b_a3b_layers_96_tokens": (QWEN3_MOE, (128, 8, 768, False), 256, 40, 96),
    "qwen3_30b_a3b_layers_9_tokens": (QWEN3_MOE, (128, 8, 768, False), 256, 0, 9),
    "256_experts_70_tokens": (SMALL, (256, 8, 256, False), 128, 20, 70),
    # Q8_0 gate / up and Q4_0 down experts: the GEMV passes at any token count
    "q8_0_q4_0_experts_40_tokens": (SMALL, (16, 4, 256, False), 128, 12, 40, None,
                                    dict(gate_quant=J.Q8_0, down_quant=J.Q4_0)),
}


@pytest.mark.parametrize("case", sorted(PREFILL_CASES))
def test_moe_prefill_matches_oracle(dev, case):
    """The batched MoE prefill (the experts' GEMMs over the prompt rows) writes every prompt token's
    trace in the decode step's layout: each token is held to the decode step's teacher-forced
    bars, and the last token's logits to the free-running oracle's token loop."""
    spec, moe, cap, pos0, n = PREFILL_CASES[case][:5]
    extra = PREFILL_CASES[case][5:]
    sample = set(extra[0]) if extra and extra[0] is not None else set(range(n))
    fmts = extra[1] if len(extra) > 1 else {}
    print(f"moe prefill {case}", flush=True)
    t, w = MS.build_moe(spec, moe, seed=80 + sorted(PREFILL_CASES).index(case), **fmts)
    m = make(spec, moe, t, cap)
    om = O.DecodeModel(spec, MS.oracle_tensors(t), cap)
    kv = prefill_rings(m, om, spec, cap, pos0, 5, dev)
    kv_free = kv.copy()
    om.model.kv_f16 = 1
    _, _, _, total = m.trace_layout()
    buf = torch.zeros(n * total, dtype=torch.uint8, device=dev)
    m.set_trace(buf)
    tokens = np.random.default_rng(7).integers(0, spec["vocab"], n).astype(np.int32)
    m.prefill(tokens, pos0)
    m.status()
    logits = torch.empty(m.logits_len(), dtype=torch.float32, device=dev)
    m.read_logits(logits)
    got = logits.cpu().numpy()
    gtok, gpos = m.read_token_pos()
    assert gpos == pos0 + n
    worst = dict(attn=0.0, gemv=0.0, xn=0.0, router=0.0, ffn=0.0, flips=0)
    for i in range(n):
        if i in sample:
            dl, dh = m.read_trace(buf[i * total:])
            wi = check_layers(m, dl, dh, t, w, spec, moe, pos0 + i, cap)
            worst = {a: worst[a] + wi[a] if a == "flips" else max(worst[a], wi[a]) for a in worst}
        free = om.moe_step(kv_free, int(tokens[i]), pos0 + i, moe, w)
    cs = check_logits(got, free, gtok, pos0 + n - 1)
    print(f"  {n} tokens ({len(sample)} checked): teacher-forced max errors " + " ".join(f"{a} {b:.1e}" for a, b in worst.items()) +
          f" | last token against the free-running oracle: rel err {rel(got, free):.2e} cos {cs:.8f}", flush=True)
    m.set_trace(None)
    m.status()
    # the untraced pass (the timed one) leaves the same logits and token
    m2 = make(spec, moe, t, cap)
    prefill_rings(m2, O.DecodeModel(spec, MS.oracle_tensors(t), cap), spec, cap, pos0, 5, dev)
    m2.prefill(tokens, pos0)
    l2 = torch.empty_like(logits)
    m2.read_logits(l2)
    assert torch.equal(l2, logits) and m2.read_token_pos() == (gtok, gpos)
    # and decoding continues from the prefilled rings
    m2.decode_step()
    m2.status()
    assert m2.read_token_pos()[1] == pos0 + n + 1
    m.close()
    m2.close()


@pytest.mark.parametrize("what", ["shared_expert", "f16_router"])
def test_moe_prefill_equals_decode_steps(dev, what):
    """jero_hip_model_prefill of a MoE model that the batched pass does not take (a shared expert,
    a router in another format than F32) runs the reference's token loop: it leaves the state the
    same tokens' decode steps leave, logits, token, position and rings bit for bit."""
    spec = SMALL
    moe = (16, 4, 256, what == "shared_expert")
    t, _ = MS.build_moe(spec, moe, seed=71, **({"router_quant": J.F16} if what == "f16_router" else {}))
    a, b = make(spec, moe, t, 128), make(spec, moe, t, 128)
    tokens = np.array([5, 17, 3, 99, 42, 7], np.int32)
    a.prefill(tokens, 10)
    for i, tk in enumerate(tokens):
        b.set_position(int(tk), 10 + i)
        b.decode_step()
    torch.cuda.synchronize()
    la = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    lb = torch.empty_like(la)
    a.read_logits(la)
    b.read_logits(lb)
    assert torch.equal(la, lb)
    assert a.read_token_pos() == b.read_token_pos()
    kvd = spec["nkv"] * spec["hd"]
    for L in range(spec["n_layers"]):
        for x, y in zip(a.kv_ptrs(L), b.kv_ptrs(L)):
            ra = torch.empty(128 * kvd, dtype=torch.float16, device=dev)
            rb = torch.empty_like(ra)
            J._memcpy(ra.data_ptr(), x, ra.numel() * 2)
            J._memcpy(rb.data_ptr(), y, rb.numel() * 2)
            assert torch.equal(ra, rb), L
    a.close()
    b.close()


def test_moe_graph_replay_matches_eager(dev):
    spec, moe = SMALL, (32, 4, 256, False)
    t, _ = MS.build_moe(spec, moe, seed=72)
    a, b = make(spec, moe, t, 128), make(spec, moe, t, 128)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        a.set_position(5, 0, stream=s)
        b.set_position(5, 0, stream=s)
    s.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        a.decode_step(stream=s)
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            a.decode_step(stream=s)
    b.decode_step()
    torch.cuda.synchronize()
    la = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    lb = torch.empty_like(la)
    for i in range(5):
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
    a.close()
    b.close()


def test_moe_model_from_gguf(dev, tmp_path):
    """A qwen3moe GGUF file (expert_count / expert_used_count / expert_feed_forward_length, stacked
    3-D expert tensors) loads to the same model as the tensors given one by one."""
    import gguf_writer as W
    spec, moe = SMALL, (16, 4, 256, False)
    E, k, F, _ = moe
    t, w = MS.build_moe(spec, moe, seed=73)
    a = "qwen3moe"
    kvs = [(f"{a}.block_count", W.U32, spec["n_layers"]), (f"{a}.embedding_length", W.U32, spec["hidden"]),
           (f"{a}.feed_forward_length", W.U32, spec["ffn"]), (f"{a}.attention.head_count", W.U32, spec["nq"]),
           (f"{a}.attention.head_count_kv", W.U32, spec["nkv"]), (f"{a}.attention.key_length", W.U32, spec["hd"]),
           (f"{a}.rope.freq_base", W.F32, spec["theta"]), (f"{a}.attention.layer_norm_rms_epsilon", W.F32, spec["eps"]),
           (f"{a}.vocab_size", W.U32, spec["vocab"]), (f"{a}.expert_count", W.U32, E),
           (f"{a}.expert_used_count", W.U32, k), (f"{a}.expert_feed_forward_length", W.U32, F)]
    ts = []
    for n, (q, arr, n_in, n_out) in t.items():
        dims = tuple(w[n][2]) if n in w and len(w[n][2]) == 3 else ((n_in, n_out) if n_out > 1 else (n_in,))
        ts.append((n, q, dims, W.as_bytes(arr)))
    path = tmp_path / "qwen3moe.gguf"
    path.write_bytes(W.gguf_bytes(a, kvs, ts))
    ma = make(spec, moe, t, 64)
    mb = J.DecodeModel.from_gguf(str(path), 64, J.KV_F16)
    assert mb.moe == (E, k, F, False)
    la = torch.empty(spec["vocab"], dtype=torch.float32, device=dev)
    lb = torch.empty_like(la)
    for m in (ma, mb):
        m.set_position(17, 0)
    for step in range(4):
        ma.decode_step()
        mb.decode_step()
        torch.cuda.synchronize()
        ma.read_logits(la)
        mb.read_logits(lb)
        assert torch.equal(la, lb), step
    ma.close()
    mb.close()


def test_moe_refusals(dev):
    spec, moe = SMALL, (16, 4, 256, False)
    t, _ = MS.build_moe(spec, moe, seed=74)
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], 64, J.KV_F16, True, moe=moe)
    for name, (quant, arr, n_in, n_out) in t.items():
        m.set_tensor(name, quant, arr, n_in, n_out)
    m.set_tensor("blk.1.exp_probs_b.bias", J.F32, np.zeros(16, np.float32), 16, 1)
    with pytest.raises(J.K3Error) as ei:
        m.finalize()
    assert ei.value.variant == "CapabilityMismatch" and "exp_probs_b" in str(ei.value)
    m.close()
    m = J.DecodeModel(spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"], spec["nq"], spec["nkv"],
                      spec["hd"], spec["eps"], spec["theta"], 64, J.KV_F16, True, moe=moe)
    for name, (quant, arr, n_in, n_out) in t.items():
        if name != "blk.0.ffn_up_exps.weight":
            m.set_tensor(name, quant, arr, n_in, n_out)
    with pytest.raises(J.K3Error) as ei:
        m.finalize()
    assert ei.value.variant == "CapabilityMismatch" and "incomplete" in str(ei.value)
    m.close()
