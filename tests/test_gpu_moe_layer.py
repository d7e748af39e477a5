"""GPU parity of the whole MoE layer, dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951), as
jero_hip.moe_layer runs it on the device: the shared expert (jero_hip_swiglu_ffn, then the routed
sum added onto it by jero_hip_moe_ffn_acc), a layer without a router (the dense FFN, each
projection project_or_deterministic_slice), per-expert tensors ffn_*_exps.{e} (stacked on the
device, or registered as one stack from host memory by jero_hip_weights_register_stacked), and the
refusals (exp_probs_b routing bias, incomplete per-expert sets).

The oracle is pyoracle.moe_layer (pinned in tests/test_oracle.py).  Routing must match exactly.
Outputs are held to 1e-3 of max(|ref|, rms(ref)): the device and the oracle quantize the f32
SwiGLU rows (and, for the shared expert, the input) to Q8_K separately, and a value that lands
within float error of a rounding boundary may round the other way (a tie flip, ~1e-3 of the
output; test_gpu_moe.py replays the device's rows through the oracle to hold the routed experts to
1e-5 without them).  Paths that quantize nothing (the deterministic dense FFN) are held to 1e-6.
"""
import numpy as np
import pytest
import torch

import decode_parity as DP
import jero_hip as J
import pyoracle as O
from qdata import rand_act, rand_float_weights, rand_weights

pytestmark = pytest.mark.gpu

TOL = 1e-3


def td(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def make_weights(H, F, E, seed, shared=True, gq=J.Q4_K, dq=J.Q6_K, sq=J.Q8_0, router_quant=J.F32, dense=False):
    """(oracle weights {name: (quant, data, dims)}, device weights {name: TensorView})."""
    w = {}
    if E:
        rq = rand_float_weights(router_quant, E, H, seed + 9) if router_quant in (J.F32, J.F16) else \
            rand_weights(router_quant, E, H, seed + 9)
        w["blk.0.ffn_gate_inp.weight"] = (router_quant, rq, [H, E])
        w["blk.0.ffn_gate_exps.weight"] = (gq, rand_weights(gq, E * F, H, seed), [H, F, E])
        w["blk.0.ffn_up_exps.weight"] = (gq, rand_weights(gq, E * F, H, seed + 1), [H, F, E])
        w["blk.0.ffn_down_exps.weight"] = (dq, rand_weights(dq, E * H, F, seed + 2), [F, H, E])
    if shared:
        rw = rand_float_weights if sq in (J.F32, J.F16, J.BF16) else rand_weights
        w["blk.0.ffn_gate_shexp.weight"] = (sq, rw(sq, 2 * F, H, seed + 5), [H, 2 * F])
        w["blk.0.ffn_up_shexp.weight"] = (sq, rw(sq, 2 * F, H, seed + 6), [H, 2 * F])
        w["blk.0.ffn_down_shexp.weight"] = (sq, rw(sq, H, 2 * F, seed + 7), [2 * F, H])
    if dense:
        w["blk.0.ffn_gate.weight"] = (gq, rand_weights(gq, F, H, seed + 11), [H, F])
        w["blk.0.ffn_up.weight"] = (gq, rand_weights(gq, F, H, seed + 12), [H, F])
        w["blk.0.ffn_down.weight"] = (dq, rand_weights(dq, H, F, seed + 13), [F, H])
    return w


def device_weights(w, dev):
    return {n: J.TensorView(n, q, dims, td(data.view(np.uint8) if data.dtype != np.uint8 else data, dev))
            for n, (q, data, dims) in w.items()}


def indexed(w):
    """The stacked expert tensors split into per-expert tensors ffn_*_exps.{e}."""
    out = dict(w)
    for kind in ("gate", "up", "down"):
        key = f"blk.0.ffn_{kind}_exps.weight"
        if key not in out:
            continue
        q, data, dims = out.pop(key)
        E = dims[2]
        per = len(data) // E
        for e in range(E):
            out[f"blk.0.ffn_{kind}_exps.{e}.weight"] = (q, data[e * per:(e + 1) * per].copy(), dims[:2])
    return out


def run(dev, w, H, E, k, F, shared, seed, tol=TOL):
    x = rand_act(H, seed)
    ref, sel_ref = O.moe_layer(x, 0, E, k, F, shared, w)
    dw = device_weights(w, dev)
    y = torch.full((H,), float("nan"), dtype=torch.float32, device=dev)  # every element is written
    sel = J.moe_layer(y, td(x, dev), 0, E, k, F, shared, dw)
    torch.cuda.synchronize()
    assert [i for i, _ in sel] == [i for i, _ in sel_ref]
    np.testing.assert_allclose([v for _, v in sel], [v for _, v in sel_ref], rtol=1e-6, atol=1e-7)
    got = y.cpu().numpy()
    err = DP.rel(got, ref)
    print(f"  H={H} E={E} k={k} F={F} shared={shared}: error {err:.2e} (selection {[i for i, _ in sel]})", flush=True)
    assert err <= tol, err
    return got, sel


@pytest.mark.parametrize("E,k", [(16, 4), (128, 8), (200, 6)])
def test_shared_expert_and_routed(dev, E, k):
    """Qwen2-MoE-style layer: shared expert (Q8_0, twice the expert width) + routed Q4_K / Q6_K
    experts, one token; E = 200 runs the routed experts' many-expert path (route, group, combine)
    whose combine adds onto the shared expert's output."""
    print(f"moe layer shared + routed E={E} k={k}", flush=True)
    H, F = 512, 256
    w = make_weights(H, F, E, 100 + E)
    with_shared, _ = run(dev, w, H, E, k, F, True, 1)
    without, _ = run(dev, w, H, E, k, F, False, 1)
    assert not np.array_equal(with_shared, without)


def test_shared_expert_formats(dev):
    """The shared expert in Q4_K, Q6_K, F16, BF16 and F32 (the f32-input GEMV), router in Q8_0."""
    H, F, E, k = 256, 256, 8, 2
    for sq in (J.Q4_K, J.Q6_K, J.F16, J.BF16, J.F32):
        print(f"moe layer shared expert quant={sq}", flush=True)
        w = make_weights(H, F, E, 200 + sq, sq=sq, router_quant=J.Q8_0)
        run(dev, w, H, E, k, F, True, 2)


def test_no_router_dense_ffn(dev):
    """No ffn_gate_inp: the shared expert (when asked for) plus the dense FFN over ffn_gate /
    ffn_up / ffn_down; the same with num_experts = 0 and with top_k = 0; an empty selection."""
    H, F = 512, 512
    print("moe layer without router", flush=True)
    w = make_weights(H, F, 0, 300, dense=True)
    run(dev, w, H, 0, 4, F, True, 3)
    run(dev, w, H, 0, 4, F, False, 3)
    w2 = make_weights(H, F, 8, 301, dense=True)
    run(dev, w2, H, 0, 4, F, True, 4)  # num_experts = 0
    run(dev, w2, H, 8, 0, F, True, 4)  # top_k = 0


def test_dense_ffn_deterministic_fallbacks(dev):
    """The dense FFN with its tensors absent, or present with the wrong element count: each
    projection is x[i % len] * scale (0.5, 0.25, 0.125); nothing is quantized, so within 1e-6;
    F = max(ffn, 4) for ffn 2."""
    H = 256
    print("moe layer deterministic dense FFN", flush=True)
    run(dev, {}, H, 0, 2, 384, False, 5, tol=1e-6)
    run(dev, {}, H, 0, 2, 2, False, 6, tol=1e-6)
    w = make_weights(H, 256, 0, 310, shared=False, dense=True)
    w["blk.0.ffn_up.weight"] = (J.Q4_K, rand_weights(J.Q4_K, 255, H, 311), [H, 255])  # wrong size
    del w["blk.0.ffn_down.weight"]
    run(dev, w, H, 0, 2, 256, False, 7)


def test_per_expert_tensors(dev):
    """ffn_*_exps.{e} tensors for every expert (stacked on the device) give the same bits as the
    stacked tensors, with and without the shared expert; the routed experts read straight from one
    stack registered from host memory (jero_hip_weights_register_stacked) give them too."""
    H, F, E, k = 512, 256, 16, 4
    print("moe layer per-expert tensors", flush=True)
    w = make_weights(H, F, E, 400)
    ix = indexed(w)
    for shared in (True, False):
        a, sa = run(dev, w, H, E, k, F, shared, 8)
        b, sb = run(dev, ix, H, E, k, F, shared, 8)
        assert sa == sb and np.array_equal(a, b)
    # the registry's stack of host tensors: the bytes of the stacked tensor, one address
    J.init(0)
    parts = {kd: [ix[f"blk.0.ffn_{kd}_exps.{e}.weight"][1] for e in range(E)] for kd in ("gate", "up", "down")}
    addr = {kd: J.weights_register_stacked(p) for kd, p in parts.items()}
    for kd, p in parts.items():
        assert J.weights_register_stacked(p) == addr[kd]  # registered again: the same stack
        got = np.empty(sum(a.nbytes for a in p), np.uint8)
        J._memcpy(got.ctypes.data, addr[kd], got.nbytes)
        assert np.array_equal(got, w[f"blk.0.ffn_{kd}_exps.weight"][1])
    x = rand_act(H, 8)
    ref, sel_ref = O.moe_layer(x, 0, E, k, F, False, w)
    logits = torch.empty((1, E), dtype=torch.float32, device=dev)
    dw = device_weights(w, dev)
    J.matvec_any(logits.view(-1), dw["blk.0.ffn_gate_inp.weight"], td(x, dev))
    nb = {kd: sum(a.nbytes for a in p) for kd, p in parts.items()}
    views = {}
    for kd, (q, dims) in (("gate", (J.Q4_K, [H, F, E])), ("up", (J.Q4_K, [H, F, E])), ("down", (J.Q6_K, [F, H, E]))):
        buf = torch.empty(nb[kd], dtype=torch.uint8, device=dev)
        J._memcpy(buf.data_ptr(), addr[kd], nb[kd])  # device-to-device copy of the registered stack
        views[kd] = J.TensorView(kd, q, dims, buf)
    y = torch.empty((1, H), dtype=torch.float32, device=dev)
    si, sw = J.dispatch_qwen3_moe_ffn(y, td(x, dev).view(1, H), logits, k, views["gate"], views["up"], views["down"])
    torch.cuda.synchronize()
    assert si.view(-1).tolist() == [i for i, _ in sel_ref]
    assert DP.rel(y.view(-1).cpu().numpy(), ref) <= TOL
    for p in parts.values():
        for a in p:
            J.weights_release(a)


def test_register_stacked_errors(dev):
    J.init(0)
    a = [np.full(512, e, np.uint8) for e in range(4)]
    J.weights_register(a[1])  # one of them registered on its own
    with pytest.raises(J.K3Error) as ei:
        J.weights_register_stacked(a)
    assert ei.value.variant == "TensorBoundsError"
    J.weights_release(a[1])
    with pytest.raises(J.K3Error) as ei:  # tensors of different sizes are no stack
        J.weights_register_stacked([a[0], a[1][:256]])
    assert ei.value.variant == "TensorBoundsError"
    b = np.zeros(1024, np.uint8)
    with pytest.raises(J.K3Error) as ei:  # overlapping tensors
        J.weights_register_stacked([b[:512], b[256:768]])
    assert ei.value.variant == "TensorBoundsError"


def test_refusals(dev):
    """exp_probs_b (DeepSeek's biased routing) and per-expert tensors missing for some experts are
    refused with CapabilityMismatch instead of running anything else."""
    H, F, E, k = 256, 256, 8, 2
    print("moe layer refusals", flush=True)
    w = make_weights(H, F, E, 500)
    dw = device_weights(w, dev)
    dw["blk.0.exp_probs_b.bias"] = J.TensorView("blk.0.exp_probs_b.bias", J.F32, [E],
                                                torch.zeros(E, dtype=torch.float32, device=dev).view(torch.uint8))
    y = torch.zeros(H, dtype=torch.float32, device=dev)
    x = td(rand_act(H, 9), dev)
    with pytest.raises(J.K3Error) as ei:
        J.moe_layer(y, x, 0, E, k, F, True, dw)
    assert ei.value.variant == "CapabilityMismatch"
    ix = device_weights(indexed(w), dev)
    del ix["blk.0.ffn_up_exps.3.weight"]
    with pytest.raises(J.K3Error) as ei:
        J.moe_layer(y, x, 0, E, k, F, True, ix)
    assert ei.value.variant == "CapabilityMismatch"
