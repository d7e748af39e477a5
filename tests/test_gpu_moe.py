"""GPU parity of the routed-expert FFN against the oracle's dispatch_qwen3_moe_ffn.

Routing (selected experts and their order) must match exactly and the weights within 1e-6.
Outputs are checked per expert, as the decode step is (decode_parity): the oracle quantizes
each token, runs each selected expert's gate/up from those (bit-identical) activation blocks and
forms silu(g) * u; the device's f32 SwiGLU rows (jero_hip_moe_trace_view) must match within
1e-5 of their rms, and the two rows' quantizations (Q8_K, or ACT_Q8 for Q8_0 / Q4_0 down
experts) may differ only by tie flips
(decode_parity.tie_flips: pre-rounding values within 0.05 quantum everywhere, each flip a +-1
crossing of a rounding boundary between them).  The oracle then runs the expert's down
projection on the device's activation blocks and combines the experts in selection order in
f32, as the reference accumulates (src/qwen_deepseek.rs:847-951); the device's outputs must
match within the north-star 1e-5 of max(|ref|, rms(ref)) per token.
"""
import numpy as np
import pytest
import torch

import decode_parity as DP
import jero_hip as J
import pyoracle as O
from qdata import rand_act, rand_weights

pytestmark = pytest.mark.gpu

MOE_TOL = 1e-5


def run_case(dev, T, E, H, F, K, gq, dq, seed, logits=None, repacked=False):
    gate = rand_weights(gq, E * F, H, seed)
    up = rand_weights(gq, E * F, H, seed + 1)
    down = rand_weights(dq, E * H, F, seed + 2)
    x = rand_act(H, seed + 3, m=T)
    if logits is None:
        logits = rand_act(E, seed + 4, m=T)
    _, si_ref, sw_ref = O.moe_ffn(logits, K, gate, up, down, gq, gq, dq, H, F, x, threads=8)
    td = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    G = J.TensorView("blk.0.ffn_gate_exps.weight", gq, [H, F, E], td(gate))
    U = J.TensorView("blk.0.ffn_up_exps.weight", gq, [H, F, E], td(up))
    D = J.TensorView("blk.0.ffn_down_exps.weight", dq, [F, H, E], td(down))
    runs = [(G, U, D)]
    if repacked:  # the load-time layouts: 16-row tiles (_T), and the GEMV planes over all rows (_R)
        for experts, gl, dl in ((True, (J.Q4_K_T, J.Q6_K_T), (J.Q4_K_T, J.Q6_K_T)),
                                (False, (J.Q4_K_R, J.Q6_K_R), (J.Q4_K_R, J.Q6_K_R))):
            Gr, Ur, Dr = (J.repack(t, experts=experts) for t in (G, U, D))
            assert Gr.quant == gl[gq == J.Q6_K] and Dr.quant == dl[dq == J.Q6_K]
            runs.append((Gr, Ur, Dr))
    first = None
    for Gx, Ux, Dx in runs:
        ws = J.moe_workspace(T, E, K, H, F, dev)
        y = torch.empty((T, H), dtype=torch.float32, device=dev)
        si, sw = J.dispatch_qwen3_moe_ffn(y, td(x), td(logits), K, Gx, Ux, Dx, workspace=ws)
        torch.cuda.synchronize()
        if first is None:
            first = (si, sw)
            np.testing.assert_array_equal(si.cpu().numpy(), si_ref)
            np.testing.assert_allclose(sw.cpu().numpy(), sw_ref, rtol=1e-6, atol=1e-7)
        else:
            assert torch.equal(si, first[0]) and torch.equal(sw, first[1])
        act = J.moe_trace_act(ws, T, E, K, H, F)
        check_experts(y.cpu().numpy(), act, x, si_ref, sw_ref, gate, up, down, gq, dq, H, F)


def check_experts(y, act, x, si, sw, gate, up, down, gq, dq, H, F):
    gb, db = O.row_bytes(gq, H) * F, O.row_bytes(dq, F) * H
    st = DP.FlipStats()
    act_err = 0.0
    for t in range(x.shape[0]):
        xq = O.quantize_act(DP.act_fmt(gq), x[t])
        ref = np.zeros(H, np.float32)
        for j, e in enumerate(si[t]):
            g = O.matvec(gq, gate[e * gb:(e + 1) * gb], H, F, xq)
            u = O.matvec(gq, up[e * gb:(e + 1) * gb], H, F, xq)
            a_or = O.swiglu(g, u)
            a_dev = act[t, j]
            act_err = max(act_err, DP.rel(a_dev, a_or))
            af = DP.act_fmt(dq)
            q_dev = O.quantize_act(af, a_dev)
            st.add(DP.tie_flips(f"token {t} slot {j}", af, F, a_or, O.quantize_act(af, a_or), a_dev, q_dev))
            ref += np.float32(sw[t, j]) * O.matvec(dq, down[e * db:(e + 1) * db], F, H, q_dev)
        err = DP.rel(y[t], ref)
        assert err <= MOE_TOL, (t, err)
    print(f"  SwiGLU rows within {act_err:.1e}; {st.flips} tie flips (farthest {st.tie_dist:.1e} quanta from its "
          f"boundary, largest pre-rounding difference {st.pre_diff:.1e})", flush=True)
    assert act_err <= MOE_TOL, act_err


@pytest.mark.parametrize("T", [1, 64])
def test_moe_qwen3_shape(dev, T):
    """Hidden 2048, 128 experts of 768, top-8; gate/up Q4_K, down Q6_K."""
    print(f"moe qwen3 T={T}", flush=True)
    run_case(dev, T, 128, 2048, 768, 8, J.Q4_K, J.Q6_K, 900 + T, repacked=True)


@pytest.mark.parametrize("T", [1, 64])
def test_moe_hidden_4096(dev, T):
    """The Qwen3-235B-A22B expert shape: hidden 4096, 128 experts of 1536, top-8 (gate/up rows of
    64 units: two units per lane of a 32-lane row group)."""
    print(f"moe hidden 4096 T={T}", flush=True)
    run_case(dev, T, 128, 4096, 1536, 8, J.Q4_K, J.Q6_K, 950 + T, repacked=True)


def test_moe_hidden_8192_small(dev):
    """Four units per lane (hidden 8192), few experts."""
    print("moe hidden 8192", flush=True)
    run_case(dev, 3, 4, 8192, 256, 2, J.Q4_K, J.Q4_K, 960)


def test_moe_small_and_q4k_down(dev):
    print("moe small", flush=True)
    run_case(dev, 5, 6, 256, 512, 2, J.Q4_K, J.Q4_K, 40, repacked=True)
    run_case(dev, 3, 16, 512, 256, 4, J.Q6_K, J.Q6_K, 41, repacked=True)


def test_moe_single_token(dev):
    """One token (two launches: gate/up routes the token itself, down sums the experts in selection
    order): Q4_K and Q6_K throughout, GGUF and repacked layouts, and the tie / NaN routing rules."""
    print("moe single token", flush=True)
    run_case(dev, 1, 6, 256, 512, 2, J.Q4_K, J.Q4_K, 45, repacked=True)
    run_case(dev, 1, 16, 512, 256, 4, J.Q6_K, J.Q6_K, 46, repacked=True)
    run_case(dev, 1, 128, 1024, 768, 16, J.Q4_K, J.Q6_K, 47)
    logits = np.array([[np.nan, 1.0, np.inf, 1.0, -np.inf, 0.5, 0.5, 2.0]], np.float32)
    run_case(dev, 1, 8, 256, 256, 3, J.Q4_K, J.Q6_K, 61, logits=logits)


def test_moe_many_tokens_per_expert(dev):
    """Four experts for 40 tokens at top-2: each expert sees ~20 tokens, several token passes.
    Two tokens or more per expert on average run the MFMA expert GEMMs (Q4_K in either layout,
    Q6_K repacked); GGUF Q6_K down runs the GEMV kernels."""
    print("moe many tokens per expert", flush=True)
    run_case(dev, 40, 4, 512, 512, 2, J.Q4_K, J.Q6_K, 42, repacked=True)
    run_case(dev, 40, 4, 512, 512, 2, J.Q4_K, J.Q4_K, 43, repacked=True)
    run_case(dev, 24, 3, 256, 768, 3, J.Q6_K, J.Q6_K, 44, repacked=True)


@pytest.mark.parametrize("T", [1, 5, 40])
def test_moe_q8_0_and_q4_0_experts(dev, T):
    """Experts in the 32-element formats, whose activations are ACT_Q8 blocks (the token rows
    quantized by the routing step or by the one-token gate/up kernel, the SwiGLU rows by the down
    kernels): Q8_0 throughout, Q4_0 throughout, and each beside a K-quant; one token, a few, and
    ~20 tokens per expert (the GEMV kernels' token passes: these formats take no MFMA path)."""
    print(f"moe q8_0 / q4_0 experts T={T}", flush=True)
    run_case(dev, T, 8, 512, 512, 4, J.Q8_0, J.Q8_0, 1100 + T)
    run_case(dev, T, 8, 512, 256, 4, J.Q4_0, J.Q4_0, 1110 + T)
    run_case(dev, T, 8, 256, 512, 2, J.Q8_0, J.Q6_K, 1120 + T)
    run_case(dev, T, 8, 256, 512, 2, J.Q4_K, J.Q4_0, 1130 + T)


def test_moe_q8_0_qwen3_shape(dev):
    """Hidden 2048 (two units per lane of a 32-lane row group), 128 experts of 768, top-8, Q8_0."""
    print("moe qwen3 shape q8_0", flush=True)
    run_case(dev, 1, 128, 2048, 768, 8, J.Q8_0, J.Q8_0, 1140)
    run_case(dev, 64, 128, 2048, 768, 8, J.Q8_0, J.Q8_0, 1141)


@pytest.mark.parametrize("T,E,K", [(130, 16, 8), (300, 64, 4), (200, 700, 16)])
def test_moe_grouping_paths(dev, T, E, K):
    """More than 1024 (token, slot) pairs, past the grouping step's per-pair rank: placed from
    per-expert token bitmasks when E * ceil(T / 32) words fit in LDS (the first two), else by
    sorting the (expert, pair) keys (the third); the experts' GEMMs and the combine read the
    lists, so the outputs check them."""
    print(f"moe grouping T={T} E={E} k={K}", flush=True)
    run_case(dev, T, E, 256, 256, K, J.Q4_K, J.Q6_K, 80 + T)


@pytest.mark.parametrize("E,K", [(200, 6), (300, 8), (700, 16)])
def test_moe_many_experts(dev, E, K):
    """Router widths above 128 experts (4, 8 and 16 expert columns per lane), top-k up to 16."""
    print(f"moe E={E} k={K}", flush=True)
    run_case(dev, 3, E, 256, 256, K, J.Q4_K, J.Q6_K, 70 + E)


def test_moe_routing_ties_and_nonfinite(dev):
    """Ties pick the lower expert id; NaN/inf logits rank last with zero probability."""
    print("moe ties", flush=True)
    E = 8
    logits = np.array([[0.1, 3.0, 0.5, 1.0, 3.0, 2.0, -1.0, 0.0],
                       [np.nan, 1.0, np.inf, 1.0, -np.inf, 0.5, 0.5, 2.0]], np.float32)
    run_case(dev, 2, E, 256, 256, 3, J.Q4_K, J.Q6_K, 60, logits=logits)


def test_moe_routing_signed_zero_total_order(dev):
    """The router ranks by f32::total_cmp (src/gemma.rs:417): +0.0 above -0.0, ties by index,
    on both the one-token path and the many-token routing."""
    print("moe signed zero", flush=True)
    nz = np.float32(-0.0)
    one = np.array([[nz, 0.0, nz, nz, 0.0, -1.0, nz, nz]], np.float32)
    run_case(dev, 1, 8, 256, 256, 3, J.Q4_K, J.Q6_K, 62, logits=one)
    two = np.array([[nz, 0.0, -2.0, -3.0, -4.0, -5.0, -6.0, -7.0], [0.0, nz, -2.0, -3.0, -4.0, -5.0, -6.0, -7.0]],
                   np.float32)
    run_case(dev, 2, 8, 256, 256, 1, J.Q4_K, J.Q6_K, 63, logits=two)


def test_moe_argument_errors(dev):
    z = torch.zeros(4096, dtype=torch.float32, device=dev)
    G = J.TensorView("g", J.Q4_K, [256, 256, 4], torch.zeros(4 * 256 * 144, dtype=torch.uint8, device=dev))
    D = J.TensorView("d", J.Q6_K, [256, 256, 4], torch.zeros(4 * 256 * 210, dtype=torch.uint8, device=dev))
    with pytest.raises(J.K3Error) as ei:
        J.dispatch_qwen3_moe_ffn(z[:256].view(1, 256), z[:256], z[:4].view(1, 4), 5, G, G, D)
    assert ei.value.variant == "CapabilityMismatch"
    with pytest.raises(J.K3Error) as ei:
        J.dispatch_qwen3_moe_ffn(z[:256].view(1, 256), z[:256], z[:4].view(1, 4), 0, G, G, D)
    assert ei.value.variant == "RoutingUnavailable"
