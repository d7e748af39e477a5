"""Random-init decoder weights (Qwen3 layout, dense or Qwen3-MoE) for the decode parity tests.

Quantized matrices are uniform random payload bytes with N(0, 0.02)-scale fields (qdata);
norm weights are 1 + 0.1 N(0, 1).  The Q4_K_M mix follows llama.cpp's public recipe:
Q6_K for attn_v / ffn_down on layers i < n/8, i >= 7n/8 or (i - n/8) % 3 == 2; Q6_K head.
"""
import numpy as np

from qdata import Q4_K, Q6_K, Q8_0, F32, rand_weights


def q6k_layers(n):
    return [i for i in range(n) if i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2]


def build(spec, seed=0, mix="q4_k_m"):
    H, F, L, V = spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"]
    Q, KV, hd = spec["nq"] * spec["hd"], spec["nkv"] * spec["hd"], spec["hd"]
    rng = np.random.default_rng(seed)
    hi = set(q6k_layers(L)) if mix == "q4_k_m" else set()
    t = {}
    s = [seed * 100]

    def mat(name, quant, n_in, n_out):
        s[0] += 1
        t[name] = (quant, rand_weights(quant, n_out, n_in, s[0]), n_in, n_out)

    def norm(name, n):
        t[name] = (F32, (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32), n, 1)

    mat("token_embd.weight", Q4_K, H, V)
    mat("output.weight", Q6_K, H, V)
    norm("output_norm.weight", H)
    for i in range(L):
        p = f"blk.{i}."
        norm(p + "attn_norm.weight", H)
        norm(p + "ffn_norm.weight", H)
        norm(p + "attn_q_norm.weight", hd)
        norm(p + "attn_k_norm.weight", hd)
        mat(p + "attn_q.weight", Q4_K, H, Q)
        mat(p + "attn_k.weight", Q4_K, H, KV)
        mat(p + "attn_v.weight", Q6_K if i in hi else Q4_K, H, KV)
        mat(p + "attn_output.weight", Q4_K, Q, H)
        mat(p + "ffn_gate.weight", Q4_K, H, F)
        mat(p + "ffn_up.weight", Q4_K, H, F)
        mat(p + "ffn_down.weight", Q6_K if i in hi else Q4_K, F, H)
    return t


def build_moe(spec, moe, seed=0, router_layers=None, shared_quant=Q8_0, router_quant=F32, down_quant=Q6_K,
              gate_quant=Q4_K):
    """A Qwen3-MoE-shaped model (the Qwen3 attention of build, then per layer
    dispatch_qwen3_moe_ffn's tensors): a router [hidden, E] of N(0, 0.02) weights (router_quant:
    F32, F16 or BF16 values, or a quantized format), the stacked gate / up experts [hidden, F, E]
    in gate_quant and down experts [F, hidden, E] in down_quant, and, when moe's use_shared is set,
    a shared expert of 2 F rows in shared_quant.  Layers not in router_layers (all by default) have
    no router: they take run_dense_swiglu_ffn with [hidden, F] gate_quant gate / up and down_quant
    down.
    moe = (E, top_k, F, use_shared).  Returns (tensors as build returns them,
    {name: (quant, data, dims)} as pyoracle.moe_layer reads them)."""
    from qdata import F16, BF16, rand_float_weights
    E, k, F, shared = moe
    H, L = spec["hidden"], spec["n_layers"]
    t = build(spec, seed)
    for i in range(L):
        for b in ("ffn_gate", "ffn_up", "ffn_down"):
            del t[f"blk.{i}.{b}.weight"]
    w = {}
    s = [seed * 100 + 50]

    def mat(name, quant, dims, rows, n_in, gen=rand_weights):
        s[0] += 1
        arr = gen(quant, rows, n_in, s[0])
        n_out = int(np.prod(dims[1:]))
        t[name] = (quant, arr, dims[0], n_out)
        w[name] = (quant, arr, list(dims))

    for i in range(L):
        p = f"blk.{i}."
        if router_layers is None or i in router_layers:
            float_router = router_quant in (F32, F16, BF16)
            mat(p + "ffn_gate_inp.weight", router_quant, (H, E), E, H, rand_float_weights if float_router else rand_weights)
            mat(p + "ffn_gate_exps.weight", gate_quant, (H, F, E), E * F, H)
            mat(p + "ffn_up_exps.weight", gate_quant, (H, F, E), E * F, H)
            mat(p + "ffn_down_exps.weight", down_quant, (F, H, E), E * H, F)
        else:
            mat(p + "ffn_gate.weight", gate_quant, (H, F), F, H)
            mat(p + "ffn_up.weight", gate_quant, (H, F), F, H)
            mat(p + "ffn_down.weight", down_quant, (F, H), H, F)
        if shared:
            mat(p + "ffn_gate_shexp.weight", shared_quant, (H, 2 * F), 2 * F, H)
            mat(p + "ffn_up_shexp.weight", shared_quant, (H, 2 * F), 2 * F, H)
            mat(p + "ffn_down_shexp.weight", shared_quant, (2 * F, H), H, 2 * F)
        nq, nd = t[p + "ffn_norm.weight"][:2]
        w[p + "ffn_norm.weight"] = (nq, nd, [H])
    return t, w


def oracle_tensors(t):
    """{name: (quant, array)} for pyoracle.DecodeModel."""
    return {k: (v[0], v[1]) for k, v in t.items()}


def _dev_weights(torch, quant, rows, k, gen, dev):
    """rows x k random blocks of `quant` generated on the device: uniform payload bytes, scale
    fields at the magnitudes rand_weights uses."""
    from qdata import BLOCK
    be, bb = BLOCK[quant]
    nb = rows * (k // be)
    b = torch.randint(0, 256, (nb, bb), dtype=torch.uint8, device=dev, generator=gen)
    u = lambda lo, hi: (torch.rand(nb, device=dev, generator=gen) * (hi - lo) + lo).half().view(torch.uint8).view(nb, 2)
    if quant == Q4_K:
        b[:, 0:2] = u(1e-4, 4e-4)
        b[:, 2:4] = u(5e-4, 2e-3)
    elif quant == Q6_K:
        b[:, 192:208] = torch.randint(-64, 64, (nb, 16), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        b[:, 208:210] = u(1e-4, 3e-4)
    elif quant == Q8_0:
        b[:, 0:2] = u(2e-4, 6e-4)
        b[:, 2:] = torch.randint(-127, 128, (nb, 32), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
    else:
        raise ValueError(quant)
    return b.reshape(-1)


def build_device(spec, dev, seed=0, mix="q4_k_m"):
    """The same model layout as build(), with the quantized matrices generated on the GPU (fast at
    the 8B shape): {name: (quant, host numpy array, n_in, n_out)} plus {name: device tensor}.
    mix "q8_0": every matrix Q8_0."""
    import torch
    H, F, L, V = spec["hidden"], spec["ffn"], spec["n_layers"], spec["vocab"]
    Q, KV, hd = spec["nq"] * spec["hd"], spec["nkv"] * spec["hd"], spec["hd"]
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    rng = np.random.default_rng(seed)
    hi = set(q6k_layers(L)) if mix == "q4_k_m" else set()
    host, on_dev = {}, {}

    def mat(name, quant, n_in, n_out):
        if mix == "q8_0":
            quant = Q8_0
        d = _dev_weights(torch, quant, n_out, n_in, gen, dev)
        on_dev[name] = d
        host[name] = (quant, d.cpu().numpy(), n_in, n_out)

    def norm(name, n):
        host[name] = (F32, (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32), n, 1)

    mat("token_embd.weight", Q4_K, H, V)
    mat("output.weight", Q6_K, H, V)
    norm("output_norm.weight", H)
    for i in range(L):
        p = f"blk.{i}."
        norm(p + "attn_norm.weight", H)
        norm(p + "ffn_norm.weight", H)
        norm(p + "attn_q_norm.weight", hd)
        norm(p + "attn_k_norm.weight", hd)
        mat(p + "attn_q.weight", Q4_K, H, Q)
        mat(p + "attn_k.weight", Q4_K, H, KV)
        mat(p + "attn_v.weight", Q6_K if i in hi else Q4_K, H, KV)
        mat(p + "attn_output.weight", Q4_K, Q, H)
        mat(p + "ffn_gate.weight", Q4_K, H, F)
        mat(p + "ffn_up.weight", Q4_K, H, F)
        mat(p + "ffn_down.weight", Q6_K if i in hi else Q4_K, F, H)
    return host, on_dev
