"""ctypes front end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline.
The function list, the reference citations and the parity pins are in oracle.h.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K, ACT_Q8 = 0, 1, 2, 8, 12, 14, 15, 100
BF16 = 30

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle` (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        P, I64, I32, F = C.c_void_p, C.c_int64, C.c_int, C.c_float
        sig = {
            "jo_f16_to_f32": (F, [C.c_uint16]),
            "jo_f32_to_f16": (C.c_uint16, [F]),
            "jo_block_elems": (I64, [I32]),
            "jo_block_bytes": (I64, [I32]),
            "jo_row_bytes": (I64, [I32, I64]),
            "jo_act_format": (I32, [I32]),
            "jo_dequantize_row": (I32, [I32, P, I64, P]),
            "jo_quantize_act_q8": (None, [P, I64, I64, P]),
            "jo_quantize_q8_k": (None, [P, I64, I64, P]),
            "jo_quantize_act": (None, [I32, P, I64, I64, P]),
            "jo_partials_per_row": (I64, [I32, I64]),
            "jo_vec_dot_row": (C.c_double, [I32, P, I64, P, P]),
            "jo_matvec": (I32, [I32, P, I64, I64, P, P, I32]),
            "jo_vec_dot": (I32, [I32, P, I64, I64, P, P, I32]),
            "jo_matvec_dequant_f64": (I32, [I32, P, I64, I64, P, P]),
            "jo_matvec_partials": (I32, [I32, P, I64, I64, P, P]),
            "jo_gemm": (I32, [I32, P, I64, I64, P, I64, P, I32]),
            "jo_gemm_i8": (None, [P, I64, P, I64, I64, P]),
            "jo_gqa_attention": (I32, [P, P, P, P, I32, I32, I32, I64, F]),
            "jo_rmsnorm": (None, [P, P, P, I64, F]),
            "jo_rope_inplace": (None, [P, I64, I32, I64, F]),
            "jo_swiglu": (None, [P, P, P, I64]),
            "jo_argmax": (I64, [P, I64]),
            "jo_select_top_k": (I32, [P, I64, I32, I32, P, P]),
            "jo_swiglu_expert": (I32, [I32, P, I32, P, I32, P, I64, I64, P, P]),
            "jo_moe_ffn": (I32, [P, I64, I64, I32, I32, P, I32, P, I32, P, I64, I64, P, P, P, P, I32]),
            "jo_decode_step": (I32, [P, P, I32, I64, P, I32]),
            "jo_decode_layer": (I32, [P, P, I64, P, I64, I32, P]),
            "jo_decode_attn": (I32, [P, P, I64, P, I64, I32, P]),
            "jo_decode_head": (I32, [P, P, P, I32, P, P]),
            "jo_read_f32_weight_or_default": (None, [I32, P, I64, I64, F, P]),
            "jo_logits_len": (I64, [I64, I32, I64]),
            "jo_embed_token": (I32, [P, C.c_uint32, P]),
            "jo_splitmix": (C.c_uint64, [C.c_uint64]),
            "jo_fill_small": (None, [C.c_uint64, I64, P]),
            "jo_isqrt": (C.c_uint64, [C.c_uint64]),
            "jo_fwd_rmsnorm": (None, [P, I64, P]),
            "jo_fwd_attention": (None, [P, P, P, I64, I64, P]),
            "jo_fwd_embed": (None, [C.c_uint64, C.c_uint32, P]),
            "jo_fwd_new": (P, [C.c_uint64, I64, I64]),
            "jo_fwd_free": (None, [P]),
            "jo_fwd_head_rows": (I64, [P]),
            "jo_fwd_len": (I64, [P]),
            "jo_fwd_reset": (None, [P]),
            "jo_fwd_set_threads": (None, [P, I32]),
            "jo_fwd_weight": (P, [P, I32, I32, P, P, P]),
            "jo_fwd_forward": (I32, [P, P, I64, I64, P]),
            "jo_fwd_sample": (C.c_uint32, [P, I64]),
            "jo_fwd_evaluate": (I32, [P, P, I64, I64, P]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(C.c_void_p) if a is not None else None


def act_format(weight_quant):
    return lib().jo_act_format(weight_quant)


def row_bytes(quant, n):
    return lib().jo_row_bytes(quant, n)


def dequantize(quant, data, rows, k):
    data = np.ascontiguousarray(data, dtype=np.uint8)
    out = np.empty((rows, k), np.float32)
    rb = row_bytes(quant, k)
    for r in range(rows):
        rc = lib().jo_dequantize_row(quant, C.c_void_p(data.ctypes.data + r * rb), k, _p(out[r]))
        assert rc == 0
    return out


def quantize_act(act_quant, x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    m, k = (1, x.shape[0]) if x.ndim == 1 else x.shape
    out = np.empty(m * row_bytes(act_quant, k), np.uint8)
    lib().jo_quantize_act(act_quant, _p(x), m, k, _p(out))
    return out


def matvec(quant, w, k, n, xq, threads=1):
    y = np.empty(n, np.float32)
    rc = lib().jo_matvec(quant, _p(w), k, n, _p(xq), _p(y), threads)
    assert rc == 0
    return y


def vec_dot(quant, w, k, n, x, threads=1):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(n, np.float32)
    rc = lib().jo_vec_dot(quant, _p(w), k, n, _p(x), _p(y), threads)
    assert rc == 0
    return y


def matvec_f64(quant, w, k, n, xq):
    y = np.empty(n, np.float64)
    rc = lib().jo_matvec_dequant_f64(quant, _p(w), k, n, _p(xq), _p(y))
    assert rc == 0
    return y


def partials(quant, w, k, n, xq):
    pp = lib().jo_partials_per_row(quant, k)
    out = np.empty((n, pp), np.int32)
    rc = lib().jo_matvec_partials(quant, _p(w), k, n, _p(xq), _p(out))
    assert rc == 0
    return out


def gemm(quant, w, k, n, xq, m, threads=1):
    y = np.empty((m, n), np.float32)
    rc = lib().jo_gemm(quant, _p(w), k, n, _p(xq), m, _p(y), threads)
    assert rc == 0
    return y


def gemm_i8(x, w):
    x = np.ascontiguousarray(x, dtype=np.int8)
    w = np.ascontiguousarray(w, dtype=np.int8)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.int32)
    lib().jo_gemm_i8(_p(x), m, _p(w), n, k, _p(out))
    return out


def requant(v, shift):
    """requant (src/forward.rs:345-350): (v + 2^(shift-1)) >> shift, clamped to [-127, 127], as int8.
    The i32 add wraps as two's complement (the reference's release build); >> is arithmetic."""
    v = np.asarray(v, np.int64)
    t = (v + (1 << (shift - 1)) + (1 << 31)) % (1 << 32) - (1 << 31)
    return np.clip(t >> shift, -127, 127).astype(np.int8)


def pack_tiles(x, rows, k, tile_rows=8, tile_k=32):
    """This library's ime::pack_tiles layout: element (r, c) at
    ((r // 8 * (k // 32) + c // 32) * 8 + r % 8) * 32 + c % 32, rows padded with zero rows."""
    t = -(-rows // tile_rows)
    p = np.zeros((t * tile_rows, k), np.int8)
    p[:rows] = np.asarray(x, np.int8).reshape(rows, k)
    return p.reshape(t, tile_rows, k // tile_k, tile_k).transpose(0, 2, 1, 3).reshape(-1).copy()


def gqa_attention(q, k, v, nq, nkv, hd, seq_len, scale):
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    out = np.empty(nq * hd, np.float32)
    rc = lib().jo_gqa_attention(_p(out), _p(q), _p(k), _p(v), nq, nkv, hd, seq_len, scale)
    assert rc == 0
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(x)
    lib().jo_rmsnorm(_p(out), _p(x), _p(w), x.size, eps)
    return out


def rope(x, hd, pos, theta):
    x = np.array(x, dtype=np.float32, copy=True)
    lib().jo_rope_inplace(_p(x), x.size, hd, pos, theta)
    return x


def swiglu(g, u):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    out = np.empty_like(g)
    lib().jo_swiglu(_p(out), _p(g), _p(u), g.size)
    return out


def argmax(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    r = lib().jo_argmax(_p(x), x.size)
    return None if r < 0 else int(r)


def select_top_k(logits, k, normalize=True):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.zeros(max(k, 1), np.int32)
    w = np.zeros(max(k, 1), np.float32)
    n = lib().jo_select_top_k(_p(logits), logits.size, k, 1 if normalize else 0, _p(idx), _p(w))
    return [(int(idx[i]), float(w[i])) for i in range(n)]


def moe_ffn(router_logits, top_k, gate, up, down, gq, uq, dq, hidden, ffn, x, threads=1):
    router_logits = np.ascontiguousarray(router_logits, dtype=np.float32)
    t, E = router_logits.shape
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(t, hidden)
    y = np.empty((t, hidden), np.float32)
    si = np.empty((t, top_k), np.int32)
    sw = np.empty((t, top_k), np.float32)
    rc = lib().jo_moe_ffn(_p(router_logits), t, E, top_k, gq, _p(gate), uq, _p(up), dq, _p(down), hidden, ffn,
                          _p(x), _p(y), _p(si), _p(sw), threads)
    assert rc == 0
    return y, si, sw


# ---- the whole MoE layer: dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951) ----
# `weights` maps GGUF names to (quant, data, dims): data the tensor's bytes (uint8) or f32 values,
# dims its GGUF shape ([n_in, rows] or [n_in, rows, n_experts]).

def _n_el(dims):
    n = 1
    for d in dims:
        n *= d
    return n


def proj_or_det(w, x, out_len, scale, threads=1):
    """project_or_deterministic_slice (src/gemma.rs:841-860): the GEMV when the tensor is present
    with exactly out_len * len(x) elements, else out[i] = x[i % len(x)] * scale."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if w is not None and _n_el(w[2]) == out_len * x.size:
        return vec_dot(w[0], w[1], x.size, out_len, x, threads)
    return (x[np.arange(out_len) % x.size] * np.float32(scale)).astype(np.float32)


def single_swiglu_expert(g, u, d, x, expert_ffn_dim, threads=1):
    """run_single_swiglu_expert (src/qwen_deepseek.rs:748-771): eff_ffn from the gate's element
    count, then matvec_any of gate and up over x, SwiGLU, matvec_any of down."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    H, ge = x.size, _n_el(g[2])
    F = ge // H if ge > 0 and ge % H == 0 else max(expert_ffn_dim, 4)
    act = swiglu(vec_dot(g[0], g[1], H, F, x, threads), vec_dot(u[0], u[1], H, F, x, threads))
    return vec_dot(d[0], d[1], F, H, act, threads)


def dense_swiglu_ffn(weights, layer, expert_ffn_dim, x, threads=1):
    """run_dense_swiglu_ffn (src/qwen_deepseek.rs:696-727)."""
    F = max(expert_ffn_dim, 4)
    name = lambda t: f"blk.{layer}.{t}.weight"
    g = proj_or_det(weights.get(name("ffn_gate")), x, F, 0.5, threads)
    u = proj_or_det(weights.get(name("ffn_up")), x, F, 0.25, threads)
    return proj_or_det(weights.get(name("ffn_down")), swiglu(g, u), len(x), 0.125, threads)


def _expert_slice(weights, stacked, indexed, e, n):
    """slice_or_lookup_expert (src/qwen_deepseek.rs:729-746): expert e of n equal parts of a 3-D
    stacked tensor, else the per-expert tensor, else None."""
    st = weights.get(stacked)
    if st is not None and len(st[2]) == 3:
        per = len(st[1]) // n
        rows = _n_el(st[2]) // n // st[2][0]
        return (st[0], st[1][e * per:(e + 1) * per], [st[2][0], rows])
    return weights.get(indexed)


def moe_layer(x, layer, num_experts, top_k, expert_ffn_dim, use_shared_expert, weights, threads=1):
    """dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951) without the exp_probs_b bias: returns
    (out [hidden] f32, [(expert, weight)])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    H = x.size
    name = lambda t: f"blk.{layer}.{t}.weight"
    out = np.zeros(H, np.float32)
    sh = [weights.get(name(t)) for t in ("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp")]
    if use_shared_expert and all(t is not None for t in sh):
        out += single_swiglu_expert(*sh, x, expert_ffn_dim, threads)
    router = weights.get(name("ffn_gate_inp"))
    if num_experts == 0 or top_k == 0 or router is None:
        out += dense_swiglu_ffn(weights, layer, expert_ffn_dim, x, threads)
        return out, []
    re = _n_el(router[2])
    eff = min(re // H, num_experts) if re > 0 and re % H == 0 else num_experts
    logits = vec_dot(router[0], router[1], H, eff, x, threads)
    sel = select_top_k(logits, top_k, True)
    ran = False
    for e, w in sel:
        parts = [_expert_slice(weights, f"blk.{layer}.ffn_{k}_exps.weight", f"blk.{layer}.ffn_{k}_exps.{e}.weight", e,
                               eff) for k in ("gate", "up", "down")]
        if all(p is not None for p in parts):
            out += np.float32(w) * single_swiglu_expert(*parts, x, expert_ffn_dim, threads)
            ran = True
    if not ran:
        out += dense_swiglu_ffn(weights, layer, expert_ffn_dim, x, threads)
    return out, sel


# ---- decode model (jo_model / jo_layer structs) ----

class JoTensor(C.Structure):
    _fields_ = [("quant", C.c_int), ("data", C.c_void_p)]


class JoLayer(C.Structure):
    _fields_ = [("attn_norm", C.c_void_p), ("ffn_norm", C.c_void_p), ("q_norm", C.c_void_p),
                ("k_norm", C.c_void_p), ("wq", JoTensor), ("wk", JoTensor), ("wv", JoTensor), ("wo", JoTensor),
                ("w_gate", JoTensor), ("w_up", JoTensor), ("w_down", JoTensor)]


class JoModel(C.Structure):
    _fields_ = [("hidden", C.c_int64), ("ffn", C.c_int64), ("n_layers", C.c_int64), ("vocab", C.c_int64),
                ("nq", C.c_int), ("nkv", C.c_int), ("hd", C.c_int), ("eps", C.c_float), ("theta", C.c_float),
                ("kv_capacity", C.c_int64), ("tok_embd", JoTensor), ("output", JoTensor),
                ("output_norm", C.c_void_p), ("layers", C.c_void_p), ("kv_f16", C.c_int),
                ("embd_rows", C.c_int64), ("out_in", C.c_int64), ("out_rows", C.c_int64), ("logits_len", C.c_int64)]


class JoLayerTrace(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("xn_attn", "q8_attn", "qkv", "q_rope", "k_rope", "attn", "q8_wo", "x_mid",
                                          "xn_ffn", "q8_ffn", "gu", "act", "q8_down")]


def act_row_bytes(weight_quant, k):
    return row_bytes(lib().jo_act_format(weight_quant), k)


def _elements(quant, arr, dims=None):
    """Element count of a tensor given as (quant, array[, n_in, n_out])."""
    if dims is not None:
        return int(dims[0]) * int(dims[1])
    a = np.asarray(arr)
    if quant == F32 and a.dtype == np.float32:
        return a.size
    be, bb = int(lib().jo_block_elems(quant)), int(lib().jo_block_bytes(quant))
    return a.nbytes // bb * be


def read_f32_weight_or_default(quant, arr, n_elements, length, default=1.0):
    """jo_read_f32_weight_or_default: arr None for an absent tensor."""
    out = np.empty(length, np.float32)
    if arr is None:
        lib().jo_read_f32_weight_or_default(quant, None, 0, length, default, _p(out))
        return out
    a = np.ascontiguousarray(arr)
    lib().jo_read_f32_weight_or_default(quant, a.ctypes.data, n_elements, length, default, _p(out))
    return out


def logits_len(vocab, head_rows):
    """jo_logits_len (infer_logits_buffer_len); head_rows None: no head tensor."""
    return int(lib().jo_logits_len(vocab, 0 if head_rows is None else 1, 0 if head_rows is None else head_rows))


class DecodeModel:
    """Holds a jo_model over numpy-owned tensors (see tests/model_spec.py for the dict layout).
    tensors: {name: (quant, array) or (quant, array, n_in, n_out)}.  Norm weights go through
    read_f32_weight_or_default (absent: ones); qk_norm (default: whether blk.0's q-norm weight is
    given) applies QK-norm with such weights.  The head is output.weight, else token_embd.weight
    (ModelWeights' tied fallback), else none; logits are infer_logits_buffer_len long."""

    def __init__(self, spec, tensors, kv_capacity, qk_norm=None):
        self._keep = []
        s = spec
        nl = s["n_layers"]
        H, hd = s["hidden"], s["hd"]
        self.layers = (JoLayer * nl)()
        if qk_norm is None:
            qk_norm = "blk.0.attn_q_norm.weight" in tensors

        def dims(name):
            v = tensors[name]
            return (v[2], v[3]) if len(v) >= 4 else None

        def t(name):
            if name not in tensors:  # a projection left out: the deterministic slice (gemma.rs:841-860)
                return JoTensor(0, None)
            quant, arr = tensors[name][:2]
            arr = np.ascontiguousarray(arr)
            self._keep.append(arr)
            return JoTensor(quant, arr.ctypes.data)

        def f(name, length, need=True):
            if not need:
                return None
            if name not in tensors:
                arr = read_f32_weight_or_default(F32, None, 0, length)
            else:
                quant, a = tensors[name][:2]
                arr = read_f32_weight_or_default(quant, a, _elements(quant, a, dims(name)), length)
            self._keep.append(arr)
            return arr.ctypes.data

        for L in range(nl):
            p = f"blk.{L}."
            self.layers[L] = JoLayer(f(p + "attn_norm.weight", H), f(p + "ffn_norm.weight", H),
                                     f(p + "attn_q_norm.weight", hd, qk_norm), f(p + "attn_k_norm.weight", hd, qk_norm),
                                     t(p + "attn_q.weight"), t(p + "attn_k.weight"), t(p + "attn_v.weight"),
                                     t(p + "attn_output.weight"), t(p + "ffn_gate.weight"), t(p + "ffn_up.weight"),
                                     t(p + "ffn_down.weight"))
        embd_rows = 0
        if "token_embd.weight" in tensors:
            q, a = tensors["token_embd.weight"][:2]
            embd_rows = _elements(q, a, dims("token_embd.weight")) // H
        head = "output.weight" if "output.weight" in tensors else (
            "token_embd.weight" if "token_embd.weight" in tensors else None)
        out_in = out_rows = 0
        if head is not None:
            q, a = tensors[head][:2]
            dm = dims(head)
            out_in, out_rows = dm if dm is not None else (H, _elements(q, a) // H)
        self.logits_len = logits_len(s["vocab"], None if head is None else out_rows)
        self.model = JoModel(s["hidden"], s["ffn"], nl, s["vocab"], s["nq"], s["nkv"], s["hd"], s["eps"],
                             s["theta"], kv_capacity, t("token_embd.weight"),
                             t(head) if head is not None else JoTensor(0, None),
                             f("output_norm.weight", H), C.cast(self.layers, C.c_void_p), 0,
                             embd_rows, out_in, out_rows, self.logits_len)
        self.kv_capacity = kv_capacity
        self.kvd = s["nkv"] * s["hd"]
        self.spec = s

    def new_kv(self):
        return np.zeros((self.spec["n_layers"], 2, self.kv_capacity, self.kvd), np.float32)

    def step(self, kv, token, pos, threads=1):
        logits = np.empty(self.logits_len, np.float32)
        rc = lib().jo_decode_step(C.byref(self.model), _p(kv), token, pos, _p(logits), threads)
        assert rc == 0
        return logits

    def embed(self, token):
        x = np.empty(self.spec["hidden"], np.float32)
        assert lib().jo_embed_token(C.byref(self.model), token, _p(x)) == 0
        return x

    def layer(self, kv, L, x, pos, threads=1, trace=True):
        """jo_decode_layer: returns (x_out, trace dict of the layer's intermediate values)."""
        s = self.spec
        H, F = s["hidden"], s["ffn"]
        qd, kvd = s["nq"] * s["hd"], s["nkv"] * s["hd"]
        ly = self.layers[L]
        x = np.array(x, np.float32, copy=True)
        tr = None
        out = {}
        if trace:
            out = dict(xn_attn=np.empty(H, np.float32), q8_attn=np.empty(act_row_bytes(ly.wq.quant, H), np.uint8),
                       qkv=np.empty(qd + 2 * kvd, np.float32), q_rope=np.empty(qd, np.float32),
                       k_rope=np.empty(kvd, np.float32), attn=np.empty(qd, np.float32),
                       q8_wo=np.empty(act_row_bytes(ly.wo.quant, qd), np.uint8), x_mid=np.empty(H, np.float32),
                       xn_ffn=np.empty(H, np.float32), q8_ffn=np.empty(act_row_bytes(ly.w_gate.quant, H), np.uint8),
                       gu=np.empty(2 * F, np.float32), act=np.empty(F, np.float32),
                       q8_down=np.empty(act_row_bytes(ly.w_down.quant, F), np.uint8))
            tr = JoLayerTrace(*[out[n].ctypes.data for n, _ in JoLayerTrace._fields_])
        rc = lib().jo_decode_layer(C.byref(self.model), _p(kv), L, _p(x), pos, threads,
                                   C.byref(tr) if tr is not None else None)
        assert rc == 0
        return x, out

    def attn(self, kv, L, x, pos, threads=1):
        """jo_decode_attn: the attention sublayer of layer L; returns x after its residual."""
        x = np.array(x, np.float32, copy=True)
        assert lib().jo_decode_attn(C.byref(self.model), _p(kv), L, _p(x), pos, threads, None) == 0
        return x

    def moe_step(self, kv, token, pos, moe, weights, threads=1, trace=None):
        """execute_token_standard_with_hidden (src/qwen_deepseek.rs:1239-1314) for a model with a
        MoE spec (Qwen3-MoE, :1286-1300): per layer the attention sublayer (jo_decode_attn), then
        RMSNorm with ffn_norm (rms_eps.max(1e-6), :1250, :1278-1284), dispatch_qwen3_moe_ffn
        (moe_layer) and the residual hidden += out (:1301-1303); then the head.  moe = (num_experts,
        top_k, expert_ffn_dim, use_shared); weights {name: (quant, data, dims)} as moe_layer reads
        them.  trace (a list, optional) receives per layer (x_mid, xn, router logits, out, sel)."""
        s = self.spec
        E, k, F, shared = moe
        eps_ffn = max(s["eps"], 1e-6)
        x = self.embed(token)
        for L in range(s["n_layers"]):
            x = self.attn(kv, L, x, pos, threads)
            norm = weights.get(f"blk.{L}.ffn_norm.weight")
            nw = read_f32_weight_or_default(norm[0], norm[1], _n_el(norm[2]), s["hidden"]) if norm is not None \
                else np.ones(s["hidden"], np.float32)
            xn = rmsnorm(x, nw, eps_ffn)
            out, sel = moe_layer(xn, L, E, k, F, shared, weights, threads)
            if trace is not None:
                router = weights.get(f"blk.{L}.ffn_gate_inp.weight")
                lg = None
                if router is not None and E > 0 and k > 0:
                    re = _n_el(router[2])
                    H = s["hidden"]
                    eff = min(re // H, E) if re > 0 and re % H == 0 else E
                    lg = vec_dot(router[0], router[1], H, eff, xn)
                trace.append((x.copy(), xn, lg, out, sel))
            x = (x + out).astype(np.float32)
        return self.head(x, threads)[0]

    def head(self, x, threads=1):
        """jo_decode_head: (logits, xn_head, q8_head)."""
        s = self.spec
        x = np.ascontiguousarray(x, np.float32)
        logits = np.empty(self.logits_len, np.float32)
        xn = np.empty(s["hidden"], np.float32)
        q8 = np.empty(act_row_bytes(self.model.output.quant, s["hidden"]), np.uint8)
        rc = lib().jo_decode_head(C.byref(self.model), _p(x), _p(logits), threads, _p(xn), _p(q8))
        assert rc == 0
        return logits, xn, q8


# ---------------------------------------------------------------- synthetic int8 ForwardModel

FWD_DIM, FWD_FFN, FWD_LAYERS = 512, 1024, 4
FWD_NAMES = ("wq", "wk", "wv", "wo", "up", "down")


def splitmix(x):
    return int(lib().jo_splitmix(x))


def fill_small(seed, n):
    out = np.empty(n, np.int8)
    lib().jo_fill_small(seed, n, _p(out))
    return out


def isqrt(v):
    return int(lib().jo_isqrt(v))


def fwd_rmsnorm(x):
    x = np.ascontiguousarray(x, np.int8).reshape(-1, FWD_DIM)
    out = np.empty_like(x)
    lib().jo_fwd_rmsnorm(_p(x), x.shape[0], _p(out))
    return out


def fwd_attention(q, k_cache, v_cache, start_pos):
    q = np.ascontiguousarray(q, np.int8).reshape(-1, FWD_DIM)
    k_cache = np.ascontiguousarray(k_cache, np.int8)
    v_cache = np.ascontiguousarray(v_cache, np.int8)
    assert k_cache.size >= (start_pos + q.shape[0]) * FWD_DIM and v_cache.size == k_cache.size
    out = np.empty_like(q)
    lib().jo_fwd_attention(_p(q), _p(k_cache), _p(v_cache), q.shape[0], start_pos, _p(out))
    return out


def fwd_embed(seed, token):
    out = np.empty(FWD_DIM, np.int8)
    lib().jo_fwd_embed(seed, token, _p(out))
    return out


def fwd_sample(logits, vocab):
    logits = np.ascontiguousarray(logits, np.int32)
    return int(lib().jo_fwd_sample(_p(logits), vocab))


class ForwardModel:
    """ForwardModel (src/forward.rs:834-1075) on the CPU: weights from (seed, vocab), a cache of
    max_positions positions."""

    def __init__(self, seed, vocab, max_positions=64, threads=1):
        self.h = lib().jo_fwd_new(seed, vocab, max_positions)
        if not self.h:
            raise ValueError("jo_fwd_new failed")
        lib().jo_fwd_set_threads(self.h, threads)
        self.vocab = vocab
        self.head_rows = int(lib().jo_fwd_head_rows(self.h))

    def close(self):
        if self.h:
            lib().jo_fwd_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def weight(self, layer, which=0):
        n, k, sh = C.c_int64(), C.c_int64(), C.c_int()
        ptr = lib().jo_fwd_weight(self.h, layer, which, C.byref(n), C.byref(k), C.byref(sh))
        assert ptr
        arr = np.ctypeslib.as_array(C.cast(ptr, C.POINTER(C.c_int8)), shape=(n.value * k.value,))
        return arr.reshape(n.value, k.value).copy(), sh.value

    @property
    def length(self):
        return int(lib().jo_fwd_len(self.h))

    def reset(self):
        lib().jo_fwd_reset(self.h)

    def forward(self, tokens, start_pos):
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.head_rows, np.int32)
        rc = lib().jo_fwd_forward(self.h, _p(t), t.size, start_pos, _p(logits))
        if rc:
            raise ValueError(f"jo_fwd_forward rc={rc}")
        return logits

    def evaluate(self, prompt, max_tokens):
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(max_tokens, 1), np.uint32)
        rc = lib().jo_fwd_evaluate(self.h, _p(p), p.size, max_tokens, _p(out))
        if rc:
            raise ValueError(f"jo_fwd_evaluate rc={rc}")
        return [int(v) for v in out[:max_tokens]]
