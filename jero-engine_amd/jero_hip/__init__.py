"""Python front end of libjero_hip.so (ctypes over the C ABI in include/jero_hip.h).

The names mirror the jero_kernels_rvv entry points the reference's recipes call
(src/gemma.rs:66-138, src/qwen_deepseek.rs:643-951): ``vec_dot_q8_0(out, weights, input)``,
``matvec_any``, ``QuantizedActQ8.quantize`` ...  Device buffers are torch tensors (torch is
used for device memory and streams only); every computation runs in the HIP library.
Errors come back as :class:`K3Error` carrying the reference's variant name.

The library must have been built (``make -C jero-engine_amd`` or ``__graft_entry__.build()``);
importing this module on a box without it raises instead of falling back to anything.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.normpath(os.path.join(HERE, "..", "libjero_hip.so"))

F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K, ACT_Q8, Q4_K_R, Q6_K_R = 0, 1, 2, 8, 12, 14, 15, 100, 112, 114
Q4_K_T, Q6_K_T = 113, 115  # stacked expert tensors in 16-row tiles (repack of a 3-D tensor)
Q4_K_G, Q6_K_P = 116, 117  # GEMM layouts (repack_gemm)
BF16 = 30
Q4_K_M = Q4_K  # the reference's QuantType::Q4_K_M names the Q4_K block format
QUANT_NAMES = {F32: "F32", F16: "F16", BF16: "BF16", Q4_0: "Q4_0", Q8_0: "Q8_0", Q4_K: "Q4_K", Q6_K: "Q6_K", Q8_K: "Q8_K",
               ACT_Q8: "ACT_Q8", Q4_K_R: "Q4_K_R", Q6_K_R: "Q6_K_R", Q4_K_G: "Q4_K_G", Q6_K_P: "Q6_K_P"}
KV_F32, KV_F16 = 0, 1

OK = 0
STATUS_NAMES = {10: "CapabilityMismatch", 11: "InsufficientLockableMemory", 12: "ContextLengthExceeded",
                14: "TensorBoundsError", 15: "RoutingUnavailable", 20: "DeviceError", 21: "InvalidArgument"}


class K3Error(RuntimeError):
    """A non-zero jero_status; ``variant`` is the K3Error variant name it mirrors."""

    def __init__(self, status, message):
        self.status = status
        self.variant = STATUS_NAMES.get(status, "Unknown")
        super().__init__(f"{self.variant}({status}): {message}")


_lib = None
_P, _I64, _I32, _SZ, _F = C.c_void_p, C.c_int64, C.c_int, C.c_size_t, C.c_float
_SIGS = {
    "jero_hip_init": (_I32, [_I32]),
    "jero_hip_last_error": (C.c_char_p, []),
    "jero_hip_status_name": (C.c_char_p, [_I32]),
    "jero_hip_row_bytes": (_I64, [_I32, _I64]),
    "jero_hip_act_format": (_I32, [_I32]),
    "jero_hip_quantize_act": (_I32, [_I32, _P, _I64, _I64, _P, _P]),
    "jero_hip_matvec": (_I32, [_I32, _P, _SZ, _I64, _I64, _P, _P, _P]),
    "jero_hip_vec_dot": (_I32, [_I32, _P, _SZ, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "jero_hip_matvec_partials": (_I32, [_I32, _P, _SZ, _I64, _I64, _P, _P, _P, _P]),
    "jero_hip_vec_dot_noalloc": (_I32, [_I32, _P, _SZ, _I64, _I64, _P, _P, _P]),
    "jero_hip_read_probe": (_I32, [_P, _SZ, _P, _P]),
    "jero_hip_weights_register": (_I32, [_P, _SZ, C.POINTER(_P)]),
    "jero_hip_weights_lookup": (_I32, [_P, _SZ, C.POINTER(_P)]),
    "jero_hip_weights_release_all": (_I32, []),
    "jero_hip_weights_release": (_I32, [_P, _SZ]),
    "jero_hip_argmax": (_I32, [_P, _I64, _P, _P, _SZ, _P]),
    "jero_hip_model_status": (_I32, [_P, _P]),
    "jero_hip_model_trace": (_I32, [_P, _P, _SZ]),
    "jero_hip_model_trace_bytes": (_I64, [_P]),
    "jero_hip_model_logits_len": (_I64, [_P]),
    "jero_hip_sync": (_I32, [_P]),
    "jero_hip_gemm": (_I32, [_I32, _P, _SZ, _I64, _I64, _P, _I64, _P, _P]),
    "jero_hip_gemm_i8": (_I32, [_P, _I64, _I64, _P, _I64, _P, _P]),
    "jero_hip_gemm_i8_requant": (_I32, [_P, _I64, _I64, _P, _I64, _I32, _P, _P]),
    "jero_hip_requant_i8": (_I32, [_P, _I64, _I32, _P, _P]),
    "jero_hip_tile_count": (_I64, [_I64]),
    "jero_hip_pack_tiles": (_I32, [_P, _I64, _I64, _P, _P]),
    "jero_hip_gemm_i8_tiles": (_I32, [_P, _I64, _P, _I64, _I64, _I64, _P, _P]),
    "jero_hip_dequantize_rows": (_I32, [_I32, _P, _SZ, _I64, _I64, _I64, _P, _P]),
    "jero_hip_repack": (_I32, [_I32, _P, _SZ, _I64, _I64, _P, C.POINTER(C.c_int), _P]),
    "jero_hip_gemm_layout_bytes": (_SZ, [_I32, _I64, _I64]),
    "jero_hip_repack_gemm": (_I32, [_I32, _P, _SZ, _I64, _I64, _P, _SZ, C.POINTER(C.c_int), _P]),
    "jero_hip_repack_experts": (_I32, [_I32, _P, _SZ, _I64, _I64, _I64, _P, C.POINTER(C.c_int), _P]),
    "jero_hip_gqa_attention": (_I32, [_P, _P, _P, _P, _I32, _I32, _I32, _I32, _I64, _F, _P, _SZ, _P]),
    "jero_hip_moe_ffn": (_I32, [_P, _P, _I64, _I64, _I32, _I32, _P, _SZ, _I32, _P, _SZ, _I32, _P, _SZ, _I64, _I64,
                                _P, _P, _P, _P, _SZ, _P]),
    "jero_hip_moe_workspace_bytes": (_SZ, [_I64, _I64, _I32, _I64, _I64]),
    "jero_hip_moe_ffn_acc": (_I32, [_P, _P, _I64, _I64, _I32, _I32, _P, _SZ, _I32, _P, _SZ, _I32, _P, _SZ, _I64,
                                    _I64, _P, _P, _P, _P, _SZ, _P]),
    "jero_hip_swiglu_ffn": (_I32, [_I32, _P, _I64, _I64, _P, _P, _P, _I32, _P, _P, _SZ, _P]),
    "jero_hip_swiglu_ffn_workspace_bytes": (_SZ, [_I64, _I64]),
    "jero_hip_weights_register_stacked": (_I32, [C.POINTER(_P), _SZ, _I64, C.POINTER(_P)]),
    "jero_hip_moe_trace_view": (_I32, [_P, _I64, _I64, _I32, _I64, _I64, C.POINTER(_P), C.POINTER(_P),
                                       C.POINTER(C.c_int)]),
    "jero_hip_model_create": (_I32, [_P, C.POINTER(_P)]),
    "jero_hip_model_set_moe": (_I32, [_P, _I64, _I32, _I64, _I32]),
    "jero_hip_model_destroy": (_I32, [_P]),
    "jero_hip_model_set_tensor": (_I32, [_P, C.c_char_p, _I32, _P, _SZ, _I64, _I64, _I32]),
    "jero_hip_model_finalize": (_I32, [_P]),
    "jero_hip_model_kv": (_I32, [_P, _I64, C.POINTER(_P), C.POINTER(_P)]),
    "jero_hip_model_state": (_I32, [_P, C.POINTER(_P), C.POINTER(_P), C.POINTER(_P)]),
    "jero_hip_model_set_position": (_I32, [_P, _I32, _I64, _P]),
    "jero_hip_decode_step": (_I32, [_P, _P]),
    "jero_hip_model_prefill": (_I32, [_P, _P, _I64, _I64, _P]),
    "jero_hip_forward_model_create": (_I32, [C.c_uint64, _I64, _I64, C.POINTER(_P)]),
    "jero_hip_forward_model_destroy": (_I32, [_P]),
    "jero_hip_forward_model_head_rows": (_I64, [_P]),
    "jero_hip_forward_model_positions": (_I64, [_P]),
    "jero_hip_forward_model_reset": (_I32, [_P]),
    "jero_hip_forward_model_weight": (_I32, [_P, _I32, _I32, C.POINTER(_P), C.POINTER(_I64), C.POINTER(_I64),
                                             C.POINTER(C.c_int)]),
    "jero_hip_forward_model_forward": (_I32, [_P, _P, _I64, _I64, _P, _P]),
    "jero_hip_forward_model_evaluate": (_I32, [_P, _P, _I64, _I64, _P, _P, _P]),
    "jero_hip_gguf_open": (_I32, [C.c_char_p, C.POINTER(_P)]),
    "jero_hip_gguf_close": (None, [_P]),
    "jero_hip_gguf_info": (_I32, [_P, C.POINTER(_I64), C.POINTER(C.c_char_p)]),
    "jero_hip_gguf_meta_int": (_I32, [_P, C.c_char_p, C.POINTER(_I64)]),
    "jero_hip_gguf_meta_float": (_I32, [_P, C.c_char_p, C.POINTER(C.c_double)]),
    "jero_hip_gguf_meta_str": (_I32, [_P, C.c_char_p, C.POINTER(C.c_char_p)]),
    "jero_hip_gguf_tensor_name": (_I32, [_P, _I64, C.POINTER(C.c_char_p)]),
    "jero_hip_gguf_tensor": (_I32, [_P, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int), C.POINTER(_I64),
                                    C.POINTER(_P), C.POINTER(_SZ)]),
    "jero_hip_gguf_upload": (_I32, [_P, C.c_char_p, C.POINTER(_P)]),
}


def lib():
    """Loads libjero_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `make -C jero-engine_amd`")
        # torch first: it loads its HIP runtime into the global namespace, so the library's HIP
        # calls bind to that same runtime and torch's device pointers and streams are valid in
        # them (loaded alone first, the library would start a second runtime that then keeps
        # torch from opening the GPU).
        import torch  # noqa: F401
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name, None)
            if fn is None:
                continue
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def declared_symbols():
    """The entry points include/jero_hip.h declares (parsed from the header)."""
    import re
    hdr = os.path.normpath(os.path.join(HERE, "..", "..", "include", "jero_hip.h"))
    text = open(hdr).read()
    return sorted(set(re.findall(r"\b(jero_hip_[a-z0-9_]+)\s*\(", text)))


def check(status):
    if status != OK:
        msg = lib().jero_hip_last_error().decode(errors="replace")
        raise K3Error(status, msg)


def _stream(stream=None):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def init(device=0):
    check(lib().jero_hip_init(device))


def row_bytes(quant, n):
    return lib().jero_hip_row_bytes(quant, n)


def act_format(weight_quant):
    return lib().jero_hip_act_format(weight_quant)


class TensorView:
    """A device-resident GGUF tensor: ``quant``, GGUF ``shape`` [n_in, n_out] and its bytes
    (a uint8 torch tensor on the device), as jero_core::TensorView is for the reference."""

    def __init__(self, name, quant, shape, data):
        self.name, self.quant, self.shape, self.data = name, quant, list(shape), data

    @property
    def n_in(self):
        return self.shape[0]

    @property
    def n_out(self):
        return self.shape[1] if len(self.shape) > 1 else 1

    def nbytes(self):
        return self.data.numel() * self.data.element_size()

    def slice_rows(self, start, count):
        rb = row_bytes(self.quant, self.n_in)
        if start < 0 or count <= 0 or start + count > self.n_out:
            raise K3Error(14, f"slice_rows [{start}, {start + count}) beyond {self.n_out} rows of '{self.name}'")
        return TensorView(self.name, self.quant, [self.n_in, count], self.data[start * rb:(start + count) * rb])

    def slice_expert(self, expert, num_experts):
        """Expert `expert` of a stacked [n_in, n_out, num_experts] tensor (src/qwen_deepseek.rs:739)."""
        rows = self.n_out
        return TensorView(f"{self.name}[{expert}]", self.quant, [self.n_in, rows],
                          self.data.view(num_experts, -1)[expert])


def quantize_act(act_quant, x, out=None, stream=None):
    """QuantizedActQ8::quantize(acts, m, k) (src/weights.rs:1416): x [m, k] or [k] f32 on device."""
    import torch
    m, k = (1, x.shape[0]) if x.dim() == 1 else x.shape
    nb = row_bytes(act_quant, k)
    if nb < 0:
        raise K3Error(14, f"k={k} is not a multiple of the {QUANT_NAMES.get(act_quant)} block")
    if out is None:
        out = torch.empty(m * nb, dtype=torch.uint8, device=x.device)
    check(lib().jero_hip_quantize_act(act_quant, _ptr(x), m, k, _ptr(out), _stream(stream)))
    return out


def matvec(weights, xq, out, stream=None):
    """y = W . x with x already in the weight format's activation blocks."""
    check(lib().jero_hip_matvec(weights.quant, _ptr(weights.data), weights.nbytes(), weights.n_in,
                                out.numel(), _ptr(xq), _ptr(out), _stream(stream)))
    return out


def weights_register(host_array):
    """Device address of a host numpy buffer's bytes (uploaded on first registration)."""
    dev = _P()
    check(lib().jero_hip_weights_register(host_array.ctypes.data, host_array.nbytes, C.byref(dev)))
    return dev.value


def weights_lookup(host_array):
    dev = _P()
    check(lib().jero_hip_weights_lookup(host_array.ctypes.data, host_array.nbytes, C.byref(dev)))
    return dev.value


def weights_release_all():
    check(lib().jero_hip_weights_release_all())


def weights_release(host_array):
    """Frees the device copies registered inside the host buffer's range (before it is unmapped)."""
    check(lib().jero_hip_weights_release(host_array.ctypes.data, host_array.nbytes))


def argmax_f32(x, out=None, workspace=None, stream=None):
    """argmax_f32 behind sample_greedy_argmax (src/engine.rs:1873-1895) on a device f32 tensor:
    returns a device int64 tensor of one element holding the first index of the largest non-NaN
    value, or -1 (None) for an empty or all-NaN input."""
    import torch
    if out is None:
        out = torch.empty(1, dtype=torch.int64, device=x.device)
    ws_p = _ptr(workspace) if workspace is not None else None
    ws_n = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().jero_hip_argmax(_ptr(x) if x.numel() else None, x.numel(), _ptr(out), ws_p, ws_n, _stream(stream)))
    return out


def sample_greedy_argmax(logits, stream=None):
    """sample_greedy_argmax (src/engine.rs:1873-1895): the token id, or None."""
    idx = int(argmax_f32(logits, stream=stream).item())
    return None if idx < 0 else idx


def sync(stream=None):
    check(lib().jero_hip_sync(_stream(stream)))


def gemm(weights, xq, m, out, stream=None):
    """Y[m, n_out] = rows of the m quantized activation rows `xq` times W: row r is matvec of
    x_r (the prefill token loop, src/qwen_deepseek.rs:2298-2312, and PackedNibbleMatrix::gemm,
    src/weights.rs:1416-1426)."""
    check(lib().jero_hip_gemm(weights.quant, _ptr(weights.data), weights.nbytes(), weights.n_in, weights.n_out,
                              _ptr(xq), m, _ptr(out), _stream(stream)))
    return out


def gemm_i8(x, w, out=None, stream=None):
    """Exact int8 product of ForwardExec::matmul (src/forward.rs:763-811): out[m, n] =
    sum_k x[m, k] * w[n, k] in int32; x [m, k], w [n, k] int8 device tensors."""
    import torch
    m, k = x.shape
    n = w.shape[0]
    if w.shape[1] != k:
        raise K3Error(14, f"gemm_i8: x has k={k}, w has k={w.shape[1]}")
    if out is None:
        out = torch.empty((m, n), dtype=torch.int32, device=x.device)
    check(lib().jero_hip_gemm_i8(_ptr(x), m, k, _ptr(w), n, _ptr(out), _stream(stream)))
    return out


def gemm_i8_requant(x, w, shift, out=None, stream=None):
    """requant_all(&ForwardExec::matmul(x, w), shift) (src/forward.rs:813-815, :957-970) in one
    launch: int8 [m, n] of the int32 product requantized as forward.rs's requant (:345-350)."""
    import torch
    m, k = x.shape
    n = w.shape[0]
    if w.shape[1] != k:
        raise K3Error(14, f"gemm_i8_requant: x has k={k}, w has k={w.shape[1]}")
    if out is None:
        out = torch.empty((m, n), dtype=torch.int8, device=x.device)
    check(lib().jero_hip_gemm_i8_requant(_ptr(x), m, k, _ptr(w), n, shift, _ptr(out), _stream(stream)))
    return out


def requant_all(raw, shift, out=None, stream=None):
    """requant_all (src/forward.rs:813-815) on a device int32 tensor."""
    import torch
    if out is None:
        out = torch.empty(raw.shape, dtype=torch.int8, device=raw.device)
    check(lib().jero_hip_requant_i8(_ptr(raw), raw.numel(), shift, _ptr(out), _stream(stream)))
    return out


class ime:
    """The ime names forward.rs imports (src/forward.rs:26-29): TILE_*, tile_count, pack_tiles,
    gemm_i8_ime, gemm_i8_vector, over this library's packed layout (jero_hip_pack_tiles)."""
    TILE_M, TILE_N, TILE_K, TILE_C = 8, 8, 32, 64

    @staticmethod
    def tile_count(rows):
        return int(lib().jero_hip_tile_count(rows))

    @staticmethod
    def pack_tiles(x, rows, k, stream=None):
        """x: [rows, k] int8 device tensor -> packed bytes (tile_count(rows) * 8 * k)."""
        import torch
        out = torch.empty(ime.tile_count(rows) * ime.TILE_N * k, dtype=torch.int8, device=x.device)
        check(lib().jero_hip_pack_tiles(_ptr(x), rows, k, _ptr(out), _stream(stream)))
        return out

    @staticmethod
    def gemm_i8_ime(a, m_tiles, packed_w, tile_range, k_chunks, emit, stream=None):
        """gemm_i8_ime (src/forward.rs:779-796): emit(mt, nt, c) for every activation tile mt and
        weight tile nt in tile_range, c the TILE_C int32 values of the 8 x 8 block (row-major)."""
        import torch
        nt0, nt1 = tile_range.start, tile_range.stop
        c = torch.empty((m_tiles, nt1 - nt0, ime.TILE_C), dtype=torch.int32, device=a.device)
        check(lib().jero_hip_gemm_i8_tiles(_ptr(a), m_tiles, _ptr(packed_w), nt0, nt1, k_chunks, _ptr(c),
                                           _stream(stream)))
        host = c.cpu().numpy()
        for mt in range(m_tiles):
            for nt in range(nt0, nt1):
                emit(mt, nt, host[mt, nt - nt0])

    @staticmethod
    def gemm_i8_vector(x, m, rows, row_range, k, emit, stream=None):
        """gemm_i8_vector (src/forward.rs:797-806): emit(row, col, v) for row < m, col in
        row_range; x [m, k] and rows [n, k] int8 device tensors."""
        out = gemm_i8(x[:m], rows[row_range.start:row_range.stop], stream=stream).cpu().numpy()
        for r in range(m):
            for j, col in enumerate(row_range):
                emit(r, col, int(out[r, j]))


def matvec_partials(weights, xq, out, partials, stream=None):
    check(lib().jero_hip_matvec_partials(weights.quant, _ptr(weights.data), weights.nbytes(), weights.n_in,
                                         out.numel(), _ptr(xq), _ptr(out), _ptr(partials), _stream(stream)))
    return out, partials


def _vec_dot(expect_quant, out, weights, inp, workspace=None, stream=None):
    if weights.quant != expect_quant:
        raise K3Error(10, f"tensor '{weights.name}' is {QUANT_NAMES.get(weights.quant)}, "
                          f"expected {QUANT_NAMES.get(expect_quant)}")
    return matvec_any(out, weights, inp, workspace, stream)


def matvec_any(out, weights, inp, workspace=None, stream=None):
    """matvec_any (src/gemma.rs:100-138): dispatch on the tensor's quantization."""
    if out.numel() == 0 or inp.numel() == 0:
        raise K3Error(14, "matvec output and input slices cannot be empty")
    ws_p = _ptr(workspace) if workspace is not None else None
    ws_n = workspace.numel() if workspace is not None else 0
    check(lib().jero_hip_vec_dot(weights.quant, _ptr(weights.data), weights.nbytes(), inp.numel(), out.numel(),
                                 _ptr(inp), _ptr(out), ws_p, ws_n, _stream(stream)))
    return out


def vec_dot_noalloc(out, weights, inp, stream=None):
    """matvec_any staged through the library's static device buffer (jero_hip_vec_dot_noalloc): no
    allocation; calls on one device must not overlap."""
    check(lib().jero_hip_vec_dot_noalloc(weights.quant, _ptr(weights.data), weights.nbytes(), inp.numel(),
                                         out.numel(), _ptr(inp), _ptr(out), _stream(stream)))
    return out


def read_probe(buf, sink, stream=None):
    """One launch that only reads buf's bytes (jero_hip_read_probe): the bandwidth ceiling of a
    kernel over the same bytes.  sink: >= 1 KiB device tensor."""
    assert sink.numel() * sink.element_size() >= 1024
    check(lib().jero_hip_read_probe(_ptr(buf), buf.numel() * buf.element_size(), _ptr(sink), _stream(stream)))


def matvec_f32(out, weights, inp, **kw):
    """matvec_f32 (src/gemma.rs:140-189): F32 weight rows dotted with the f32 input."""
    return _vec_dot(F32, out, weights, inp, **kw)


def vec_dot_f16(out, weights, inp, **kw):
    return _vec_dot(F16, out, weights, inp, **kw)


def vec_dot_bf16(out, weights, inp, **kw):
    return _vec_dot(BF16, out, weights, inp, **kw)


def vec_dot_q8_0(out, weights, inp, **kw):
    return _vec_dot(Q8_0, out, weights, inp, **kw)


def vec_dot_q4_0(out, weights, inp, **kw):
    return _vec_dot(Q4_0, out, weights, inp, **kw)


def vec_dot_q4_k_m(out, weights, inp, **kw):
    """BaselineKernel::vec_dot_q4_k_m (src/gemma.rs:82)."""
    return _vec_dot(Q4_K, out, weights, inp, **kw)


def vec_dot_q6_k(out, weights, inp, **kw):
    return _vec_dot(Q6_K, out, weights, inp, **kw)


def repack(weights, stream=None, experts=None):
    """Load-time re-layout (repack_tensor_parallel, src/weights.rs:914-955): returns a new
    TensorView in a device layout of the same byte count.  A 2-D tensor: Q4_K -> Q4_K_R,
    Q6_K -> Q6_K_R (the GEMV layouts).  A stacked expert tensor [n_in, rows, n_experts] with rows a
    multiple of 16: Q4_K -> Q4_K_T, Q6_K -> Q6_K_T (16-row tiles, for dispatch_qwen3_moe_ffn);
    experts=False repacks it as rows * n_experts rows of the 2-D layout instead."""
    import torch
    dst = torch.empty(weights.nbytes(), dtype=torch.uint8, device=weights.data.device)
    q = C.c_int(0)
    rows = 1
    for d in weights.shape[1:]:
        rows *= d
    if experts is None:
        experts = len(weights.shape) == 3 and weights.shape[1] % 16 == 0
    if experts:
        check(lib().jero_hip_repack_experts(weights.quant, _ptr(weights.data), weights.nbytes(), weights.n_in,
                                            weights.shape[1], weights.shape[2], _ptr(dst), C.byref(q),
                                            _stream(stream)))
    else:
        check(lib().jero_hip_repack(weights.quant, _ptr(weights.data), weights.nbytes(), weights.n_in, rows,
                                    _ptr(dst), C.byref(q), _stream(stream)))
    return TensorView(weights.name, q.value, weights.shape, dst)


def gemm_layout_bytes(quant, n_in, n_out):
    return lib().jero_hip_gemm_layout_bytes(quant, n_in, n_out)


def repack_gemm(weights, stream=None):
    """Load-time re-layout of a Q4_K / Q6_K tensor (GGUF or the _R layouts) for the prefill GEMM
    (the RepackedWeight role, src/weights.rs:914-955): returns a TensorView of quant Q4_K_G (the
    Q4_K quants in the MFMA fragment order, scales unpacked) or Q6_K_P (exact int8 planes) for gemm()."""
    import torch
    n = gemm_layout_bytes(weights.quant, weights.n_in, weights.n_out)
    if n == 0:
        raise K3Error(10, f"repack_gemm: no GEMM layout for quant {weights.quant} at {weights.shape}")
    dst = torch.empty(n, dtype=torch.uint8, device=weights.data.device)
    q = C.c_int(0)
    check(lib().jero_hip_repack_gemm(weights.quant, _ptr(weights.data), weights.nbytes(), weights.n_in,
                                     weights.n_out, _ptr(dst), n, C.byref(q), _stream(stream)))
    return TensorView(weights.name, q.value, weights.shape, dst)


def gqa_causal_attention_f32(out, q, k, v, n_heads_q, n_heads_kv, head_dim, seq_len, scale, workspace=None,
                             stream=None):
    """gqa_causal_attention_f32 (src/qwen_deepseek.rs:669-691); k, v: [seq][n_kv*hd] f32 or f16."""
    import torch
    kv_dtype = KV_F16 if k.dtype == torch.float16 else KV_F32
    ws_p = _ptr(workspace) if workspace is not None else None
    ws_n = workspace.numel() * workspace.element_size() if workspace is not None else 0
    check(lib().jero_hip_gqa_attention(_ptr(out), _ptr(q), _ptr(k), _ptr(v), kv_dtype, n_heads_q, n_heads_kv,
                                       head_dim, seq_len, scale, ws_p, ws_n, _stream(stream)))
    return out


def dispatch_qwen3_moe_ffn(out, norm_ffn_in, router_logits, top_k, gate, up, down, workspace=None, stream=None,
                           accumulate=False):
    """The routed experts of dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951) from router
    logits.  gate/up/down: stacked TensorViews with shape [n_in, rows_per_expert, n_experts].
    accumulate: the routed sum is added onto out (jero_hip_moe_ffn_acc).  Returns (sel_idx [T, k]
    int32, sel_w [T, k] f32) device tensors."""
    import torch
    T = router_logits.shape[0] if router_logits.dim() == 2 else 1
    E = router_logits.shape[-1]
    hidden, ffn = gate.shape[0], gate.shape[1]
    sel_idx = torch.empty((T, top_k), dtype=torch.int32, device=out.device)
    sel_w = torch.empty((T, top_k), dtype=torch.float32, device=out.device)
    if workspace is None:
        need = lib().jero_hip_moe_workspace_bytes(T, E, top_k, hidden, ffn)
        workspace = torch.empty(need, dtype=torch.uint8, device=out.device)
    fn = lib().jero_hip_moe_ffn_acc if accumulate else lib().jero_hip_moe_ffn
    check(fn(_ptr(norm_ffn_in), _ptr(router_logits), T, E, top_k, gate.quant, _ptr(gate.data), gate.nbytes(),
             up.quant, _ptr(up.data), up.nbytes(), down.quant, _ptr(down.data), down.nbytes(), hidden, ffn, _ptr(out),
             _ptr(sel_idx), _ptr(sel_w), _ptr(workspace), workspace.numel(), _stream(stream)))
    return sel_idx, sel_w


class HipTensor(C.Structure):
    """jero_hip_tensor."""
    _fields_ = [("quant", C.c_int), ("dev", C.c_void_p), ("bytes", C.c_size_t), ("n_elements", C.c_int64)]

    @classmethod
    def of(cls, view):
        if view is None:
            return cls(0, None, 0, 0)
        n = 1
        for d in view.shape:
            n *= d
        return cls(view.quant, view.data.data_ptr(), view.nbytes(), n)


FFN_SHARED_EXPERT, FFN_DENSE = 0, 1


def swiglu_ffn(mode, out, x, ffn, gate, up, down, accumulate=False, workspace=None, stream=None):
    """run_single_swiglu_expert (mode FFN_SHARED_EXPERT, src/qwen_deepseek.rs:748-771) or
    run_dense_swiglu_ffn (FFN_DENSE, :696-727, each projection project_or_deterministic_slice; a
    None tensor is absent) on one token row x [hidden]: out = (out if accumulate else 0) + r
    (jero_hip_swiglu_ffn)."""
    H = x.numel()
    ws_p, ws_n = (_ptr(workspace), workspace.numel()) if workspace is not None else (None, 0)
    g, u, d = HipTensor.of(gate), HipTensor.of(up), HipTensor.of(down)
    check(lib().jero_hip_swiglu_ffn(mode, _ptr(x), H, ffn, C.byref(g), C.byref(u), C.byref(d), int(bool(accumulate)),
                                    _ptr(out), ws_p, ws_n, _stream(stream)))
    return out


def weights_register_stacked(host_arrays):
    """Device address of n equal-sized host buffers registered as one stacked tensor
    (jero_hip_weights_register_stacked)."""
    n = len(host_arrays)
    if n == 0 or any(a.nbytes != host_arrays[0].nbytes for a in host_arrays):
        raise K3Error(14, "weights_register_stacked: the tensors of a stack must all have the same size")
    arr = (_P * n)(*[a.ctypes.data for a in host_arrays])
    dev = _P()
    check(lib().jero_hip_weights_register_stacked(arr, host_arrays[0].nbytes, n, C.byref(dev)))
    return dev.value


def _n_elements(view):
    n = 1
    for d in view.shape:
        n *= d
    return n


def moe_layer(out, norm_ffn_in, layer, num_experts, top_k, expert_ffn_dim, use_shared_expert, weights, stream=None):
    """dispatch_qwen3_moe_ffn (src/qwen_deepseek.rs:847-951) in full, on the device: `weights` maps
    GGUF names to device TensorViews (ModelWeights).  out [hidden] = the shared expert (when
    use_shared_expert and all three ffn_*_shexp tensors are present) + the routed experts over the
    router ffn_gate_inp, or + the dense FFN (ffn_gate / ffn_up / ffn_down, each
    project_or_deterministic_slice) when there is no router or no expert to route to.  The routed
    experts come from the stacked ffn_*_exps tensors (3-D) or, for each of gate / up / down
    apart, the per-expert tensors ffn_*_exps.{e} of every expert (slice_or_lookup_expert,
    :729-746), stacked on the device.  Returns the selection [(expert, weight)] (empty after the
    dense FFN).  Refused (CapabilityMismatch): exp_probs_b routing bias (DeepSeek's biased
    selection, :909-918) and per-expert tensors missing for some experts (the reference would
    skip those experts)."""
    import torch
    H = norm_ffn_in.numel()
    name = lambda t: f"blk.{layer}.{t}.weight"
    if f"blk.{layer}.exp_probs_b.bias" in weights:
        raise K3Error(10, f"layer {layer}: exp_probs_b routing bias (biased expert selection) is not supported on the "
                          "device")
    shexp = [weights.get(name(t)) for t in ("ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp")]
    shared = bool(use_shared_expert) and all(t is not None for t in shexp)
    if shared:
        swiglu_ffn(FFN_SHARED_EXPERT, out, norm_ffn_in, expert_ffn_dim, *shexp, accumulate=False, stream=stream)
    router = weights.get(name("ffn_gate_inp"))
    if num_experts == 0 or top_k == 0 or router is None:
        swiglu_ffn(FFN_DENSE, out, norm_ffn_in, expert_ffn_dim, weights.get(name("ffn_gate")),
                   weights.get(name("ffn_up")), weights.get(name("ffn_down")), accumulate=shared, stream=stream)
        return []
    re = _n_elements(router)
    eff = min(re // H, num_experts) if re > 0 and re % H == 0 else num_experts
    logits = torch.empty((1, eff), dtype=torch.float32, device=out.device)
    matvec_any(logits.view(-1), router, norm_ffn_in, stream=stream)

    def experts(kind):
        st = weights.get(f"blk.{layer}.ffn_{kind}_exps.weight")
        if st is not None and len(st.shape) == 3:
            return TensorView(st.name, st.quant, [st.shape[0], _n_elements(st) // (st.shape[0] * eff), eff], st.data)
        per = [weights.get(f"blk.{layer}.ffn_{kind}_exps.{e}.weight") for e in range(eff)]
        missing = [e for e, t in enumerate(per) if t is None]
        if missing:
            raise K3Error(10, f"layer {layer}: no ffn_{kind}_exps tensor for experts {missing[:8]} (the device runs "
                              "only complete expert sets)")
        q, nb = per[0].quant, per[0].nbytes()
        if any(t.quant != q or t.nbytes() != nb for t in per):
            raise K3Error(10, f"layer {layer}: per-expert ffn_{kind}_exps tensors differ in format or size")
        return TensorView(f"blk.{layer}.ffn_{kind}_exps", q, [per[0].shape[0], _n_elements(per[0]) // per[0].shape[0],
                                                            eff], torch.cat([t.data.reshape(-1) for t in per]))

    g, u, d = experts("gate"), experts("up"), experts("down")
    k = min(top_k, eff)
    g_rows = g.shape[1]  # run_single_swiglu_expert's eff_ffn of an expert slice (:757-762)
    x2 = norm_ffn_in.view(1, H)
    sel_idx, sel_w = dispatch_qwen3_moe_ffn(out.view(1, H), x2, logits, k, TensorView(g.name, g.quant, [H, g_rows, eff], g.data),
                                            TensorView(u.name, u.quant, [H, g_rows, eff], u.data),
                                            TensorView(d.name, d.quant, [g_rows, H, eff], d.data), stream=stream,
                                            accumulate=shared)
    if stream is not None:
        stream.synchronize()
    else:
        torch.cuda.synchronize()
    return list(zip(sel_idx.view(-1).tolist(), sel_w.view(-1).tolist()))


def moe_workspace(n_tokens, n_experts, top_k, hidden, ffn, device="cuda"):
    import torch
    need = lib().jero_hip_moe_workspace_bytes(n_tokens, n_experts, top_k, hidden, ffn)
    return torch.empty(need, dtype=torch.uint8, device=device)


def moe_trace_act(workspace, n_tokens, n_experts, top_k, hidden, ffn):
    """The f32 SwiGLU rows of the last jero_hip_moe_ffn call on `workspace` (synchronize first), as
    a numpy array [n_tokens, top_k, ffn] in (token, slot) order (jero_hip_moe_trace_view)."""
    import numpy as np
    act, rows, ident = _P(), _P(), C.c_int()
    check(lib().jero_hip_moe_trace_view(_ptr(workspace), n_tokens, n_experts, top_k, hidden, ffn, C.byref(act),
                                        C.byref(rows), C.byref(ident)))
    n = n_tokens * top_k
    a = np.empty((n, ffn), np.float32)
    _memcpy(a.ctypes.data, act.value, a.nbytes)
    if ident.value:
        order = np.arange(n)
    else:
        order = np.empty(n, np.int32)
        _memcpy(order.ctypes.data, rows.value, order.nbytes)
    return a[order].reshape(n_tokens, top_k, ffn)


def dequantize_rows(weights, row0, n_rows, out, stream=None):
    """dequantize_token_row for rows [row0, row0 + n_rows)."""
    check(lib().jero_hip_dequantize_rows(weights.quant, _ptr(weights.data), weights.nbytes(), weights.n_in, row0,
                                         n_rows, _ptr(out), _stream(stream)))
    return out


def dequantize_token_row(weights, row, out, stream=None):
    return dequantize_rows(weights, row, 1, out, stream)


# ---------------------------------------------------------------- device-resident decoder

class ModelConfig(C.Structure):
    """jero_model_config."""
    _fields_ = [("hidden", C.c_int64), ("ffn", C.c_int64), ("n_layers", C.c_int64), ("vocab", C.c_int64),
                ("n_heads_q", C.c_int), ("n_heads_kv", C.c_int), ("head_dim", C.c_int), ("rms_eps", C.c_float),
                ("rope_theta", C.c_float), ("kv_capacity", C.c_int64), ("kv_dtype", C.c_int), ("qk_norm", C.c_int)]


_hip = None


def _memcpy(dst_ptr, src_ptr, nbytes):
    """Synchronous device/host copy through the HIP runtime (hipMemcpyDefault)."""
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [_P, _P, _SZ, C.c_int]
        _hip.hipMemcpy.restype = C.c_int
    rc = _hip.hipMemcpy(C.c_void_p(dst_ptr), C.c_void_p(src_ptr), nbytes, 4)
    if rc != 0:
        raise K3Error(20, f"hipMemcpy failed ({rc})")


class ForwardModel:
    """The synthetic all-int8 transformer of src/forward.rs (ForwardModel::new, :879-903) on the
    device: weights generated from (seed, vocab), a K/V cache of max_positions positions.
    forward() mirrors ForwardModel::forward (:930-976) and evaluate() the token loop of
    ForwardModel::evaluate (:995-1043)."""

    DIM, FFN, LAYERS = 512, 1024, 4
    NAMES = ("wq", "wk", "wv", "wo", "up", "down")

    def __init__(self, seed, vocab, max_positions=64):
        h = C.c_void_p()
        check(lib().jero_hip_forward_model_create(C.c_uint64(seed), vocab, max_positions, C.byref(h)))
        self.h = h
        self.vocab = vocab
        self.max_positions = max_positions
        self.head_rows = int(lib().jero_hip_forward_model_head_rows(h))

    def close(self):
        if self.h:
            lib().jero_hip_forward_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def positions(self):
        """Positions in the K/V cache: the start_pos the next forward() must pass."""
        return int(lib().jero_hip_forward_model_positions(self.h))

    def reset(self):
        check(lib().jero_hip_forward_model_reset(self.h))

    def weight(self, layer, which=0):
        """(device pointer, n, k, shift) of layer's matrix `which` (0..5: wq wk wv wo up down), or of
        the LM head for layer -1."""
        w, n, k, sh = C.c_void_p(), C.c_int64(), C.c_int64(), C.c_int()
        check(lib().jero_hip_forward_model_weight(self.h, layer, which, C.byref(w), C.byref(n), C.byref(k),
                                                  C.byref(sh)))
        return w.value, n.value, k.value, sh.value

    def forward(self, tokens, start_pos, logits, stream=None):
        """One forward pass over host `tokens` at start_pos (== positions); logits: int32 device
        tensor of head_rows values."""
        import numpy as np
        t = np.ascontiguousarray(tokens, np.uint32)
        check(lib().jero_hip_forward_model_forward(self.h, C.c_void_p(t.ctypes.data), t.size, start_pos,
                                                   _ptr(logits), _stream(stream)))

    def evaluate(self, prompt, max_tokens, stream=None, timing=False):
        """Prefill over prompt, then greedy decode until max_tokens tokens: the generated ids
        (and, with timing, the (prefill_ms, decode_ms) the device took)."""
        import numpy as np
        p = np.ascontiguousarray(prompt, np.uint32)
        out = np.zeros(max(max_tokens, 1), np.uint32)
        ms = np.zeros(2, np.float32)
        check(lib().jero_hip_forward_model_evaluate(self.h, C.c_void_p(p.ctypes.data), p.size, max_tokens,
                                                    C.c_void_p(out.ctypes.data), C.c_void_p(ms.ctypes.data),
                                                    _stream(stream)))
        toks = [int(v) for v in out[:max_tokens]]
        return (toks, (float(ms[0]), float(ms[1]))) if timing else toks


class DecodeModel:
    """A device-resident decoder (Qwen3 / Llama layout, dense or, with moe, Qwen3-MoE): the
    ArchRecipe::decode_step path of the reference (src/qwen_deepseek.rs:1441-1460) with ctx state
    (token, position, logits) held on the device.  moe = (num_experts, top_k, expert_ffn_dim,
    use_shared), the recipe's MoeDispatchSpec (jero_hip_model_set_moe)."""

    def __init__(self, hidden, ffn, n_layers, vocab, n_heads_q, n_heads_kv, head_dim, rms_eps, rope_theta,
                 kv_capacity, kv_dtype=KV_F16, qk_norm=True, moe=None):
        self.cfg = ModelConfig(hidden, ffn, n_layers, vocab, n_heads_q, n_heads_kv, head_dim, rms_eps, rope_theta,
                               kv_capacity, kv_dtype, 1 if qk_norm else 0)
        h = C.c_void_p()
        check(lib().jero_hip_model_create(C.byref(self.cfg), C.byref(h)))
        self.h = h
        self.moe = tuple(moe) if moe is not None else None
        if moe is not None:
            E, k, F, shared = moe
            check(lib().jero_hip_model_set_moe(self.h, E, k, F, 1 if shared else 0))

    def close(self):
        if self.h:
            lib().jero_hip_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @classmethod
    def from_gguf(cls, path, kv_capacity, kv_dtype=KV_F16):
        """Builds and finalizes a model from a GGUF file: hyperparameters by
        GGUFFile.hyperparams, every tensor copied from the mapped file."""
        g = path if isinstance(path, GGUFFile) else GGUFFile(path)
        try:
            hp = g.hyperparams()
            m = cls(hp["hidden"], hp["ffn"], hp["n_layers"], hp["vocab"], hp["n_heads_q"], hp["n_heads_kv"],
                    hp["head_dim"], hp["rms_eps"], hp["rope_theta"], kv_capacity, kv_dtype, hp["qk_norm"],
                    hp.get("moe"))
            names = ["token_embd.weight", "output.weight", "output_norm.weight"]
            per = ["attn_norm", "ffn_norm", "attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                   "ffn_down"] + (["attn_q_norm", "attn_k_norm"] if hp["qk_norm"] else [])
            if hp.get("moe"):
                per += ["ffn_gate_inp", "ffn_gate_exps", "ffn_up_exps", "ffn_down_exps", "ffn_gate_shexp",
                        "ffn_up_shexp", "ffn_down_shexp"]
            names += [f"blk.{i}.{b}.weight" for i in range(hp["n_layers"]) for b in per]
            present = set(g.tensor_names())
            if hp.get("moe"):  # the routing bias is refused at finalize (select_experts_with_optional_bias)
                names += [n for n in present if n.endswith(".exp_probs_b.bias")]
            for name in names:
                # an absent tensor takes the reference's default (norms 1.0, the projections'
                # deterministic slice, the tied head, embed_token's deterministic row)
                if name not in present:
                    continue
                t = g.tensor(name)
                n_out = 1
                for d in t["dims"][1:t["n_dims"]]:
                    n_out *= d
                check(lib().jero_hip_model_set_tensor(m.h, name.encode(), t["quant"], C.c_void_p(t["host"]),
                                                      t["nbytes"], t["dims"][0], n_out, 0))
            m.finalize()
            return m
        finally:
            if g is not path:
                g.close()

    def set_tensor(self, name, quant, data, n_in, n_out):
        """data: a numpy array (host) or a torch tensor (host or device) holding the GGUF bytes."""
        import numpy as np
        if isinstance(data, np.ndarray):
            arr = np.ascontiguousarray(data)
            ptr, nbytes, on_dev = arr.ctypes.data, arr.nbytes, 0
        else:
            ptr, nbytes, on_dev = data.data_ptr(), data.numel() * data.element_size(), 1 if data.is_cuda else 0
        check(lib().jero_hip_model_set_tensor(self.h, name.encode(), quant, C.c_void_p(ptr), nbytes, n_in, n_out,
                                              on_dev))

    def finalize(self):
        check(lib().jero_hip_model_finalize(self.h))

    def kv_ptrs(self, layer):
        k, v = C.c_void_p(), C.c_void_p()
        check(lib().jero_hip_model_kv(self.h, layer, C.byref(k), C.byref(v)))
        return k.value, v.value

    def write_kv(self, layer, k, v):
        """Copies torch tensors k, v ([capacity][n_kv*hd] in the cache dtype) into layer's rings."""
        kp, vp = self.kv_ptrs(layer)
        _memcpy(kp, k.data_ptr(), k.numel() * k.element_size())
        _memcpy(vp, v.data_ptr(), v.numel() * v.element_size())

    def state_ptrs(self):
        t, p, l = C.c_void_p(), C.c_void_p(), C.c_void_p()
        check(lib().jero_hip_model_state(self.h, C.byref(t), C.byref(p), C.byref(l)))
        return t.value, p.value, l.value

    def set_position(self, token, pos, stream=None):
        check(lib().jero_hip_model_set_position(self.h, token, pos, _stream(stream)))

    def prefill(self, tokens, pos0, stream=None):
        """run_prefill_with_hidden over `tokens` from position pos0 in one pass
        (jero_hip_model_prefill): leaves the last token's logits, the greedy next token and
        position pos0 + len(tokens)."""
        import numpy as np
        if hasattr(tokens, "data_ptr"):  # an int32 torch tensor in host memory (pinned: the upload is asynchronous)
            import torch
            if tokens.dtype != torch.int32 or tokens.device.type != "cpu" or not tokens.is_contiguous():
                raise K3Error(21, "prefill: a tensor of tokens must be contiguous int32 in host memory")
            check(lib().jero_hip_model_prefill(self.h, tokens.data_ptr(), tokens.numel(), pos0, _stream(stream)))
            return
        t = np.ascontiguousarray(np.asarray(tokens, np.int32))
        check(lib().jero_hip_model_prefill(self.h, t.ctypes.data, t.size, pos0, _stream(stream)))

    def decode_step(self, stream=None):
        check(lib().jero_hip_decode_step(self.h, _stream(stream)))

    TRACE_FIELDS = ("x_in", "xn_attn", "q8_attn", "qkv", "q_rope", "k_rope", "attn", "q8_wo", "x_mid", "xn_ffn",
                    "q8_ffn", "gu", "act", "q8_down")

    def trace_layout(self):
        """{field: (byte offset in a layer record, numpy dtype, count)}, the layer record size
        and the head fields' offsets, as jero_hip_model_trace documents them."""
        import numpy as np
        c = self.cfg
        H, F, Q, KV = c.hidden, c.ffn, c.n_heads_q * c.head_dim, c.n_heads_kv * c.head_dim
        r16 = lambda n: (n + 15) // 16 * 16
        A = lambda n: r16(max(n // 32 * 36, n // 256 * 292 if n % 256 == 0 else 0))
        f4, u8 = np.float32, np.uint8
        spec = [(f4, H), (f4, H), (u8, A(H)), (f4, Q + 2 * KV), (f4, Q), (f4, KV), (f4, Q), (u8, A(Q)), (f4, H),
                (f4, H), (u8, A(H)), (f4, 2 * F), (f4, F), (u8, A(F))]
        out, off = {}, 0
        for name, (dt, n) in zip(self.TRACE_FIELDS, spec):
            nb = r16(n * np.dtype(dt).itemsize)
            out[name] = (off, dt, n if dt is f4 else nb)
            off += nb
        tail = off * c.n_layers
        head = {"x_final": (tail, f4, H), "xn_head": (tail + r16(4 * H), f4, H),
                "q8_head": (tail + 2 * r16(4 * H), u8, A(H)), "rope_cs": (tail + 2 * r16(4 * H) + A(H), f4, c.head_dim)}
        total = tail + 2 * r16(4 * H) + A(H) + r16(4 * c.head_dim)
        assert total == lib().jero_hip_model_trace_bytes(self.h), "trace layout disagrees with the library"
        return out, off, head, total

    def set_trace(self, buf):
        """Records every later decode step's intermediate values into the uint8 device tensor
        `buf` (None: off)."""
        if buf is None:
            check(lib().jero_hip_model_trace(self.h, None, 0))
        else:
            check(lib().jero_hip_model_trace(self.h, _ptr(buf), buf.numel()))

    def read_trace(self, buf):
        """The trace in `buf` as ([per-layer dict of numpy arrays], head dict)."""
        import numpy as np
        fields, layer_bytes, head, total = self.trace_layout()
        raw = buf[:total].cpu().numpy()

        def view(off, dt, n):
            return raw[off:off + n * np.dtype(dt).itemsize].view(dt).copy()

        layers = [{k: view(L * layer_bytes + o, dt, n) for k, (o, dt, n) in fields.items()}
                  for L in range(self.cfg.n_layers)]
        return layers, {k: view(o, dt, n) for k, (o, dt, n) in head.items()}

    def status(self, stream=None):
        """Waits for the stream; raises K3Error CapabilityMismatch once a step found no argmax
        (all-NaN logits), as the reference's engine fails closed (src/engine.rs:636-641)."""
        check(lib().jero_hip_model_status(self.h, _stream(stream)))

    def logits_len(self):
        """Logits per step: infer_logits_buffer_len once finalized (jero_hip_model_logits_len)."""
        return int(lib().jero_hip_model_logits_len(self.h))

    def read_logits(self, out):
        """Copies the last step's logits into the float32 device tensor `out` (at least
        logits_len() long; its first logits_len() values are written)."""
        n = self.logits_len()
        assert out.numel() >= n, f"logits buffer of {out.numel()} values, the model writes {n}"
        _, _, lp = self.state_ptrs()
        _memcpy(out.data_ptr(), lp, n * 4)
        return out

    def read_token_pos(self):
        import numpy as np
        tp, pp, _ = self.state_ptrs()
        t = np.zeros(1, np.int32)
        p = np.zeros(1, np.int64)
        _memcpy(t.ctypes.data, tp, 4)
        _memcpy(p.ctypes.data, pp, 8)
        return int(t[0]), int(p[0])


class GGUFFile:
    """A mapped GGUF v2/v3 model file (LockedModelWeights' weight source, src/weights.rs:338-570)."""

    def __init__(self, path):
        h = C.c_void_p()
        check(lib().jero_hip_gguf_open(os.fsencode(path), C.byref(h)))
        self.h = h
        n, a = _I64(), C.c_char_p()
        check(lib().jero_hip_gguf_info(h, C.byref(n), C.byref(a)))
        self.n_tensors, self.arch = n.value, a.value.decode()

    def close(self):
        if self.h:
            lib().jero_hip_gguf_close(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def meta_int(self, key, default=None):
        v = _I64()
        rc = lib().jero_hip_gguf_meta_int(self.h, key.encode(), C.byref(v))
        if rc and default is not None:
            return default
        check(rc)
        return v.value

    def meta_float(self, key, default=None):
        v = C.c_double()
        rc = lib().jero_hip_gguf_meta_float(self.h, key.encode(), C.byref(v))
        if rc and default is not None:
            return default
        check(rc)
        return v.value

    def meta_str(self, key):
        v = C.c_char_p()
        check(lib().jero_hip_gguf_meta_str(self.h, key.encode(), C.byref(v)))
        return v.value.decode()

    def tensor_names(self):
        out = []
        for i in range(self.n_tensors):
            v = C.c_char_p()
            check(lib().jero_hip_gguf_tensor_name(self.h, i, C.byref(v)))
            out.append(v.value.decode())
        return out

    def tensor(self, name):
        """ModelWeights::tensor (src/weights.rs:1097-1144), with the tied output.weight fallback:
        {quant, n_dims, dims (4, row length first), host (mapped address), nbytes}."""
        q, nd, dims, host, nb = C.c_int(), C.c_int(), (_I64 * 4)(), C.c_void_p(), _SZ()
        check(lib().jero_hip_gguf_tensor(self.h, name.encode(), C.byref(q), C.byref(nd), dims, C.byref(host),
                                         C.byref(nb)))
        return dict(quant=q.value, n_dims=nd.value, dims=list(dims), host=host.value, nbytes=nb.value)

    def tensor_bytes(self, name):
        """The tensor's bytes as a read-only numpy view of the mapping (valid until close)."""
        import numpy as np
        t = self.tensor(name)
        buf = (C.c_uint8 * t["nbytes"]).from_address(t["host"])
        a = np.frombuffer(buf, np.uint8)
        a.flags.writeable = False
        return a

    def tensor_view(self, name, device="cuda", repack_layout=False):
        """The tensor copied to a device TensorView (shape as in the file, row length first).
        repack_layout: Q4_K / Q6_K re-laid out on the device like a load-time repack
        (src/weights.rs:914-955): 2-D tensors to Q4_K_R / Q6_K_R, stacked expert tensors
        [n_in, rows, n_experts] with rows a multiple of 16 to Q4_K_T / Q6_K_T."""
        import torch
        t = self.tensor(name)
        dst = torch.empty(t["nbytes"], dtype=torch.uint8, device=device)
        _memcpy(dst.data_ptr(), t["host"], t["nbytes"])
        v = TensorView(name, t["quant"], t["dims"][:t["n_dims"]], dst)
        if repack_layout and v.quant in (Q4_K, Q6_K):
            v = repack(v)
            torch.cuda.synchronize(dst.device)
        return v

    def upload(self, name):
        """Device address of the tensor, copied to HBM once through the weight registry."""
        dev = C.c_void_p()
        check(lib().jero_hip_gguf_upload(self.h, name.encode(), C.byref(dev)))
        return dev.value

    def hyperparams(self):
        """GgufHyperparams::from_metadata (src/capability.rs:212-285) for the dense decoder:
        metadata first, tensor shapes where a key is absent (block count from the highest
        blk.N, head_count_kv = head_count, key_length from blk.0.attn_k's width, vocab from the
        LM head / embedding rows)."""
        a = self.arch
        names = set(self.tensor_names())
        emb = self.tensor("token_embd.weight")
        hidden = self.meta_int(f"{a}.embedding_length", 0) or emb["dims"][0]
        n_layers = self.meta_int(f"{a}.block_count", 0)
        if not n_layers:
            n_layers = 1 + max([int(n.split(".")[1]) for n in names if n.startswith("blk.")], default=-1)
        nq = self.meta_int(f"{a}.attention.head_count")
        nkv = self.meta_int(f"{a}.attention.head_count_kv", 0) or nq
        hd = self.meta_int(f"{a}.attention.key_length", 0)
        if not hd:
            k = self.tensor("blk.0.attn_k.weight")
            hd = k["dims"][1] // nkv if k["dims"][1] % nkv == 0 else hidden // nq
        ffn = self.meta_int(f"{a}.feed_forward_length", 0)
        if not ffn and "blk.0.ffn_gate.weight" in names:
            ffn = self.tensor("blk.0.ffn_gate.weight")["dims"][1]
        vocab = self.meta_int(f"{a}.vocab_size", 0) or self.tensor("output.weight")["dims"][1]
        eps = self.meta_float(f"{a}.attention.layer_norm_rms_epsilon", 1e-6)
        theta = self.meta_float(f"{a}.rope.freq_base", 10000.0)
        # MoE (GgufHyperparams' expert_count, expert_used_count, expert_feed_forward_length and
        # expert_shared_count, src/capability.rs:58-65, 428-455): the Qwen3-MoE recipe's spec
        moe = None
        n_exp = self.meta_int(f"{a}.expert_count", 0)
        if n_exp:
            top_k = self.meta_int(f"{a}.expert_used_count", 0)
            f_exp = self.meta_int(f"{a}.expert_feed_forward_length", 0) or \
                self.meta_int(f"{a}.expert.feed_forward_length", 0)
            if not f_exp and "blk.0.ffn_gate_exps.weight" in names:
                f_exp = self.tensor("blk.0.ffn_gate_exps.weight")["dims"][1]
            shared = self.meta_int(f"{a}.expert_shared_count", 0) or self.meta_int(f"{a}.expert.shared_count", 0)
            moe = (n_exp, top_k, f_exp, shared > 0)
        ffn = ffn or (moe[2] if moe else 0)
        return dict(hidden=hidden, ffn=ffn, n_layers=n_layers, vocab=vocab, n_heads_q=nq, n_heads_kv=nkv,
                    head_dim=hd, rms_eps=eps, rope_theta=theta, qk_norm="blk.0.attn_q_norm.weight" in names, moe=moe)
