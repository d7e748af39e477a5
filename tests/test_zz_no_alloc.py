"""jero_hip_vec_dot_noalloc (activation staged in the library's static device array) against
jero_hip_vec_dot (staged in a caller workspace) through the C ABI: bit-identical outputs on two
calls in a row, the second with a smaller input, for every weight format; sizes beyond the
static array are rejected."""
import ctypes as C

import numpy as np
import pytest
import torch

import jero_hip as J
from qdata import rand_act, rand_float_weights, rand_weights

pytestmark = pytest.mark.gpu


def call(fn, quant, w, n_in, n_out, x, y, *extra):
    J.check(fn(quant, C.c_void_p(w.data_ptr()), w.numel(), n_in, n_out, C.c_void_p(x.data_ptr()),
               C.c_void_p(y.data_ptr()), *extra, J._stream()))


@pytest.mark.parametrize("quant", [J.Q4_K, J.Q6_K, J.Q8_0, J.Q4_0, J.F32, J.F16, J.BF16])
def test_noalloc_matches_vec_dot(dev, quant):
    """The quantized formats stage the activation in the static array; F32 / F16 / BF16 rows take
    the f32 input unstaged (their own branch of the entry point)."""
    print(f"vec_dot_noalloc quant={quant}", flush=True)
    lib = J.lib()
    floats = quant in (J.F32, J.F16, J.BF16)
    for i, (n_in, n_out) in enumerate(((8192, 3000), (1024, 77))):  # second call smaller
        gen = rand_float_weights if floats else rand_weights
        w = torch.from_numpy(gen(quant, n_out, n_in, 300 + i)).to(dev)
        x = torch.from_numpy(rand_act(n_in, 310 + i)).to(dev)
        y0 = torch.empty(n_out, dtype=torch.float32, device=dev)
        y1 = torch.full((n_out,), float("nan"), dtype=torch.float32, device=dev)
        ws = torch.empty(4 * n_in if floats else J.row_bytes(J.act_format(quant), n_in), dtype=torch.uint8, device=dev)
        call(lib.jero_hip_vec_dot, quant, w, n_in, n_out, x, y0, C.c_void_p(ws.data_ptr()), ws.numel())
        call(lib.jero_hip_vec_dot_noalloc, quant, w, n_in, n_out, x, y1)
        torch.cuda.synchronize()
        assert torch.equal(y0, y1), (quant, n_in)


def test_noalloc_rejects_oversized_input(dev):
    n_in = 131072  # Q8_K blocks of 149504 bytes: above the 128 KiB static buffer
    w = torch.zeros(J.row_bytes(J.Q4_K, n_in), dtype=torch.uint8, device=dev)
    x = torch.zeros(n_in, dtype=torch.float32, device=dev)
    y = torch.zeros(1, dtype=torch.float32, device=dev)
    with pytest.raises(J.K3Error) as ei:
        call(J.lib().jero_hip_vec_dot_noalloc, J.Q4_K, w, n_in, 1, x, y)
    assert ei.value.variant == "CapabilityMismatch"
