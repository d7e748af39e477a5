"""Device copies of host weight tensors (the binding path for mmaped GGUF bytes): one upload per
tensor, sub-range views map to the matching device bytes, and a GEMV on a registered row slice
equals the same rows of the whole tensor (the reference's partition invariance,
tests/wave1_engine_regression_test.rs:1286-1295)."""
import ctypes as C

import numpy as np
import pytest
import torch

import jero_hip as J
import pyoracle as O
from qdata import rand_act, rand_weights

pytestmark = pytest.mark.gpu


def matvec_dev(quant, w_dev, nbytes, k, n, xq, y):
    J.check(J.lib().jero_hip_matvec(quant, C.c_void_p(w_dev), nbytes, k, n, C.c_void_p(xq.data_ptr()),
                                    C.c_void_p(y.data_ptr()), J._stream()))


def test_register_slice_and_release(dev):
    k, n = 1024, 512
    w = rand_weights(J.Q4_K, n, k, 4242)
    rb = J.row_bytes(J.Q4_K, k)
    x = rand_act(k, 4243)
    xq = J.quantize_act(J.Q8_K, torch.from_numpy(x).to(dev))
    d0 = J.weights_register(w)
    assert J.weights_register(w) == d0                       # second registration: same bytes
    y = torch.empty(n, device=dev)
    matvec_dev(J.Q4_K, d0, w.nbytes, k, n, xq, y)
    ref = O.matvec(J.Q4_K, w, k, n, xq.cpu().numpy(), threads=4)
    full = y.cpu().numpy()
    assert np.max(np.abs(full - ref)) <= 1e-5 * max(np.abs(ref).max(), 1e-30)
    # a row slice view of the host tensor maps inside the registered copy
    start, count = 100, 37
    view = w[start * rb:(start + count) * rb]
    dv = J.weights_lookup(view)
    assert dv == d0 + start * rb
    assert J.weights_register(view) == dv
    ys = torch.empty(count, device=dev)
    matvec_dev(J.Q4_K, dv, view.nbytes, k, count, xq, ys)
    assert np.array_equal(ys.cpu().numpy(), full[start:start + count])
    # partial overlap with a bigger range is rejected; unregistered bytes are not found
    bigger = np.concatenate([w, w])
    with pytest.raises(J.K3Error) as e:
        J.weights_lookup(bigger)
    assert e.value.variant == "TensorBoundsError"
    J.weights_release_all()
    with pytest.raises(J.K3Error):
        J.weights_lookup(w)
    J.sync()


def test_release_range_and_gguf_close(dev, tmp_path):
    """jero_hip_weights_release frees the copies inside a host range; gguf_close does it for the
    mapping, so a second file mapped at the same addresses uploads its own bytes, never the
    first file's stale copy."""
    import gguf_writer as W
    a = rand_weights(J.Q4_K, 8, 512, 77)
    b = rand_weights(J.Q4_K, 8, 512, 78)
    assert not np.array_equal(a, b)
    d = J.weights_register(a)
    J.weights_release(a)
    with pytest.raises(J.K3Error):
        J.weights_lookup(a)
    assert J.weights_register(a) is not None
    J.weights_release(a)
    paths = []
    for i, arr in enumerate((a, b)):
        p = tmp_path / f"m{i}.gguf"
        p.write_bytes(W.gguf_bytes("llama", [], [("w", J.Q4_K, (512, 8), arr.tobytes())]))
        paths.append(p)
    assert paths[0].stat().st_size == paths[1].stat().st_size
    for p, arr in zip(paths, (a, b)):
        g = J.GGUFFile(str(p))
        host = g.tensor_bytes("w")
        dv = g.upload("w")
        back = np.zeros(arr.nbytes, np.uint8)
        J._memcpy(back.ctypes.data, dv, arr.nbytes)
        np.testing.assert_array_equal(back, arr)
        g.close()
        with pytest.raises(J.K3Error):
            J.weights_lookup(host)  # released with the mapping
    J.sync()
    del d
