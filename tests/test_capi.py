"""The C ABI without a GPU: the library loads, exports every declared entry point, and
rejects bad arguments with the K3Error-mirroring status before touching the device."""
import ctypes as C

import pytest

import jero_hip as J


def test_library_exports_every_declared_symbol():
    lib = J.lib()
    declared = J.declared_symbols()
    assert len(declared) >= 8
    missing = [s for s in declared if not hasattr(lib, s)]
    assert missing == []


def test_status_names_mirror_k3error():
    lib = J.lib()
    names = {s: lib.jero_hip_status_name(s).decode() for s in (0, 10, 11, 12, 14, 15, 20, 21)}
    assert names[10] == "CapabilityMismatch"
    assert names[14] == "TensorBoundsError"
    assert names[11] == "InsufficientLockableMemory"
    assert names[15] == "RoutingUnavailable"


def test_row_bytes_and_act_formats():
    assert J.row_bytes(J.Q4_K, 4096) == 16 * 144
    assert J.row_bytes(J.Q6_K, 4096) == 16 * 210
    assert J.row_bytes(J.Q8_0, 4096) == 128 * 34
    assert J.row_bytes(J.Q8_K, 4096) == 16 * 292
    assert J.row_bytes(J.ACT_Q8, 4096) == 128 * 36
    assert J.row_bytes(J.Q4_K, 100) == -1
    assert J.act_format(J.Q4_K) == J.Q8_K and J.act_format(J.Q6_K) == J.Q8_K
    assert J.act_format(J.Q8_0) == J.ACT_Q8 and J.act_format(J.Q4_0) == J.ACT_Q8
    assert J.act_format(J.F32) == J.F32 and J.act_format(J.F16) == J.F32 and J.act_format(J.BF16) == J.F32
    assert J.act_format(J.Q8_K) == -1


def _matvec(quant, w, nbytes, n_in, n_out, xq, y):
    return J.lib().jero_hip_matvec(quant, w, nbytes, n_in, n_out, xq, y, None)


def test_matvec_argument_errors_before_launch():
    fake = C.c_void_p(0x10000)  # never dereferenced: every call below fails validation first
    assert _matvec(J.Q4_K, None, 1 << 20, 256, 4, fake, fake) == 21             # null weights
    assert _matvec(J.Q4_K, fake, 1 << 20, 0, 4, fake, fake) == 14               # empty input
    assert _matvec(J.Q4_K, fake, 1 << 20, 256, 0, fake, fake) == 14             # empty output
    assert _matvec(J.Q4_K, fake, 1 << 20, 100, 4, fake, fake) == 14             # not a block multiple
    assert _matvec(J.Q4_K, fake, 144 * 4 - 1, 256, 4, fake, fake) == 14         # tensor too small
    assert _matvec(3, fake, 1 << 20, 256, 4, fake, fake) == 10                  # unsupported quant (Q4_1)
    assert _matvec(J.Q4_K, fake, 1 << 62, 256 * ((1 << 22) + 1), 1, fake, fake) == 10  # n_in above 2^30
    assert _matvec(J.Q4_K, C.c_void_p(0x10002), 1 << 20, 256, 4, fake, fake) == 21  # misaligned


def test_k3error_carries_variant_and_message():
    with pytest.raises(J.K3Error) as ei:
        J.check(_matvec(J.Q4_K, C.c_void_p(0x10000), 10, 256, 4, C.c_void_p(0x10000), C.c_void_p(0x10000)))
    assert ei.value.variant == "TensorBoundsError"
    assert "bytes" in str(ei.value)


def test_quantize_argument_errors():
    lib = J.lib()
    fake = C.c_void_p(0x10000)
    assert lib.jero_hip_quantize_act(J.Q4_K, fake, 1, 256, fake, None) == 10
    assert lib.jero_hip_quantize_act(J.Q8_K, fake, 1, 100, fake, None) == 14
    assert lib.jero_hip_quantize_act(J.Q8_K, None, 1, 256, fake, None) == 21


def test_read_probe_argument_errors():
    lib = J.lib()
    fake = C.c_void_p(0x10000)
    assert lib.jero_hip_read_probe(None, 1024, fake, None) == 21
    assert lib.jero_hip_read_probe(fake, 1024, None, None) == 21
    assert lib.jero_hip_read_probe(C.c_void_p(0x10008), 1024, fake, None) == 21  # misaligned
    assert lib.jero_hip_read_probe(fake, 1000, fake, None) == 21  # not a multiple of 16
    assert lib.jero_hip_read_probe(fake, 0, fake, None) == 21


def test_int8_entry_argument_errors():
    lib = J.lib()
    fake = C.c_void_p(0x10000)
    assert lib.jero_hip_requant_i8(fake, 16, 0, fake, None) == 21      # shift 0
    assert lib.jero_hip_requant_i8(fake, 16, 32, fake, None) == 21     # shift above 31
    assert lib.jero_hip_requant_i8(None, 16, 7, fake, None) == 21
    assert lib.jero_hip_requant_i8(fake, 0, 7, fake, None) == 14
    assert lib.jero_hip_gemm_i8_requant(fake, 4, 64, fake, 4, 0, fake, None) == 21
    assert lib.jero_hip_gemm_i8_requant(fake, 0, 64, fake, 4, 7, fake, None) == 14
    assert lib.jero_hip_pack_tiles(fake, 8, 48, fake, None) == 14      # k not a multiple of 32
    assert lib.jero_hip_pack_tiles(fake, 0, 64, fake, None) == 14
    assert lib.jero_hip_gemm_i8_tiles(fake, 1, fake, 2, 2, 2, fake, None) == 14   # empty tile range
    assert lib.jero_hip_gemm_i8_tiles(C.c_void_p(0x10002), 1, fake, 0, 1, 2, fake, None) == 21  # misaligned
    assert lib.jero_hip_gemm_i8_tiles(fake, 1, fake, 0, 1, 1 << 13, fake, None) == 10  # k = 2^18: int32 overflow
    assert [lib.jero_hip_tile_count(r) for r in (0, 1, 8, 9, 512)] == [0, 1, 1, 2, 64]
