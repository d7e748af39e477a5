"""GPU parity of the int8 forward path's entry points: requant (forward.rs:345-350) fused into the
int8 product or alone, and the packed-tile product (ime::gemm_i8_ime) with the reference's own
callbacks (matmul_rows, src/forward.rs:763-811), plus the ring-slice call shape of
gqa_causal_attention_f32 (src/qwen_deepseek.rs:660-677).  Integer results are bit-exact against
int64 numpy products and the oracle's requant."""
import numpy as np
import pytest
import torch

import jero_hip as J
import pyoracle as O

pytestmark = pytest.mark.gpu


def to_dev(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def rand_i8(rng, shape, lo=-128, hi=128):
    return rng.integers(lo, hi, size=shape, dtype=np.int64).astype(np.int8)


@pytest.mark.parametrize("shift", [1, 7, 12, 31])
def test_requant_all_bit_exact(dev, shift):
    rng = np.random.default_rng(shift)
    raw = rng.integers(-(1 << 31), 1 << 31, size=100003, dtype=np.int64).astype(np.int32)
    raw[:8] = [2147483647, -2147483648, 0, -1, 1, 127 << shift if shift < 24 else 5, -(1 << 30), 1 << 30]
    out = J.requant_all(to_dev(raw, dev), shift).cpu().numpy()
    assert np.array_equal(out, O.requant(raw, shift))


@pytest.mark.parametrize("m,k,n,shift", [(512, 512, 512, 9), (37, 80, 45, 6), (5, 33, 7, 3), (130, 4096, 260, 14),
                                         (64, 8192, 128, 16)])
def test_gemm_i8_requant_bit_exact(dev, m, k, n, shift):
    print(f"gemm_i8_requant m={m} k={k} n={n} shift={shift}", flush=True)
    rng = np.random.default_rng(m + k + n + shift)
    x = rand_i8(rng, (m, k), -8, 8)  # forward.rs's fill_small range
    w = rand_i8(rng, (n, k))
    out = J.gemm_i8_requant(to_dev(x, dev), to_dev(w, dev), shift).cpu().numpy()
    ref = O.requant(x.astype(np.int64) @ w.astype(np.int64).T, shift)
    assert np.array_equal(out, ref)


@pytest.mark.parametrize("rows,k", [(13, 64), (512, 512), (8, 32), (1, 96)])
def test_pack_tiles_device_layout(dev, rows, k):
    rng = np.random.default_rng(rows * k)
    x = rand_i8(rng, (rows, k))
    p = J.ime.pack_tiles(to_dev(x, dev), rows, k).cpu().numpy()
    assert np.array_equal(p, O.pack_tiles(x, rows, k))


@pytest.mark.parametrize("m,k,n,tiles", [(13, 512, 64, (0, 8)), (512, 512, 512, (0, 64)), (100, 1024, 512, (16, 40)),
                                         (1, 32, 8, (0, 1)), (37, 4096, 200, (3, 25))])
def test_gemm_i8_ime_callback(dev, m, k, n, tiles):
    """matmul_rows' IME branch (src/forward.rs:779-796) over the packed operands: rows >= m and
    columns outside the tile range are not written; every written value equals the int64 product."""
    print(f"gemm_i8_ime m={m} k={k} n={n} tiles={tiles}", flush=True)
    rng = np.random.default_rng(m * 31 + k + n)
    x = rand_i8(rng, (m, k))
    w_rows = rand_i8(rng, (n, k))
    n_pad = J.ime.tile_count(n) * J.ime.TILE_N
    a = J.ime.pack_tiles(to_dev(x, dev), m, k)
    pw = J.ime.pack_tiles(to_dev(w_rows, dev), n, k)
    abs_rows = range(tiles[0] * 8, min(tiles[1] * 8, n_pad))
    out = np.full((m, n_pad), -7, np.int64)

    def emit(mt, nt, c):
        for i in range(J.ime.TILE_M):
            row = mt * J.ime.TILE_M + i
            if row >= m:
                break
            for j in range(J.ime.TILE_N):
                col = nt * J.ime.TILE_N + j
                if abs_rows.start <= col < abs_rows.stop:
                    out[row, col] = c[i * J.ime.TILE_N + j]

    J.ime.gemm_i8_ime(a, J.ime.tile_count(m), pw, range(*tiles), k // J.ime.TILE_K, emit)
    w_pad = np.zeros((n_pad, k), np.int64)
    w_pad[:n] = w_rows
    ref = x.astype(np.int64) @ w_pad.T
    cols = list(abs_rows)
    assert np.array_equal(out[:, cols], ref[:, cols])
    others = [c for c in range(n_pad) if c not in abs_rows]
    assert (out[:, others] == -7).all()


def test_gemm_i8_vector_callback(dev):
    """gemm_i8_vector (src/forward.rs:797-806): emit(row, col, v) for every row < m, col in the range."""
    rng = np.random.default_rng(11)
    m, k, n = 9, 512, 64
    x = rand_i8(rng, (m, k))
    rows = rand_i8(rng, (n, k))
    got = {}
    J.ime.gemm_i8_vector(to_dev(x, dev), m, to_dev(rows, dev), range(16, 40), k,
                         lambda r, c, v: got.__setitem__((r, c), v))
    ref = x.astype(np.int64) @ rows.astype(np.int64).T
    assert sorted(got) == [(r, c) for r in range(m) for c in range(16, 40)]
    assert all(got[(r, c)] == ref[r, c] for r, c in got)


@pytest.mark.parametrize("capacity,pos", [(64, 10), (64, 63), (64, 200), (300, 299)])
def test_attention_ring_slice_call_shape(dev, capacity, pos):
    """The call site's shape (src/qwen_deepseek.rs:660-677): the new k/v written at slot = pos %
    capacity of an f32 ring, attention over the first active_len = min(pos + 1, capacity) rows."""
    nq, nkv, hd = 8, 2, 64
    kv_dim = nkv * hd
    rng = np.random.default_rng(capacity + pos)
    k_ring = rng.standard_normal((capacity, kv_dim)).astype(np.float32)
    v_ring = rng.standard_normal((capacity, kv_dim)).astype(np.float32)
    q = rng.standard_normal(nq * hd).astype(np.float32)
    slot, active = pos % capacity, min(pos + 1, capacity)
    k_ring[slot] = rng.standard_normal(kv_dim)
    v_ring[slot] = rng.standard_normal(kv_dim)
    scale = 1.0 / np.sqrt(hd)
    kd, vd = to_dev(k_ring, dev), to_dev(v_ring, dev)
    out = torch.empty(nq * hd, dtype=torch.float32, device=dev)
    J.gqa_causal_attention_f32(out, to_dev(q, dev), kd[:active], vd[:active], nq, nkv, hd, active, scale)
    ref = O.gqa_attention(q, k_ring[:active], v_ring[:active], nq, nkv, hd, active, scale)
    got = out.cpu().numpy().astype(np.float64)
    r = np.asarray(ref, np.float64)
    s = max(float(np.sqrt(np.mean(r ** 2))), 1e-30)
    assert float(np.max(np.abs(got - r) / np.maximum(np.abs(r), s))) < 1e-3


def test_attention_context_length_exceeded(dev):
    z = torch.zeros(1024, dtype=torch.float32, device=dev)
    with pytest.raises(J.K3Error) as ei:
        J.gqa_causal_attention_f32(z, z, z, z, 4, 2, 64, 131073, 1.0)
    assert ei.value.variant == "ContextLengthExceeded"
