"""Variant index formats on the CPU: packing known answers (worked out by
hand from the reference's byte formulas), round trips and the reference's
own packing cases, the oracle's reconstructions against explicit loops, and
HelixLinear with pair codebooks (int16 and 12-bit packed) on its CPU path."""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate.helix_linear import HelixLinear
from helix_substrate.index_packing import (pack_6bit, pack_12bit, unpack_6bit, unpack_12bit,
                                           unpack_12bit_rows)


def test_pack_12bit_known_answer():
    # (0, 4095) -> [0x00, 0xF0, 0xFF]; (1, 2048) -> [0x01, 0x00, 0x80];
    # (100, 3999 = 0xF9F) -> [0x64, 0xF0, 0xF9]
    vals = torch.tensor([0, 4095, 1, 2048, 100, 3999], dtype=torch.int16)
    want = [0x00, 0xF0, 0xFF, 0x01, 0x00, 0x80, 0x64, 0xF0, 0xF9]
    assert pack_12bit(vals).tolist() == want
    assert oracle.pack_12bit_np(vals.numpy()).tolist() == want
    assert torch.equal(unpack_12bit(torch.tensor(want, dtype=torch.uint8), 6), vals)


def test_pack_6bit_known_answer():
    # codec spec: byte0 = q0 | q1 << 6, byte1 = q1 >> 2 | q2 << 4, byte2 = q2 >> 4 | q3 << 2
    q = torch.tensor([63, 0, 0, 63, 1, 2, 3, 4, 0x2A, 0x15, 0x3C, 0x03], dtype=torch.uint8)
    want = [63, 0, 252,
            1 | (2 << 6), (2 >> 2) | (3 << 4), (3 >> 4) | (4 << 2),
            (0x2A | (0x15 << 6)) & 255, ((0x15 >> 2) | (0x3C << 4)) & 255, (0x3C >> 4) | (0x03 << 2)]
    assert pack_6bit(q).tolist() == want
    assert oracle.unpack_6bit_np(np.array(want, np.uint8), 12).tolist() == q.tolist()
    assert torch.equal(unpack_6bit(torch.tensor(want, dtype=torch.uint8), 12), q)


def test_packing_round_trips_and_errors():
    g = torch.Generator().manual_seed(0)
    v = torch.randint(0, 4096, (100000,), generator=g, dtype=torch.int32).to(torch.int16)
    p = pack_12bit(v)
    assert p.numel() == 150000 and torch.equal(unpack_12bit(p, 100000), v)
    np.testing.assert_array_equal(oracle.unpack_12bit_np(p.numpy(), 100000), v.numpy())
    m = v.reshape(100, 1000)
    assert torch.equal(unpack_12bit_rows(pack_12bit(m), 10, 20, 1000), m[10:20])
    assert torch.equal(unpack_12bit_rows(pack_12bit(m), 99, 100, 1000), m[99:100])
    q = torch.randint(0, 64, (4096,), generator=g, dtype=torch.int32).to(torch.uint8)
    assert torch.equal(unpack_6bit(pack_6bit(q), 4096), q)
    with pytest.raises(ValueError, match="even"):
        pack_12bit(torch.tensor([1, 2, 3], dtype=torch.int16))
    with pytest.raises(ValueError, match="4096"):
        pack_12bit(torch.tensor([4096, 0], dtype=torch.int16))
    with pytest.raises(ValueError):
        pack_6bit(torch.tensor([64, 0, 0, 0]))


def test_packed_streams_are_little_endian_bitfields():
    # field i of the 12-bit stream sits at bit 12 i; of the 6-bit one at bit 6 i
    g = torch.Generator().manual_seed(1)
    v = torch.randint(0, 4096, (8,), generator=g, dtype=torch.int32)
    big = int.from_bytes(bytes(pack_12bit(v.to(torch.int16)).tolist()), "little")
    assert [(big >> (12 * i)) & 0xFFF for i in range(8)] == v.tolist()
    q = torch.randint(0, 64, (16,), generator=g, dtype=torch.int32)
    big = int.from_bytes(bytes(pack_6bit(q).tolist()), "little")
    assert [(big >> (6 * i)) & 63 for i in range(16)] == q.tolist()


def test_reconstruct_oracles_against_loops():
    rs = np.random.RandomState(2)
    cb = rs.randn(37, 2).astype(np.float32)
    idx = rs.randint(0, 37, (3, 5))
    w = oracle.reconstruct_vq2_np(idx, cb, [1, 29], [7.0, -7.0])
    for o in range(3):
        for j in range(10):
            want = cb[idx[o, j // 2], j % 2]
            if o * 10 + j == 1:
                want = 7.0
            if o * 10 + j == 29:
                want = -7.0
            assert w[o, j] == want
    q = rs.randint(0, 64, (2, 8))
    s = rs.uniform(0.5, 1.5, (2, 2)).astype(np.float32)
    off = rs.randn(2, 2).astype(np.float32)
    w6 = oracle.reconstruct_af6_np(q, s, off, 4)
    for o in range(2):
        for i in range(8):
            assert w6[o, i] == np.float32(np.float32(q[o, i] * s[o, i // 4]) + off[o, i // 4])


def _pair_layer(out=64, inp=128, k=4096, packed=False, sidecar=True, seed=3):
    g = torch.Generator().manual_seed(seed)
    cb = torch.randn(k, 2, generator=g) * 0.02
    idx = torch.randint(0, k, (out, inp // 2), generator=g, dtype=torch.int32).to(torch.int16)
    pos = val = None
    if sidecar:
        pos = torch.randperm(out * inp, generator=g)[: out * inp // 100].sort().values
        val = torch.randn(pos.numel(), generator=g)
    bias = torch.randn(out, generator=g)
    ind = pack_12bit(idx) if packed else idx
    m = HelixLinear(inp, out, cb, ind, sidecar_positions=pos, sidecar_values=val, bias=bias,
                    vector_dim=2)
    W = oracle.reconstruct_vq2_np(idx.numpy(), cb.numpy(),
                                  None if pos is None else pos.numpy(),
                                  None if val is None else val.numpy())
    return m, W, bias.numpy()


@pytest.mark.parametrize("packed", [False, True])
def test_pair_helix_linear_cpu(packed):
    m, W, b = _pair_layer(packed=packed)
    assert m.vector_dim == 2 and m.index_packing == ("12bit" if packed else None)
    np.testing.assert_array_equal(m.decode_weight().numpy(), W)
    for start, end in [(0, 16), (10, 26), (48, 64)]:
        np.testing.assert_array_equal(m._dequant_tile(start, end).numpy(), W[start:end])
    x = torch.randn(3, 128)
    y = m(x).numpy()
    np.testing.assert_allclose(y, oracle.linear_f64(x.numpy(), W, b), rtol=1e-5, atol=1e-5)
    # sidecar deltas are value - reconstruction at the position
    rows, cols = m._sidecar_rows, m._sidecar_cols
    m2, W2, _ = _pair_layer(packed=packed, sidecar=False)
    np.testing.assert_array_equal(m._sc_delta.numpy(),
                                  (m._sc_val - torch.from_numpy(W2)[rows, cols]).numpy())


def test_pair_shell_and_recompute():
    shell = HelixLinear.from_quantized_config(128, 64, n_clusters=4096, vector_dim=2,
                                              index_packing="12bit")
    assert shell.index_packing == "12bit" and shell.indices.dtype == torch.uint8
    assert shell.indices.shape == (64 * 64 * 3 // 2,)
    plain = HelixLinear.from_quantized_config(128, 64, n_clusters=4096, vector_dim=2)
    assert plain.index_packing is None and plain.indices.shape == (64, 64)
    assert plain.indices.dtype == torch.int16
    g = torch.Generator().manual_seed(4)
    shell.register_buffer("indices", pack_12bit(torch.randint(0, 4096, (64 * 64,), generator=g)))
    shell.register_buffer("codebook", torch.randn(4096, 2, generator=g))
    shell._recompute_derived()
    assert shell.index_packing == "12bit" and (shell._idx_rows, shell._idx_cols) == (64, 64)
    assert shell.vector_dim == 2
    # 25% less index storage than int16
    m16, _, _ = _pair_layer(out=3584 // 28, inp=7168 // 28 * 2 // 2 * 2, sidecar=False)
    mp, _, _ = _pair_layer(out=3584 // 28, inp=7168 // 28 * 2 // 2 * 2, packed=True, sidecar=False)
    assert mp.indices.numel() * 1 == m16.indices.numel() * 2 * 3 // 4
