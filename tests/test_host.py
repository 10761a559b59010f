"""Host-side logic on the CPU: CSR layout, CDNAv3 files, HelixLinear API surface.

Mirrors the reference's host tests (tests/test_helix_linear.py,
tests/test_hxq_writer_reader.py, tests/test_sidecar_v3.py) against the oracle.
"""
import numpy as np
import pytest
import torch
import torch.nn as nn

import oracle
from helix_substrate import synth
from helix_substrate.generate_sidecars_v3 import read_sidecar_v3, write_sidecar_npz
from helix_substrate.helix_linear import (HelixLinear, _tensor_name_to_module_path,
                                          load_cdna_factors, load_helix_linear_from_cdnav3,
                                          swap_summary, swap_to_helix)
from helix_substrate.hxq_format import build_sidecar_csr, compressed_bytes
from helix_substrate.hxq_reader_v3 import CDNAv3Reader
from helix_substrate.hxq_writer_v3 import CDNAv3Writer


def _module(L, bias=None):
    T = synth.to_torch(L)
    out_f, in_f = T["indices"].shape
    return HelixLinear(in_f, out_f, T["codebook"], T["indices"], T["sidecar_positions"],
                       T["sidecar_values"], bias=bias, group_scale=T["group_scale"],
                       group_offset=T["group_offset"], group_size=L["group_size"])


def _oracle_w(L):
    return oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"],
                              L["group_size"], L["sidecar_positions"], L["sidecar_values"])


def test_sidecar_npz_known_values(tmp_path):
    # reference tests/test_sidecar_v3.py:79-94 (+ the exact fp16 values)
    pos = np.array([0, 5, 100, 999], np.int64)
    val = np.array([1.5, -2.3, 0.01, 100.0], np.float32)
    r = write_sidecar_npz(pos, val, tmp_path / "sidecar.npz")
    assert r["num_corrections"] == 4 and r["size_bytes"] > 0
    p2, v2 = read_sidecar_v3(tmp_path / "sidecar.npz")
    np.testing.assert_array_equal(p2, pos)
    np.testing.assert_allclose(v2, val, atol=0.1)
    np.testing.assert_array_equal(v2, np.array([1.5, -2.30078125, 0.01000213623046875, 100.0], np.float32))


def test_csr_identities():
    L = synth.make_layer_np(50, 128, seed=3, density=0.02)
    T = synth.to_torch(L)
    csr = build_sidecar_csr(T["sidecar_positions"], T["sidecar_values"], T["indices"],
                            T["codebook"], T["group_scale"], T["group_offset"], 128)
    pos = L["sidecar_positions"]
    np.testing.assert_array_equal(csr.rows.numpy(), pos // 128)   # sorted input keeps order
    np.testing.assert_array_equal(csr.cols.numpy(), pos % 128)
    counts = np.bincount(pos // 128, minlength=50)
    np.testing.assert_array_equal(np.diff(csr.row_ptr.numpy()), counts)
    W = oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"], 128)
    np.testing.assert_array_equal(csr.vq.numpy(), W.ravel()[pos])          # W_affine at pos
    np.testing.assert_array_equal(csr.delta.numpy(), (L["sidecar_values"] - W.ravel()[pos]))


def test_csr_stable_for_unsorted_and_repeated_positions():
    idx = torch.zeros(4, 16, dtype=torch.uint8)
    cb = torch.zeros(256)
    pos = torch.tensor([40, 3, 40, 17], dtype=torch.int64)
    val = torch.tensor([1.0, 2.0, 3.0, 4.0])
    csr = build_sidecar_csr(pos, val, idx, cb)
    # row-major order, one entry per position: the last stored value of 40 wins
    assert csr.row_ptr.tolist() == [0, 1, 2, 3, 3]
    assert csr.col.tolist() == [3, 1, 8]
    assert csr.val.tolist() == [2.0, 4.0, 3.0]
    pos2 = torch.tensor([9, 2, 9, 9, 5, 2], dtype=torch.int64)
    csr2 = build_sidecar_csr(pos2, torch.arange(6, dtype=torch.float32), idx, cb)
    assert csr2.col.tolist() == [2, 5, 9] and csr2.val.tolist() == [5.0, 4.0, 3.0]
    with pytest.raises(ValueError):
        build_sidecar_csr(torch.tensor([64]), torch.tensor([1.0]), idx, cb)


def test_decode_weight_bit_exact_cpu():
    L = synth.make_layer_np(300, 256, seed=9, density=0.01)
    m = _module(L)
    W = m.decode_weight().numpy()
    np.testing.assert_array_equal(W.view(np.uint32), _oracle_w(L).view(np.uint32))
    # _dequant_tile(0, all) == decode_weight; sub-tiles concatenate (tests/test_fused_parity.py:73-109)
    tiles = [m._dequant_tile(r, min(r + 64, 300)) for r in range(0, 300, 64)]
    np.testing.assert_array_equal(torch.cat(tiles).numpy(), W)


def test_short_codebook_kernel_copy_is_padded():
    """Scalar-codebook kernels read 256 entries: a k < 256 codebook gets a
    zero-padded kernel copy (_kcb); the saved codebook keeps k entries, and
    the kernel wrappers refuse a short codebook."""
    from helix_substrate import _hxq
    L = synth.make_layer_np(40, 128, seed=5, sidecar=False)
    L["codebook"] = np.sort(np.random.RandomState(1).standard_normal(37).astype(np.float32))
    L["indices"] = np.random.RandomState(2).randint(0, 37, (40, 128)).astype(np.uint8)
    m = _module(L)
    assert m.codebook.numel() == 37 and m.state_dict()["codebook"].numel() == 37
    assert not any("kcb" in k for k in m.state_dict())
    assert m._kcb.numel() == 256
    assert torch.equal(m._kcb[:37], m.codebook) and not m._kcb[37:].any()
    np.testing.assert_array_equal(m.decode_weight().numpy(), _oracle_w(L))
    with pytest.raises(ValueError):
        _hxq._need_cb256(m.codebook)
    _hxq._need_cb256(m._kcb)
    # the padded copy follows the codebook: in-place edits, load_state_dict
    m.codebook.mul_(2.0)
    assert torch.equal(m._kcb[:37], m.codebook)
    sd = {k: v.clone() for k, v in m.state_dict().items()}
    sd["codebook"] = sd["codebook"] + 1.0
    m.load_state_dict(sd, strict=False)
    assert torch.equal(m._kcb[:37], sd["codebook"]) and not m._kcb[37:].any()
    # a full 256-entry codebook is used as is (no copy to go stale)
    m2 = _module(synth.make_layer_np(8, 128, seed=6, sidecar=False))
    assert m2._kcb is m2.codebook


@pytest.mark.parametrize("cast", ["bfloat16", "half", "double"])
def test_dtype_cast_keeps_hxq_state_fp32(cast):
    """module.bfloat16() / .half() / .double() (e.g. model.to(dtype) after loading)
    must not round the codebook, affine, sidecar or bias the kernels read as fp32."""
    L = synth.make_layer_np(96, 256, seed=12, density=0.01)
    b = torch.linspace(-1, 1, 96)
    m = getattr(_module(L, bias=b), cast)()
    for name in HelixLinear._FP32_STATE:
        t = getattr(m, name, None)
        assert t is None or t.dtype == torch.float32, (name, t.dtype)
    assert m.indices.dtype == torch.uint8
    np.testing.assert_array_equal(m.decode_weight().numpy().view(np.uint32),
                                  _oracle_w(L).view(np.uint32))
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(1))
    yr = oracle.linear_f64(x.numpy(), _oracle_w(L), b.numpy())
    y = m(x)
    assert y.dtype == torch.float32
    assert np.abs(y.numpy() - yr).max() / np.abs(yr).max() < 1e-5


def test_kernel_wrappers_refuse_16bit_state():
    from helix_substrate import _hxq
    with pytest.raises(RuntimeError, match="float32"):
        _hxq._need_f32(bias=torch.zeros(4, dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="int32"):
        _hxq._need_i32(sc_col=torch.zeros(4, dtype=torch.int64))
    _hxq._need_f32(bias=None, group_scale=torch.zeros(2))


@pytest.mark.parametrize("shape", [(256,), (3, 256), (2, 3, 256)])
def test_forward_cpu_matches_oracle(shape):
    L = synth.make_layer_np(96, 256, seed=4)
    b = torch.linspace(-1, 1, 96)
    m = _module(L, bias=b)
    x = torch.randn(*shape, generator=torch.Generator().manual_seed(0))
    y = m(x)
    assert y.shape == (*shape[:-1], 96) and y.dtype == x.dtype
    yr = oracle.linear_f64(x.reshape(-1, 256).numpy(), _oracle_w(L), b.numpy())
    rel = np.abs(y.reshape(-1, 96).numpy() - yr).max() / np.abs(yr).max()
    assert rel < 1e-5


def test_cdnav3_roundtrip(tmp_path):
    L = synth.make_layer_np(64, 256, seed=12, density=0.01)
    w = CDNAv3Writer(tmp_path)
    d = w.write_quantized("model.layers.0.mlp.up_proj.weight", L["codebook"], L["indices"],
                          L["sidecar_positions"], L["sidecar_values"], L["group_scale"],
                          L["group_offset"], 128)
    r = CDNAv3Reader(d)
    assert r.shape == (64, 256) and r.has_affine and r.verify_codebook()
    np.testing.assert_array_equal(r.reconstruct(), _oracle_w(L))
    np.testing.assert_array_equal(r.reconstruct_block(10, 40), _oracle_w(L)[10:40])
    m = load_helix_linear_from_cdnav3(d)
    np.testing.assert_array_equal(m.decode_weight().numpy(), _oracle_w(L))
    facs = load_cdna_factors(tmp_path)
    assert list(facs) == ["model.layers.0.mlp.up_proj"]


def test_reader_without_affine_is_reference_layout(tmp_path):
    L = synth.make_layer_np(32, 128, seed=13, affine=False, density=0.02)
    d = CDNAv3Writer(tmp_path).write_quantized("w", L["codebook"], L["indices"],
                                               L["sidecar_positions"], L["sidecar_values"])
    r = CDNAv3Reader(d)
    assert not r.has_affine
    exp = L["codebook"][L["indices"]].copy()
    exp.ravel()[L["sidecar_positions"]] = L["sidecar_values"]
    np.testing.assert_array_equal(r.reconstruct(), exp)


def test_state_dict_roundtrip_through_quantized_shell():
    L = synth.make_layer_np(48, 128, seed=6)
    m = _module(L, bias=torch.ones(48))
    sd = {k: v for k, v in m.state_dict().items() if not k.startswith("_")}
    shell = HelixLinear.from_quantized_config(128, 48, group_size=128)
    shell.load_state_dict(sd, strict=False)
    shell._recompute_derived()
    x = torch.randn(2, 128)
    torch.testing.assert_close(shell(x), m(x), rtol=0, atol=0)


def test_swap_to_helix_and_summary():
    L = synth.make_layer_np(32, 64, seed=8)
    model = nn.Sequential(nn.Linear(64, 32), nn.ReLU())
    model = swap_to_helix(model, {"0": _module(L)})
    assert isinstance(model[0], HelixLinear)
    s = swap_summary(model)
    assert s["helix_modules"] == 1 and s["linear_modules"] == 0
    with pytest.raises(ValueError):
        swap_to_helix(nn.Sequential(nn.Linear(16, 32)), {"0": _module(L)})


def test_sidecar_policy_always_off_drops_corrections():
    L = synth.make_layer_np(32, 128, seed=10, density=0.05)
    m = _module(L)
    x = torch.randn(1, 128)
    m.set_sidecar_policy("always_off")
    y = m(x)
    W0 = oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"], 128)
    yr = oracle.linear_f64(x.numpy(), W0)
    assert np.abs(y.numpy() - yr).max() / np.abs(yr).max() < 1e-5
    assert m.get_sidecar_policy_stats()["skip_count"] == 1


def test_tensor_name_mapping():
    assert _tensor_name_to_module_path("model.layers.3.self_attn.q_proj.weight") == \
        "model.layers.3.self_attn.q_proj"
    assert _tensor_name_to_module_path("blk.2.ffn_down.weight") == "model.layers.2.mlp.down_proj"
    assert _tensor_name_to_module_path("output.weight") == "lm_head"


def test_compressed_bytes_config0():
    # 4,194,304 idx + 1,024 cb + 262,144 s/o + 8,196 row_ptr + 33,552 CSR
    assert compressed_bytes(2048, 2048, 128, 4194) == 4194304 + 1024 + 262144 + 8196 + 33552


def test_rejects_unsupported_shapes():
    L = synth.make_layer_np(8, 128, seed=1)
    T = synth.to_torch(L)
    with pytest.raises(ValueError):               # affine groups must divide in_features
        HelixLinear(120, 8, T["codebook"], T["indices"][:, :120],
                    group_scale=torch.ones(8, 1), group_offset=torch.zeros(8, 1), group_size=128)
    with pytest.raises(NotImplementedError):      # scalar codebooks hold <= 4096 entries
        HelixLinear(128, 8, torch.zeros(4097), T["indices"])


@pytest.mark.parametrize("in_f,kw", [(120, {}), (100, {}), (1, {}), (4000, {"group_size": 32}),
                                     (96, {"group_size": 48})])
def test_any_in_features_kernel_layout(in_f, kw):
    """in_features that are not a multiple of 64: the kernels' padded copy of
    the index rows (zero columns up to the next multiple of 64) and the
    affine's zero groups; the CPU forward is unchanged (oracle)."""
    L = (synth.make_layer_np(40, in_f, seed=in_f, density=0.01, **kw) if kw else
         synth.make_layer_np(40, in_f, seed=in_f, density=0.01, affine=False))
    m = _module(L)
    kp = -(-in_f // 64) * 64
    assert m._kin == kp
    assert m._kidx.shape == (40, kp)
    assert torch.equal(m._kidx[:, :in_f], m.indices) and not m._kidx[:, in_f:].any()
    if kw:
        G = kw["group_size"]
        assert m._affine_t.shape == (-(-kp // G), 40, 2)
        assert not m._affine_t[in_f // G:].any()
    x = torch.randn(3, in_f, generator=torch.Generator().manual_seed(1))
    W = oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"],
                           L["group_size"], L["sidecar_positions"], L["sidecar_values"])
    np.testing.assert_allclose(m(x).numpy(), oracle.linear_f64(x.numpy(), W), rtol=1e-5, atol=1e-6)


def test_forward_wave_threaded_tiles_match_oracle(monkeypatch):
    """HELIX_WAVE_TILES=1: the threaded tile path (reference _forward_wave) gives
    the oracle contraction, like the sequential tiles."""
    monkeypatch.setenv("HELIX_WAVE_TILES", "1")
    L = synth.make_layer_np(700, 512, seed=21, density=0.01)   # 3 tiles, ragged last
    b = torch.linspace(-1, 1, 700)
    m = _module(L, bias=b)
    assert m._wave_enabled
    x = torch.randn(5, 512, generator=torch.Generator().manual_seed(2))
    threads = torch.get_num_threads()
    y = m(x)
    assert m._last_dispatch_path == "wave" and torch.get_num_threads() == threads
    yr = oracle.linear_f64(x.numpy(), _oracle_w(L), b.numpy())
    assert np.abs(y.numpy() - yr).max() / np.abs(yr).max() < 1e-5
    monkeypatch.setenv("HELIX_WAVE_TILES", "0")
    m2 = _module(L, bias=b)
    torch.testing.assert_close(m2(x), y, rtol=1e-6, atol=1e-6)
    assert m2._last_dispatch_path == "naive"


def test_sidecar_row_groups_order():
    """Prefill sidecar order: per 64-row group, by column then row; repeated
    positions keep their stored order (the last copy is applied last)."""
    from helix_substrate.hxq_format import sidecar_row_groups
    rows = torch.tensor([0, 0, 5, 5, 63, 64, 64, 130, 130])
    cols = torch.tensor([9, 3, 3, 3, 1, 7, 2, 0, 0])
    val = torch.arange(9, dtype=torch.float32)
    ptr, key, v = sidecar_row_groups(rows, cols, val, out_f=140, in_f=16)
    assert ptr.tolist() == [0, 5, 7, 9]
    k = key.long()
    assert ((k >> 6).tolist(), (k & 63).tolist()) == ([1, 3, 3, 3, 9, 2, 7, 0, 0],
                                                     [63, 0, 5, 5, 0, 0, 0, 2, 2])
    assert v.tolist() == [4.0, 1.0, 2.0, 3.0, 0.0, 6.0, 5.0, 7.0, 8.0]
    # one pointer per (group, 64-column step): the first entry at that step or later
    ptr, key, v = sidecar_row_groups(torch.tensor([0, 0, 0, 70]), torch.tensor([130, 10, 64, 199]),
                                     torch.arange(4, dtype=torch.float32), out_f=100, in_f=200)
    assert ptr.tolist() == [0, 1, 2, 3, 3, 3, 3, 3, 4]
    assert (key.long() >> 6).tolist() == [10, 64, 130, 199] and v.tolist() == [1.0, 2.0, 0.0, 3.0]
