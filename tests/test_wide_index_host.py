"""Scalar codebooks above 256 entries (uint16 on disk, int16 in memory) and
the per-tensor policy routing of the writer, on the CPU.

Follows the reference's own tests of the k > 256 path
(tests/test_k512_uint16.py:26-40 round trip and meta, :86-107 k = 256 stays
uint8, :109-131 missing index_dtype, :133-151 block reconstruction,
:200-296 HelixLinear forward, memory_savings, loading and the quantized
shell) and its policy table (helix_substrate/tensor_policy.py:188-259,
:291-323).
"""
import json

import numpy as np
import pytest
import torch

import oracle
from helix_substrate.helix_linear import HelixLinear, load_helix_linear_from_cdnav3
from helix_substrate.hxq_reader_v3 import CDNAv3Reader
from helix_substrate.hxq_writer_v3 import CDNAv3Writer, compress_model
from helix_substrate.tensor_policy import (TensorClass, TensorPolicy, classify_tensor,
                                           get_default_policy, get_policy)


def test_reconstruct_np_wide_indices_known_answer():
    cb = np.arange(512, dtype=np.float32) * 0.5
    idx = np.array([[300, 511], [0, 257]], np.uint16)
    np.testing.assert_array_equal(oracle.reconstruct_np(idx, cb), [[150.0, 255.5], [0.0, 128.5]])
    # below 256 the wide gather equals the C restatement on uint8 indices
    rs = np.random.RandomState(0)
    i8 = rs.randint(0, 256, (16, 64)).astype(np.uint8)
    cb256 = rs.standard_normal(256).astype(np.float32)
    gs = rs.uniform(0.9, 1.1, (16, 2)).astype(np.float32)
    go = rs.normal(0, 1e-3, (16, 2)).astype(np.float32)
    a = oracle.reconstruct_np(i8.astype(np.uint16), cb256, gs, go, 32)
    b = oracle.reconstruct(i8, cb256, gs, go, 32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    with pytest.raises(ValueError):
        oracle.reconstruct(i8.astype(np.uint16), cb256)


def _k512_policy(sidecar=False, percentile=99.9):
    return TensorPolicy(tensor_class=TensorClass.UNKNOWN, storage_mode="codebook",
                        n_clusters=512, sidecar_enabled=sidecar, use_kmeans=True,
                        percentile=percentile)


def test_k512_write_read_roundtrip(tmp_path):
    t = np.random.RandomState(42).randn(128, 256).astype(np.float32)
    stats = CDNAv3Writer(tmp_path).write_tensor(t, "test.weight", policy=_k512_policy())
    d = tmp_path / "test_weight.cdnav3"
    meta = json.loads((d / "meta.json").read_text())
    assert meta["index_dtype"] == "uint16" and meta["n_clusters"] == 512
    assert (d / "indices.bin").stat().st_size == 128 * 256 * 2
    assert stats["cosine_no_sidecar"] > 0.99
    r = CDNAv3Reader(d)
    W = r.reconstruct()
    idx = np.fromfile(d / "indices.bin", np.uint16).reshape(128, 256)
    assert idx.max() >= 256                              # really uses the wide range
    np.testing.assert_array_equal(W, oracle.reconstruct_np(idx, np.load(d / "codebook.npy")))
    np.testing.assert_array_equal(r.reconstruct_block(16, 32), W[16:32])


def test_k256_still_uint8_and_missing_index_dtype(tmp_path):
    t = np.random.RandomState(42).randn(64, 128).astype(np.float32)
    pol = TensorPolicy(TensorClass.UNKNOWN, "codebook", n_clusters=256, sidecar_enabled=False)
    CDNAv3Writer(tmp_path).write_tensor(t, "test.weight", policy=pol)
    d = tmp_path / "test_weight.cdnav3"
    meta = json.loads((d / "meta.json").read_text())
    assert meta["index_dtype"] == "uint8" and (d / "indices.bin").stat().st_size == 64 * 128
    W = CDNAv3Reader(d).reconstruct()
    del meta["index_dtype"]
    (d / "meta.json").write_text(json.dumps(meta))
    np.testing.assert_array_equal(CDNAv3Reader(d).reconstruct(), W)


def test_k512_with_sidecar_and_helix_linear(tmp_path):
    t = np.random.RandomState(7).randn(96, 256).astype(np.float32)
    stats = CDNAv3Writer(tmp_path).write_tensor(
        t, "blk.0.ffn_down.weight", policy=_k512_policy(sidecar=True, percentile=99.5))
    assert stats["num_outliers"] > 0 and stats["cosine_with_sidecar"] >= stats["cosine_no_sidecar"]
    d = tmp_path / "blk_0_ffn_down_weight.cdnav3"
    hl = load_helix_linear_from_cdnav3(d)
    assert hl.codebook.shape[0] == 512 and hl.indices.dtype == torch.int16
    W = CDNAv3Reader(d).reconstruct()
    np.testing.assert_array_equal(hl.decode_weight().numpy().view(np.uint32), W.view(np.uint32))
    x = torch.randn(3, 256, generator=torch.Generator().manual_seed(0))
    y = hl(x)
    yr = oracle.linear_f64(x.numpy(), W)
    assert np.abs(y.numpy() - yr).max() / np.abs(yr).max() < 1e-5


def test_k512_module_constructor_memory_and_shell():
    out_f, in_f = 64, 128
    cb = torch.randn(512)
    idx = torch.randint(0, 512, (out_f, in_f), dtype=torch.int16)
    hl = HelixLinear(in_features=in_f, out_features=out_f, codebook=cb, indices=idx,
                     tensor_name="test_k512")
    assert hl.indices.dtype == torch.int16
    assert hl(torch.randn(2, in_f)).shape == (2, out_f)
    s = hl.memory_savings()
    assert s["dense_bytes"] == out_f * in_f * 4
    assert s["compressed_bytes"] == 512 * 4 + out_f * in_f * 2
    # int64 indices into a 512-entry codebook are stored as int16 (reference :166-176)
    hl2 = HelixLinear(in_f, out_f, cb, idx.long())
    assert hl2.indices.dtype == torch.int16 and torch.equal(hl2.indices, idx)
    k256 = HelixLinear(in_f, out_f, torch.randn(256), torch.randint(0, 256, (out_f, in_f),
                                                                    dtype=torch.uint8))
    assert k256.memory_savings()["compressed_bytes"] == 256 * 4 + out_f * in_f
    shell = HelixLinear.from_quantized_config(in_features=128, out_features=64, n_clusters=512)
    assert shell.codebook.shape[0] == 512 and shell.indices.dtype == torch.int16
    # a state dict from the full module fills the shell
    shell.load_state_dict(hl.state_dict(), strict=False)
    shell._recompute_derived()
    x = torch.randn(4, in_f)
    torch.testing.assert_close(shell(x), hl(x), rtol=0, atol=0)


def test_k512_with_affine_cpu():
    rs = np.random.RandomState(3)
    cb = np.sort(rs.standard_normal(700).astype(np.float32) * 0.02)
    idx = rs.randint(0, 700, (40, 256)).astype(np.uint16)
    gs = rs.uniform(0.95, 1.05, (40, 2)).astype(np.float32)
    go = rs.normal(0, 1e-4, (40, 2)).astype(np.float32)
    pos = np.sort(rs.choice(40 * 256, 30, replace=False)).astype(np.int64)
    val = rs.standard_normal(30).astype(np.float32)
    hl = HelixLinear(256, 40, torch.from_numpy(cb), torch.from_numpy(idx.astype(np.int16)),
                     torch.from_numpy(pos), torch.from_numpy(val), group_scale=torch.from_numpy(gs),
                     group_offset=torch.from_numpy(go), group_size=128)
    W = oracle.reconstruct_np(idx, cb, gs, go, 128, pos, val)
    np.testing.assert_array_equal(hl.decode_weight().numpy().view(np.uint32), W.view(np.uint32))
    assert hl.kernel_bytes() == 40 * 256 * 2 + 700 * 4 + 40 * 2 * 8 + 41 * 4 + 30 * 8


# ---------------------------------------------------------------------------
# policy routing
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("name,shape,cls", [
    ("blk.3.attn_q.weight", (8, 8), TensorClass.ATTENTION_QK),
    ("blk.3.attn_v.weight", (8, 8), TensorClass.ATTENTION_VO),
    ("blk.0.ffn_down.weight", (8, 8), TensorClass.FFN),
    ("token_embd.weight", (8, 8), TensorClass.EMBEDDING),
    ("output.weight", (8, 8), TensorClass.LM_HEAD),
    ("model.layers.2.self_attn.k_proj.weight", (8, 8), TensorClass.ATTENTION_QK),
    ("model.layers.2.self_attn.o_proj.weight", (8, 8), TensorClass.ATTENTION_VO),
    ("model.layers.2.mlp.up_proj.weight", (8, 8), TensorClass.FFN),
    ("model.layers.2.input_layernorm.weight", (8, 8), TensorClass.NORM),
    ("model.layers.2.self_attn.q_proj.bias", (8,), TensorClass.NORM),     # 1-D
    ("model.embed_tokens.weight", (8, 8), TensorClass.EMBEDDING),
    ("lm_head.weight", (8, 8), TensorClass.LM_HEAD),
    ("backbone.layers.1.mixer.in_proj.weight", (8, 8), TensorClass.FFN),
    ("backbone.layers.1.mixer.dt_proj.weight", (8, 8), TensorClass.UNKNOWN),
    ("backbone.embedding.weight", (8, 8), TensorClass.EMBEDDING),
    ("something.else", (8, 8), TensorClass.UNKNOWN),
])
def test_classify_tensor(name, shape, cls):
    assert classify_tensor(name, shape) == cls


def test_default_policies():
    qk = get_policy("model.layers.0.self_attn.q_proj.weight", (4, 4))
    assert (qk.percentile, qk.max_corrections, qk.block_rows) == (99.95, 512, 16)
    vo = get_default_policy(TensorClass.ATTENTION_VO)
    assert (vo.percentile, vo.max_corrections, vo.storage_mode) == (99.9, 512, "codebook+sidecar")
    unk = get_policy("x.weight", (4, 4))
    assert (unk.percentile, unk.max_corrections, unk.block_rows) == (99.9, 256, 32)
    for c in (TensorClass.NORM, TensorClass.EMBEDDING):
        p = get_default_policy(c)
        assert p.storage_mode == "exact" and p.n_clusters == 0 and not p.sidecar_enabled
    assert all(get_default_policy(c).n_clusters == 256 for c in TensorClass
               if c not in (TensorClass.NORM, TensorClass.EMBEDDING))


def test_write_tensor_routes_by_policy(tmp_path):
    rs = np.random.RandomState(1)
    t = rs.randn(64, 256).astype(np.float32)
    w = CDNAv3Writer(tmp_path)
    w.write_tensor(t, "model.layers.0.self_attn.q_proj.weight")
    meta = json.loads((tmp_path / "model_layers_0_self_attn_q_proj_weight.cdnav3" /
                       "meta.json").read_text())
    assert meta["percentile"] == 99.95 and meta["tensor_class"] == "attention_qk"
    # 1-D and exact classes are written exact (fp16 .npy)
    st = w.write_tensor(rs.randn(64).astype(np.float32), "model.norm.weight")
    assert st["storage_mode"] == "exact" and (tmp_path / "model_norm_weight.npy").exists()
    st = w.write_tensor(t, "model.embed_tokens.weight")
    assert st["storage_mode"] == "exact"
    # overrides replace policy fields
    w.write_tensor(t, "z.weight", max_corrections=7)
    z = json.loads((tmp_path / "z_weight.cdnav3" / "meta.json").read_text())
    assert z["num_outliers"] == 7 and z["tensor_class"] == "unknown"
    with pytest.raises(NotImplementedError):
        w.write_tensor(t, "m.weight", policy=TensorPolicy(TensorClass.NORM, "morpho"))


def test_compress_model_uses_class_policies(tmp_path):
    tr = pytest.importorskip("transformers")
    torch.manual_seed(0)
    cfg = tr.Qwen2Config(hidden_size=128, intermediate_size=256, num_hidden_layers=1,
                         num_attention_heads=4, num_key_value_heads=2, vocab_size=64)
    model = tr.Qwen2ForCausalLM(cfg).eval()
    compress_model(model, tmp_path)
    pct = {}
    for d in tmp_path.glob("*.cdnav3"):
        m = json.loads((d / "meta.json").read_text())
        pct[m["tensor_name"].split(".")[-2]] = (m["percentile"], m["tensor_class"])
    assert pct["q_proj"] == (99.95, "attention_qk") and pct["k_proj"] == (99.95, "attention_qk")
    assert pct["v_proj"] == (99.9, "attention_vo") and pct["o_proj"] == (99.9, "attention_vo")
    assert pct["gate_proj"] == (99.9, "ffn") and pct["down_proj"] == (99.9, "ffn")


def test_pair_indices_uint8_up_to_256_entries(tmp_path):
    """Pair codebooks of <= 256 entries are written with uint8 indices
    (reference hxq_writer_v3.py:187: uint16 only above 256 entries)."""
    rs = np.random.RandomState(4)
    cb = rs.standard_normal((200, 2)).astype(np.float32)
    idx = rs.randint(0, 200, (32, 64)).astype(np.uint16)
    d = CDNAv3Writer(tmp_path).write_quantized("p.weight", cb, idx)
    meta = json.loads((d / "meta.json").read_text())
    assert meta["index_dtype"] == "uint8" and meta["vector_dim"] == 2
    assert (d / "indices.bin").stat().st_size == 32 * 64
    hl = load_helix_linear_from_cdnav3(d)
    assert hl.vector_dim == 2
    W = oracle.reconstruct_vq2_np(idx, cb)
    np.testing.assert_array_equal(hl.decode_weight().numpy(), W)
