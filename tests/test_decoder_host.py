"""Oracle pinning for the decode-loop glue (CPU only): RMSNorm, RoPE and GQA
attention against closed forms, so the GPU decoder test compares against a
pinned restatement of transformers' Qwen2 math."""
import numpy as np

import oracle


def test_rmsnorm_closed_form():
    x = np.array([[3.0, -4.0]])
    out = oracle.rmsnorm_np(x, [1.0, 2.0], 0.0)
    np.testing.assert_allclose(out, [[3 / np.sqrt(12.5), -8 / np.sqrt(12.5)]], rtol=1e-15)


def test_rope_identity_norm_and_relative_position():
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 5, 8))
    k = rng.standard_normal((1, 5, 8))
    pos = np.arange(5)
    qr, kr = oracle.rope_np(q, pos, 1e4), oracle.rope_np(k, pos, 1e4)
    np.testing.assert_allclose(qr[0, 0], q[0, 0], rtol=0, atol=0)          # position 0
    np.testing.assert_allclose(np.linalg.norm(qr, axis=-1), np.linalg.norm(q, axis=-1), rtol=1e-13)
    # q(m).k(n) depends on m - n only: shift both positions by 3
    a = oracle.rope_np(q[:, :1], [1], 1e4)[0, 0] @ oracle.rope_np(k[:, :1], [4], 1e4)[0, 0]
    b = oracle.rope_np(q[:, :1], [4], 1e4)[0, 0] @ oracle.rope_np(k[:, :1], [7], 1e4)[0, 0]
    assert abs(a - b) < 1e-12
    # 2-D rotation of the first pair by pos * theta^0 = pos radians
    x = np.zeros((1, 1, 2)); x[0, 0, 0] = 1.0
    np.testing.assert_allclose(oracle.rope_np(x, [0.5], 1e4)[0, 0], [np.cos(0.5), np.sin(0.5)], rtol=1e-14)


def test_attention_closed_forms():
    rng = np.random.default_rng(1)
    v = rng.standard_normal((2, 6, 4))
    k = rng.standard_normal((2, 6, 4))
    q = np.zeros((4, 6, 4))                       # zero query -> causal running mean of v
    out = oracle.causal_gqa_attention_np(q, k, v)
    for h in range(4):
        for t in range(6):
            np.testing.assert_allclose(out[h, t], v[h // 2, :t + 1].mean(0), rtol=1e-13)
    # first position attends only to itself
    q = rng.standard_normal((4, 6, 4))
    out = oracle.causal_gqa_attention_np(q, k, v)
    np.testing.assert_allclose(out[:, 0], v[[0, 0, 1, 1], 0], rtol=1e-13)
