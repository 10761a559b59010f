"""hxq_gemm_noalloc (no allocation, split-K partials in the library's static
per-device scratch) against hxq_gemm_ws with a caller workspace, through the
C ABI: identical kernels and K split, so identical outputs; two calls in a
row, the second on a smaller problem."""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate import _hxq, synth
from helix_substrate.helix_linear import HelixLinear

pytestmark = pytest.mark.gpu


def _module(out_f, in_f, seed, dev, density=0.001):
    L = synth.make_layer_np(out_f, in_f, seed=seed, sigma=0.015, density=density)
    T = synth.to_torch(L)
    m = HelixLinear(in_f, out_f, T["codebook"], T["indices"], T["sidecar_positions"],
                    T["sidecar_values"], bias=torch.linspace(-1, 1, out_f),
                    group_scale=T["group_scale"], group_offset=T["group_offset"],
                    group_size=128).to(dev)
    W = oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"], 128,
                           L["sidecar_positions"], L["sidecar_values"])
    return m, W


def _args(m, x):
    return (x, m.indices, m._kcb, m._affine_t, m.group_size, m._sc_row_ptr, m._sc_col,
            m._sc_val, m.bias)


def test_noalloc_matches_workspace_entry_point(dev):
    assert _hxq.lib().hxq_gemm_noalloc_max_bytes() == 64 << 20
    # first call: kv-like shape, K split 8 ways (partials in the scratch);
    # second call: a smaller split problem that reuses the same scratch
    for (mr, out_f, in_f, seed) in ((1024, 512, 3584, 1), (40, 128, 512, 2)):
        print(f"gemm_noalloc m={mr} out={out_f} in={in_f}", flush=True)
        need = _hxq.lib().hxq_gemm_workspace_bytes(mr, out_f, in_f)
        assert 0 < need <= 64 << 20
        m, W = _module(out_f, in_f, seed, dev)
        x = torch.randn(mr, in_f, generator=torch.Generator().manual_seed(seed)).to(torch.bfloat16)
        xd = x.to(dev)
        for out_dtype in (torch.float32, torch.bfloat16):
            ref = _hxq.gemm(*_args(m, xd), out_dtype=out_dtype)               # hxq_gemm_ws
            got = _hxq.gemm_noalloc(*_args(m, xd), out_dtype=out_dtype)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), (mr, out_dtype)
        # and the BASELINE bar against the fp64 oracle
        y = got.float().cpu().numpy()
        yr = oracle.linear_np(x.float().numpy(), W, m.bias.cpu().numpy())
        assert np.abs(y - yr).max() / np.abs(yr).max() <= 2e-2


def test_noalloc_unsplit_shape_and_scratch_bound(dev):
    # many output tiles: no K split, no scratch touched
    m, W = _module(4096, 256, 3, dev)
    x = torch.randn(2048, 256, device=dev).to(torch.bfloat16)
    assert _hxq.lib().hxq_gemm_workspace_bytes(2048, 4096, 256) == 0
    assert torch.equal(_hxq.gemm_noalloc(*_args(m, x)), _hxq.gemm(*_args(m, x)))
    # the split plan keeps ksplit x output tiles <= 256, so no shape's partials
    # exceed 32 MiB: the static 64 MiB array covers every plan (the size check
    # in the entry point guards against future plans)
    worst = max(_hxq.lib().hxq_gemm_workspace_bytes(mr, o, k)
                for mr in (1, 100, 128, 1000, 4000, 8064, 16256, 20000)
                for o in (64, 256, 300, 512, 1024, 4096) for k in (256, 1024, 3584, 18944))
    assert 0 < worst <= 32 << 20 <= _hxq.lib().hxq_gemm_noalloc_max_bytes()
