"""GPU parity of the GEMV's final pass at its edges, against the fp64 oracle
(fp32 activations, 1e-5 max-relative).

The final pass gives each output row up to 64 lanes and reduces them in a
fixed order; the sidecar products of a block's first 512 entries come from
LDS, later ones from memory.  These cases reach the ends of both ranges:
blocks of 512 rows (one lane per row) whose sidecar lists exceed 512 entries,
and one-row blocks (64 lanes per row) whose row alone has more than 512
entries."""
import numpy as np
import pytest
import torch

import oracle
from helix_substrate import synth
from helix_substrate.helix_linear import HelixLinear

pytestmark = pytest.mark.gpu


def _run(dev, out_f, in_f, group, density, seed):
    L = synth.make_layer_np(out_f, in_f, seed=seed, group_size=group, density=density)
    T = synth.to_torch(L)
    m = HelixLinear(in_f, out_f, T["codebook"], T["indices"], T["sidecar_positions"],
                    T["sidecar_values"], group_scale=T["group_scale"],
                    group_offset=T["group_offset"], group_size=group).to(dev)
    x = torch.randn(1, in_f, generator=torch.Generator().manual_seed(seed))
    print(f"gemv epilogue out={out_f} in={in_f} density={density} "
          f"entries={len(L['sidecar_positions'])}", flush=True)
    y = m(x.to(dev))
    assert m._last_dispatch_path == "hip_gemv"
    W = oracle.reconstruct(L["indices"], L["codebook"], L["group_scale"], L["group_offset"],
                           L["group_size"], L["sidecar_positions"], L["sidecar_values"])
    ref = oracle.linear_f64(x.numpy(), W)
    rel = float(np.abs(y.cpu().numpy().astype(np.float64) - ref).max() / np.abs(ref).max())
    assert rel <= 1e-5, rel


def test_gemv_512_row_blocks_with_long_sidecar_lists(dev):
    # 262144 rows over 512 blocks: 512 rows per block, one lane per row; about
    # 670 sidecar entries per block (past the 512 staged in LDS)
    _run(dev, 262144, 64, 64, 0.02, 5)


def test_gemv_one_row_blocks_with_long_sidecar_rows(dev):
    # 64 rows over 64 blocks: 64 lanes per row; about 655 entries in each row
    _run(dev, 64, 8192, 128, 0.08, 6)
