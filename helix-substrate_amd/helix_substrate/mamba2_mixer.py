"""Mamba2 mixer with HXQ-compressed projections around the chunked scan.

Mirrors the reference's patched mixer forward ``_chunked_scan_forward``
(``mamba_scan_chunked.py:239-387``) -- the same split of ``in_proj``'s
output, causal conv1d + SiLU, ``dt = clamp(softplus(dt + dt_bias),
time_step_min)``, chunked scan with ``D``, gated RMSNorm and ``out_proj`` --
for the prefill form and the single-token (cached) form.

On a GPU every stage is a HIP launch: ``in_proj`` (HXQ GEMM, or GEMV for a
token), ``hxq_mamba2_conv_split`` / ``hxq_mamba2_conv_step``, the scan
(``hxq_ssm_chunk_scan`` / ``hxq_ssm_decode_step``), ``hxq_gated_rmsnorm``
and ``out_proj``.  On the CPU the same math runs as torch ops (the
reference's CPU path: ``HelixLinear`` tiles, ``sequential_scan``).
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

from . import _hxq
from .helix_linear import HelixLinear
from .mamba_scan_chunked import DEFAULT_CHUNK_SIZE, sequential_scan


class HelixMamba2Mixer(nn.Module):
    """Attributes follow the HF mixer the reference patches (in_proj, conv1d,
    dt_bias, A_log, D, norm, out_proj, time_step_min, n_groups,
    ssm_state_size, num_heads, head_dim, intermediate_size, conv_kernel_size)."""

    def __init__(self, in_proj: HelixLinear, out_proj: HelixLinear, conv_weight, conv_bias,
                 dt_bias, A_log, D, norm_weight, *, num_heads, head_dim, ssm_state_size,
                 n_groups=1, eps=1e-5, time_step_min=0.0, time_step_max=float("inf"),
                 d_mlp=0, chunk_size=DEFAULT_CHUNK_SIZE):
        super().__init__()
        self.in_proj, self.out_proj = in_proj, out_proj
        self.num_heads, self.head_dim = int(num_heads), int(head_dim)
        self.ssm_state_size, self.n_groups = int(ssm_state_size), int(n_groups)
        self.intermediate_size = self.num_heads * self.head_dim
        self.conv_dim = self.intermediate_size + 2 * self.n_groups * self.ssm_state_size
        self.d_mlp = int(d_mlp)
        self.conv_kernel_size = int(conv_weight.shape[-1])
        self.time_step_min, self.time_step_max = float(time_step_min), float(time_step_max)
        self.variance_epsilon = float(eps)
        self.chunk_size = int(chunk_size)
        proj_width = (2 * self.d_mlp + 2 * self.intermediate_size
                      + 2 * self.n_groups * self.ssm_state_size + self.num_heads)
        if in_proj.out_features != proj_width:
            raise ValueError(f"in_proj has {in_proj.out_features} outputs, expected {proj_width}")
        self.register_buffer("conv_weight", conv_weight.reshape(self.conv_dim, -1).float().contiguous())
        self.register_buffer("conv_bias", None if conv_bias is None else conv_bias.float().contiguous())
        self.register_buffer("dt_bias", dt_bias.float().contiguous())
        self.register_buffer("A_log", A_log.float().contiguous())
        self.register_buffer("D", D.float().reshape(-1).contiguous())
        self.register_buffer("norm_weight", norm_weight.float().contiguous())

    # -- splits of in_proj's output (reference :256-261) ----------------------
    def _split(self, proj):
        d, I, cd, H = self.d_mlp, self.intermediate_size, self.conv_dim, self.num_heads
        gate = proj[..., 2 * d:2 * d + I]
        xbc = proj[..., 2 * d + I:2 * d + I + cd]
        dt = proj[..., 2 * d + I + cd:2 * d + I + cd + H]
        return gate, xbc, dt

    def _dt(self, dt):
        dt = F.softplus(dt.float() + self.dt_bias)
        return torch.clamp(dt, self.time_step_min, self.time_step_max)

    def new_state(self, batch, device):
        """(conv_state fp32 [b, conv_dim, width], ssm_state fp32 [b, H, P, N]), zeros."""
        return (torch.zeros(batch, self.conv_dim, self.conv_kernel_size, device=device),
                torch.zeros(batch, self.num_heads, self.head_dim, self.ssm_state_size,
                            device=device))

    # -- prefill ---------------------------------------------------------------
    def forward(self, hidden_states, state=None):
        """hidden_states [b, L, d_model] -> [b, L, d_model].  `state`, if given,
        is (conv_state, ssm_state) and receives the states after the sequence
        (the sequence starts from zero state, as the reference's prefill)."""
        if hidden_states.is_cuda:
            return self._forward_hip(hidden_states, state)
        return self._forward_cpu(hidden_states, state)

    def _forward_hip(self, hs, state):
        b, L, _ = hs.shape
        dtype = hs.dtype
        proj = self.in_proj(hs)                                      # [b, L, proj_width]
        x, B, C, dt = _hxq.mamba2_conv_split(
            proj.contiguous(), self.conv_weight, self.conv_bias, self.dt_bias, self.time_step_min,
            self.time_step_max, self.d_mlp, self.intermediate_size, self.n_groups,
            self.ssm_state_size, self.num_heads,
            conv_state=None if state is None else state[0])
        A = -torch.exp(self.A_log)
        y, h = _hxq.ssm_chunk_scan(x, dt, A, B, C, self.D, None, chunk=self.chunk_size,
                                   out_dtype=torch.float32, want_final=state is not None)
        if state is not None:
            state[1].copy_(h)
        gate, _, _ = self._split(proj.view(b * L, -1))
        z = _hxq.gated_rmsnorm(y.view(b * L, -1), gate, self.norm_weight, self.variance_epsilon,
                               out_dtype=dtype)
        return self.out_proj(z).view(b, L, -1)

    def _forward_cpu(self, hs, state):
        b, L, _ = hs.shape
        dtype = hs.dtype
        proj = self.in_proj(hs)
        gate, xbc, dt = self._split(proj)
        W = self.conv_kernel_size
        xt = F.pad(xbc.float().transpose(1, 2), (W - 1, 0))
        conv = F.conv1d(xt, self.conv_weight.unsqueeze(1), self.conv_bias, groups=self.conv_dim)
        xbc_a = F.silu(conv).transpose(1, 2)                         # [b, L, conv_dim]
        if state is not None:
            state[0].copy_(xt[:, :, -W:])
        I, GN = self.intermediate_size, self.n_groups * self.ssm_state_size
        x = xbc_a[..., :I].reshape(b, L, self.num_heads, self.head_dim)
        B = xbc_a[..., I:I + GN].reshape(b, L, self.n_groups, self.ssm_state_size)
        C = xbc_a[..., I + GN:].reshape(b, L, self.n_groups, self.ssm_state_size)
        rep = self.num_heads // self.n_groups
        B, C = B.repeat_interleave(rep, dim=2), C.repeat_interleave(rep, dim=2)
        A = -torch.exp(self.A_log)
        h0 = torch.zeros(b, self.num_heads, self.head_dim, self.ssm_state_size)
        y, h = sequential_scan(h0, self._dt(dt), A, x, B, C, self.D[:, None])
        if state is not None:
            state[1].copy_(h)
        z = self._gated_norm(y.reshape(b, L, -1), gate.float())
        return self.out_proj(z.to(dtype))

    def _gated_norm(self, y, gate):
        h = y.float() * F.silu(gate.float())
        var = h.pow(2).mean(-1, keepdim=True)
        return self.norm_weight * (h * torch.rsqrt(var + self.variance_epsilon))

    # -- single token ------------------------------------------------------------
    def step(self, hidden_state, state):
        """hidden_state [b, d_model] (one token); state = (conv_state, ssm_state),
        updated in place.  Returns [b, d_model]."""
        conv_state, ssm_state = state
        b = hidden_state.shape[0]
        dtype = hidden_state.dtype
        proj = self.in_proj(hidden_state)                            # [b, proj_width]
        if hidden_state.is_cuda:
            x, B, C, dt = _hxq.mamba2_conv_step(
                proj.contiguous(), conv_state, self.conv_weight, self.conv_bias, self.dt_bias,
                self.time_step_min, self.time_step_max, self.d_mlp, self.intermediate_size,
                self.n_groups, self.ssm_state_size, self.num_heads)
            A = -torch.exp(self.A_log)
            y = _hxq.ssm_decode_step(ssm_state, x, dt, A, B, C, self.D)
            gate, _, _ = self._split(proj)
            z = _hxq.gated_rmsnorm(y.view(b, -1), gate, self.norm_weight, self.variance_epsilon,
                                   out_dtype=dtype)
            return self.out_proj(z)
        gate, xbc, dt = self._split(proj)
        conv_state.copy_(torch.roll(conv_state, shifts=-1, dims=-1))
        conv_state[:, :, -1] = xbc.float()
        v = (conv_state * self.conv_weight).sum(-1)
        if self.conv_bias is not None:
            v = v + self.conv_bias
        v = F.silu(v)
        I, GN = self.intermediate_size, self.n_groups * self.ssm_state_size
        x = v[:, :I].reshape(b, self.num_heads, self.head_dim)
        rep = self.num_heads // self.n_groups
        B = v[:, I:I + GN].reshape(b, self.n_groups, -1).repeat_interleave(rep, dim=1)
        C = v[:, I + GN:].reshape(b, self.n_groups, -1).repeat_interleave(rep, dim=1)
        dtv = self._dt(dt)                                           # [b, H]
        A = -torch.exp(self.A_log)
        dA = torch.exp(dtv * A)[:, :, None, None]
        ssm_state.copy_(ssm_state * dA + (dtv[:, :, None] * x)[..., None] * B[:, :, None, :])
        y = (ssm_state * C[:, :, None, :]).sum(-1) + self.D[None, :, None] * x
        z = self._gated_norm(y.reshape(b, -1), gate.float())
        return self.out_proj(z.to(dtype))


def mamba2_13b_dims():
    """Benchmark config 3 (Mamba2-1.3B): d_model 2048, d_inner 4096, 64 heads of
    64, d_state 128, 1 group, conv width 4; in_proj 8512 x 2048, out_proj
    2048 x 4096."""
    return {"d_model": 2048, "num_heads": 64, "head_dim": 64, "ssm_state_size": 128,
            "n_groups": 1, "conv_width": 4}


def random_mixer_params(d_model, num_heads, head_dim, ssm_state_size, n_groups, conv_width,
                        seed=0, device="cpu"):
    """Random-init non-projection parameters of a Mamba2 mixer (the HF init
    ranges: dt from [1e-3, 0.1] log-uniform through inverse softplus, A in
    [1, 16])."""
    g = torch.Generator(device="cpu").manual_seed(seed)
    I = num_heads * head_dim
    conv_dim = I + 2 * n_groups * ssm_state_size
    bound = 1.0 / math.sqrt(conv_width)
    dt = torch.exp(torch.rand(num_heads, generator=g) * (math.log(0.1) - math.log(1e-3))
                   + math.log(1e-3))
    p = {"conv_weight": (torch.rand(conv_dim, conv_width, generator=g) * 2 - 1) * bound,
         "conv_bias": (torch.rand(conv_dim, generator=g) * 2 - 1) * bound,
         "dt_bias": dt + torch.log(-torch.expm1(-dt)),
         "A_log": torch.log(torch.rand(num_heads, generator=g) * 15 + 1),
         "D": torch.ones(num_heads),
         "norm_weight": 1.0 + 0.1 * torch.randn(I, generator=g)}
    return {k: v.to(device) for k, v in p.items()}
