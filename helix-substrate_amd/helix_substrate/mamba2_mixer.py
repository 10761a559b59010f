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
from .ssm_scan import DEFAULT_CHUNK_SIZE, sequential_scan


class HelixMamba2Mixer(nn.Module):
    """Attributes follow the HF mixer the reference patches (in_proj, conv1d,
    dt_bias, A_log, D, norm, out_proj, time_step_min, n_groups,
    ssm_state_size, num_heads, head_dim, intermediate_size, conv_kernel_size)."""

    def __init__(self, in_proj: HelixLinear, out_proj: HelixLinear, conv_weight, conv_bias,
                 dt_bias, A_log, D, norm_weight, *, num_heads, head_dim, ssm_state_size,
                 n_groups=1, eps=1e-5, time_step_min=0.0, time_step_max=float("inf"),
                 d_mlp=0, chunk_size=DEFAULT_CHUNK_SIZE, norm_group_size=None):
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
        # gated RMSNorm groups: the whole d_inner (Mamba2) or d_inner / n_groups (Zamba2)
        self.norm_group_size = int(norm_group_size or self.intermediate_size)
        if self.intermediate_size % self.norm_group_size:
            raise ValueError("norm_group_size must divide the intermediate size")
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
                               group_size=self.norm_group_size, out_dtype=dtype)
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
        hg = h.unflatten(-1, (-1, self.norm_group_size))
        hg = hg * torch.rsqrt(hg.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.norm_weight * hg.flatten(-2)

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
                                   group_size=self.norm_group_size, out_dtype=dtype)
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


    # -- transformers' mixer contract --------------------------------------------
    @classmethod
    def from_hf(cls, mod):
        """Build from a transformers 5.x ``Mamba2Mixer`` or ``Zamba2MambaMixer``.
        ``in_proj`` / ``out_proj`` are the HF module's own (``HelixLinear`` once
        the HXQ quantizer has replaced them, else ``nn.Linear``); the small
        parameters are copied to fp32.  dt is clamped to the module's
        ``time_step_limit`` (Zamba2: ``(time_step_min, inf)``); the gated norm
        takes the module's group size (Zamba2) or the whole d_inner (Mamba2)."""
        lo, hi = getattr(mod, "time_step_limit", (0.0, float("inf")))
        norm = mod.norm
        det = lambda t: None if t is None else t.detach()
        return cls(mod.in_proj, mod.out_proj, det(mod.conv1d.weight), det(mod.conv1d.bias),
                   det(mod.dt_bias), det(mod.A_log), det(mod.D), det(norm.weight),
                   num_heads=mod.num_heads, head_dim=mod.head_dim,
                   ssm_state_size=mod.ssm_state_size, n_groups=mod.n_groups,
                   eps=norm.variance_epsilon, time_step_min=lo, time_step_max=hi,
                   chunk_size=mod.chunk_size, norm_group_size=getattr(norm, "group_size", None))

    def hf_forward(self, hidden_states, cache_params=None, attention_mask=None, layer_idx=0):
        """transformers' mixer forward (``Mamba2Mixer.forward`` /
        ``Zamba2MambaMixer.forward``, transformers 5.x) on device tensors, every
        stage a HIP launch.  With ``cache_params`` (HF's linear-attention cache)
        it covers the three cases the HF forward has: prefill (stores the last
        ``conv_kernel_size`` raw xBC columns and the fp32 final SSM state),
        a multi-token continuation (the cached columns are prepended to the
        convolution's input and the cached state is the scan's initial state)
        and the single-token step (conv state and SSM state updated in place).
        A 2-D ``attention_mask`` zeroes padded positions before in_proj and
        after the convolution, as HF's ``apply_mask_to_padding_states``."""
        if not hidden_states.is_cuda:
            raise RuntimeError("hf_forward runs the HIP kernels: pass device tensors")
        b, L, _ = hidden_states.shape
        dtype = hidden_states.dtype
        mask = attention_mask
        if mask is not None and bool((mask == 1).all()):
            mask = None
        hs = hidden_states if mask is None else (hidden_states * mask[:, :, None]).to(dtype)
        proj = self.in_proj(hs).contiguous()                          # [b, L, proj_width]
        d, I, cd, H = self.d_mlp, self.intermediate_size, self.conv_dim, self.num_heads
        G, N, W = self.n_groups, self.ssm_state_size, self.conv_kernel_size
        A = -torch.exp(self.A_log)
        conv = (self.conv_weight, self.conv_bias, self.dt_bias, self.time_step_min,
                self.time_step_max, d, I, G, N, H)
        layer = None if cache_params is None else cache_params.layers[layer_idx]
        use_prev = cache_params is not None and cache_params.has_previous_state(layer_idx)
        if use_prev and L == 1 and not layer.record_past:
            conv_state, ssm_state = layer.conv_states[0], layer.recurrent_states[0]
            cs = _f32_view(conv_state)
            x, B, C, dt = _hxq.mamba2_conv_step(proj[:, 0].contiguous(), cs, *conv)
            h = _f32_view(ssm_state)
            y = _hxq.ssm_decode_step(h, x, dt, A, B, C, self.D)         # [b, H, P] fp32
            if cs is not conv_state:
                conv_state.copy_(cs)
            if h is not ssm_state:
                ssm_state.copy_(h)
            y = y.reshape(b, 1, I)
        else:
            src, prefix = proj, 0
            if cache_params is not None:
                xbc_t = proj[..., 2 * d + I:2 * d + I + cd].transpose(1, 2)   # [b, cd, L]
                full = cache_params.update_conv_state(xbc_t, layer_idx, conv_kernel_size=W)
                if use_prev:
                    # continuation: the cached raw columns go in front of the new
                    # ones, their gate / dt slots zero (those rows are dropped)
                    prefix = full.shape[-1] - L
                    src = proj.new_zeros(b, prefix + L, proj.shape[-1])
                    src[:, :prefix, 2 * d + I:2 * d + I + cd] = \
                        full[..., :prefix].transpose(1, 2).to(proj.dtype)
                    src[:, prefix:] = proj
            x, B, C, dt = _hxq.mamba2_conv_split(src, *conv)
            if prefix:
                x, B, C, dt = (t[:, prefix:].contiguous() for t in (x, B, C, dt))
            if mask is not None:
                m = mask[:, :, None, None]
                x, B, C = ((t * m).to(t.dtype) for t in (x, B, C))
            h0 = layer.recurrent_states[0] if use_prev else None
            y, h = _hxq.ssm_chunk_scan(x, dt, A, B, C, self.D, h0, chunk=self.chunk_size,
                                       out_dtype=torch.float32, want_final=cache_params is not None)
            if cache_params is not None:
                cache_params.update_recurrent_state(h, layer_idx=layer_idx)
            y = y.reshape(b, L, I)
        gate = proj.view(b * L, -1)[:, 2 * d:2 * d + I]
        z = _hxq.gated_rmsnorm(y.view(b * L, I), gate, self.norm_weight, self.variance_epsilon,
                               group_size=self.norm_group_size, out_dtype=dtype)
        return self.out_proj(z).view(b, L, -1)


def _f32_view(t):
    """t itself when fp32 and contiguous (updated in place), else an fp32 copy
    (copied back by the caller)."""
    return t if t.dtype == torch.float32 and t.is_contiguous() else t.float().contiguous()


def hf_core(mod):
    """The HelixMamba2Mixer behind a transformers mixer module (built on first
    use and kept on the module outside its parameters and submodules; rebuilt
    when a parameter is replaced, moved or modified in place)."""
    params = (mod.conv1d.weight, mod.conv1d.bias, mod.dt_bias, mod.A_log, mod.D, mod.norm.weight)
    key = tuple(None if p is None else (p.data_ptr(), p._version, str(p.device)) for p in params)
    core = mod.__dict__.get("_helix_core")
    if (core is None or core._hf_key != key or core.in_proj is not mod.in_proj
            or core.out_proj is not mod.out_proj):
        core = HelixMamba2Mixer.from_hf(mod).to(mod.dt_bias.device)
        core._hf_key = key
        mod.__dict__["_helix_core"] = core
    return core


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
