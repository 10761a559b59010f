"""Mixture-of-experts FFN over HXQ-compressed experts (OLMoE-shaped SwiGLU).

The reference has no MoE kernel: its quantizer swaps ``nn.Linear`` experts for
``HelixLinear`` one by one (``hf_quantizer.py:231-249``), so a MoE block runs
one ``HelixLinear.forward`` (``helix_linear.py:318-361``) per expert
projection on that expert's tokens, inside the HF block (transformers 5.15.0
``models/olmoe/modeling_olmoe.py``: router ``OlmoeTopKRouter.forward``
:337-346, experts ``OlmoeExperts.forward`` :301-325).  ``HelixMoeExperts``
keeps exactly that math -- per expert ``down(silu(gate(x)) * up(x))``,
combined with the router's softmax top-k weights (OLMoE:
``norm_topk_prob=False``) -- but runs all
experts of a layer as grouped HIP launches over one expert-sorted token list:

  route   softmax + top-k + expert-sorted assignment lists  (hxq_moe_route)
  ffn     gate/up grouped GEMM with silu*mul epilogue, down grouped GEMM,
          ordered weighted combine                          (hxq_moe_ffn)

Expert weights are stacked into banks (``stack_bank``): indices [E, out, in],
codebooks [E, 256], affine [E, out, in/G] (and its GEMM layout [E, in/G, out,
2]), and one CSR sidecar whose row pointers [E, out+1] are absolute offsets
into the concatenated entries.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F
from torch import nn

from . import _hxq
from .hxq_format import sidecar_row_groups


def _csr_of(positions, values, out_f, in_f, device):
    """Row-major CSR of one matrix's sidecar (replacement values), order kept."""
    if positions is None or len(positions) == 0:
        return (torch.zeros(out_f + 1, dtype=torch.int32, device=device),
                torch.zeros(0, dtype=torch.int32, device=device),
                torch.zeros(0, dtype=torch.float32, device=device))
    pos = torch.as_tensor(positions, device=device).to(torch.int64)
    val = torch.as_tensor(values, device=device).to(torch.float32)
    order = torch.sort(pos, stable=True).indices
    pos, val = pos[order], val[order]
    rows = pos // in_f
    cols = (pos % in_f).to(torch.int32)
    counts = torch.bincount(rows, minlength=out_f)
    rp = torch.zeros(out_f + 1, dtype=torch.int64, device=device)
    rp[1:] = torch.cumsum(counts, 0)
    return rp.to(torch.int32), cols, val


def stack_bank(layers, device=None):
    """Stack per-expert HXQ layers (dicts as made by ``synth.make_layer_*`` or read
    from CDNAv3 directories) into one expert bank for the grouped kernels."""
    E = len(layers)
    dev = torch.device(device) if device is not None else torch.as_tensor(
        layers[0]["indices"]).device
    idx = torch.stack([torch.as_tensor(L["indices"]).to(dev) for L in layers]).contiguous()
    _, out_f, in_f = idx.shape
    cb = torch.stack([torch.as_tensor(L["codebook"]).to(dev).float() for L in layers]).contiguous()
    if cb.shape[1] != 256:
        raise ValueError("expert banks take 256-entry codebooks (uint8 indices)")
    affine = layers[0].get("group_scale") is not None
    gs = go = None
    if affine:
        gs = torch.stack([torch.as_tensor(L["group_scale"]).to(dev).float()
                          for L in layers]).contiguous()
        go = torch.stack([torch.as_tensor(L["group_offset"]).to(dev).float()
                          for L in layers]).contiguous()
    rps, cols, vals = [], [], []
    gptrs, gkeys, gvals = [], [], []
    base = 0
    for L in layers:
        rp, c, v = _csr_of(L.get("sidecar_positions"), L.get("sidecar_values"), out_f, in_f, dev)
        rps.append(rp + base)
        cols.append(c)
        vals.append(v)
        if in_f % 64 == 0:
            # the register-dequant kernel's order (per 64 rows, by column; the
            # step pointers absolute into the concatenated lists)
            rows = torch.repeat_interleave(torch.arange(out_f, device=dev),
                                           (rp[1:] - rp[:-1]).to(torch.int64))
            gp, gk, gv = sidecar_row_groups(rows, c, v, out_f, in_f)
            gptrs.append(gp + base)
            gkeys.append(gk)
            gvals.append(gv)
        base += int(c.numel())
    if base >= 2 ** 31:
        raise ValueError("too many sidecar entries for 32-bit offsets")
    # the grouped GEMM reads the affine factors as [E, K/G, out, 2]
    ga = None if gs is None else torch.stack([gs.transpose(1, 2), go.transpose(1, 2)], dim=-1).contiguous()
    return {"indices": idx, "codebook": cb, "group_scale": gs, "group_offset": go,
            "group_affine": ga,
            "group_size": int(layers[0].get("group_size") or 0) if affine else 0,
            "sc_row_ptr": torch.stack(rps).contiguous(),
            "sc_col": torch.cat(cols).contiguous(), "sc_val": torch.cat(vals).contiguous(),
            "sc_grp_ptr": torch.stack(gptrs).contiguous() if gptrs else None,
            "sc_grp_key": torch.cat(gkeys).contiguous() if gptrs else None,
            "sc_grp_val": torch.cat(gvals).contiguous() if gptrs else None}


def bank_to(bank, device):
    return {k: (v.to(device) if isinstance(v, torch.Tensor) else v) for k, v in bank.items()}


def decode_expert(bank, e):
    """Dense fp32 weight of expert e (torch, any device): cb[idx] -> affine
    fl(fl(cb*s)+o) -> sidecar replacement."""
    idx = bank["indices"][e].long()
    W = bank["codebook"][e][idx]
    if bank.get("group_scale") is not None:
        G = bank["group_size"]
        s = bank["group_scale"][e].repeat_interleave(G, dim=1)
        o = bank["group_offset"][e].repeat_interleave(G, dim=1)
        W = (W * s) + o
    rp = bank["sc_row_ptr"][e].long()
    lo, hi = int(rp[0]), int(rp[-1])
    if hi > lo:
        rows = torch.repeat_interleave(torch.arange(W.shape[0], device=W.device), rp[1:] - rp[:-1])
        cols = bank["sc_col"][lo:hi].long()
        W = W.clone()
        W[rows, cols] = bank["sc_val"][lo:hi]  # later duplicates win (CSR order)
    return W


def route_cpu(logits, top_k, renormalize=False):
    """Router on the host: softmax over experts, top-k by logit (ties -> lower
    id), optional renormalisation; returns (ids int64 [T, k], weights f32)."""
    p = torch.softmax(logits.float(), dim=-1)
    order = torch.sort(-logits.float(), dim=-1, stable=True).indices[:, :top_k]
    w = torch.gather(p, 1, order)
    if renormalize:
        w = w / w.sum(dim=-1, keepdim=True)
    return order, w


class HelixMoeExperts(nn.Module):
    """All experts of one SwiGLU MoE layer, HXQ-compressed.

    ``forward(x, router_logits)`` -> y with y[t] = sum_s w[t,s] *
    down_e(silu(gate_e(x_t)) * up_e(x_t)); on a GPU the three grouped HIP
    launches above, on the CPU a per-expert torch loop with the same math.
    """

    def __init__(self, gate_bank, up_bank, down_bank, top_k=8, norm_topk_prob=False):
        super().__init__()
        self.top_k = int(top_k)
        self.norm_topk_prob = bool(norm_topk_prob)
        self.banks = {"gate": gate_bank, "up": up_bank, "down": down_bank}
        self.num_experts, self.intermediate, self.hidden = gate_bank["indices"].shape
        self._last_dispatch_path = None

    @classmethod
    def from_layers(cls, gate_layers, up_layers, down_layers, device=None, **kw):
        return cls(stack_bank(gate_layers, device), stack_bank(up_layers, device),
                   stack_bank(down_layers, device), **kw)

    @classmethod
    def from_helix_linears(cls, gates, ups, downs, **kw):
        """Build from per-expert ``HelixLinear`` modules (e.g. after ``swap_to_helix``)."""
        def layers(mods):
            out = []
            for m in mods:
                out.append({"indices": m.indices, "codebook": m._kcb,
                            "group_scale": getattr(m, "group_scale", None),
                            "group_offset": getattr(m, "group_offset", None),
                            "group_size": getattr(m, "group_size", 0),
                            "sidecar_positions": m.sidecar_positions
                            if m.sidecar_positions.numel() else None,
                            "sidecar_values": m.sidecar_values
                            if m.sidecar_values.numel() else None})
            return out
        return cls.from_layers(layers(gates), layers(ups), layers(downs), **kw)

    def to(self, *args, **kwargs):
        dev = torch.device(args[0]) if args and not isinstance(args[0], torch.dtype) \
            else kwargs.get("device")
        if dev is not None:
            self.banks = {k: bank_to(b, dev) for k, b in self.banks.items()}
        return self

    def route(self, router_logits):
        if router_logits.is_cuda:
            return _hxq.moe_route(router_logits, self.top_k, self.norm_topk_prob)
        return route_cpu(router_logits, self.top_k, self.norm_topk_prob)

    def forward(self, x, router_logits):
        shape = x.shape
        x2 = x.reshape(-1, shape[-1])
        if x2.is_cuda:
            if x2.dtype not in (torch.bfloat16, torch.float16, torch.float32):
                x2 = x2.float()
            r = _hxq.moe_route(router_logits.reshape(x2.shape[0], -1), self.top_k,
                               self.norm_topk_prob)
            y = _hxq.moe_ffn(x2.contiguous(), r, self.banks["gate"], self.banks["up"],
                             self.banks["down"], out_dtype=x.dtype)
            self._last_dispatch_path = "hip_moe"
            return y.reshape(shape)
        ids, w = route_cpu(router_logits.reshape(x2.shape[0], -1), self.top_k,
                           self.norm_topk_prob)
        xf = x2.float()
        y = torch.zeros(x2.shape[0], self.hidden, dtype=torch.float32)
        for e in range(self.num_experts):
            tok, slot = torch.nonzero(ids == e, as_tuple=True)
            if tok.numel() == 0:
                continue
            xe = xf[tok]
            h = F.silu(xe @ decode_expert(self.banks["gate"], e).T) * (
                xe @ decode_expert(self.banks["up"], e).T)
            o = h @ decode_expert(self.banks["down"], e).T
            y.index_add_(0, tok, o * w[tok, slot].unsqueeze(1))
        self._last_dispatch_path = "cpu_moe"
        return y.to(x.dtype).reshape(shape)


def olmoe_router_logits(n_tokens, n_experts, seed=0, device="cpu"):
    """Benchmark config 4 router logits: N(0, 1) [n_tokens, n_experts]."""
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(n_tokens, n_experts, generator=g, device=device)


def expert_load(ids, n_experts):
    """Tokens per expert of a routing (numpy, for reports)."""
    return np.bincount(np.asarray(ids).reshape(-1), minlength=n_experts)
