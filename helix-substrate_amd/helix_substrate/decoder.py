"""Batch-1 greedy decoder (Qwen2-shaped) whose projections are HXQ HelixLinear.

The reference measures decode tok/s with HF models whose q/k/v/o/gate/up/down
``nn.Linear`` were swapped for ``HelixLinear`` (``swap_to_helix``,
``helix_linear.py``; benchmark config 1: Qwen2.5-3B).  This module is that
decode loop on MI355X: every projection is an HXQ GEMV launch (q/k/v share one,
gate/up share one), and the glue -- residual add + RMSNorm, RoPE + KV-cache
append, GQA attention, SiLU(gate) * up, the uncompressed bf16 LM head and the
greedy argmax -- are small HIP kernels (``hxq_decode.hip``).  The token id and
position live in device memory and the argmax kernel advances them, so one
captured HIP graph per step replays the whole generation with no host sync.

Math: transformers' Qwen2 (``models/qwen2/modeling_qwen2.py``); the residual
stream is kept in fp32, activations entering the GEMVs are bf16.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _hxq, synth
from .helix_linear import HelixLinear


@dataclass
class DecoderConfig:
    hidden: int
    n_layers: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    intermediate: int
    vocab: int
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    max_seq: int = 512


QWEN25_3B = DecoderConfig(hidden=2048, n_layers=36, n_heads=16, n_kv_heads=2, head_dim=128,
                          intermediate=11008, vocab=151936)
QWEN25_7B = DecoderConfig(hidden=3584, n_layers=28, n_heads=28, n_kv_heads=4, head_dim=128,
                          intermediate=18944, vocab=152064)

_PROJ = ("q", "k", "v", "o", "gate", "up", "down")


def _mats(mods):
    return [{"indices": m.indices, "codebook": m._kcb, "group_scale": m.group_scale,
             "group_offset": m.group_offset, "sc_row_ptr": m._sc_row_ptr, "sc_col": m._sc_col,
             "sc_delta": m._sc_delta, "bias": m.bias} for m in mods]


class HelixDecoder:
    """Weights: per layer HelixLinear q/k/v (with bias, as Qwen2), o, gate, up,
    down and fp32 RMSNorm weights; a bf16 embedding tied to the LM head."""

    def __init__(self, cfg: DecoderConfig, layers, embed, final_norm):
        self.cfg = cfg
        self.layers = layers
        self.embed = embed
        self.final_norm = final_norm
        self.device = embed.device
        self._graph = None
        self._alloc()

    # -- construction ---------------------------------------------------------
    @classmethod
    def synthetic(cls, cfg: DecoderConfig, seed=0, device="cuda", layer_fn=None):
        """Random-init weights, every projection HXQ-encoded per the config-0
        recipe (``synth.make_layer_torch``); q/k/v biases ~ N(0, 0.02)."""
        dev = torch.device(device)
        g = torch.Generator(device=dev).manual_seed(seed)
        H, I, D = cfg.hidden, cfg.intermediate, cfg.head_dim
        shapes = {"q": (cfg.n_heads * D, H), "k": (cfg.n_kv_heads * D, H),
                  "v": (cfg.n_kv_heads * D, H), "o": (H, cfg.n_heads * D), "gate": (I, H),
                  "up": (I, H), "down": (H, I)}
        make = layer_fn or (lambda o, i, s: synth.make_layer_torch(o, i, seed=s, device=dev))
        layers = []
        for li in range(cfg.n_layers):
            L = {}
            for pi, name in enumerate(_PROJ):
                o, i = shapes[name]
                w = make(o, i, seed * 1000003 + 16 * li + pi)
                bias = (torch.randn(o, generator=g, device=dev) * 0.02) if name in "qkv" else None
                L[name] = HelixLinear(i, o, torch.as_tensor(w["codebook"]).to(dev),
                                      torch.as_tensor(w["indices"]).to(dev),
                                      torch.as_tensor(w["sidecar_positions"]).to(dev),
                                      torch.as_tensor(w["sidecar_values"]).to(dev), bias=bias,
                                      group_scale=torch.as_tensor(w["group_scale"]).to(dev),
                                      group_offset=torch.as_tensor(w["group_offset"]).to(dev),
                                      group_size=w["group_size"])
            L["in_norm"] = 1.0 + 0.1 * torch.randn(H, generator=g, device=dev)
            L["post_norm"] = 1.0 + 0.1 * torch.randn(H, generator=g, device=dev)
            layers.append(L)
        embed = (torch.randn(cfg.vocab, H, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        final_norm = 1.0 + 0.1 * torch.randn(H, generator=g, device=dev)
        return cls(cfg, layers, embed, final_norm)

    def _alloc(self):
        c, dev = self.cfg, self.device
        H, I, D = c.hidden, c.intermediate, c.head_dim
        f32 = dict(dtype=torch.float32, device=dev)
        bf = dict(dtype=torch.bfloat16, device=dev)
        nq, nkv = c.n_heads * D, c.n_kv_heads * D
        self.x = torch.zeros(1, H, **f32)               # residual stream (ping-pong pair)
        self.x2 = torch.zeros(1, H, **f32)
        self.h = torch.zeros(1, H, **bf)                # normed activation
        self.qkv = torch.zeros(nq + 2 * nkv, **f32)
        self.q = torch.zeros(nq, **f32)
        self.attn = torch.zeros(1, nq, **bf)
        self.o = torch.zeros(1, H, **f32)
        self.g = torch.zeros(1, I, **f32)
        self.u = torch.zeros(1, I, **f32)
        self.act = torch.zeros(1, I, **bf)
        self.dn = torch.zeros(1, H, **f32)
        self.logits = torch.zeros(c.vocab, **f32)
        self.tok = torch.zeros(1, dtype=torch.int32, device=dev)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self._argmax_ws = torch.empty(2048, dtype=torch.uint8, device=dev)
        self.kc = [torch.zeros(c.max_seq, c.n_kv_heads, D, **bf) for _ in self.layers]
        self.vc = [torch.zeros(c.max_seq, c.n_kv_heads, D, **bf) for _ in self.layers]
        self._qkv_mats = [_mats([L["q"], L["k"], L["v"]]) for L in self.layers]
        self._gu_mats = [_mats([L["gate"], L["up"]]) for L in self.layers]
        self._down_mats = [_mats([L["down"]]) for L in self.layers]
        self._qkv_outs = [self.qkv[:nq].view(1, -1), self.qkv[nq:nq + nkv].view(1, -1),
                          self.qkv[nq + nkv:].view(1, -1)]
        gs = {L["q"].group_size for L in self.layers} | {L["down"].group_size for L in self.layers}
        if len(gs) != 1:
            raise ValueError("all projections must share one group size")
        self._group = gs.pop()

    # -- one token --------------------------------------------------------------
    def _step_launches(self, fused=True):
        """All launches of one decode step for token self.tok at self.pos; ends
        with argmax into self.tok and ++pos.  fused: the norms are folded into
        the GEMV prologues and RoPE / KV append into the attention launch (6
        launches per layer instead of 9)."""
        c = self.cfg
        if not fused:
            return self._step_launches_unfused()
        xa, xb = self.x, self.x2
        xa.copy_(self.embed.index_select(0, self.tok.long()))
        delta = None
        for li, L in enumerate(self.layers):
            # r = xa + delta -> xb; h = norm(r) -> q/k/v
            _hxq.gemv_multi_rmsnorm(xa, delta, L["in_norm"], c.rms_eps, xb, self._qkv_mats[li],
                                    self._group, outs=self._qkv_outs)
            _hxq.attn_rope_decode(self.qkv, self.pos, c.n_heads, c.n_kv_heads, c.head_dim,
                                  c.rope_theta, self.kc[li], self.vc[li], self.attn)
            Lo = L["o"]
            _hxq.gemv(self.attn, Lo.indices, Lo._kcb, Lo.group_scale, Lo.group_offset,
                      Lo.group_size, Lo._sc_row_ptr, Lo._sc_col, Lo._sc_delta, Lo.bias,
                      out=self.o)
            # r = xb + o -> xa; h = norm(r) -> gate/up
            _hxq.gemv_multi_rmsnorm(xb, self.o, L["post_norm"], c.rms_eps, xa, self._gu_mats[li],
                                    self._group, outs=[self.g, self.u])
            # SiLU stays a separate kernel: the down GEMV reads bf16 act (K = 11008)
            # far cheaper than fp32 gate and up in every block
            _hxq.silu_mul(self.g, self.u, self.act)
            Ld = L["down"]
            _hxq.gemv(self.act, Ld.indices, Ld._kcb, Ld.group_scale, Ld.group_offset,
                      Ld.group_size, Ld._sc_row_ptr, Ld._sc_col, Ld._sc_delta, Ld.bias,
                      out=self.dn)
            delta = self.dn
        _hxq.add_rmsnorm(xa, delta, self.final_norm, c.rms_eps, self.h)
        _hxq.dense_gemv_bf16(self.embed, self.h, self.logits)
        _hxq.argmax(self.logits, self.tok, self.pos, self._argmax_ws)

    def _step_launches_unfused(self):
        c = self.cfg
        self.x.copy_(self.embed.index_select(0, self.tok.long()))
        delta = None
        for li, L in enumerate(self.layers):
            _hxq.add_rmsnorm(self.x, delta, L["in_norm"], c.rms_eps, self.h)
            _hxq.gemv_multi(self.h, self._qkv_mats[li], self._group, outs=self._qkv_outs)
            _hxq.rope_kv_append(self.qkv, self.pos, c.n_heads, c.n_kv_heads, c.head_dim,
                                c.rope_theta, self.q, self.kc[li], self.vc[li])
            _hxq.attn_decode(self.q, self.kc[li], self.vc[li], self.pos, c.n_heads, c.n_kv_heads,
                             c.head_dim, self.attn)
            Lo = L["o"]
            _hxq.gemv(self.attn, Lo.indices, Lo._kcb, Lo.group_scale, Lo.group_offset,
                      Lo.group_size, Lo._sc_row_ptr, Lo._sc_col, Lo._sc_delta, Lo.bias,
                      out=self.o)
            _hxq.add_rmsnorm(self.x, self.o, L["post_norm"], c.rms_eps, self.h)
            _hxq.gemv_multi(self.h, self._gu_mats[li], self._group, outs=[self.g, self.u])
            _hxq.silu_mul(self.g, self.u, self.act)
            Ld = L["down"]
            _hxq.gemv(self.act, Ld.indices, Ld._kcb, Ld.group_scale, Ld.group_offset,
                      Ld.group_size, Ld._sc_row_ptr, Ld._sc_col, Ld._sc_delta, Ld.bias,
                      out=self.dn)
            delta = self.dn
        _hxq.add_rmsnorm(self.x, delta, self.final_norm, c.rms_eps, self.h)
        _hxq.dense_gemv_bf16(self.embed, self.h, self.logits)
        _hxq.argmax(self.logits, self.tok, self.pos, self._argmax_ws)

    def reset(self):
        for t in self.kc + self.vc:
            t.zero_()
        self.pos.zero_()

    def prefill(self, prompt_ids):
        """Feed the prompt token by token (teacher forced); leaves the greedy
        successor of the last prompt token in self.tok."""
        ids = torch.as_tensor(prompt_ids, dtype=torch.int32, device=self.device)
        if ids.numel() >= self.cfg.max_seq:
            raise ValueError("prompt longer than max_seq")
        for t in range(ids.numel()):
            self.tok.copy_(ids[t:t + 1])
            self._step_launches()

    def capture(self):
        """Capture one decode step in a HIP graph (weights and buffers fixed)."""
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            self._graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self._graph, stream=s):
                self._step_launches()
        torch.cuda.current_stream(self.device).wait_stream(s)
        return self._graph

    def generate(self, n_new, use_graph=True):
        """Greedy-decode n_new tokens after prefill; returns their ids (device
        int32 [n_new]).  Each step replays the captured graph; the only host
        synchronisation is the final copy."""
        if int(self.pos.item()) + n_new > self.cfg.max_seq:
            raise ValueError("generation would exceed max_seq")
        out = torch.empty(n_new, dtype=torch.int32, device=self.device)
        for t in range(n_new):
            out[t:t + 1].copy_(self.tok)
            if use_graph:
                self._graph.replay()
            else:
                self._step_launches()
        return out

    # -- one launch per token (persistent kernel) ---------------------------------
    def persistent_init(self):
        """Prepare hxq_decoder_step: one cooperative launch runs a whole token
        (every layer, LM head and argmax) with grid barriers between stages;
        same math as _step_launches.  Shares this decoder's buffers (token,
        position, caches, logits)."""
        c = self.cfg
        n = len(self.layers)
        arr = (_hxq.HxqDecoderLayer * n)()
        for i, L in enumerate(self.layers):
            arr[i] = _hxq.HxqDecoderLayer(
                *(_hxq.hxq_matrix_of(L[name]) for name in _PROJ),
                L["in_norm"].data_ptr(), L["post_norm"].data_ptr(), self.kc[i].data_ptr(),
                self.vc[i].data_ptr())
        desc = _hxq.HxqDecoder(c.hidden, n, c.n_heads, c.n_kv_heads, c.head_dim, c.intermediate,
                               c.vocab, c.max_seq, self._group, c.rms_eps, c.rope_theta,
                               ctypes.addressof(arr), self.embed.data_ptr(),
                               self.final_norm.data_ptr(), self.tok.data_ptr(),
                               self.pos.data_ptr(), self.logits.data_ptr())
        ws = torch.empty(_hxq.decoder_workspace_bytes(desc), dtype=torch.uint8, device=self.device)
        _hxq.decoder_init(desc, ws)
        self._p_layers, self._p_desc, self._p_ws = arr, desc, ws
        return self

    def step_persistent(self, n_steps=1, out_ids=None):
        """n_steps greedy steps, one launch each (no host synchronisation)."""
        if getattr(self, "_p_desc", None) is None:
            self.persistent_init()
        _hxq.decoder_step(self._p_desc, self._p_ws, n_steps, out_ids)

    def persistent_error(self):
        """0 when every step completed; 1 = a grid barrier timed out; 2 = bad
        token / position.  Synchronises the stream."""
        return _hxq.decoder_error(self._p_desc, self._p_ws)

    def generate_persistent(self, n_new):
        """generate() through the one-launch-per-token kernel."""
        if int(self.pos.item()) + n_new > self.cfg.max_seq:
            raise ValueError("generation would exceed max_seq")
        out = torch.empty(n_new, dtype=torch.int32, device=self.device)
        self.step_persistent(n_new, out)
        return out

    def close(self):
        """Release device state in a fixed order before the process exits: wait for
        queued work, destroy the captured graph, then drop the persistent
        workspace (flags, layer table) and its host descriptors."""
        torch.cuda.synchronize(self.device)
        if self._graph is not None:
            self._graph.reset()
            self._graph = None
        self._p_desc = self._p_layers = self._p_ws = None
        torch.cuda.synchronize(self.device)

    def hxq_bytes_per_token(self):
        return sum(L[n].kernel_bytes() for L in self.layers for n in _PROJ)
