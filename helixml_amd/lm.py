"""Byte-level SSM language model on the C ABI.

The reference's byte LM example (examples/ssm_byte_lm/src/main.rs:104-130) builds an S4Block and
a Linear(d_model, 256) head and feeds random tensors; the configured model is
12 x (RMSNorm + MambaBlock) with a 256-entry byte embedding and a 256-way head. This module is
that model, pre-norm with a residual stream:

    x = embed[tokens]                                    (fp32 residual stream)
    for each layer: x += MambaBlock(RMSNorm(x))          (hx_mamba_layer_fwd / _decode)
    logits = RMSNorm_f(x) . W_head^T                     (hx_rmsnorm_fwd + hx_gemm_bf16)

``prefill`` runs whole sequences and returns the per-layer decode state (the scan's last state
and the conv window); ``decode_step`` advances every sequence by one token from that state.
Every value is computed by libhelix_hip.so; torch provides device memory and the stream.
"""
from __future__ import annotations

import math
from typing import Dict, List, Optional

import torch

from . import _ffi
from .ssm import _ptr, _stream, keep_for_stream, on_launch_stream

_F32, _BF16 = _ffi.HX_F32, _ffi.HX_BF16


@on_launch_stream
def embedding(tokens, table, out=None, stream=None):
    """out[t] = table[tokens[t]] (hx_embedding_fwd); tokens int32 of any shape (made contiguous)."""
    if tokens.dtype != torch.int32:
        raise _ffi.DTypeMismatch(f"tokens: expected torch.int32, got {tokens.dtype}")
    tokens = tokens.contiguous()
    n = tokens.numel()
    vocab, dim = table.shape
    if out is None:
        out = torch.empty((*tokens.shape, dim), device=table.device, dtype=torch.float32)
    _ffi.call("hx_embedding_fwd", n, vocab, dim, _ptr(tokens), _ptr(table), _ptr(out), _stream(stream))
    return out


@on_launch_stream
def rmsnorm(x, weight, eps=1e-5, out_dtype=torch.float32, out=None, stream=None):
    """nn::RMSNorm::forward (crates/nn/src/lib.rs:258-285) over the last dim (hx_rmsnorm_fwd)."""
    dim = x.shape[-1]
    rows = x.numel() // dim
    if out is None:
        out = torch.empty(x.shape, device=x.device, dtype=out_dtype)
    od = _F32 if out.dtype == torch.float32 else _BF16
    _ffi.call("hx_rmsnorm_fwd", rows, dim, _ptr(x), _ptr(weight), float(eps), od, _ptr(out),
              _stream(stream))
    return out


@on_launch_stream
def conv1d_step(x, weight, bias, state, out=None, stream=None):
    """One recurrent step of the causal conv (hx_conv1d_step); x [batch, dim] (rows may be
    strided), state [batch, width-1, dim] fp32 advanced in place."""
    bt, dim = x.shape
    width = weight.shape[1]
    if out is None:
        out = torch.empty((bt, dim), device=x.device, dtype=x.dtype)
    dt = _F32 if x.dtype == torch.float32 else _BF16
    _ffi.call("hx_conv1d_step", bt, dim, width, dt, _ptr(x), x.stride(0), _ptr(weight), _ptr(bias),
              _ptr(state), _ptr(out), _stream(stream))
    return out


LAYER_KEYS = ("w_in", "conv_w", "conv_b", "w_x", "w_dt", "dt_bias", "A", "D", "w_out")


class ByteLM:
    """12 x (RMSNorm + MambaBlock) byte LM with the config-5 shape by default (d_model 512,
    d_state 16, d_conv 4, expand 2, dt_rank 32, vocab 256). Weights are drawn from a seeded
    generator with the reference's Linear init N(0, sqrt(2/fan_in)) (crates/nn/src/lib.rs:67-77),
    RMSNorm weights 1 (lib.rs:231), and the Mamba-specific A = -(n+1), D = 1, dt_bias =
    softplus^-1 of a log-uniform dt in [1e-3, 1e-1]. Projections are stored bf16, the rest fp32."""

    def __init__(self, n_layers=12, d_model=512, d_state=16, d_conv=4, expand=2, dt_rank=None,
                 vocab=256, eps=1e-5, device="cuda", seed=0x48454C49):
        self.n_layers, self.d_model, self.d_state, self.d_conv = n_layers, d_model, d_state, d_conv
        self.d_inner = d_model * expand
        self.dt_rank = dt_rank or math.ceil(d_model / 16)
        self.vocab, self.eps, self.device = vocab, eps, torch.device(device)
        g = torch.Generator().manual_seed(seed)
        di, r, N, dm = self.d_inner, self.dt_rank, d_state, d_model
        bf, f32 = torch.bfloat16, torch.float32

        def lin(out_f, in_f):
            return (torch.randn((out_f, in_f), generator=g) * math.sqrt(2.0 / in_f)).to(self.device, bf)

        self.embed = torch.randn((vocab, dm), generator=g).to(self.device, f32)
        self.layers: List[Dict[str, torch.Tensor]] = []
        for _ in range(n_layers):
            dt0 = torch.exp(torch.rand(di, generator=g) * (math.log(0.1) - math.log(1e-3)) + math.log(1e-3))
            self.layers.append(dict(
                norm_w=torch.ones(dm, dtype=f32, device=self.device),
                w_in=lin(2 * di, dm),
                conv_w=((torch.rand((di, d_conv), generator=g) * 2 - 1) / math.sqrt(d_conv)).to(self.device),
                conv_b=((torch.rand(di, generator=g) * 2 - 1) / math.sqrt(d_conv)).to(self.device),
                w_x=lin(r + 2 * N, di),
                w_dt=lin(di, r),
                dt_bias=(dt0 + torch.log(-torch.expm1(-dt0))).to(self.device, f32),
                A=(-torch.arange(1, N + 1, dtype=f32)).repeat(di, 1).to(self.device),
                D=torch.ones(di, dtype=f32, device=self.device),
                w_out=lin(dm, di),
            ))
        self.norm_f = torch.ones(dm, dtype=f32, device=self.device)
        self.w_head = lin(vocab, dm)
        self._ws: Optional[torch.Tensor] = None

    # ------------------------------------------------------------------ helpers
    def _workspace(self, batch, seqlen):
        need = int(_ffi.lib().hx_mamba_layer_workspace_size(batch, seqlen, self.d_model, self.d_inner,
                                                            self.dt_rank, self.d_state))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, device=self.device, dtype=torch.uint8)
        return self._ws

    def new_state(self, batch):
        """Zero decode state: per layer (ssm_state [B, d_inner, N], conv_state [B, d_conv-1, d_inner])."""
        return [(torch.zeros((batch, self.d_inner, self.d_state), device=self.device),
                 torch.zeros((batch, max(self.d_conv - 1, 1), self.d_inner), device=self.device))
                for _ in range(self.n_layers)]

    def _head(self, x, stream):
        rows = x.numel() // self.d_model
        xn = rmsnorm(x, self.norm_f, self.eps, out_dtype=torch.bfloat16, stream=stream)
        logits = torch.empty((*x.shape[:-1], self.vocab), device=self.device, dtype=torch.float32)
        _ffi.call("hx_gemm_bf16", rows, self.vocab, self.d_model, _ptr(xn), self.d_model,
                  _ptr(self.w_head), self.d_model, None, 0, _F32, _ptr(logits), self.vocab,
                  self.vocab, None, 0, self.vocab, None, 0, _stream(stream))
        return logits

    # ------------------------------------------------------------------ forward
    @on_launch_stream
    def prefill(self, tokens, state=None, stream=None):
        """tokens int32 [batch, seqlen] -> (logits fp32 [batch, seqlen, vocab], decode state).
        ``state`` (from new_state) receives each layer's final scan state and conv window."""
        bt, L = tokens.shape
        x = embedding(tokens, self.embed, stream=stream)
        ws = self._workspace(bt, L)
        keep_for_stream(ws, stream)
        if state is None:
            state = self.new_state(bt)
        s = _stream(stream)
        for p, (ssm_st, conv_st) in zip(self.layers, state):
            _ffi.call("hx_mamba_layer_fwd", bt, L, self.d_model, self.d_inner, self.d_state,
                      self.dt_rank, self.d_conv, _ptr(x), _ptr(p["norm_w"]), float(self.eps),
                      *[_ptr(p[k]) for k in LAYER_KEYS], _ptr(ssm_st), _ptr(conv_st), _ptr(ws),
                      ws.numel(), s)
        return self._head(x, stream), state

    @on_launch_stream
    def decode_step(self, tokens, state, stream=None, workspace=None):
        """tokens int32 [batch] -> logits fp32 [batch, vocab]; advances ``state`` in place.
        ``workspace`` (uint8 device tensor of at least hx_mamba_layer_workspace_size(batch, 1,
        ...) bytes) replaces the model's shared workspace."""
        bt = tokens.shape[0]
        x = embedding(tokens, self.embed, stream=stream)
        ws = self._workspace(bt, 1) if workspace is None else workspace
        if workspace is None:
            keep_for_stream(ws, stream)
        s = _stream(stream)
        for p, (ssm_st, conv_st) in zip(self.layers, state):
            _ffi.call("hx_mamba_layer_decode", bt, self.d_model, self.d_inner, self.d_state,
                      self.dt_rank, self.d_conv, _ptr(x), _ptr(p["norm_w"]), float(self.eps),
                      *[_ptr(p[k]) for k in LAYER_KEYS], _ptr(ssm_st), _ptr(conv_st), _ptr(ws),
                      ws.numel(), s)
        return self._head(x, stream)

    def decode_graph(self, state, stream=None):
        """Captures one decode step for ``state``'s batch into a HIP graph (torch.cuda.CUDAGraph
        over the C ABI's launches: no host round trips, no allocations, no memsets in the step).
        Returns ``step(tokens) -> logits``: it copies the tokens into the graph's input buffer
        and replays; ``state`` is advanced in place exactly as by decode_step. The logits tensor
        is the graph's output buffer, overwritten by the next replay."""
        bt = state[0][0].shape[0]
        tok = torch.zeros((bt,), dtype=torch.int32, device=self.device)
        # the graph's own workspace: the captured launches hold its raw address, so it must live
        # as long as the graph and never be replaced (the model's shared workspace is, whenever
        # a longer prefill needs more)
        need = int(_ffi.lib().hx_mamba_layer_workspace_size(bt, 1, self.d_model, self.d_inner,
                                                            self.dt_rank, self.d_state))
        ws = torch.empty(need, device=self.device, dtype=torch.uint8)
        # warm up on a copy of the state so capture sees allocated buffers
        scratch = [(s.clone(), c.clone()) for s, c in state]
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self.decode_step(tok, scratch, workspace=ws)
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            logits = self.decode_step(tok, state, workspace=ws)

        def step(tokens):
            tok.copy_(tokens)
            g.replay()
            return logits

        step.graph = g
        step.workspace = ws
        step.tokens = tok
        step.state = state
        return step

    def host_params(self):
        """Every parameter as float32 numpy arrays (for the CPU oracle in tests)."""
        f = lambda t: t.float().cpu().numpy()  # noqa: E731
        return dict(embed=f(self.embed), norm_f=f(self.norm_f), w_head=f(self.w_head),
                    layers=[{k: f(v) for k, v in p.items()} for p in self.layers])
