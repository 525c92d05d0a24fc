"""The MTP verify step around the MoE expert path, on the device.

The reference's verify round (runtime/deepseek_v4_ssd/native_qwen.py:604-656) runs the
anchor and its drafts through the model in one call (``engine.verify([anchor, *drafts])``;
the native engine sends those <= 8 rows through the expert pair path,
Native/QwenNative/engine.mm:869, :2198-2235) and then accepts drafts with
``Sampler.verify`` (native_qwen.py:389-408; dspark._verify, dspark.py:857-904).

Here the decoder layers are reduced to their MoE halves with the pre-norm residual glue
(attention and KV state are outside the expert path):
    x_l = bf16(rmsnorm(r_l)),  (indices, weights) = DeepSeek gate over the layer's router
    logits (sigmoid, bias select, group-limited), r_{l+1} = r_l + MoE_l(x_l),
then logits = x_L head^T in fp32 (wm_linear_bf16) and greedy acceptance
(wm_mtp_verify_greedy); rejection acceptance takes the same logits through
``mtp_verify_rejection``. Every step is a library kernel, so one call can be captured
in a HIP graph.
"""
from __future__ import annotations

import torch

import ctypes

from . import _lib
from .ops import (SCORE_FUNCS, FP8Experts, _ptr, _stream, linear_bf16, moe_fp8, mtp_verify_greedy, residual_rmsnorm,
                  route_scored)


class VerifyStep:
    """M = n + 1 rows (the accepted token and n drafts) through ``len(layers)`` FP8 MoE
    layers, the LM head and greedy acceptance."""

    def __init__(self, layers: list[FP8Experts], shared: list[FP8Experts], biases: list[torch.Tensor],
                 head: torch.Tensor, k: int = 8, score_func: str = "sigmoid", route_scale: float = 2.5,
                 n_groups: int = 8, topk_groups: int = 4, eps: float = 1e-6):
        if not layers or len(shared) != len(layers) or len(biases) != len(layers):
            raise ValueError("one shared expert and one bias per layer are required")
        if head.dtype != torch.bfloat16 or head.dim() != 2 or head.shape[1] != layers[0].hidden:
            raise ValueError("head must be bf16 [vocab, hidden]")
        self.layers, self.shared, self.biases, self.head = layers, shared, biases, head
        self.k, self.score_func, self.route_scale = k, score_func, route_scale
        self.n_groups, self.topk_groups, self.eps = n_groups, topk_groups, eps
        # the C entry's host arrays: the layer tables, the shared tables, the bias pointers
        self._tables = (_lib.FP8ExpertsC * len(layers))(*[t.c_struct() for t in layers])
        self._shared = (_lib.FP8ExpertsC * len(shared))(*[t.c_struct() for t in shared])
        self._biases = (ctypes.c_void_p * len(biases))(*[b.data_ptr() if b is not None else None for b in biases])
        self._ws = None

    def moe_layers(self, router_logits: torch.Tensor, residual: torch.Tensor, trace: list | None = None):
        """router_logits fp32 [L, M, E]; residual fp32 [M, H], updated in place. Returns the
        last bf16 rmsnorm x_L. ``trace`` (a list) receives (x_l, residual after layer l) copies."""
        x = residual_rmsnorm(residual, None, self.eps)
        for l, (table, sh, bias) in enumerate(zip(self.layers, self.shared, self.biases)):
            idx, w = route_scored(router_logits[l], bias, self.k, self.score_func, self.route_scale, True,
                                  self.n_groups, self.topk_groups)
            y = moe_fp8(x, idx, w, table, sh, None)
            x_in = x
            x = residual_rmsnorm(residual, y, self.eps)
            if trace is not None:
                trace.append((x_in.clone(), residual.clone()))
        return x

    def __call__(self, router_logits: torch.Tensor, residual: torch.Tensor, drafts: torch.Tensor,
                 trace: list | None = None):
        """(acceptance int32[2] = (accepted drafts, next token), vocab logits fp32 [M, V])."""
        x = self.moe_layers(router_logits, residual, trace)
        logits = linear_bf16(x, self.head)
        return mtp_verify_greedy(logits, drafts), logits

    def native(self, router_logits: torch.Tensor, residual: torch.Tensor, drafts: torch.Tensor):
        """The same step through the library's one C entry (wm_verify_step_fp8): the calls a
        native caller binds instead of composing them. Returns (acceptance, logits) as
        __call__ does; residual is updated in place."""
        L, M = len(self.layers), residual.shape[0]
        H, E, V = self.layers[0].hidden, self.layers[0].count, self.head.shape[0]
        if router_logits.shape != (L, M, E) or router_logits.dtype != torch.float32 or not router_logits.is_contiguous():
            raise ValueError("router_logits must be contiguous fp32 [layers, rows, experts]")
        if residual.dtype != torch.float32 or not residual.is_contiguous() or residual.shape != (M, H):
            raise ValueError("residual must be contiguous fp32 [rows, hidden]")
        lib = _lib.load()
        need = lib.wm_verify_step_fp8_workspace_size(M, self.k, V, ctypes.byref(self._tables[0]))
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(need, dtype=torch.uint8, device=residual.device)
        logits = torch.empty(M, V, dtype=torch.float32, device=residual.device)
        acceptance = torch.empty(2, dtype=torch.int32, device=residual.device)
        d = drafts.to(torch.int32).contiguous()
        _lib.call("wm_verify_step_fp8", L, _ptr(router_logits), _ptr(residual), M, self._tables, self._shared,
                  self._biases, self.k, SCORE_FUNCS[self.score_func], float(self.route_scale), self.n_groups,
                  self.topk_groups, float(self.eps), _ptr(self.head), V, _ptr(d), _ptr(logits), _ptr(acceptance),
                  _ptr(self._ws), self._ws.numel(), _stream(residual.device))
        return acceptance, logits
