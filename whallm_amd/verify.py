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

from .ops import (FP8Experts, linear_bf16, moe_fp8, mtp_verify_greedy, residual_rmsnorm, route_scored)


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
