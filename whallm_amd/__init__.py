"""MI355X-native (gfx950) MoE expert path: HIP kernels behind a C ABI, with a
torch-facing layer that keeps the reference runtime's expert-FFN operator
signatures (runtime/deepseek_v4_ssd/qwen4_exp.py:763-1051, model.py:318-546)."""

from . import _lib
from .ops import (FP8Experts, MXFP4Experts, combine_pairs, dequant_mxfp4, dequant_fp8_blocks, dequant_fp8_e8m0, experts_fp8, experts_mxfp4,
                  linear_bf16, mlp_bf16, moe_fp8, moe_mxfp4, mtp_verify_greedy, mtp_verify_rejection, norm_router, permute, prefill_layout, repack_router,
                  route_scored, route_softmax_topk, split_rows_e2m3, split_rows_e4m3)

__all__ = [
    "FP8Experts", "MXFP4Experts", "combine_pairs", "dequant_mxfp4", "dequant_fp8_blocks", "dequant_fp8_e8m0", "experts_fp8", "experts_mxfp4",
    "linear_bf16", "mlp_bf16", "moe_fp8", "moe_mxfp4",
    "mtp_verify_greedy", "mtp_verify_rejection", "norm_router", "permute", "repack_router", "prefill_layout", "route_scored", "route_softmax_topk",
    "split_rows_e2m3", "split_rows_e4m3",
]
