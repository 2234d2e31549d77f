"""Operator API of the DP-SGD hot path (names of flashdp/core/__init__.py:1-11).

Every operator runs on the HIP kernels of libflashdp_hip.so; there is no CPU
fallback.  ``wgrad_clip``, ``colsum_clip``, ``layernorm_fwd`` and
``layernorm_bwd_clip`` are the general entry points the layers use (they add
out_scale, injected noise and per-sample norm/factor outputs); ``dgrad`` is
the layers' input gradient.
"""
from .wgrad import (
    wgrad_clip,
    wgrad_status,
    set_wgrad_launch,
    set_expiry_check,
    bmtm_clip,
    bmm_clip,
    mm_clip,
    mm_fused,
    linear_weight_flashdp,
    conv1d_weight_flashdp,
)
from .colsum import (
    colsum_clip,
    linear_bias_grad_clip,
    conv1d_bias_grad_clip,
    layernorm_dw_clip,
    layernorm_db_clip,
)
from .layernorm import (
    layernorm_fwd,
    layernorm_bwd_clip,
    layernorm_fwd_fused,
    layernorm_bwd_clip_fused,
    layernorm_dwdb_fused,
)
from .inputgrad import dgrad, dgrad_choices, input_grad, set_dgrad
from .utils import RuntimeAutoTuner, supported_acc_dtypes

__all__ = [
    "wgrad_clip", "wgrad_status", "set_wgrad_launch", "set_expiry_check", "bmtm_clip", "bmm_clip", "mm_clip", "mm_fused", "linear_weight_flashdp",
    "conv1d_weight_flashdp", "colsum_clip", "linear_bias_grad_clip", "conv1d_bias_grad_clip",
    "layernorm_dw_clip", "layernorm_db_clip", "layernorm_fwd", "layernorm_bwd_clip",
    "layernorm_fwd_fused", "layernorm_bwd_clip_fused", "layernorm_dwdb_fused",
    "dgrad", "dgrad_choices", "input_grad", "set_dgrad", "RuntimeAutoTuner", "supported_acc_dtypes",
]
