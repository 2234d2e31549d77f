from .linear import DPLinear
from .layernorm import DPLayerNorm
from .transformers_conv1d import DPConv1D
from .utils import DPParameter

__all__ = ["DPLinear", "DPLayerNorm", "DPConv1D", "DPParameter"]
