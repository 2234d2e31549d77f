"""MI355X-native FlashDP DP-SGD hot path.

Same import surface as the reference package (flashdp/__init__.py:1-8):
DPLinear, DPLayerNorm, DPConv1D, wrap_with_flashdp_layers, dp_supported_modules.
The clipped-gradient math runs in hand-written HIP kernels for gfx950 loaded
from libflashdp_hip.so (built by ``python -m flashdp4review_amd.build``).
"""
from .layers.linear import DPLinear
from .layers.layernorm import DPLayerNorm
from .layers.transformers_conv1d import DPConv1D
from .api.wrap_model import dp_supported_modules, wrap_with_flashdp_layers
from .layers.utils import (get_noise_convention, get_wgrad_precision, set_noise_convention,
                           set_wgrad_precision)

__version__ = "0.1.0"

__all__ = ["DPLinear", "DPLayerNorm", "DPConv1D", "wrap_with_flashdp_layers",
           "dp_supported_modules", "set_noise_convention", "get_noise_convention",
           "set_wgrad_precision", "get_wgrad_precision"]
