from .wrap_model import dp_supported_modules, wrap_with_flashdp_layers

__all__ = ["wrap_with_flashdp_layers", "dp_supported_modules"]
