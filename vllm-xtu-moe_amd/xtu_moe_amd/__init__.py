"""MI355X-native (gfx950) quantized MoE expert path with the xiaotu-moe operator surface."""
from . import _lib, formats  # noqa: F401

__all__ = ["_lib", "formats"]
