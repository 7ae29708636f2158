"""Platform entry for the codec decode stage."""

from .rocm import ROCmCodecPlatform, current_platform

__all__ = ["ROCmCodecPlatform", "current_platform"]
