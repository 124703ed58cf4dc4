"""Lazy access to the compiled HIP library."""

from ._wrapper import is_cuda_extension_available

__all__ = ["is_cuda_extension_available"]
