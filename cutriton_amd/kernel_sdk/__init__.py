"""Kernel Pack ABI (specs) and producer (builder) for the gfx950 kernels."""

from .spec import (
    ArgumentSpec,
    KernelSpec,
    KernelVariant,
    clear_registry,
    register,
    registered_specs,
)

__all__ = [
    "ArgumentSpec",
    "KernelSpec",
    "KernelVariant",
    "clear_registry",
    "register",
    "registered_specs",
]
