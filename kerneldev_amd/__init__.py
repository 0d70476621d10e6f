"""kerneldev_amd -- MI355X-native hierarchical-mask flash attention.

A from-scratch gfx950 implementation of KernelDev's attention hot path behind
the reference's ``flash_attention()`` signature (``original_kernel.py:2096``).
``model.MultiHeadAttention`` adopts it with an import swap::

    from kerneldev_amd import flash_attention
"""
from .attention import AttentionPlan, build_plan, build_plan_from_tokens, flash_attention, plan_views  # noqa: F401
from .hadamard import generate_hadamard_signs, hadamard_transform  # noqa: F401
from .metadata import derive_metadata  # noqa: F401

__all__ = ["flash_attention", "build_plan", "build_plan_from_tokens", "AttentionPlan", "plan_views", "derive_metadata", "generate_hadamard_signs",
           "hadamard_transform"]
__version__ = "0.1.0"
