"""slideformer_amd: MI355X-native LayerAdam step (fused AdamW + bf16 copy + grad-norm clip).

``from slideformer_amd import LayerAdam`` replaces ``from optimizer import LayerAdam``
of the reference (optimizer/__init__.py:4).
"""
from .layer_adam import LayerAdam, SUPPORTED_TRIPLES

__all__ = ["LayerAdam", "SUPPORTED_TRIPLES"]
