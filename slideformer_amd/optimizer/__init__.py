"""Import path of the reference (``optimizer/__init__.py:4``): ``from slideformer_amd.optimizer import LayerAdam``."""
from ..layer_adam import LayerAdam

__all__ = ["LayerAdam"]
