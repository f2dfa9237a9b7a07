"""Encoder forwards assembled from the hot-path kernels (GEMMs through torch /
hipBLASLt); used for end-to-end throughput and parity of whole layers."""
from .modernbert import ModernBertLayerWeights, ModernBertWeights, modernbert_forward, random_weights
from .mt5 import mt5_layer_forward

__all__ = ["ModernBertLayerWeights", "ModernBertWeights", "modernbert_forward", "random_weights",
           "mt5_layer_forward"]
