"""Encoder forwards assembled from the hot-path kernels (GEMMs through torch /
hipBLASLt); used for end-to-end throughput and parity of whole layers."""
from .modernbert import ModernBertLayerWeights, ModernBertWeights, modernbert_forward, random_weights

__all__ = ["ModernBertLayerWeights", "ModernBertWeights", "modernbert_forward", "random_weights"]
