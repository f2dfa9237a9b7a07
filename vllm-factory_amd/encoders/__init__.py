"""Encoder forwards assembled from the hot-path kernels (GEMMs through torch /
hipBLASLt); used for end-to-end throughput and parity of whole layers."""
from .deberta import (DebertaLayerWeights, DebertaWeights, deberta_forward, deberta_forward_flat,
                      deberta_layer_forward)
from .modernbert import (ModernBertLayerWeights, ModernBertWeights, modernbert_forward,
                         modernbert_forward_positions, random_weights)
from .mt5 import mt5_layer_forward

__all__ = ["DebertaLayerWeights", "DebertaWeights", "deberta_forward", "deberta_forward_flat",
           "deberta_layer_forward",
           "ModernBertLayerWeights", "ModernBertWeights", "modernbert_forward",
           "modernbert_forward_positions", "random_weights",
           "mt5_layer_forward"]
