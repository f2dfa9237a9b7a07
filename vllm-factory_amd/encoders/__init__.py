"""Encoder forwards assembled from the hot-path kernels (GEMMs through torch /
hipBLASLt); used for end-to-end throughput and parity of whole layers."""
from .deberta import (DebertaLayerWeights, DebertaV1LayerWeights, DebertaV1Weights, DebertaWeights,
                      deberta_forward, deberta_forward_flat, deberta_layer_forward,
                      deberta_v1_forward, deberta_v1_layer_forward, random_weights_v1)
from .modernbert import (ModernBertLayerWeights, ModernBertWeights, modernbert_colbert_forward,
                         modernbert_forward, modernbert_forward_positions, random_weights)
from .mt5 import mt5_encoder_flat, mt5_layer_forward

__all__ = ["DebertaLayerWeights", "DebertaV1LayerWeights", "DebertaV1Weights", "DebertaWeights",
           "deberta_forward", "deberta_forward_flat", "deberta_layer_forward",
           "deberta_v1_forward", "deberta_v1_layer_forward", "random_weights_v1",
           "ModernBertLayerWeights", "ModernBertWeights", "modernbert_colbert_forward",
           "modernbert_forward",
           "modernbert_forward_positions", "random_weights",
           "mt5_encoder_flat", "mt5_layer_forward"]
