from kla.layers.common import MLP, CausalConv1d, RMSNorm, l2_norm
from kla.layers.kla_layer import KLALayer, KLALayerState

__all__ = ["CausalConv1d", "KLALayer", "KLALayerState", "MLP", "RMSNorm", "l2_norm"]
