"""Layers with the reference's fields and geometry (salt_core/layers/__init__.py)."""
from salt_amd.layers.base import LayerOutput
from salt_amd.layers.conv import ConvLayer, ConvSpec, conv
from salt_amd.layers.fc import FCLayer, FCSpec, fc

__all__ = ["ConvLayer", "ConvSpec", "FCLayer", "FCSpec", "LayerOutput", "conv", "fc"]
