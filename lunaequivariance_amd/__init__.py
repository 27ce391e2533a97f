"""MI355X-native fused tensor-product convolution (UVU, and UUU).

Drop-in for the ``TensorProductConv`` path of LunaEquivariance: the same
module and functional API, with kernels emitted per irreps configuration and
compiled for gfx950 (CDNA4) behind a C-ABI library.
"""

from .irreps import Irrep, Irreps
from .layout import TensorProductConfig, TensorProductPaths, Instruction
from .graph import LunaTPGraph, make_graph
from .interface import prepare_tensor_product, tensor_product, tensor_product_conv
from .modules import TensorProduct, TensorProductConv
from .uvu_conv import create_uvu_conv_operator
from .uuu_conv import create_uuu_conv_operator
from .cg import wigner_3j
from . import ops  # registers the lunatp:: dispatcher operators

__all__ = [
    "Irrep", "Irreps", "TensorProductConfig", "TensorProductPaths", "Instruction",
    "LunaTPGraph", "make_graph", "prepare_tensor_product", "tensor_product",
    "tensor_product_conv", "TensorProduct", "TensorProductConv", "create_uvu_conv_operator",
    "create_uuu_conv_operator", "wigner_3j",
]
