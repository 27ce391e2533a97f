"""``TensorProductConv`` module (``src/modules/tensorproduct.py:119-206``)."""

from __future__ import annotations

from collections.abc import Mapping

import torch

from .graph import make_graph
from .interface import tensor_product_conv
from .layout import TensorProductConfig
from .uuu_conv import create_uuu_conv_operator
from .uvu_conv import create_uvu_conv_operator


class TensorProduct(torch.nn.Module):
    """Row-wise tensor product (``src/modules/tensorproduct.py:19-116``).

    ``uvw``: shared weights in fp32 on matrix-core kernels, fp64 and per-row
    weights through the row form of the UVW convolution.  ``uvu`` and ``uuu``:
    the convolution kernels over the identity graph (matrices only).  Weights
    are the configuration's registered parameter unless given.
    """

    def __init__(self, irreps_in1, irreps_in2=None, irreps_out=None, instructions=None,
                 in1_var=None, in2_var=None, out_var=None, irrep_normalization=None,
                 path_normalization=None, internal_weights=None, shared_weights=None, *, dtype=None):
        super().__init__()
        if isinstance(irreps_in1, torch.nn.Module):
            if any(value is not None for value in (
                    irreps_in2, irreps_out, instructions, in1_var, in2_var, out_var,
                    irrep_normalization, path_normalization, internal_weights, shared_weights)):
                raise TypeError("Pass either an existing tensor product or irreps and path options")
            tp = irreps_in1
        else:
            if irreps_in2 is None or irreps_out is None or instructions is None:
                raise TypeError("irreps_in2, irreps_out and instructions are required")
            tp = TensorProductConfig(
                irreps_in1, irreps_in2, irreps_out, instructions,
                in1_var=in1_var, in2_var=in2_var, out_var=out_var,
                irrep_normalization=irrep_normalization, path_normalization=path_normalization,
                internal_weights=internal_weights, shared_weights=shared_weights,
            )
            if dtype is not None and tp.weight.dtype != dtype:
                tp.to(dtype=dtype)
        modes = {ins.connection_mode for ins in tp.instructions}
        if len(modes) != 1 or not modes <= {"uuu", "uvu", "uvw"}:
            raise ValueError("TensorProduct requires one connection mode: uuu, uvu or uvw")
        self.mode = modes.pop()
        weight = getattr(tp, "weight", None)
        if dtype is None:
            dtype = weight.dtype if isinstance(weight, torch.Tensor) else torch.float32
        self.op = self._make_op(tp, dtype)
        self.tp = tp
        self.irreps_in1, self.irreps_in2, self.irreps_out = tp.irreps_in1, tp.irreps_in2, tp.irreps_out
        self.instructions = tp.instructions
        self.weight_numel = tp.weight_numel
        self.internal_weights, self.shared_weights = tp.internal_weights, tp.shared_weights

    @property
    def weight(self):
        return self.tp.weight

    def _make_op(self, tp, dtype):
        if self.mode == "uvw":
            from .uvw import LunaTPUVW

            return LunaTPUVW(tp, dtype=dtype)
        from .rowwise import LunaTPRows

        return LunaTPRows(tp, dtype=dtype)

    def _apply(self, fn, recurse=True):
        dtype = fn(torch.empty(0, dtype=self.op.compute_dtype)).dtype
        result = super()._apply(fn, recurse=recurse)
        if dtype in (torch.float32, torch.float64) and dtype != self.op.compute_dtype:
            self.op = self._make_op(self.tp, dtype)
        return result

    def forward(self, x, y, weight=None):
        if weight is None and self.internal_weights:
            weight = self.tp.weight
        return self.op.run(x, y, weight)


class TensorProductConv(torch.nn.Module):
    """Fused tensor product on every edge, summed at destination nodes.

    Pass irreps and instructions, an existing configuration (or e3nn-like
    module with the same attributes), or prebuilt metadata with ``mode="uvu"`` or
    ``mode="uuu"``.  uvu, uuu and uvw instructions are supported.
    Build topology with ``create_graph`` and pass ``graph=`` on every call.
    """

    def __init__(self, irreps_in1, irreps_in2=None, irreps_out=None, instructions=None,
                 in1_var=None, in2_var=None, out_var=None, irrep_normalization=None,
                 path_normalization=None, internal_weights=None, shared_weights=None, *,
                 dtype=None, mode=None):
        super().__init__()
        metadata = isinstance(irreps_in1, Mapping)
        if metadata or isinstance(irreps_in1, torch.nn.Module):
            if any(value is not None for value in (
                    irreps_in2, irreps_out, instructions, in1_var, in2_var, out_var,
                    irrep_normalization, path_normalization, internal_weights, shared_weights)):
                raise TypeError(
                    "Pass either an existing tensor product/metadata or irreps and path options")
            tp = irreps_in1
        else:
            if irreps_in2 is None or irreps_out is None or instructions is None:
                raise TypeError("irreps_in2, irreps_out and instructions are required")
            tp = TensorProductConfig(
                irreps_in1, irreps_in2, irreps_out, instructions,
                in1_var=in1_var, in2_var=in2_var, out_var=out_var,
                irrep_normalization=irrep_normalization, path_normalization=path_normalization,
                internal_weights=internal_weights, shared_weights=shared_weights,
            )
            if dtype is not None and tp.weight.dtype != dtype:
                tp.to(dtype=dtype)
        if metadata:
            if mode not in ("uuu", "uvu"):
                raise ValueError('Prebuilt metadata requires mode="uuu" or mode="uvu"')
            dtype = torch.float32 if dtype is None else dtype
        else:
            modes = {ins.connection_mode for ins in tp.instructions}
            if len(modes) != 1 or not modes <= {"uuu", "uvu", "uvw"}:
                raise ValueError("TensorProductConv requires one connection mode: uuu, uvu or uvw")
            inferred = modes.pop()
            if mode is not None and mode != inferred:
                raise ValueError("mode must match the tensor-product instructions")
            mode = inferred
            weight = getattr(tp, "weight", None)
            if dtype is None:
                dtype = weight.dtype if isinstance(weight, torch.Tensor) else torch.get_default_dtype()
        if metadata and mode not in ("uvu", "uuu"):
            raise ValueError('Prebuilt metadata requires mode="uuu" or mode="uvu"')
        from .uvw_conv import create_uvw_conv_operator

        self.mode = mode + "_conv"
        self._factory = {"uuu": create_uuu_conv_operator, "uvu": create_uvu_conv_operator,
                         "uvw": create_uvw_conv_operator}[mode]
        self.op = self._factory(tp, dtype=dtype)
        if metadata:
            self.weight_numel = tp["weight_numel"]
            self.internal_weights = self.shared_weights = False
        else:
            self.tp = tp
            self.irreps_in1, self.irreps_in2, self.irreps_out = tp.irreps_in1, tp.irreps_in2, tp.irreps_out
            self.instructions = tp.instructions
            self.weight_numel = tp.weight_numel
            self.internal_weights, self.shared_weights = tp.internal_weights, tp.shared_weights

    @property
    def weight(self):
        """The configuration's registered weight (internal weights) or its empty buffer."""
        return self.tp.weight

    def _apply(self, fn, recurse=True):
        dtype = fn(torch.empty(0, dtype=self.op.compute_dtype)).dtype
        result = super()._apply(fn, recurse=recurse)
        if dtype in (torch.float32, torch.float64) and dtype != self.op.compute_dtype:
            self.op = self._factory(self.op.meta if not hasattr(self, "tp") else self.tp, dtype=dtype)
        return result

    @staticmethod
    def create_graph(src, dst, num_nodes=None, **kwargs):
        """Prepare shared topology once per batch."""
        return make_graph(src, dst, num_nodes, **kwargs)

    def forward(self, x, edge_attr, weight=None, *, graph, **kwargs):
        if weight is None and self.internal_weights:
            weight = self.tp.weight
        return tensor_product_conv(x, edge_attr, weight, graph=graph, config=self.op, **kwargs)


__all__ = ["TensorProduct", "TensorProductConv"]
