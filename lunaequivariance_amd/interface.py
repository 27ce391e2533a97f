"""Functional API: preparation and calls with explicit weights.

Mirrors ``prepare_tensor_product`` / ``tensor_product_conv``
(``src/lunatp/interface.py:147-262``) for the UVU, UUU and UVW convolutions
and the row-wise products of all three modes.
"""

from __future__ import annotations

from collections.abc import Mapping
from copy import copy
from functools import lru_cache

import torch

from .irreps import Irreps
from .layout import TensorProductPaths
from .uuu_conv import LunaTPUUUConv, create_uuu_conv_operator
from .uvu_conv import LunaTPUVUConv, create_uvu_conv_operator


def _unsupported(mode: str, convolution: bool):
    kind = "convolution" if convolution else "tensor product"
    raise NotImplementedError(f"{mode} {kind} is not part of this MI355X build")


def prepare_tensor_product(irreps_in1, irreps_in2=None, irreps_out=None, instructions=None, *,
                           in1_var=None, in2_var=None, out_var=None,
                           irrep_normalization=None, path_normalization=None, shared_weights=False,
                           dtype=torch.float32, convolution=False, mode=None):
    """Prepare paths and kernels once for repeated calls (``lunatp/interface.py:147-193``)."""
    if isinstance(irreps_in1, Mapping):
        if not convolution or mode not in ("uuu", "uvu"):
            raise ValueError('Metadata requires convolution=True and mode="uuu" or "uvu"')
        factory = create_uuu_conv_operator if mode == "uuu" else create_uvu_conv_operator
        return factory(irreps_in1, dtype=dtype)
    if isinstance(irreps_in1, TensorProductPaths):
        paths = copy(irreps_in1)
    else:
        if irreps_in2 is None or irreps_out is None or instructions is None:
            raise TypeError("All three irreps and instructions are required")
        paths = TensorProductPaths(
            irreps_in1, irreps_in2, irreps_out, instructions,
            in1_var=in1_var, in2_var=in2_var, out_var=out_var,
            irrep_normalization=irrep_normalization, path_normalization=path_normalization,
            internal_weights=False, shared_weights=shared_weights,
        )
    paths.dtype = dtype
    modes = {ins.connection_mode for ins in paths.instructions}
    if len(modes) != 1 or not modes <= {"uuu", "uvu", "uvw"}:
        raise ValueError("Tensor products require one connection mode: uuu, uvu or uvw")
    inferred = modes.pop()
    if mode is not None and mode != inferred:
        raise ValueError("mode must match the tensor-product instructions")
    if not convolution:
        if inferred == "uvw":
            from .uvw import LunaTPUVW
            return LunaTPUVW(paths, dtype=dtype)
        from .rowwise import LunaTPRows

        return LunaTPRows(paths, dtype=dtype)
    if inferred == "uuu":
        return create_uuu_conv_operator(paths, dtype=dtype)
    if inferred == "uvw":
        from .uvw_conv import LunaTPUVWConv

        return LunaTPUVWConv(paths, dtype=dtype)
    if inferred != "uvu":
        _unsupported(inferred, True)
    return create_uvu_conv_operator(paths, dtype=dtype)


@lru_cache(maxsize=128)
def _cached(irreps_in1, irreps_in2, irreps_out, instructions, in1_var, in2_var, out_var,
            irrep_normalization, path_normalization, shared_weights, dtype, convolution):
    return prepare_tensor_product(
        irreps_in1, irreps_in2, irreps_out, [tuple(i) for i in instructions],
        in1_var=in1_var, in2_var=in2_var, out_var=out_var,
        irrep_normalization=irrep_normalization, path_normalization=path_normalization,
        shared_weights=shared_weights, dtype=dtype, convolution=convolution,
    )


def _config_from_arguments(x, irreps_in1, irreps_in2, irreps_out, instructions, in1_var, in2_var,
                           out_var, irrep_normalization, path_normalization, shared_weights,
                           convolution):
    if irreps_in1 is None or irreps_in2 is None or irreps_out is None or instructions is None:
        raise TypeError("Supply irreps and instructions, or a prepared config")
    return _cached(
        str(Irreps(irreps_in1)), str(Irreps(irreps_in2)), str(Irreps(irreps_out)),
        tuple(tuple(i) for i in instructions),
        None if in1_var is None else tuple(in1_var),
        None if in2_var is None else tuple(in2_var),
        None if out_var is None else tuple(out_var),
        irrep_normalization, path_normalization, shared_weights, x.dtype, convolution,
    )


def tensor_product(x, y, weight=None, *, irreps_in1=None, irreps_in2=None, irreps_out=None,
                   instructions=None, in1_var=None, in2_var=None, out_var=None,
                   irrep_normalization=None, path_normalization=None, shared_weights=False,
                   config=None):
    """Independent per-row tensor products (``lunatp/interface.py:210-235``)."""
    if config is None:
        config = _config_from_arguments(x, irreps_in1, irreps_in2, irreps_out, instructions,
                                        in1_var, in2_var, out_var, irrep_normalization,
                                        path_normalization, shared_weights, False)
    return config.run(x, y, weight)


def tensor_product_conv(x, edge_attr, weight=None, *, graph, irreps_in1=None, irreps_in2=None,
                        irreps_out=None, instructions=None, in1_var=None, in2_var=None,
                        out_var=None, irrep_normalization=None, path_normalization=None,
                        shared_weights=False, config=None, **kwargs):
    """Contract edge messages and sum them at destinations (``lunatp/interface.py:238-262``)."""
    if config is None:
        config = _config_from_arguments(x, irreps_in1, irreps_in2, irreps_out, instructions,
                                        in1_var, in2_var, out_var, irrep_normalization,
                                        path_normalization, shared_weights, True)
    return config.run(x, edge_attr, weight, graph=graph, **kwargs)


__all__ = ["prepare_tensor_product", "tensor_product", "tensor_product_conv",
           "create_uvu_conv_operator", "LunaTPUVUConv", "create_uuu_conv_operator", "LunaTPUUUConv"]
