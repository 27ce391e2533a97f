"""Tensor-product paths with e3nn normalisation.

Restates ``TensorProductPaths`` / ``TensorProductConfig`` of the reference
(``src/lunatp/utils/layout.py:238-438``), which follow e3nn 0.6.0: with
``irrep_normalization="component"`` and ``path_normalization="element"`` each
instruction gets ``path_weight = sqrt(alpha)`` with
``alpha = (2 l_out + 1) / sum(in1_var * in2_var * fan) * out_var * user_weight``
where the sum runs over instructions sharing the output and ``fan`` is
``mul_in2`` for uvu, ``mul_in1 * mul_in2`` for uvw and 1 for uuu.
"""

from __future__ import annotations

from math import prod, sqrt
from typing import Any, NamedTuple

import torch

from .irreps import Irreps


class Instruction(NamedTuple):
    i_in1: int
    i_in2: int
    i_out: int
    connection_mode: str
    has_weight: bool
    path_weight: float
    path_shape: tuple


def _fan(mode: str, mul1: int, mul2: int) -> int:
    return {"uvw": mul1 * mul2, "uvu": mul2, "uuu": 1}[mode]


class TensorProductPaths:
    """Normalised paths of a tensor product, without parameters."""

    dtype: torch.dtype = torch.float32

    def __init__(self, irreps_in1, irreps_in2, irreps_out, instructions, *,
                 in1_var=None, in2_var=None, out_var=None,
                 irrep_normalization=None, path_normalization=None,
                 internal_weights=None, shared_weights=None):
        irrep_normalization = "component" if irrep_normalization is None else irrep_normalization
        path_normalization = "element" if path_normalization is None else path_normalization
        if irrep_normalization not in ("component", "norm", "none"):
            raise AssertionError(f"irrep_normalization={irrep_normalization!r}")
        if path_normalization not in ("element", "path", "none"):
            raise AssertionError(f"path_normalization={path_normalization!r}")
        self.irreps_in1 = Irreps(irreps_in1)
        self.irreps_in2 = Irreps(irreps_in2)
        self.irreps_out = Irreps(irreps_out)
        raw = []
        for entry in instructions:
            entry = tuple(entry)
            if len(entry) == 5:
                entry = entry + (1.0,)
            i1, i2, io, mode, has_weight, user_weight = entry
            shape = {
                "uvw": (self.irreps_in1[i1].mul, self.irreps_in2[i2].mul, self.irreps_out[io].mul),
                "uvu": (self.irreps_in1[i1].mul, self.irreps_in2[i2].mul),
                "uuu": (self.irreps_in1[i1].mul,),
            }[mode]
            raw.append(Instruction(i1, i2, io, mode, has_weight, user_weight, shape))

        def variances(values, irreps, name):
            if values is None:
                return [1.0] * len(irreps)
            values = [float(v) for v in values]
            if len(values) != len(irreps):
                raise AssertionError(f"Len of {name} must be equal to len(irreps)")
            return values

        v1 = variances(in1_var, self.irreps_in1, "ir1_var")
        v2 = variances(in2_var, self.irreps_in2, "ir2_var")
        vo = variances(out_var, self.irreps_out, "out_var")

        normalized = []
        for ins in raw:
            a, b, o = self.irreps_in1[ins.i_in1], self.irreps_in2[ins.i_in2], self.irreps_out[ins.i_out]
            if a.ir.p * b.ir.p != o.ir.p:
                raise AssertionError("parity violation")
            if not abs(a.ir.l - b.ir.l) <= o.ir.l <= a.ir.l + b.ir.l:
                raise AssertionError("degree violates the triangle inequality")
            if ins.connection_mode not in ("uuu", "uvw", "uvu"):
                raise AssertionError("unknown connection mode")
            if ins.connection_mode == "uuu" and not a.mul == b.mul == o.mul:
                raise AssertionError("UUU requires equal input and output multiplicities")
            alpha = {"component": o.ir.dim, "norm": a.ir.dim * b.ir.dim, "none": 1}[irrep_normalization]
            if path_normalization == "element":
                x = sum(
                    v1[other.i_in1] * v2[other.i_in2]
                    * _fan(other.connection_mode, self.irreps_in1[other.i_in1].mul,
                           self.irreps_in2[other.i_in2].mul)
                    for other in raw if other.i_out == ins.i_out
                )
            elif path_normalization == "path":
                x = v1[ins.i_in1] * v2[ins.i_in2] * _fan(ins.connection_mode, a.mul, b.mul)
                x *= len([other for other in raw if other.i_out == ins.i_out])
            else:
                x = 1
            if x > 0.0:
                alpha /= x
            alpha *= vo[ins.i_out]
            alpha *= ins.path_weight
            normalized.append(ins._replace(path_weight=sqrt(alpha)))
        self.instructions = normalized
        if shared_weights is False and internal_weights is None:
            internal_weights = False
        if shared_weights is None:
            shared_weights = True
        if internal_weights is None:
            internal_weights = shared_weights and any(i.has_weight for i in self.instructions)
        if not (shared_weights or not internal_weights):
            raise AssertionError("internal weights require shared weights")
        self.internal_weights = internal_weights
        self.shared_weights = shared_weights
        self.weight_numel = sum(prod(i.path_shape) for i in self.instructions if i.has_weight)

    @classmethod
    def from_tensor_product(cls, tp: Any) -> "TensorProductPaths":
        """Copy the static path attributes of a configuration or e3nn-like module."""
        if isinstance(tp, cls):
            return tp
        paths = cls.__new__(cls)
        for name in ("irreps_in1", "irreps_in2", "irreps_out", "internal_weights",
                     "shared_weights", "weight_numel"):
            setattr(paths, name, getattr(tp, name))
        paths.irreps_in1 = Irreps(str(paths.irreps_in1))
        paths.irreps_in2 = Irreps(str(paths.irreps_in2))
        paths.irreps_out = Irreps(str(paths.irreps_out))
        paths.instructions = [Instruction(*tuple(i)) for i in tp.instructions]
        weight = getattr(tp, "weight", None)
        paths.dtype = weight.dtype if isinstance(weight, torch.Tensor) else torch.get_default_dtype()
        return paths


class TensorProductConfig(torch.nn.Module):
    """Normalised paths plus the optional registered shared weight.

    ``src/lunatp/utils/layout.py:409-438``: internal weights are a Parameter of
    ``randn(weight_numel)``; otherwise ``weight`` is an empty buffer whose dtype
    records the configuration's dtype.
    """

    def __init__(self, irreps_in1, irreps_in2, irreps_out, instructions, *,
                 in1_var=None, in2_var=None, out_var=None,
                 irrep_normalization=None, path_normalization=None,
                 internal_weights=None, shared_weights=None):
        super().__init__()
        paths = TensorProductPaths(
            irreps_in1, irreps_in2, irreps_out, instructions,
            in1_var=in1_var, in2_var=in2_var, out_var=out_var,
            irrep_normalization=irrep_normalization, path_normalization=path_normalization,
            internal_weights=internal_weights, shared_weights=shared_weights,
        )
        for name in ("irreps_in1", "irreps_in2", "irreps_out", "instructions",
                     "internal_weights", "shared_weights", "weight_numel"):
            setattr(self, name, getattr(paths, name))
        if self.internal_weights and self.weight_numel > 0:
            self.weight = torch.nn.Parameter(torch.randn(self.weight_numel))
        else:
            self.register_buffer("weight", torch.Tensor())


__all__ = ["Instruction", "TensorProductPaths", "TensorProductConfig"]
