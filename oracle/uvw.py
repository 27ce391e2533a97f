"""Dense fp64 restatement of the shared-weight UVW tensor product (oracle).

e3nn's ``connection_mode="uvw"`` as lowered by the reference
(``src/lunatp/uvw/kernels/utils.py:100-190``): per instruction with path
weight ``pw``, ``out[b, io][w, k] += pw * sum_{u v i j} C_ijk W[u, v, w]
x[b, i1][u, i] y[b, i2][v, j]``, W the instruction's slice of the shared
weight in ``[u, v, w]`` order.  TEST INFRASTRUCTURE ONLY.
"""

from __future__ import annotations

import math

import torch

from .uvu_conv import offsets, parse_irreps
from .wigner import wigner_3j


def uvw_path_weights(in1, in2, out, instructions):
    """component + element normalisation: (2 l_out + 1) / sum(mul1 * mul2) over paths into the output."""
    weights = []
    for i1, i2, io, *_ in instructions:
        fan = sum(in1[a][0] * in2[b][0] for a, b, o, *_ in instructions if o == io)
        weights.append(math.sqrt((2 * out[io][1] + 1) / fan))
    return weights


def uvw_tensor_product(irreps_in1, irreps_in2, irreps_out, instructions, x, y, weight):
    in1, in2, out = parse_irreps(irreps_in1), parse_irreps(irreps_in2), parse_irreps(irreps_out)
    x_off, _ = offsets(in1)
    y_off, _ = offsets(in2)
    o_off, out_dim = offsets(out)
    B = x.shape[0]
    result = x.new_zeros((B, out_dim))
    w_off = 0
    for (i1, i2, io, *_), pw in zip(instructions, uvw_path_weights(in1, in2, out, instructions)):
        m1, l1, _ = in1[i1]
        m2, l2, _ = in2[i2]
        m3, l3, _ = out[io]
        d1, d2, d3 = 2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1
        cg = torch.tensor(wigner_3j(l1, l2, l3), dtype=x.dtype)
        xb = x[:, x_off[i1]: x_off[i1] + m1 * d1].reshape(B, m1, d1)
        yb = y[:, y_off[i2]: y_off[i2] + m2 * d2].reshape(B, m2, d2)
        W = weight[w_off: w_off + m1 * m2 * m3].reshape(m1, m2, m3)
        piece = pw * torch.einsum("ijk,bui,bvj,uvw->bwk", cg, xb, yb, W).reshape(B, m3 * d3)
        result = result + torch.nn.functional.pad(piece, (o_off[io], out_dim - o_off[io] - m3 * d3))
        w_off += m1 * m2 * m3
    return result
