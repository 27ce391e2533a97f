"""Dense fp64 restatement of the reference's oracle for the UVU and UUU convolutions.

The reference checks its kernels against e3nn's ``o3.TensorProduct`` applied
to ``x[src]`` followed by ``index_add`` over ``dst``
(``src/utils/testing.py:12-70``, ``tests/lunatp/test_uvu_conv.py:37-41``), with
the operation documented in ``docs/operators/tensor_product_conv.md``
("Equivalent e3nn computation").  For a uvu instruction ``(i1, i2, io)`` with
normalised path weight ``pw`` (``src/lunatp/utils/layout.py:323-370``) and edge
multiplicity ``m2``:

    msg[e, io][u, k] = pw * sum_{v, i, j} C[i, j, k] x[src_e, i1][u, i]
                                          y[e, i2][v, j] w[e, off + u*m2 + v]
    out[n] = sum_{e: dst_e = n} env_e * msg[e]

For a uvw instruction every input pair (u, v) feeds every output channel w,
``msg[e, io][w, k] = pw * sum C[i, j, k] x[src_e, i1][u, i] y[e, i2][v, j]
W[e, off + (u*m2 + v)*mo + w]`` (e3nn's weight layout), with W the per-edge
weights or the shared row repeated (the reference's UVW conv tests use the same
oracle, ``tests/lunatp/test_uvw_conv.py:33-50``).

For a uuu instruction (``docs/operators/tensor_product.md:100-106``; the
reference's UUU conv tests use the same e3nn-then-``index_add`` oracle,
``tests/lunatp/test_uuu_conv.py:30-45``) the channels are matched instead of
mixed, and unweighted paths use weight 1:

    msg[e, io][u, k] = pw * sum_{i, j} C[i, j, k] x[src_e, i1][u, i] y[e, i2][u, j]
                       * (w[e, off + u] if has_weight else 1)

with ``off`` advancing by ``mul`` over weighted uuu instructions only.

The scalar-path features (``src/utils/testing.py:55-70``) are the per-edge
``msg`` columns of instructions whose output has l = 0, before ``env``,
concatenated in output order.  Everything is differentiable torch fp64 code,
so gradients of any order come from autograd.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from .wigner import wigner_3j


def parse_irreps(text: str):
    """[(mul, l, parity)] of an e3nn irreps string."""
    out = []
    for chunk in text.replace(" ", "").split("+"):
        if not chunk:
            continue
        mul, ir = chunk.split("x") if "x" in chunk else ("1", chunk)
        out.append((int(mul), int(ir[:-1]), 1 if ir[-1] == "e" else -1))
    return out


def path_weights(in1, in2, out, instructions, irrep_normalization="component",
                 path_normalization="element", in1_var=None, in2_var=None, out_var=None):
    """sqrt(alpha) per instruction (``layout.py:323-370``).

    alpha = a_irrep / x * out_var[io] * user_weight, with a_irrep = 2 l3 + 1
    ("component"), (2 l1 + 1)(2 l2 + 1) ("norm") or 1 ("none"), and x = the sum
    over the instructions into the same output of in1_var * in2_var * fan
    ("element"), this instruction's in1_var * in2_var * fan times the number of
    instructions into its output ("path"), or 1 ("none"); fan = mul2 (uvu),
    mul1 * mul2 (uvw), 1 (uuu).  Variances default to 1 per irrep block.
    """
    v1 = [1.0] * len(in1) if in1_var is None else [float(v) for v in in1_var]
    v2 = [1.0] * len(in2) if in2_var is None else [float(v) for v in in2_var]
    vo = [1.0] * len(out) if out_var is None else [float(v) for v in out_var]
    if (len(v1), len(v2), len(vo)) != (len(in1), len(in2), len(out)):
        raise ValueError("one variance per irrep block is required")

    def fan(ins):
        mode = ins[3]
        return v1[ins[0]] * v2[ins[1]] * {"uvu": in2[ins[1]][0], "uvw": in1[ins[0]][0] * in2[ins[1]][0],
                                          "uuu": 1}[mode]

    weights = []
    for ins in instructions:
        i1, i2, io, mode, _has_w, *rest = ins
        user = rest[0] if rest else 1.0
        l1, l2, l3 = in1[i1][1], in2[i2][1], out[io][1]
        alpha = {"component": 2 * l3 + 1, "norm": (2 * l1 + 1) * (2 * l2 + 1), "none": 1}[irrep_normalization]
        if path_normalization == "element":
            x = sum(fan(other) for other in instructions if other[2] == io)
        elif path_normalization == "path":
            x = fan(ins) * sum(1 for other in instructions if other[2] == io)
        else:
            x = 1
        if x > 0:
            alpha /= x
        weights.append(math.sqrt(alpha * vo[io] * user))
    return weights


def offsets(irreps):
    out, start = [], 0
    for mul, l, _ in irreps:
        out.append(start)
        start += mul * (2 * l + 1)
    return out, start


def edge_messages(in1, in2, out, instructions, x_src, y, w, weights=None):
    """Per-edge messages [E, out_dim] and the per-instruction output pieces."""
    if weights is None:
        weights = path_weights(in1, in2, out, instructions)
    x_off, _ = offsets(in1)
    y_off, _ = offsets(in2)
    o_off, out_dim = offsets(out)
    E = y.shape[0]
    pieces = []
    w_off = 0
    msg = x_src.new_zeros((E, out_dim))
    for (i1, i2, io, mode, has_w, *_), pw in zip(instructions, weights):
        m1, l1, _ = in1[i1]
        m2, l2, _ = in2[i2]
        mo, l3, _ = out[io]
        d1, d2, d3 = 2 * l1 + 1, 2 * l2 + 1, 2 * l3 + 1
        cg = torch.tensor(wigner_3j(l1, l2, l3), dtype=x_src.dtype)
        xb = x_src[:, x_off[i1]: x_off[i1] + m1 * d1].reshape(E, m1, d1)
        yb = y[:, y_off[i2]: y_off[i2] + m2 * d2].reshape(E, m2, d2)
        if mode == "uvu":
            wb = w[:, w_off: w_off + m1 * m2].reshape(E, m1, m2)
            piece = pw * torch.einsum("ijk,eui,evj,euv->euk", cg, xb, yb, wb).reshape(E, mo * d3)
            w_off += m1 * m2
        elif mode == "uuu":
            if not m1 == m2 == mo:
                raise ValueError("uuu instructions need equal multiplicities")
            wb = w[:, w_off: w_off + m1] if has_w else xb.new_ones((E, m1))
            piece = pw * torch.einsum("ijk,eui,euj,eu->euk", cg, xb, yb, wb).reshape(E, mo * d3)
            w_off += m1 if has_w else 0
        elif mode == "uvw":
            wb = w[:, w_off: w_off + m1 * m2 * mo].reshape(E, m1, m2, mo)
            piece = pw * torch.einsum("ijk,eui,evj,euvw->ewk", cg, xb, yb, wb).reshape(E, mo * d3)
            w_off += m1 * m2 * mo
        else:
            raise ValueError("oracle covers uvu, uuu and uvw instructions")
        pieces.append((io, piece))
        msg = msg + torch.nn.functional.pad(piece, (o_off[io], out_dim - o_off[io] - mo * d3))
    return msg, pieces


def conv(irreps_in1, irreps_in2, irreps_out, instructions, x, y, w, src, dst, num_nodes,
             env=None, return_l0=False, normalization=None):
    """Reference semantics of ``TensorProductConv(...)(x, y, w, graph=..., env=, return_l0_feat=)``
    for uvu or uuu instructions.  ``normalization``: keyword arguments of
    ``path_weights`` (irrep/path normalisation and variances); defaults otherwise."""
    in1, in2, out = parse_irreps(irreps_in1), parse_irreps(irreps_in2), parse_irreps(irreps_out)
    src = torch.as_tensor(src).long()
    dst = torch.as_tensor(dst).long()
    weights = path_weights(in1, in2, out, instructions, **(normalization or {}))
    msg, pieces = edge_messages(in1, in2, out, instructions, x[src], y, w, weights)
    scaled = msg if env is None else msg * env.reshape(-1, 1)
    result = x.new_zeros((num_nodes, msg.shape[1])).index_add(0, dst, scaled)
    if not return_l0:
        return result
    scalars = sorted([(io, piece) for io, piece in pieces if out[io][1] == 0], key=lambda t: t[0])
    l0 = torch.cat([p for _, p in scalars], 1) if scalars else msg[:, :0]
    return result, l0


def brute_force(irreps_in1, irreps_in2, irreps_out, instructions, x, y, w, src, dst, num_nodes):
    """Scalar loop version of ``uvu_conv`` for tiny problems (pins the einsum form)."""
    in1, in2, out = parse_irreps(irreps_in1), parse_irreps(irreps_in2), parse_irreps(irreps_out)
    weights = path_weights(in1, in2, out, instructions)
    x_off, _ = offsets(in1)
    y_off, _ = offsets(in2)
    o_off, out_dim = offsets(out)
    x, y, w = (np.asarray(t, dtype=np.float64) for t in (x, y, w))
    result = np.zeros((num_nodes, out_dim))
    for e in range(len(src)):
        w_off = 0
        for (i1, i2, io, mode, has_w, *_), pw in zip(instructions, weights):
            m1, l1, _ = in1[i1]
            m2, l2, _ = in2[i2]
            _, l3, _ = out[io]
            cg = wigner_3j(l1, l2, l3)
            mo = out[io][0]
            # (u, v, output channel, weight index): uvu keeps u and mixes v;
            # uuu matches u = v; uvw mixes both into every output channel.
            if mode == "uvu":
                quads = [(u, v, u, w_off + u * m2 + v) for u in range(m1) for v in range(m2)]
            elif mode == "uuu":
                quads = [(u, u, u, w_off + u if has_w else None) for u in range(m1)]
            else:
                quads = [(u, v, o, w_off + (u * m2 + v) * mo + o)
                         for u in range(m1) for v in range(m2) for o in range(mo)]
            for u, v, o, windex in quads:
                weight = 1.0 if windex is None else w[e, windex]
                for i in range(2 * l1 + 1):
                    for j in range(2 * l2 + 1):
                        for k in range(2 * l3 + 1):
                            c = cg[i, j, k]
                            if c == 0.0:
                                continue
                            result[dst[e], o_off[io] + o * (2 * l3 + 1) + k] += (
                                pw * c * x[src[e], x_off[i1] + u * (2 * l1 + 1) + i]
                                * y[e, y_off[i2] + v * (2 * l2 + 1) + j] * weight)
            w_off += {"uvu": m1 * m2, "uuu": m1 if has_w else 0, "uvw": m1 * m2 * mo}[mode]
    return result


uvu_conv = conv  # the name the uvu tests and fixtures use
