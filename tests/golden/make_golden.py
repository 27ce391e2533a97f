"""Writes the golden fixtures of the UVU, UUU and UVW convolutions from the CPU oracle.

Run from the repository root: ``python tests/golden/make_golden.py [names...]``
(all fixtures, or only the named uuu/uvw ones).
Each ``.npz`` holds the problem (irreps, instructions, graph, inputs) and
fp64 outputs: the forward, first-order gradients for a seed ``g`` and
second-order derivatives of ``<gx,rx> + <gy,ry> + <gw,rw>`` for directions
(rx, ry, rw).  Inputs are small enough that the files stay under 1 MB.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle.uvu_conv import parse_irreps, uvu_conv  # noqa: E402


def all_paths(in1, in2, out):
    a, b, c = parse_irreps(in1), parse_irreps(in2), parse_irreps(out)
    result = []
    for i, (_, l1, p1) in enumerate(a):
        for j, (_, l2, p2) in enumerate(b):
            for k, (_, l3, p3) in enumerate(c):
                if abs(l1 - l2) <= l3 <= l1 + l2 and p1 * p2 == p3:
                    result.append((i, j, k, "uvu", True))
    return result


def weight_numel(in1, in2, instructions, out=None):
    """Weights per edge: mul1*mul2 per uvu path, mul1 per weighted uuu path, mul1*mul2*mul3 per uvw path."""
    a, b = parse_irreps(in1), parse_irreps(in2)
    c = parse_irreps(out) if out is not None else None
    total = 0
    for i, j, k, mode, has_w, *_ in instructions:
        if mode == "uvu":
            total += a[i][0] * b[j][0]
        elif mode == "uuu":
            total += a[i][0] if has_w else 0
        else:
            total += a[i][0] * b[j][0] * c[k][0]
    return total


def make_case(name, in1, in2, out, instructions, nodes, src, dst, seed, env=False):
    gen = torch.Generator().manual_seed(seed)
    dims = [sum(m * (2 * l + 1) for m, l, _ in parse_irreps(t)) for t in (in1, in2, out)]
    E = len(src)
    x = torch.randn(nodes, dims[0], generator=gen, dtype=torch.float64)
    y = torch.randn(E, dims[1], generator=gen, dtype=torch.float64)
    w = torch.randn(E, weight_numel(in1, in2, instructions, out), generator=gen, dtype=torch.float64)
    e = torch.rand(E, generator=gen, dtype=torch.float64) if env else None
    g = torch.randn(nodes, dims[2], generator=gen, dtype=torch.float64)
    rx, ry, rw = (torch.randn(t.shape, generator=gen, dtype=torch.float64) for t in (x, y, w))
    leaves = [t.clone().requires_grad_() for t in (x, y, w)]
    out_t = uvu_conv(in1, in2, out, instructions, *leaves, src, dst, nodes, env=e)
    gx, gy, gw = torch.autograd.grad(out_t, leaves, g, create_graph=True)
    second = torch.autograd.grad((gx, gy, gw), leaves, (rx, ry, rw))
    arrays = dict(x=x, y=y, w=w, g=g, rx=rx, ry=ry, rw=rw, out=out_t.detach(), gx=gx.detach(),
                  gy=gy.detach(), gw=gw.detach(), hx=second[0], hy=second[1], hw=second[2])
    if e is not None:
        arrays["env"] = e
    meta = dict(in1=in1, in2=in2, out=out, instructions=[list(i) for i in instructions], nodes=nodes)
    np.savez_compressed(
        ROOT / "tests" / "golden" / f"{name}.npz",
        meta=np.array(json.dumps(meta)),
        src=np.asarray(src, dtype=np.int64), dst=np.asarray(dst, dtype=np.int64),
        **{k: v.numpy() for k, v in arrays.items()},
    )


def main(only=None):
    if only:
        return extra_cases(only)
    # The reference's standard problem shape (tests/conftest.py:8-70): 7 nodes, 19 edges.
    gen = torch.Generator().manual_seed(731)
    src = torch.randint(7, (19,), generator=gen)
    dst = torch.sort(torch.randint(7, (19,), generator=gen))[0]
    in1, in2 = "32x0e+32x1o", "1x0e+1x1o"
    make_case("reference_problem", in1, in2, in1, all_paths(in1, in2, in1), 7, src, dst, 731)
    # Config 1 at 1/32 scale: 31 atoms, 16 edges each.
    gen = torch.Generator().manual_seed(0)
    nodes = 31
    src = torch.randint(nodes, (nodes * 16,), generator=gen)
    dst = torch.arange(nodes).repeat_interleave(16)
    make_case("config1_small", "32x1o", "1x1o", "32x0e", [(0, 0, 0, "uvu", True)], nodes, src, dst, 1)
    # Edge multiplicity > 1, repeated instructions, summed outputs and an envelope
    # (tests/lunatp/test_uvu_conv.py:378-452 shape).
    src = torch.tensor([1, 0, 1, 2, 0, 1, 2, 0, 1])
    dst = torch.tensor([0, 0, 0, 1, 1, 1, 2, 2, 2])
    instructions = [(0, 0, 0, "uvu", True), (0, 0, 0, "uvu", True), (1, 1, 0, "uvu", True),
                    (0, 1, 1, "uvu", True), (1, 0, 1, "uvu", True)]
    make_case("multi_edge_env", "33x0e+33x1o+1x2e", "2x0e+3x1o+1x2e", "33x0e+33x1o+1x2e", instructions, 5, src,
              dst, 2, env=True)
    # lmax = 3, every uvu path, one output block per path (the config 2 layer at 4 channels).
    parity = lambda l: "e" if l % 2 == 0 else "o"
    in1 = "+".join(f"4x{l}{parity(l)}" for l in range(4))
    sh = "+".join(f"1x{l}{parity(l)}" for l in range(4))
    outs, instructions = [], []
    for i, (m1, l1, p1) in enumerate(parse_irreps(in1)):
        for j, (_, l2, p2) in enumerate(parse_irreps(sh)):
            for l3 in range(abs(l1 - l2), min(l1 + l2, 3) + 1):
                instructions.append((i, j, len(outs), "uvu", True))
                outs.append(f"{m1}x{l3}{'e' if p1 * p2 == 1 else 'o'}")
    gen = torch.Generator().manual_seed(3)
    src = torch.randint(12, (60,), generator=gen)
    dst = torch.sort(torch.randint(12, (60,), generator=gen))[0]
    make_case("lmax3_paths", in1, sh, "+".join(outs), instructions, 12, src, dst, 3)
    extra_cases(None)


def extra_cases(only):
    """The uuu and uvw convolutions on the reference's standard problem shape."""
    gen = torch.Generator().manual_seed(731)
    src = torch.randint(7, (19,), generator=gen)
    dst = torch.sort(torch.randint(7, (19,), generator=gen))[0]
    ir = "32x0e+32x1o"
    if not only or "uuu_reference" in only:
        a = parse_irreps(ir)
        uuu = [(i, j, k, "uuu", n != 1) for n, (i, j, k) in enumerate(
            (i, j, k) for i, (_, l1, p1) in enumerate(a) for j, (_, l2, p2) in enumerate(a)
            for k, (_, l3, p3) in enumerate(a) if abs(l1 - l2) <= l3 <= l1 + l2 and p1 * p2 == p3)]
        make_case("uuu_reference", ir, ir, ir, uuu, 7, src, dst, 733, env=True)
    if not only or "uvw_reference" in only:
        sh, narrow = "1x0e+1x1o", "16x0e+16x1o"  # 16 channels keep the per-edge uvw weights small
        uvw = [(i, j, k, "uvw", True) for i, j, k, *_ in all_paths(narrow, sh, narrow)]
        make_case("uvw_reference", narrow, sh, narrow, uvw, 7, src, dst, 734, env=True)


if __name__ == "__main__":
    main(sys.argv[1:] or None)
