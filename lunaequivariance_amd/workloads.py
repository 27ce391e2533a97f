"""Synthetic workloads of the benchmark configurations (inputs only).

* ``periodic_radius_graph``: atoms uniform in a periodic cube at a given
  density, directed edges i -> j for every pair closer than the cutoff under
  the minimum-image convention (no self loops), sorted by destination.
* ``spherical_harmonics``: e3nn real spherical harmonics with component
  normalisation (``|Y_l|^2 = 2l+1``) of unit edge vectors, l <= 4, in the
  Cartesian form of ``src/o3/spherical_harmonics/kernels/forward.py:21-57``.
* ``mace_irreps``: the lmax-``L`` MACE-style uvu layer of configs 2-4: every
  allowed uvu path, one output block per path.
"""

from __future__ import annotations

import math

import torch

from .irreps import Irreps


def periodic_radius_graph(num_atoms: int, density: float = 0.1, cutoff: float = 5.0, *,
                          seed: int = 0, device="cpu", chunk: int = 2048):
    """(src, dst, positions, edge_vectors, box) with edges sorted by dst (stable)."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    box = (num_atoms / density) ** (1.0 / 3.0)
    pos = (torch.rand(num_atoms, 3, generator=gen, dtype=torch.float64) * box).to(device)
    srcs, dsts = [], []
    for start in range(0, num_atoms, chunk):
        block = pos[start:start + chunk]
        delta = pos[None, :, :] - block[:, None, :]          # [b, N, 3]: pos[src] - pos[dst]
        delta -= box * torch.round(delta / box)
        dist2 = (delta * delta).sum(-1)
        dst_local, src = torch.nonzero(dist2 < cutoff * cutoff, as_tuple=True)
        dst = dst_local + start
        keep = src != dst
        srcs.append(src[keep])
        dsts.append(dst[keep])
    src = torch.cat(srcs)
    dst = torch.cat(dsts)
    order = torch.argsort(dst, stable=True)
    src, dst = src[order], dst[order]
    vec = pos[src] - pos[dst]
    vec -= box * torch.round(vec / box)
    return src, dst, pos, vec, box


def spherical_harmonics(lmax: int, vectors: torch.Tensor) -> torch.Tensor:
    """[n, (lmax+1)^2] real harmonics of the normalised vectors, degrees 0..lmax <= 4."""
    if lmax > 4:
        raise ValueError("degrees up to 4 are provided")
    v = vectors / vectors.norm(dim=-1, keepdim=True)
    x, y, z = v.unbind(-1)
    s = math.sqrt
    out = [torch.ones_like(x)]
    sh1 = [s(3.0) * x, s(3.0) * y, s(3.0) * z]
    y2, x2z2 = y * y, x * x + z * z
    sh2 = [s(15.0) * x * z, s(15.0) * x * y, s(5.0) * (y2 - 0.5 * x2z2), s(15.0) * y * z,
           0.5 * s(15.0) * (z * z - x * x)]
    rad2 = x2z2 + y2
    sh3 = [s(7.0 / 6.0) * (sh2[0] * z + sh2[4] * x), s(7.0) * y * sh2[0],
           s(35.0 / 8.0) * y * sh2[1] - s(21.0 / 24.0) * rad2 * sh1[0],
           s(35.0 / 9.0) * y * sh2[2] - s(28.0 / 27.0) * rad2 * sh1[1],
           s(35.0 / 8.0) * y * sh2[3] - s(21.0 / 24.0) * rad2 * sh1[2],
           s(7.0) * y * sh2[4], s(7.0 / 6.0) * (sh2[4] * z - sh2[0] * x)]
    sh4 = [s(9.0 / 8.0) * (sh3[0] * z + sh3[6] * x), s(9.0) * y * sh3[0],
           s(63.0 / 12.0) * y * sh3[1] - s(45.0 / 60.0) * rad2 * sh2[0],
           s(63.0 / 15.0) * y * sh3[2] - s(72.0 / 75.0) * rad2 * sh2[1],
           s(63.0 / 16.0) * y * sh3[3] - s(81.0 / 80.0) * rad2 * sh2[2],
           s(63.0 / 15.0) * y * sh3[4] - s(72.0 / 75.0) * rad2 * sh2[3],
           s(63.0 / 12.0) * y * sh3[5] - s(45.0 / 60.0) * rad2 * sh2[4],
           s(9.0) * y * sh3[6], s(9.0 / 8.0) * (sh3[6] * z - sh3[0] * x)]
    degrees = [out, sh1, sh2, sh3, sh4][: lmax + 1]
    return torch.stack([c for d in degrees for c in d], dim=-1)


def mace_irreps(channels: int, lmax: int = 3):
    """(irreps_in1, sh irreps, irreps_out, instructions) with every uvu path up to lmax."""
    parity = lambda l: "e" if l % 2 == 0 else "o"
    in1 = "+".join(f"{channels}x{l}{parity(l)}" for l in range(lmax + 1))
    sh = "+".join(f"1x{l}{parity(l)}" for l in range(lmax + 1))
    outs, instructions = [], []
    for i, (mul, ir1) in enumerate(Irreps(in1)):
        for j, (_, ir2) in enumerate(Irreps(sh)):
            for ir3 in ir1 * ir2:
                if ir3.l <= lmax:
                    instructions.append((i, j, len(outs), "uvu", True))
                    outs.append(f"{mul}x{ir3}")
    return in1, sh, "+".join(outs), instructions


__all__ = ["periodic_radius_graph", "spherical_harmonics", "mace_irreps"]
