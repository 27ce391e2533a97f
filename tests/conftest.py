"""Shared fixtures.  Tests marked ``gpu`` need an MI355X (HIP device)."""

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X)")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no HIP GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def all_uvu_instructions(in1, in2, out):
    from lunaequivariance_amd import Irreps

    a, b, c = Irreps(in1), Irreps(in2), Irreps(out)
    return [(i, j, k, "uvu", True) for i, (_, x) in enumerate(a) for j, (_, y) in enumerate(b)
            for k, (_, z) in enumerate(c) if z in x * y]


def mace_irreps(channels, lmax=3):
    """irreps_in1, SH irreps and one output block per allowed uvu path (l <= lmax)."""
    from lunaequivariance_amd import Irreps

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


@pytest.fixture
def make_problem():
    """The reference's standard small problem (``tests/conftest.py:8-70``): seed 731,
    irreps 32x0e+32x1o, edge irreps 1x0e+1x1o, all uvu paths, 7 nodes and 19 edges,
    x and y created transposed (non-contiguous)."""

    def build(dtype=torch.float64, device="cpu"):
        gen = torch.Generator().manual_seed(731)
        in1, in2 = "32x0e+32x1o", "1x0e+1x1o"
        instructions = all_uvu_instructions(in1, in2, in1)
        from lunaequivariance_amd import TensorProductConfig

        tp = TensorProductConfig(in1, in2, in1, instructions, internal_weights=False, shared_weights=False)
        nodes, items = 7, 19
        x = torch.randn(tp.irreps_in1.dim, nodes, generator=gen, dtype=dtype).t()
        y = torch.randn(tp.irreps_in2.dim, items, generator=gen, dtype=dtype).t()
        w = torch.randn(items, tp.weight_numel, generator=gen, dtype=dtype)
        src = torch.randint(nodes, (items,), generator=gen)
        dst = torch.sort(torch.randint(nodes, (items,), generator=gen))[0]
        return tp, instructions, x.to(device), y.to(device), w.to(device), src, dst

    return build
