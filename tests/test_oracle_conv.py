"""The CPU oracle of the UVU convolution against fixed facts (no GPU)."""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.uvu_conv import brute_force, parse_irreps, path_weights, uvu_conv
from oracle.sh import spherical_harmonics
from tests.conftest import all_uvu_instructions

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_oracle_matches_brute_force(make_problem):
    tp, instructions, x, y, w, src, dst = make_problem()
    in1, in2 = "32x0e+32x1o", "1x0e+1x1o"
    dense = uvu_conv(in1, in2, in1, instructions, x, y, w, src, dst, 7)
    loops = brute_force(in1, in2, in1, instructions, x, y, w, src.numpy(), dst.numpy(), 7)
    assert np.allclose(dense.numpy(), loops, atol=1e-12)


def test_oracle_brute_force_multi_edge():
    in1, in2, out = "3x0e+3x1o+1x2e", "2x0e+3x1o+1x2e", "3x0e+3x1o+1x2e"
    instructions = [(0, 0, 0, "uvu", True), (0, 0, 0, "uvu", True), (1, 1, 0, "uvu", True),
                    (0, 1, 1, "uvu", True), (1, 0, 1, "uvu", True), (2, 2, 2, "uvu", True)]
    gen = torch.Generator().manual_seed(1)
    dims = [sum(m * (2 * l + 1) for m, l, _ in parse_irreps(t)) for t in (in1, in2, out)]
    x = torch.randn(4, dims[0], generator=gen, dtype=torch.float64)
    y = torch.randn(6, dims[1], generator=gen, dtype=torch.float64)
    wn = sum(parse_irreps(in1)[i][0] * parse_irreps(in2)[j][0] for i, j, *_ in instructions)
    w = torch.randn(6, wn, generator=gen, dtype=torch.float64)
    src = torch.tensor([0, 3, 1, 2, 2, 0])
    dst = torch.tensor([0, 0, 1, 1, 3, 3])
    dense = uvu_conv(in1, in2, out, instructions, x, y, w, src, dst, 4)
    loops = brute_force(in1, in2, out, instructions, x, y, w, src.numpy(), dst.numpy(), 4)
    assert np.allclose(dense.numpy(), loops, atol=1e-12)


def test_config1_closed_form():
    """32x1o x 1x1o -> 32x0e: message = w * <x_src, y> / sqrt(3) (examples/basic_uvu_conv.py:33-41)."""
    gen = torch.Generator().manual_seed(0)
    x = torch.randn(10, 96, generator=gen, dtype=torch.float64)
    y = torch.randn(40, 3, generator=gen, dtype=torch.float64)
    w = torch.randn(40, 32, generator=gen, dtype=torch.float64)
    src = torch.randint(10, (40,), generator=gen)
    dst = torch.arange(10).repeat_interleave(4)
    out = uvu_conv("32x1o", "1x1o", "32x0e", [(0, 0, 0, "uvu", True)], x, y, w, src, dst, 10)
    msg = (x[src].reshape(40, 32, 3) * y[:, None, :]).sum(-1) * w / math.sqrt(3)
    assert torch.allclose(out, torch.zeros(10, 32, dtype=torch.float64).index_add(0, dst, msg), atol=1e-13)


def test_path_weights_match_package():
    """The oracle's restated normalisation agrees with the package's."""
    from lunaequivariance_amd import TensorProductConfig

    in1, sh = "8x0e+8x1o+8x2e", "1x0e+1x1o+1x2e"
    out = "8x0e+8x1o+8x2e+8x1e+8x2o"
    instructions = all_uvu_instructions(in1, sh, out)
    for norm in ("element", "path", "none"):
        tp = TensorProductConfig(in1, sh, out, instructions, internal_weights=False, shared_weights=False,
                                 path_normalization=norm)
        expected = path_weights(parse_irreps(in1), parse_irreps(sh), parse_irreps(out), instructions,
                                path_normalization=norm)
        assert [i.path_weight for i in tp.instructions] == pytest.approx(expected, rel=1e-14)


def test_path_weight_values():
    """component + element normalisation: alpha = (2 l_out + 1) / (number of paths into
    the output times mul_in2); each path into 8x1o from 1x1o, 1x0e, 1x2e gets sqrt(3/3) = 1."""
    in1, sh, out = "8x0e+8x1o+8x2e", "1x0e+1x1o+1x2e", "8x1o"
    instructions = all_uvu_instructions(in1, sh, out)
    weights = path_weights(parse_irreps(in1), parse_irreps(sh), parse_irreps(out), instructions)
    n = len(instructions)
    assert weights == pytest.approx([math.sqrt(3 / n)] * n)


def test_oracle_gradcheck_and_gradgradcheck():
    in1, in2 = "2x0e+2x1o", "1x0e+1x1o"
    instructions = all_uvu_instructions(in1, in2, in1)
    gen = torch.Generator().manual_seed(5)
    x = torch.randn(3, 8, generator=gen, dtype=torch.float64, requires_grad=True)
    y = torch.randn(5, 4, generator=gen, dtype=torch.float64, requires_grad=True)
    w = torch.randn(5, 2 * len(instructions), generator=gen, dtype=torch.float64, requires_grad=True)
    src, dst = torch.tensor([0, 2, 1, 1, 0]), torch.tensor([0, 0, 1, 2, 2])
    fn = lambda a, b, c: uvu_conv(in1, in2, in1, instructions, a, b, c, src, dst, 3)
    assert torch.autograd.gradcheck(fn, (x, y, w))
    assert torch.autograd.gradgradcheck(fn, (x, y, w))


def rotation(seed):
    rng = np.random.default_rng(seed)
    q, r = np.linalg.qr(rng.normal(size=(3, 3)))
    q = q @ np.diag(np.sign(np.diag(r)))
    return q if np.linalg.det(q) > 0 else -q


def block_diag_d(irreps, R, rng):
    """Block-diagonal D(R) for an irreps string; parity only matters for reflections."""
    v = rng.normal(size=(300, 3))
    A = spherical_harmonics(4, v)
    B = spherical_harmonics(4, v @ R.T)
    blocks = []
    for mul, l, _ in parse_irreps(irreps):
        D, *_ = np.linalg.lstsq(A[l], B[l], rcond=None)
        blocks += [D.T] * mul
    size = sum(b.shape[0] for b in blocks)
    out = np.zeros((size, size))
    at = 0
    for b in blocks:
        out[at:at + len(b), at:at + len(b)] = b
        at += len(b)
    return torch.tensor(out)


def test_oracle_equivariance(make_problem):
    """Rotating inputs rotates outputs (tests/lunatp/test_uvu_conv.py:149-164 recipe)."""
    tp, instructions, x, y, w, src, dst = make_problem()
    in1, in2 = "32x0e+32x1o", "1x0e+1x1o"
    R = rotation(3)
    rng = np.random.default_rng(4)
    D1, D2 = block_diag_d(in1, R, rng), block_diag_d(in2, R, rng)
    out = uvu_conv(in1, in2, in1, instructions, x, y, w, src, dst, 7)
    rotated = uvu_conv(in1, in2, in1, instructions, x @ D1.T, y @ D2.T, w, src, dst, 7)
    assert torch.allclose(rotated, out @ D1.T, atol=1e-10)


def load_golden(name):
    data = np.load(GOLDEN / f"{name}.npz")
    meta = json.loads(str(data["meta"]))
    meta["instructions"] = [tuple(i) for i in meta["instructions"]]
    return meta, {k: torch.tensor(data[k]) for k in data.files if k != "meta"}


@pytest.mark.parametrize("name", ["reference_problem", "config1_small", "multi_edge_env", "lmax3_paths",
                                  "uuu_reference", "uvw_reference"])
def test_golden_fixtures(name):
    """The oracle still reproduces its committed fixtures (forward, first and second order)."""
    meta, t = load_golden(name)
    leaves = [t[k].clone().requires_grad_() for k in ("x", "y", "w")]
    out = uvu_conv(meta["in1"], meta["in2"], meta["out"], meta["instructions"], *leaves, t["src"], t["dst"],
                   meta["nodes"], env=t.get("env"))
    assert torch.allclose(out, t["out"], atol=1e-12)
    first = torch.autograd.grad(out, leaves, t["g"], create_graph=True)
    for a, k in zip(first, ("gx", "gy", "gw")):
        assert torch.allclose(a, t[k], atol=1e-12)
    second = torch.autograd.grad(first, leaves, (t["rx"], t["ry"], t["rw"]))
    for a, k in zip(second, ("hx", "hy", "hw")):
        assert torch.allclose(a, t[k], atol=1e-12)


# Closed forms of layout.py:323-370 with non-unit variances, written out by hand.
# Two uvu paths 0e x 0e -> 0e and 1o x 1o -> 0e, edge multiplicity 2, variances
# in1 = (2, 3), in2 = (5, 7), out = (11):
#   element: x = 2*5*2 + 3*7*2 = 62 for both paths;
#   path:    x = 2*5*2*2 = 40 and 3*7*2*2 = 84 (two paths into the output);
#   none:    x = 1.
# The "norm" irrep normalisation multiplies by d1*d2 = 1 and 9 instead of d3 = 1.
VAR_CASE = dict(in1="3x0e+3x1o", in2="2x0e+2x1o", out="3x0e",
                instructions=[(0, 0, 0, "uvu", True), (1, 1, 0, "uvu", True)],
                variances=dict(in1_var=[2.0, 3.0], in2_var=[5.0, 7.0], out_var=[11.0]))
VAR_EXPECTED = {
    ("component", "element"): [math.sqrt(11 / 62), math.sqrt(11 / 62)],
    ("component", "path"): [math.sqrt(11 / 40), math.sqrt(11 / 84)],
    ("component", "none"): [math.sqrt(11), math.sqrt(11)],
    ("norm", "element"): [math.sqrt(11 / 62), math.sqrt(9 * 11 / 62)],
    ("norm", "path"): [math.sqrt(11 / 40), math.sqrt(9 * 11 / 84)],
    ("none", "none"): [math.sqrt(11), math.sqrt(11)],
}


@pytest.mark.parametrize("irrep_norm,path_norm", sorted(VAR_EXPECTED))
def test_path_weights_with_variances_closed_form(irrep_norm, path_norm):
    c = VAR_CASE
    weights = path_weights(parse_irreps(c["in1"]), parse_irreps(c["in2"]), parse_irreps(c["out"]),
                           c["instructions"], irrep_normalization=irrep_norm, path_normalization=path_norm,
                           **c["variances"])
    assert weights == pytest.approx(VAR_EXPECTED[irrep_norm, path_norm], rel=1e-15)


def test_path_weights_user_weight_and_component_dimension():
    """1o x 0e -> 1o and 1o x 1e -> 1o into 3x1o, edge multiplicity 2, in1 var 2, in2 vars
    (5, 7), out var 4, user path weights 0.5 and 1: element x = 2*5*2 + 2*7*2 = 48, so
    alpha = 3 * 4 / 48 times the user weight."""
    instructions = [(0, 0, 0, "uvu", True, 0.5), (0, 1, 0, "uvu", True, 1.0)]
    weights = path_weights(parse_irreps("3x1o"), parse_irreps("2x0e+2x1e"), parse_irreps("3x1o"), instructions,
                           in1_var=[2.0], in2_var=[5.0, 7.0], out_var=[4.0])
    assert weights == pytest.approx([math.sqrt(0.5 * 12 / 48), math.sqrt(12 / 48)], rel=1e-15)


def test_path_weights_reject_wrong_variance_lengths():
    with pytest.raises(ValueError):
        path_weights(parse_irreps("3x0e"), parse_irreps("1x0e"), parse_irreps("3x0e"), [(0, 0, 0, "uvu", True)],
                     in1_var=[1.0, 2.0])


@pytest.mark.parametrize("irrep_norm,path_norm", sorted(VAR_EXPECTED))
def test_package_normalisation_with_variances_matches_pinned_oracle(irrep_norm, path_norm):
    from lunaequivariance_amd import TensorProductConfig

    c = VAR_CASE
    tp = TensorProductConfig(c["in1"], c["in2"], c["out"], c["instructions"], internal_weights=False,
                             shared_weights=False, irrep_normalization=irrep_norm, path_normalization=path_norm,
                             **c["variances"])
    assert [i.path_weight for i in tp.instructions] == pytest.approx(VAR_EXPECTED[irrep_norm, path_norm],
                                                                     rel=1e-14)


def test_conv_uses_normalisation_arguments():
    """Doubling out_var scales the convolution by sqrt(2); "none"/"none" equals the
    unnormalised brute force times sqrt(out_var)."""
    c = VAR_CASE
    gen = torch.Generator().manual_seed(9)
    x = torch.randn(4, 12, generator=gen, dtype=torch.float64)
    y = torch.randn(6, 8, generator=gen, dtype=torch.float64)
    w = torch.randn(6, 12, generator=gen, dtype=torch.float64)
    src, dst = torch.tensor([0, 1, 3, 2, 2, 0]), torch.tensor([0, 0, 1, 2, 3, 3])
    args = (c["in1"], c["in2"], c["out"], c["instructions"], x, y, w, src, dst, 4)
    base = uvu_conv(*args, normalization=dict(c["variances"]))
    doubled = uvu_conv(*args, normalization=dict(c["variances"], out_var=[22.0]))
    assert torch.allclose(doubled, base * math.sqrt(2), rtol=1e-13, atol=0)
    plain = uvu_conv(*args, normalization=dict(irrep_normalization="none", path_normalization="none"))
    brute = brute_force(*args)
    # brute_force uses the default (component, element) weights: both paths sqrt(1 / (2 + 2)).
    assert torch.allclose(plain * 0.5, torch.as_tensor(brute), rtol=1e-12, atol=1e-13)
