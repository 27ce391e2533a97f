"""Host-side API: configuration, metadata lowering and argument errors (no GPU)."""

import math

import pytest
import torch

import lunaequivariance_amd as lunaeq
from lunaequivariance_amd.uvu_conv import build_uvu_conv_metadata, l0_feature_layout
from tests.conftest import all_uvu_instructions


def config(in1="4x0e+4x1o", in2="1x0e+1x1o", out="4x0e+4x1o", instructions=None, **kw):
    instructions = instructions or all_uvu_instructions(in1, in2, out)
    kw.setdefault("internal_weights", False)
    kw.setdefault("shared_weights", False)
    return lunaeq.TensorProductConfig(in1, in2, out, instructions, **kw)


def test_irreps_parsing_and_layout():
    irreps = lunaeq.Irreps("32x0e + 32x1o+1x2e")
    assert irreps.dim == 32 + 96 + 5
    assert [s.start for s in irreps.slices()] == [0, 32, 128]
    assert str(irreps) == "32x0e+32x1o+1x2e"
    assert lunaeq.Irrep("3y") == lunaeq.Irrep(3, -1)
    assert list(lunaeq.Irrep("1o") * lunaeq.Irrep("1o")) == [lunaeq.Irrep(l, 1) for l in range(3)]
    with pytest.raises(ValueError):
        lunaeq.Irreps("3xq")


def test_metadata_lowering_offsets_and_terms():
    tp = config("2x0e+2x1o", "2x0e+1x1o", "2x0e+2x1o",
                [(0, 0, 0, "uvu", True), (1, 1, 0, "uvu", True), (1, 0, 1, "uvu", True)])
    meta = build_uvu_conv_metadata(tp, torch.float64)
    specs = meta["generated_specs"]
    # instruction 0 has two edge channels -> two specs with weight stride 2
    assert [s["weight_offset"] for s in specs] == [0, 1, 4, 6, 7]
    assert [s.get("weight_stride", 1) for s in specs] == [2, 2, 1, 2, 2]
    assert [s["y_offset"] for s in specs] == [0, 1, 2, 0, 1]
    assert [s["x_offset"] for s in specs] == [0, 0, 2, 2, 2]
    assert meta["weight_numel"] == tp.weight_numel == 4 + 2 + 4
    # 1o x 1o -> 0e: c = delta / sqrt(3) times the path weight
    pw = tp.instructions[1].path_weight
    terms = specs[2]["terms"]
    assert [(i, j, k) for i, j, k, _ in terms] == [(0, 0, 0), (1, 1, 0), (2, 2, 0)]
    assert terms[0][3] == pytest.approx(pw / math.sqrt(3))


def test_l0_layout_groups_edge_copies():
    tp = config("2x0e+2x1o", "2x0e+1x1o", "2x0e+2x1o",
                [(0, 0, 0, "uvu", True), (1, 1, 0, "uvu", True), (1, 0, 1, "uvu", True)])
    specs = build_uvu_conv_metadata(tp)["generated_specs"]
    offsets, width = l0_feature_layout(specs)
    assert offsets == {0: 0, 1: 0, 2: 2}
    assert width == 4


def test_uvu_requirements():
    with pytest.raises(ValueError, match="internal_weights"):
        build_uvu_conv_metadata(config(internal_weights=True, shared_weights=True))
    with pytest.raises(ValueError, match="shared_weights"):
        build_uvu_conv_metadata(config(shared_weights=True))
    bad = config("4x0e", "1x0e", "2x0e", [(0, 0, 0, "uvu", True)])
    with pytest.raises(ValueError, match="multiplicities"):
        build_uvu_conv_metadata(bad)


def test_module_constructors_and_errors():
    tp = config()
    conv = lunaeq.TensorProductConv(tp)
    assert conv.mode == "uvu_conv" and conv.weight_numel == tp.weight_numel
    direct = lunaeq.TensorProductConv("4x0e+4x1o", "1x0e+1x1o", "4x0e+4x1o",
                                      all_uvu_instructions("4x0e+4x1o", "1x0e+1x1o", "4x0e+4x1o"),
                                      internal_weights=False, shared_weights=False, dtype=torch.float64)
    assert direct.op.compute_dtype == torch.float64
    assert direct.op.spec == lunaeq.TensorProductConv(tp, dtype=torch.float64).op.spec
    with pytest.raises(TypeError):
        lunaeq.TensorProductConv(tp, "1x0e")
    with pytest.raises(TypeError):
        lunaeq.TensorProductConv("4x0e")
    with pytest.raises(ValueError, match="mode"):
        lunaeq.TensorProductConv(tp, mode="uuu")
    meta = build_uvu_conv_metadata(tp)
    with pytest.raises(ValueError, match="mode"):
        lunaeq.TensorProductConv(meta)
    from_meta = lunaeq.TensorProductConv(meta, mode="uvu")
    assert from_meta.weight_numel == tp.weight_numel


def test_module_dtype_conversion_rebuilds_operator():
    conv = lunaeq.TensorProductConv(config())
    assert conv.op.compute_dtype == torch.float32
    conv.double()
    assert conv.op.compute_dtype == torch.float64
    conv.float()
    assert conv.op.compute_dtype == torch.float32


def test_prepare_tensor_product():
    in1, in2 = "4x0e+4x1o", "1x0e+1x1o"
    instructions = all_uvu_instructions(in1, in2, in1)
    op = lunaeq.prepare_tensor_product(in1, in2, in1, instructions, convolution=True)
    assert op.mode == "uvu_conv" and op.compute_dtype == torch.float32
    op64 = lunaeq.prepare_tensor_product(in1, in2, in1, instructions, convolution=True, dtype=torch.float64)
    assert op64.compute_dtype == torch.float64
    with pytest.raises(ValueError, match="mode"):
        lunaeq.prepare_tensor_product(in1, in2, in1, instructions, convolution=True, mode="uvw")
    with pytest.raises(TypeError):
        lunaeq.prepare_tensor_product(in1, in2, convolution=True)
    meta = build_uvu_conv_metadata(config())
    assert lunaeq.prepare_tensor_product(meta, convolution=True, mode="uvu").mode == "uvu_conv"
    with pytest.raises(ValueError):
        lunaeq.prepare_tensor_product(meta, convolution=False, mode="uvu")


def test_schedule_collisions_and_phases():
    """Merged outputs (several paths into one block) need a zeroed output and
    accumulation; one output block per path does not."""
    in1, sh = "8x0e+8x1o+8x2e", "1x0e+1x1o+1x2e"
    merged = lunaeq.TensorProductConv(in1, sh, "8x0e+8x1o+8x2e+8x1e+8x2o",
                                      all_uvu_instructions(in1, sh, "8x0e+8x1o+8x2e+8x1e+8x2o"),
                                      internal_weights=False, shared_weights=False)
    assert merged.op.plan.info.fwd_needs_zero == 1
    assert merged.op.plan.info.num_fwd_launches >= 2
    from lunaequivariance_amd.workloads import mace_irreps

    a, b, c, i = mace_irreps(8, 2)
    separate = lunaeq.TensorProductConv(a, b, c, i, internal_weights=False, shared_weights=False)
    assert separate.op.plan.info.fwd_needs_zero == 0
    assert separate.op.plan.info.num_fwd_launches == 1
