"""The C-ABI library: exported symbols, plans, errors and emitted code (no GPU)."""

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest
import torch

from lunaequivariance_amd import _native
from lunaequivariance_amd.uvu_conv import NativePlan, create_uvu_conv_operator
from lunaequivariance_amd.workloads import mace_irreps

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lunaeq_amd.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(luna_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_native.LIBRARY_PATH))
    names = declared_functions()
    assert "luna_uvu_conv_fwd" in names and "luna_uvu_conv_bwd" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_native.PROTOTYPES), "ctypes prototypes and header differ"


def test_version_and_device_count_without_gpu():
    lib = _native.lib()
    assert b"gfx950" in lib.luna_version()
    assert lib.luna_device_count() >= 0


def op_for(channels=8, lmax=2, dtype=torch.float32):
    from lunaequivariance_amd import TensorProductConfig

    in1, sh, out, instructions = mace_irreps(channels, lmax)
    tp = TensorProductConfig(in1, sh, out, instructions, internal_weights=False, shared_weights=False)
    return create_uvu_conv_operator(tp, dtype=dtype)


def test_plan_info_matches_metadata():
    op = op_for()
    info = op.plan.info
    assert (info.in1_dim, info.in2_dim, info.out_dim, info.weight_numel) == (
        op.in1_dim, op.in2_dim, op.out_dim, op.weight_numel)
    assert info.num_paths == len(op.generated_specs)
    assert info.dtype_bits == 32
    assert info.fwd_needs_zero == 0 and info.num_fwd_launches == 1


@pytest.mark.parametrize("text,message", [
    ("nonsense", "LUNAUVU1"),
    ("LUNAUVU1 16 4 4 4 4 1 0\n0 0 0 0 1 4 1 1 1 -1 0", "dtype"),
    ("LUNAUVU1 32 4 1 4 4 1 0\n0 0 0 0 1 8 1 1 1 -1 0", "in1_dim"),
    ("LUNAUVU1 32 4 1 4 4 1 0\n0 0 0 0 1 4 1 1 1 -1 1 0 0 3 1.0", "coefficient index"),
    ("LUNAUVU1 32 4 1 4 4 1 0\n0 0 0 0 1 0 1 1 1 -1 0", "positive channels"),
])
def test_bad_specs_are_rejected(text, message):
    with pytest.raises(RuntimeError, match=message):
        NativePlan(text)


def test_workspace_size():
    op = op_for()
    size = ctypes.c_size_t()
    _native.check(_native.lib().luna_uvu_conv_bwd_workspace(op.plan.handle, 10, 100, ctypes.byref(size)),
                  "workspace")
    parts = op.plan.info.gy_parts * 100 * (op.in2_dim + 1) * 4
    msgs = 100 * op.in1_dim * 4
    round_up = lambda n: (n + 255) // 256 * 256
    assert size.value == round_up(parts) + round_up(msgs)


def test_launch_argument_errors():
    """Argument checks fail before any device work (safe with or without a GPU)."""
    lib = _native.lib()
    op = op_for()
    with pytest.raises(RuntimeError, match="null plan"):
        _native.check(lib.luna_uvu_conv_fwd(None, None, None, None, None, None, None, None, None, None, 5, 5, None),
                      "fwd")
    with pytest.raises(RuntimeError, match="negative"):
        _native.check(lib.luna_uvu_conv_fwd(op.plan.handle, None, None, None, None, None, None, None, None, None,
                                            -1, 5, None), "fwd")
    with pytest.raises(RuntimeError, match="null tensor"):
        _native.check(lib.luna_uvu_conv_fwd(op.plan.handle, None, None, None, None, None, None, None, None, None,
                                            4, 0, None), "fwd")
    with pytest.raises(RuntimeError, match="null"):
        _native.check(lib.luna_uvu_conv_bwd(op.plan.handle, *([None] * 15), None, 0, 4, 4, None), "bwd")


def test_precompile_emits_gfx950_code_without_packed_fp32(tmp_path, monkeypatch):
    """hipRTC compiles the emitted kernels here (no GPU needed); the code objects
    contain no packed-FP32 instructions."""
    monkeypatch.setenv("LUNAEQ_AMD_CACHE", str(tmp_path))
    for dtype in (torch.float32, torch.float64):
        op = op_for(dtype=dtype)
        op.plan.precompile()
    objects = sorted(tmp_path.glob("*.co"))
    assert len(objects) == 4
    objdump = shutil.which("llvm-objdump") or "/opt/rocm/llvm/bin/llvm-objdump"
    if not Path(objdump).exists():
        pytest.skip("llvm-objdump not available")
    for path in objects:
        text = subprocess.run([objdump, "-d", "--mcpu=gfx950", str(path)], capture_output=True, text=True).stdout
        assert "luna_uvu_" in text
        assert not re.search(r"\bv_pk_(fma|mul|add)_f32\b", text), path.name


def test_product_path_has_no_cpu_fallback():
    """The forward on CPU tensors raises instead of computing on the host."""
    from lunaequivariance_amd import TensorProductConv, make_graph

    in1, sh, out, instructions = mace_irreps(4, 1)
    conv = TensorProductConv(in1, sh, out, instructions, internal_weights=False, shared_weights=False)
    graph = make_graph(torch.tensor([0, 1]), torch.tensor([0, 1]), 2)
    x = torch.randn(2, conv.irreps_in1.dim)
    with pytest.raises(RuntimeError, match="GPU"):
        conv(x, torch.randn(2, conv.irreps_in2.dim), torch.randn(2, conv.weight_numel), graph=graph)


def test_fp64_backward_splits_large_groups():
    """fp64 backward groups holding more than 24 output seeds run as two path
    subsets that add their gy partials in LDS into one slot per channel chunk;
    fp32 keeps one wave per group and chunk, and the two chunk waves of a group
    share one partial slot (they add their partials in LDS)."""
    # lmax=3, 128 channels: input blocks l=0..3 hold 16, 39, 51, 50 seeds.
    f32 = op_for(channels=128, lmax=3, dtype=torch.float32).plan.info
    f64 = op_for(channels=128, lmax=3, dtype=torch.float64).plan.info
    assert f32.gy_parts == 4
    assert f64.gy_parts == 1 + 3 * 2


def test_graph_entry_points_check_arguments():
    """The graph builder's argument checks fail before any device work."""
    lib = _native.lib()
    size = ctypes.c_size_t()
    _native.check(lib.luna_graph_workspace(20000, 1047038, ctypes.byref(size)), "workspace")
    assert size.value > 20000 * 4
    with pytest.raises(RuntimeError, match="negative"):
        _native.check(lib.luna_graph_workspace(-1, 5, ctypes.byref(size)), "workspace")
    with pytest.raises(RuntimeError, match="int32"):
        _native.check(lib.luna_graph_workspace(1 << 31, 5, ctypes.byref(size)), "workspace")
    with pytest.raises(RuntimeError, match="index_bits"):
        _native.check(lib.luna_graph_bounds(None, None, 16, 0, None, None), "bounds")
    with pytest.raises(RuntimeError, match="null"):
        _native.check(lib.luna_graph_bounds(None, None, 32, 4, None, None), "bounds")
    with pytest.raises(RuntimeError, match="null table"):
        _native.check(lib.luna_graph_build(None, None, 32, 4, 0, *([None] * 15), 0, None), "build")
