"""In-tree build of the C-ABI library and warm-up of the kernel cache.

``build_library`` compiles ``csrc/*.cpp`` with hipcc for gfx950 into
``liblunaeq_amd.so`` next to this file.  ``precompile`` emits and compiles
(hipRTC, gfx950) the kernels of the given configurations into the on-disk
code-object cache, so a GPU host loads them without compiling.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCES = ["common.cpp", "uvu_schedule.cpp", "uvu_emit.cpp", "uvu_runtime.cpp", "uvw.cpp", "graph.cpp", "uuu.cpp", "uvu_noalloc.hip", "placement.hip"]
HIP_FLAGS = [
    "--offload-arch=gfx950", "-O2", "-fPIC", "-shared", "-std=c++17", "-Wno-format-security",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build_library(verbose: bool = False) -> Path:
    hipcc = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
    target = PACKAGE_DIR / "liblunaeq_amd.so"
    tmp = target.with_suffix(f".so.tmp{os.getpid()}")
    command = [hipcc, *HIP_FLAGS, *[str(PACKAGE_DIR / "csrc" / s) for s in SOURCES],
               "-lhiprtc", "-o", str(tmp)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + result.stdout + result.stderr)
    if verbose:
        print(" ".join(command))
    os.replace(tmp, target)
    return target


def standard_operators():
    """Operators of the benchmark and test configurations (fp32 and fp64)."""
    import torch

    from .layout import TensorProductConfig
    from .uvu_conv import create_uvu_conv_operator
    from .irreps import Irreps

    def all_paths(a, b, c):
        a, b, c = Irreps(a), Irreps(b), Irreps(c)
        return [(i, j, k, "uvu", True) for i, (_, x) in enumerate(a) for j, (_, y) in enumerate(b)
                for k, (_, z) in enumerate(c) if z in x * y]

    def mace(channels):
        in1 = "+".join(f"{channels}x{l}{'e' if l % 2 == 0 else 'o'}" for l in range(4))
        sh = "1x0e+1x1o+1x2e+1x3o"
        outs, instructions = [], []
        a, b = Irreps(in1), Irreps(sh)
        for i, (mul, ir1) in enumerate(a):
            for j, (_, ir2) in enumerate(b):
                for ir3 in ir1 * ir2:
                    if ir3.l <= 3:
                        instructions.append((i, j, len(outs), "uvu", True))
                        outs.append(f"{mul}x{ir3}")
        return in1, sh, "+".join(outs), instructions

    configs = [
        ("32x1o", "1x1o", "32x0e", [(0, 0, 0, "uvu", True)]),
        ("32x0e+32x1o", "1x0e+1x1o", "32x0e+32x1o", all_paths("32x0e+32x1o", "1x0e+1x1o", "32x0e+32x1o")),
        mace(128),
        mace(64),
    ]
    ops = []
    for in1, in2, out, instructions in configs:
        tp = TensorProductConfig(in1, in2, out, instructions, internal_weights=False, shared_weights=False)
        for dtype in (torch.float32, torch.float64):
            ops.append(create_uvu_conv_operator(tp, dtype=dtype))
    return ops


def uvw_operators():
    """The shared-weight UVW layer of config 5 (fp32)."""
    from .irreps import Irreps
    from .layout import TensorProductPaths
    from .uvw import LunaTPUVW

    ir, sh = "64x0e+64x1o+64x2e", "1x0e+1x1o+1x2e"
    a, b = Irreps(ir), Irreps(sh)
    instructions = [(i, j, k, "uvw", True) for i, (_, x) in enumerate(a) for j, (_, y) in enumerate(b)
                    for k, (_, z) in enumerate(a) if z in x * y]
    paths = TensorProductPaths(ir, sh, ir, instructions, shared_weights=True, internal_weights=False)
    return [LunaTPUVW(paths)]


def uuu_operators():
    """UUU convolutions of the benchmark (64 channels per degree, lmax 2-4, fp32)
    and of the reference's standard test problem (fp32 and fp64)."""
    import torch

    from .irreps import Irreps
    from .layout import TensorProductConfig
    from .uuu_conv import create_uuu_conv_operator

    def config(ir):
        a = Irreps(ir)
        paths = [(i, j, k, "uuu", True) for i, (_, x) in enumerate(a) for j, (_, y) in enumerate(a)
                 for k, (_, z) in enumerate(a) if z in x * y]
        return TensorProductConfig(ir, ir, ir, paths, internal_weights=False, shared_weights=False)

    ops = []
    for lmax in (2, 3, 4):
        ir = "+".join(f"64x{l}{'e' if l % 2 == 0 else 'o'}" for l in range(lmax + 1))
        ops.append(create_uuu_conv_operator(config(ir), dtype=torch.float32))
    for dtype in (torch.float32, torch.float64):
        ops.append(create_uuu_conv_operator(config("32x0e+32x1o"), dtype=dtype))
    return ops


def precompile() -> int:
    from . import _native

    _native.check(_native.lib().luna_graph_precompile(_native.cache_dir().encode()), "luna_graph_precompile")
    count = 1
    for op in standard_operators() + uvw_operators() + uuu_operators():
        op.plan.precompile()
        count += 1
    return count


if __name__ == "__main__":
    build_library(verbose=True)
    print("precompiled", precompile(), "operators")
