"""GPU parity of the matrix-core UVW tensor product against the fp64 oracle.

Tolerance: max abs error <= 1e-5 * max|ref| + 1e-7 (fp32), for the forward
and each derivative order.
"""

import pytest
import torch

import lunaequivariance_amd as lunaeq
from oracle.uvw import uvw_tensor_product
from tests.test_oracle_uvw import uvw_instructions
from tests.test_uvu_conv_gpu import assert_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("in1,in2,out,rows", [
    ("64x0e+64x1o+64x2e", "1x0e+1x1o+1x2e", "64x0e+64x1o+64x2e", 100),     # config 5 layer
    ("8x0e+8x1o", "1x0e+1x1o", "8x0e+8x1o+8x1e", 33),                       # narrow, padded tiles
    ("96x0e+16x1o", "1x0e+2x1o", "48x0e+40x1o+8x2e", 70),                   # K > 64, mul2 = 2, odd mul3
    ("32x0e+32x1o", "1x0e+1x1o", "48x0e+50x1o+8x2e", 70),                   # LDS-copied, 64-wide and narrow units
    ("64x0e+32x1o", "2x0e+1x1o", "64x0e+64x1o", 50),                        # mul2 = 2 with 32-w seed chunks
    ("16x0e+16x1o", "1x0e+1x1o", "64x0e+64x1o+16x2e", 45),                  # two LDS-copied chunks per path
    ("64x0e+64x1o+64x2e", "1x0e+1x1o+1x2e", "64x0e+64x1o+64x2e", 600),     # config 5 layer, 3 weight chunks
    ("256x0e+256x2e", "1x0e+1x1o+1x2e", "256x0e+256x2e", 300),              # LDS-copy union over paths
    ("192x0e+192x3o", "1x0e+1x3o", "192x0e+192x3o", 260),                   # wide degree-3 blocks
])
def test_uvw_forward_and_two_orders(in1, in2, out, rows):
    instructions = uvw_instructions(in1, in2, out)
    tp = lunaeq.TensorProduct(in1, in2, out, instructions, shared_weights=True, internal_weights=False)
    gen = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, tp.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(rows, tp.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn(tp.weight_numel, generator=gen, dtype=torch.float64) / 8
    ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
    ref = uvw_tensor_product(in1, in2, out, instructions, *ref_in)
    dev_in = [t.to(DEV, torch.float32).requires_grad_() for t in (x, y, w)]
    act = tp(*dev_in[:2], dev_in[2])
    assert_close(act, ref, torch.float32, "forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    ref_first = torch.autograd.grad(ref, ref_in, g, create_graph=True)
    dev_first = torch.autograd.grad(act, dev_in, g.to(DEV, torch.float32), create_graph=True)
    for n, (a, r) in enumerate(zip(dev_first, ref_first)):
        assert_close(a, r, torch.float32, f"first-order {n}")
    dirs = [torch.randn(r.shape, generator=gen, dtype=torch.float64) for r in ref_first]
    ref_second = torch.autograd.grad(ref_first, ref_in, dirs)
    dev_second = torch.autograd.grad(dev_first, dev_in, [d.to(DEV, torch.float32) for d in dirs])
    for n, (a, r) in enumerate(zip(dev_second, ref_second)):
        assert_close(a, r, torch.float32, f"second-order {n}")


def test_uvw_internal_weights_and_functional_api():
    ir, sh = "16x0e+16x1o", "1x0e+1x1o"
    instructions = uvw_instructions(ir, sh, ir)
    tp = lunaeq.TensorProduct(ir, sh, ir, instructions, shared_weights=True, internal_weights=True).to(DEV)
    x = torch.randn(40, tp.irreps_in1.dim, device=DEV)
    y = torch.randn(40, tp.irreps_in2.dim, device=DEV)
    out = tp(x, y)
    ref = uvw_tensor_product(ir, sh, ir, instructions, x.double().cpu(), y.double().cpu(),
                             tp.weight.detach().double().cpu())
    assert_close(out, ref, torch.float32, "internal weights")
    op = lunaeq.prepare_tensor_product(ir, sh, ir, instructions, shared_weights=True)
    again = lunaeq.tensor_product(x, y, tp.weight.detach(), config=op)
    assert_close(again, ref, torch.float32, "functional")
    out.sum().backward()
    assert tp.weight.grad is not None and tp.weight.grad.shape == (tp.weight_numel,)


@pytest.mark.parametrize("dtype,shared", [(torch.float64, True), (torch.float32, False), (torch.float64, False)])
def test_uvw_rows_fp64_and_per_row_weights(dtype, shared):
    """fp64 and per-row weights run the row form of the UVW convolution (identity graph)."""
    from oracle.uvu_conv import conv as oracle_conv

    in1, in2, out, rows = "12x0e+8x1o", "1x0e+2x1o", "8x0e+12x1o+4x2e", 37
    instructions = uvw_instructions(in1, in2, out)
    tp = lunaeq.TensorProduct(in1, in2, out, instructions, shared_weights=shared, internal_weights=False,
                              dtype=dtype)
    assert tp.op.rows_op is not None
    gen = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, tp.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(rows, tp.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn((tp.weight_numel,) if shared else (rows, tp.weight_numel), generator=gen, dtype=torch.float64)
    ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
    ids = torch.arange(rows)
    ref = oracle_conv(in1, in2, out, instructions, ref_in[0], ref_in[1],
                      ref_in[2].expand(rows, -1) if shared else ref_in[2], ids, ids, rows)
    if shared:
        assert torch.allclose(ref, uvw_tensor_product(in1, in2, out, instructions, x, y, w), atol=1e-12)
    dev_in = [t.to(DEV, dtype).requires_grad_() for t in (x, y, w)]
    act = tp(*dev_in)
    assert_close(act, ref, dtype, "forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    ref_first = torch.autograd.grad(ref, ref_in, g, create_graph=True)
    dev_first = torch.autograd.grad(act, dev_in, g.to(DEV, dtype), create_graph=True)
    for n, (a, r) in enumerate(zip(dev_first, ref_first)):
        assert_close(a, r, dtype, f"first-order {n}")
    dirs = [torch.randn(r.shape, generator=gen, dtype=torch.float64) for r in ref_first]
    ref_second = torch.autograd.grad(ref_first, ref_in, dirs, allow_unused=True)
    dev_second = torch.autograd.grad(dev_first, dev_in, [d.to(DEV, dtype) for d in dirs], allow_unused=True)
    for n, (a, r) in enumerate(zip(dev_second, ref_second)):
        if r is None:
            assert a is None or not a.count_nonzero()
            continue
        assert_close(torch.zeros_like(r) if a is None else a, r, dtype, f"second-order {n}")


def test_uvw_module_dtype_switch():
    ir, sh = "8x0e+8x1o", "1x0e+1x1o"
    instructions = uvw_instructions(ir, sh, ir)
    tp = lunaeq.TensorProduct(ir, sh, ir, instructions, shared_weights=True, internal_weights=True).to(DEV)
    assert tp.op.rows_op is None
    tp.double()
    assert tp.op.compute_dtype == torch.float64 and tp.op.rows_op is not None
    x = torch.randn(20, tp.irreps_in1.dim, device=DEV, dtype=torch.float64)
    y = torch.randn(20, tp.irreps_in2.dim, device=DEV, dtype=torch.float64)
    ref = uvw_tensor_product(ir, sh, ir, instructions, x.cpu(), y.cpu(), tp.weight.detach().cpu())
    assert_close(tp(x, y), ref, torch.float64, "fp64 after .double()")


@pytest.mark.parametrize("rows", [0, 1, 45])
def test_uvw_degree3_and_tiny_batches(rows):
    """Output blocks of degree 3 (seven components: 32-channel tiles) beside 64-wide
    units, on an empty batch, a single row and a ragged one."""
    in1, in2, out = "64x0e+32x1o", "1x0e+1x1o+1x2e", "64x0e+64x1o+32x3o"
    instructions = uvw_instructions(in1, in2, out)
    tp = lunaeq.TensorProduct(in1, in2, out, instructions, shared_weights=True, internal_weights=False)
    gen = torch.Generator().manual_seed(7 + rows)
    x = torch.randn(rows, tp.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(rows, tp.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn(tp.weight_numel, generator=gen, dtype=torch.float64) / 8
    ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
    ref = uvw_tensor_product(in1, in2, out, instructions, *ref_in)
    dev_in = [t.to(DEV, torch.float32).requires_grad_() for t in (x, y, w)]
    act = tp(*dev_in)
    assert act.shape == (rows, tp.irreps_out.dim)
    assert_close(act, ref, torch.float32, "forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    ref_first = torch.autograd.grad(ref, ref_in, g)
    dev_first = torch.autograd.grad(act, dev_in, g.to(DEV, torch.float32))
    for n, (a, r) in enumerate(zip(dev_first, ref_first)):
        assert a.shape == r.shape
        assert_close(a, r, torch.float32, f"first-order {n}")


def test_uvw_wide_blocks():
    """128- and 64-channel blocks with degree-3 components: large LDS-copied rows
    in the weight gradient next to 32-channel forward tiles."""
    in1, in2, out = "128x0e+64x3o", "1x0e+1x3o", "128x0e+64x3o"
    instructions = uvw_instructions(in1, in2, out)
    tp = lunaeq.TensorProduct(in1, in2, out, instructions, shared_weights=True, internal_weights=False)
    rows = 300
    gen = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, tp.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(rows, tp.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn(tp.weight_numel, generator=gen, dtype=torch.float64) / 16
    ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
    ref = uvw_tensor_product(in1, in2, out, instructions, *ref_in)
    dev_in = [t.to(DEV, torch.float32).requires_grad_() for t in (x, y, w)]
    act = tp(*dev_in)
    assert_close(act, ref, torch.float32, "forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    ref_first = torch.autograd.grad(ref, ref_in, g)
    dev_first = torch.autograd.grad(act, dev_in, g.to(DEV, torch.float32))
    for n, (a, r) in enumerate(zip(dev_first, ref_first)):
        assert_close(a, r, torch.float32, f"first-order {n}")


def _random_layouts(count, seed):
    import random

    rnd = random.Random(seed)
    muls = [8, 16, 24, 32, 48, 64, 96, 128]

    def irreps(lmax, pick):
        return "+".join(f"{pick()}x{l}{'e' if l % 2 == 0 else 'o'}" for l in range(lmax + 1))

    out = []
    while len(out) < count:
        a = irreps(rnd.randint(1, 3), lambda: rnd.choice(muls))
        b = irreps(rnd.randint(1, 3), lambda: rnd.choice([1, 1, 2]))
        c = irreps(rnd.randint(1, 3), lambda: rnd.choice(muls))
        if uvw_instructions(a, b, c):
            out.append((a, b, c, rnd.choice([1, 17, 70, 257])))
    return out


@pytest.mark.parametrize("in1,in2,out,rows", _random_layouts(6, 1))
def test_uvw_random_layouts(in1, in2, out, rows):
    """Seeded random layouts (multiplicities 8-128, degrees up to 3, one or two
    edge copies): every kernel variant and launch split against the oracle."""
    instructions = uvw_instructions(in1, in2, out)
    tp = lunaeq.TensorProduct(in1, in2, out, instructions, shared_weights=True, internal_weights=False)
    gen = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, tp.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(rows, tp.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn(tp.weight_numel, generator=gen, dtype=torch.float64) / 8
    ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
    ref = uvw_tensor_product(in1, in2, out, instructions, *ref_in)
    dev_in = [t.to(DEV, torch.float32).requires_grad_() for t in (x, y, w)]
    act = tp(*dev_in)
    assert_close(act, ref, torch.float32, "forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    ref_first = torch.autograd.grad(ref, ref_in, g)
    dev_first = torch.autograd.grad(act, dev_in, g.to(DEV, torch.float32))
    for n, (a, r) in enumerate(zip(dev_first, ref_first)):
        assert_close(a, r, torch.float32, f"first-order {n}")


def test_uvw_graph_capture_replays():
    """Forward and backward (whose weight-gradient half runs on a library stream,
    forked from and joined back to the capturing stream) captured in a HIP graph
    and replayed with new inputs, each replay against eager."""
    ir, sh = "64x0e+64x1o+64x2e", "1x0e+1x1o+1x2e"
    instructions = uvw_instructions(ir, sh, ir)
    tp = lunaeq.TensorProduct(ir, sh, ir, instructions, shared_weights=True, internal_weights=False)
    rows = 600
    gen = torch.Generator().manual_seed(5)
    shapes = [(rows, tp.irreps_in1.dim), (rows, tp.irreps_in2.dim), (tp.weight_numel,), (rows, tp.irreps_out.dim)]
    sx, sy, sw, sg = (torch.randn(s, generator=gen).to(DEV) for s in shapes)
    sx.requires_grad_(), sy.requires_grad_(), sw.requires_grad_()

    def step():
        o = tp(sx, sy, sw)
        return (o, *torch.autograd.grad(o, (sx, sy, sw), sg))

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(side)
    captured = torch.cuda.CUDAGraph()
    with torch.cuda.graph(captured):
        static = step()
    for replay in range(3):
        new = [torch.randn(s, generator=gen).to(DEV) for s in shapes]
        with torch.no_grad():
            for dst, src in zip((sx, sy, sw, sg), new):
                dst.copy_(src)
        captured.replay()
        torch.cuda.synchronize()
        ex, ey, ew = (t.clone().requires_grad_() for t in new[:3])
        eo = tp(ex, ey, ew)
        expected = (eo, *torch.autograd.grad(eo, (ex, ey, ew), new[3]))
        for n, (a, b) in enumerate(zip(static, expected)):
            scale = b.abs().max()
            assert (a - b).abs().max() <= 1e-5 * scale + 1e-6, f"replay {replay}, output {n}"


def test_uvw_row_block_fastest_grid(monkeypatch):
    """The grid order the launches fall back to above 65,535 row blocks (row block
    fastest, LUNAEQ_AMD_UVW_TF=0 forces it here): same results as the oracle."""
    monkeypatch.setenv("LUNAEQ_AMD_UVW_TF", "0")
    ir, sh = "64x0e+64x1o+64x2e", "1x0e+1x1o+1x2e"
    instructions = uvw_instructions(ir, sh, ir)
    tp = lunaeq.TensorProduct(ir, sh, ir, instructions, shared_weights=True, internal_weights=False)
    rows = 600
    gen = torch.Generator().manual_seed(8)
    x = torch.randn(rows, tp.irreps_in1.dim, generator=gen, dtype=torch.float64)
    y = torch.randn(rows, tp.irreps_in2.dim, generator=gen, dtype=torch.float64)
    w = torch.randn(tp.weight_numel, generator=gen, dtype=torch.float64) / 8
    ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
    ref = uvw_tensor_product(ir, sh, ir, instructions, *ref_in)
    dev_in = [t.to(DEV, torch.float32).requires_grad_() for t in (x, y, w)]
    act = tp(*dev_in)
    assert_close(act, ref, torch.float32, "forward")
    g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
    for n, (a, r) in enumerate(zip(torch.autograd.grad(act, dev_in, g.to(DEV, torch.float32)),
                                   torch.autograd.grad(ref, ref_in, g))):
        assert_close(a, r, torch.float32, f"first-order {n}")


@pytest.mark.parametrize("copied", [0, 1])
@pytest.mark.parametrize("in1,in2,out,rows", [
    ("64x0e+64x1o+64x2e", "1x0e+1x1o+1x2e", "64x0e+64x1o+64x2e", 90),      # config 5 layer
    ("96x0e+16x1o", "1x0e+2x1o", "48x0e+40x1o+8x2e", 70),                   # K > 64: two rounds of K tiles
    ("16x0e+16x1o", "1x0e+1x1o", "64x0e+64x1o+16x2e", 45),                  # several chunks per path
    ("64x0e+64x1o+64x2e+64x3o", "1x0e+1x1o+1x2e+1x3o", "64x0e+64x1o+64x2e+64x3o", 40),
])
def test_uvw_gx_gy_staging_modes(monkeypatch, copied, in1, in2, out, rows):
    """gx and gy with the seed and weight chunks copied straight to LDS one chunk
    ahead (LUNAEQ_AMD_UVW_BDMA=1) and staged through registers (0), whichever the
    layout would pick by itself: both against the oracle."""
    import lunaequivariance_amd.interface as itf
    monkeypatch.setenv("LUNAEQ_AMD_UVW_BDMA", str(copied))
    itf._cached.cache_clear()
    try:
        instructions = uvw_instructions(in1, in2, out)
        tp = lunaeq.TensorProduct(in1, in2, out, instructions, shared_weights=True, internal_weights=False)
        gen = torch.Generator().manual_seed(rows + copied)
        x = torch.randn(rows, tp.irreps_in1.dim, generator=gen, dtype=torch.float64)
        y = torch.randn(rows, tp.irreps_in2.dim, generator=gen, dtype=torch.float64)
        w = torch.randn(tp.weight_numel, generator=gen, dtype=torch.float64) / 8
        ref_in = [t.clone().requires_grad_() for t in (x, y, w)]
        ref = uvw_tensor_product(in1, in2, out, instructions, *ref_in)
        dev_in = [t.to(DEV, torch.float32).requires_grad_() for t in (x, y, w)]
        act = tp(*dev_in)
        g = torch.randn(ref.shape, generator=gen, dtype=torch.float64)
        for n, (a, r) in enumerate(zip(torch.autograd.grad(act, dev_in[:2], g.to(DEV, torch.float32)),
                                       torch.autograd.grad(ref, ref_in[:2], g))):
            assert_close(a, r, torch.float32, f"{'gx' if n == 0 else 'gy'}, copied={copied}")
    finally:
        itf._cached.cache_clear()
