"""HIP adaLN modulation and gated residual against the oracle (MI355X).

The kernels compute in fp32 and round once, so:

* ``adaln_modulate`` is within one unit in the last place (of the output
  dtype) of the fp64 result rounded once (``oracle.norm.adaln_modulate_exact``);
  the only freedom is the fp32 summation order of the row statistics;
* ``gated_residual`` is bit-identical to the fp32 product and fp32 sum
  rounded once (``oracle.norm.gated_residual_fp32``).

Both also pass the reference suite's own comparison against the reference
expression with its per-op roundings (``test/test_ops.py:12-15,33-44``: max
relative error below 2e-2), on the reference's shapes.
"""

from __future__ import annotations

import pytest
import torch

import dexter_amd.ops as ops
from dexter_amd.registry import select_spec
from oracle import norm as onorm

from _util import close_rel

pytestmark = pytest.mark.gpu
DT = torch.bfloat16


def _ulp(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """One unit in the last place of ``dtype`` at each value of ``t`` (fp64)."""
    fi = torch.finfo(dtype)
    mag = t.abs().clamp_min(fi.tiny)
    return torch.exp2(torch.floor(torch.log2(mag))) * fi.eps


def assert_within_one_ulp(got: torch.Tensor, exact: torch.Tensor, terms: torch.Tensor, what=""):
    """``got`` (any float dtype) within one ulp of the fp64 ``exact`` result plus
    the error fp32 arithmetic may make, and equal to ``exact`` rounded once on
    nearly every element.

    ``terms`` bounds the magnitudes the kernel adds up for each element (for
    adaLN ``|normed * gain| + |shift| + |gain|``, the last for the absolute
    error of the fp32 row statistics): fp32 sums and products are within a few
    2^-24 of them, which matters only where the terms cancel to a small result
    or the output itself is f32. The bound allows 2^-18.
    """
    assert got.shape == exact.shape, f"{what}: shape {tuple(got.shape)} != {tuple(exact.shape)}"
    g = got.detach().cpu()
    e = exact.detach().cpu().double()
    assert torch.isfinite(g).all(), f"{what}: non-finite output"
    tol = _ulp(e, g.dtype) + 2.0 ** -18 * terms.detach().cpu().double().expand_as(e)
    bad = (g.double() - e).abs() > tol
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements beyond the bound, worst excess "
                           f"{((g.double() - e).abs() - tol).max().item():.3e}")
    if g.dtype != torch.float32:
        differ = (g != e.to(g.dtype)).float().mean().item()
        assert differ < 0.01, f"{what}: {differ:.2%} of elements not the correctly rounded value"


def _adaln_inputs(shape, mod_shape, dtype=DT, mod_dtype=None, seed=0, device="cuda", scale_mag=1.0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g).to(dtype)
    md = mod_dtype or dtype
    scale = (scale_mag * torch.randn(*mod_shape, generator=g)).to(md)
    shift = torch.randn(*mod_shape, generator=g).to(md)
    return x.to(device), scale.to(device), shift.to(device)


def _check_adaln(x, scale, shift, eps=1e-6, what=""):
    got = ops.adaln_modulate(x, scale, shift, eps)
    xc, sc, sh = x.cpu(), scale.cpu(), shift.cpu()
    exact = onorm.adaln_modulate_exact(xc, sc, sh, eps, out_dtype=torch.float64)
    assert got.dtype == torch.promote_types(torch.promote_types(x.dtype, scale.dtype), shift.dtype)
    zero = torch.zeros((), dtype=torch.float64)
    normed = onorm.adaln_modulate_exact(xc, zero, zero, eps, out_dtype=torch.float64)
    gain = (1 + sc.double()).abs()
    terms = (normed.abs() * gain + sh.double().abs() + gain)
    assert_within_one_ulp(got, exact, terms, what)
    return got


# ------------------------------------------------------------- adaLN -----

def test_adaln_selects_the_hip_kernel(device):
    x, s, b = _adaln_inputs((1, 8, 256), (1, 1, 256))
    assert select_spec("norm", "adaln", x, s, b).name == "hip_adaln_gfx950"
    assert select_spec("norm", "gated_residual", x, x, s).name == "hip_gated_residual_gfx950"


@pytest.mark.parametrize("shape", [(1, 125, 3072), (2, 64, 5120)])
def test_adaln_reference_cases(device, shape):
    """The reference's own test (test/test_ops.py:33-38), plus the one-ulp bar."""
    x, s, b = _adaln_inputs(shape, (shape[0], 1, shape[2]), seed=shape[1])
    got = _check_adaln(x, s, b, what=str(shape))
    close_rel(got, onorm.adaln_modulate(x.cpu(), s.cpu(), b.cpu(), 1e-6))


@pytest.mark.parametrize("case", ["C1", "C2", "14B"])
def test_adaln_workload_sizes(device, case):
    """The activations around attention at the bench's shapes: C1 (83 tokens of
    Wan-5B), C2 (the 8,192-token prefill) and the Wan-14B chunk (913 x 5120)."""
    shape = {"C1": (1, 83, 3072), "C2": (1, 8192, 3072), "14B": (1, 913, 5120)}[case]
    x, s, b = _adaln_inputs(shape, (1, 1, shape[2]), seed=7)
    _check_adaln(x, s, b, what=case)


@pytest.mark.parametrize("mod", ["full", "batch_row", "vector", "single_row", "unbind_view"])
def test_adaln_modulation_broadcasts(device, mod):
    b_, l_, c_ = 3, 17, 1024
    g = torch.Generator().manual_seed(3)
    x = torch.randn(b_, l_, c_, generator=g).to(DT).to(device)
    if mod == "unbind_view":
        # The Wan block: (modulation + e).unsqueeze(2).unbind(1) gives [B, 1, C]
        # views with batch stride 6C (models/dreamzero/model.py:266-267).
        m = torch.randn(b_, 6, 1, c_, generator=g).to(DT).to(device)
        parts = m.unbind(dim=1)
        s, sh = parts[1], parts[0]
        assert not s.is_contiguous()
    else:
        mshape = {"full": (b_, l_, c_), "batch_row": (b_, 1, c_), "vector": (c_,),
                  "single_row": (1, 1, c_)}[mod]
        s = torch.randn(*mshape, generator=g).to(DT).to(device)
        sh = torch.randn(*mshape, generator=g).to(DT).to(device)
    _check_adaln(x, s, sh, what=mod)


@pytest.mark.parametrize("xdt,mdt", [
    (torch.float16, torch.float16), (torch.float32, torch.float32),
    (torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16),
    (torch.bfloat16, torch.float16), (torch.float16, torch.float32),
])
def test_adaln_dtypes_and_promotion(device, xdt, mdt):
    x, s, b = _adaln_inputs((2, 33, 768), (2, 1, 768), dtype=xdt, mod_dtype=mdt, seed=5)
    _check_adaln(x, s, b, what=f"{xdt}/{mdt}")


@pytest.mark.parametrize("cols", [1, 7, 8, 64, 100, 1001, 4104, 16384, 32768])
def test_adaln_row_widths(device, cols):
    """Ragged widths take the element-wise variant; 32768 bf16 columns use 16 waves."""
    x, s, b = _adaln_inputs((1, 5, cols), (1, 1, cols), seed=cols)
    if cols == 1:
        # A one-column LayerNorm is 0; the output is shift.
        got = ops.adaln_modulate(x, s, b)
        assert torch.equal(got, b.expand_as(got))
        return
    _check_adaln(x, s, b, what=f"C={cols}")


def test_adaln_strided_and_misaligned_rows(device):
    g = torch.Generator().manual_seed(11)
    big = torch.randn(2, 9, 1536, generator=g).to(DT).to(device)
    s = torch.randn(2, 1, 1024, generator=g).to(DT).to(device)
    b = torch.randn(2, 1, 1024, generator=g).to(DT).to(device)
    x = big[:, :, 256:1280]  # row stride 1536, 16-byte aligned: the vector path
    _check_adaln(x, s, b, what="strided")
    x = big[:, :, 3:1027]    # 6-byte offset: the element-wise path
    _check_adaln(x, s, b, what="misaligned")
    flat = torch.randn(1 + 4 * 512, generator=g).to(DT).to(device)
    x = flat[1:].view(1, 4, 512)
    _check_adaln(x, s[:1, :, :512], b[:1, :, :512], what="offset base")


def test_adaln_edge_rows(device):
    c = 512
    x = torch.full((1, 4, c), 0.5, dtype=DT, device=device)  # constant rows: normed = 0
    s = torch.randn(1, 1, c, dtype=DT, device=device)
    b = torch.randn(1, 1, c, dtype=DT, device=device)
    assert torch.equal(ops.adaln_modulate(x, s, b), b.expand(1, 4, c))
    # Outliers (x20, as in the ragged-batch config) and large eps.
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 40, c, generator=g)
    x[torch.rand(x.shape, generator=g) < 0.01] *= 20
    x = x.to(DT).to(device)
    _check_adaln(x, s, b, eps=1e-6, what="outliers")
    _check_adaln(x, s, b, eps=0.5, what="eps 0.5")


def test_adaln_empty_and_4d(device):
    x = torch.empty(2, 0, 256, dtype=DT, device=device)
    s = torch.randn(2, 1, 256, dtype=DT, device=device)
    assert ops.adaln_modulate(x, s, s).shape == (2, 0, 256)
    x, s, b = _adaln_inputs((2, 3, 5, 256), (2, 1, 1, 256), seed=4)
    _check_adaln(x, s, b, what="4d")
    x, s, b = _adaln_inputs((7, 256), (256,), seed=6)
    _check_adaln(x, s, b, what="2d")


def test_adaln_broadcast_over_batch_of_x(device):
    """x [1, L, C] against [B, 1, C] modulation gives [B, L, C], as torch broadcasting does."""
    x, _, _ = _adaln_inputs((1, 6, 512), (1, 1, 512), seed=12)
    _, s, b = _adaln_inputs((1, 6, 512), (3, 1, 512), seed=13)
    got = _check_adaln(x, s, b, what="x broadcast")
    assert got.shape == (3, 6, 512)


# --------------------------------------------------------- gated residual -----

def _check_gated(x, y, gate, what=""):
    got = ops.gated_residual(x, y, gate)
    ref = onorm.gated_residual_fp32(x.cpu(), y.cpu(), gate.cpu())
    assert got.dtype == ref.dtype and got.shape == ref.shape, what
    assert torch.equal(got.cpu(), ref), (
        f"{what}: {int((got.cpu() != ref).sum())} elements differ from the fp32 form")
    return got


def test_gated_residual_reference_case(device):
    """The reference's own test (test/test_ops.py:41-45): bit-exact to the
    single-rounding form, and within the suite's tolerance of the reference."""
    g = torch.Generator().manual_seed(1)
    x = torch.randn(1, 125, 3072, generator=g).to(DT).to(device)
    y = torch.randn(1, 125, 3072, generator=g).to(DT).to(device)
    gate = torch.randn(1, 1, 3072, generator=g).to(DT).to(device)
    got = _check_gated(x, y, gate, "reference case")
    close_rel(got, onorm.gated_residual(x.cpu(), y.cpu(), gate.cpu()))


@pytest.mark.parametrize("case", ["C1", "C2", "14B"])
def test_gated_residual_workload_sizes(device, case):
    shape = {"C1": (1, 83, 3072), "C2": (1, 8192, 3072), "14B": (1, 913, 5120)}[case]
    g = torch.Generator().manual_seed(2)
    x = torch.randn(*shape, generator=g).to(DT).to(device)
    y = torch.randn(*shape, generator=g).to(DT).to(device)
    gate = torch.randn(1, 1, shape[2], generator=g).to(DT).to(device)
    _check_gated(x, y, gate, case)


@pytest.mark.parametrize("xdt,gdt", [
    (torch.float16, torch.float16), (torch.float32, torch.float32),
    (torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16), (torch.bfloat16, torch.float16),
])
def test_gated_residual_dtypes(device, xdt, gdt):
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 21, 640, generator=g).to(xdt).to(device)
    y = torch.randn(2, 21, 640, generator=g).to(xdt).to(device)
    gate = torch.randn(2, 1, 640, generator=g).to(gdt).to(device)
    _check_gated(x, y, gate, f"{xdt}/{gdt}")


@pytest.mark.parametrize("form", ["full", "vector", "unbind_view", "ragged", "misaligned",
                                  "mixed_xy"])
def test_gated_residual_shapes(device, form):
    g = torch.Generator().manual_seed(4)
    b_, l_, c_ = 2, 19, 1001 if form == "ragged" else 1024
    x = torch.randn(b_, l_, c_, generator=g).to(DT).to(device)
    y = torch.randn(b_, l_, c_, generator=g).to(DT).to(device)
    if form == "full":
        gate = torch.randn(b_, l_, c_, generator=g).to(DT).to(device)
    elif form == "vector":
        gate = torch.randn(c_, generator=g).to(DT).to(device)
    elif form == "unbind_view":
        gate = torch.randn(b_, 6, 1, c_, generator=g).to(DT).to(device).unbind(1)[2]
    elif form == "misaligned":
        big = torch.randn(b_, l_, c_ + 5, generator=g).to(DT).to(device)
        x = big[:, :, 5:]
        gate = torch.randn(b_, 1, c_, generator=g).to(DT).to(device)
    elif form == "mixed_xy":
        y = y.float()
        gate = torch.randn(b_, 1, c_, generator=g).to(DT).to(device)
    else:
        gate = torch.randn(b_, 1, c_, generator=g).to(DT).to(device)
    _check_gated(x, y, gate, form)


def test_gated_residual_closed_forms_on_device(device):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 33, 512, generator=g).to(DT).to(device)
    y = torch.randn(1, 33, 512, generator=g).to(DT).to(device)
    zero = torch.zeros(1, 1, 512, dtype=DT, device=device)
    assert torch.equal(ops.gated_residual(x, y, zero), x)
    one = torch.ones(1, 1, 512, dtype=DT, device=device)
    assert torch.equal(ops.gated_residual(x, y, one), x + y)
    assert ops.gated_residual(x[:, :0], y[:, :0], one).shape == (1, 0, 512)


def test_block_pair_in_a_graph_replays_like_eager(device):
    """adaLN -> (stand-in for attention) -> gated residual, captured once and
    replayed several times with eager work between replays; every replay
    equals the eager result bit for bit."""
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 83, 3072, generator=g).to(DT).to(device)
    mod = torch.randn(1, 6, 1, 3072, generator=g).to(DT).to(device)
    shift1, scale1, gate1 = mod.unbind(1)[:3]

    def block():
        h = ops.adaln_modulate(x, scale1, shift1, 1e-6)
        return ops.gated_residual(x, h, gate1)

    eager = block()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        block()  # warm the allocator on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = block()
    for i in range(4):
        x.add_(0)  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
