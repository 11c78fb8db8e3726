"""eg_split_bf16x6 + eg_gemm_bf16x6 (the PLE projections' GEMM with fp32
accuracy on the bf16 matrix cores: three bf16 planes an operand, six plane
products) against float64 products of the same fp32 operands.

The split: hi = rne(x), mid = rne(x - hi), lo = rne(x - hi - mid) as torch's
own bf16 rounding gives them, and hi + mid + lo = x exactly for fp32 values of
any 24-bit mantissa.  The GEMM, three bars:
* random data held to the fp32 GEMM's own worst-case bound,
  |C - C64| <= (k + 2) 2^-24 (|A| |B|^T);
* single products (A and B permutations with full 24-bit mantissas and
  power-of-two scales, so every output is one a*b): within 8 2^-24 |a b| of
  the exact product.  The six passes' products (hi*hi, mid*hi, hi*mid,
  mid*mid, lo*hi, hi*lo) are all larger than that on such data (mid*mid, the
  smallest, ~2^-18 |a b|), so a missing or doubled pass fails it, as does a
  plane read in the wrong place; gemm_x3 on the same data (16 mantissa bits)
  is off by ~2^-17;
* the shapes of the other GEMM tests: partial tiles, two K segments (two
  launches), two column groups, accumulation, the last round's K ranges and
  equal K pieces on a ragged shape (one launch over both plane sets)."""
from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _full_mantissa(shape, g, dev, e_lo=-6, e_hi=6):
    """fp32 values with all 24 significand bits random."""
    mant = torch.randint(1 << 23, 1 << 24, shape, generator=g, device=dev).double()
    sign = torch.randint(0, 2, shape, generator=g, device=dev).double() * 2 - 1
    expo = torch.randint(e_lo, e_hi, shape, generator=g, device=dev).double()
    return (sign * mant * 2.0 ** (expo - 23)).float()


def _check_f32_bound(got, k, a, b, a2=None, b2=None, base=None):
    a64, b64 = a.double(), b.double()
    exp = a64 @ b64.T
    bound = a64.abs() @ b64.abs().T
    if a2 is not None:
        exp += a2.double() @ b2.double().T
        bound += a2.double().abs() @ b2.double().abs().T
    if base is not None:
        exp += base.double()
        bound += base.double().abs()
    torch.cuda.synchronize()
    err = (got.double() - exp).abs()
    tol = (k + 2) * 2.0 ** -24
    worst = float((err / (bound + 1e-30)).max())
    assert bool((err <= tol * bound + 1e-30).all()), f"max err / bound {worst:.3e} > {tol:.3e}"
    return worst


def test_split_three_planes_exact(cuda):
    from engraft_ngram_amd.ple import SplitPlanes
    _say("eg_split_bf16x6 planes")
    g = torch.Generator(device=cuda).manual_seed(61)
    x = _full_mantissa((37, 100), g, cuda, -30, 30)
    x[0, :4] = torch.tensor([0.0, -0.0, 1.0, -3.0], device=cuda)
    p = SplitPlanes(x, three=True)
    assert p.kp == 128 and p.lo2 is not None
    hi, mid, lo = (t[:, :100].float() for t in (p.hi, p.lo, p.lo2))
    assert torch.equal(hi, x.bfloat16().float())
    assert torch.equal(mid, (x - hi).bfloat16().float())
    assert torch.equal(lo, (x - hi - mid).bfloat16().float())
    assert torch.equal(hi.double() + mid.double() + lo.double(), x.double())
    for t in (p.hi, p.lo, p.lo2):
        assert not bool(t[:, 100:].float().any()), "padding must be zero"
    # the first two planes are eg_split_bf16's
    p2 = SplitPlanes(x)
    assert torch.equal(p2.hi, p.hi) and torch.equal(p2.lo, p.lo) and p2.lo2 is None


@pytest.mark.parametrize("m,n,k", [(96, 160, 256), (300, 136, 512)])
def test_gemm_x6_single_products(cuda, m, n, k):
    """C[i, j] = a_i b_j 2^(e_i + f_j) where A's row i and B's row j share
    their one nonzero column, else 0."""
    from engraft_ngram_amd.ple import gemm_x3, gemm_x6
    _say(f"gemm_x6 single products m={m} n={n} k={k}")
    g = torch.Generator(device=cuda).manual_seed(m + n + k)
    cols_a = torch.randperm(k, generator=g, device=cuda)[:m]
    cols_b = torch.cat([cols_a[torch.randperm(m, generator=g, device=cuda)[:n // 2]],
                        torch.randperm(k, generator=g, device=cuda)[:n - n // 2]])
    va, vb = _full_mantissa((m,), g, cuda), _full_mantissa((n,), g, cuda)
    a = torch.zeros((m, k), device=cuda)
    b = torch.zeros((n, k), device=cuda)
    a[torch.arange(m, device=cuda), cols_a] = va
    b[torch.arange(n, device=cuda), cols_b] = vb
    exact = a.double() @ b.double().T
    mag = exact.abs()
    got = gemm_x6(a, b)
    torch.cuda.synchronize()
    assert bool(((got.double() - exact).abs() <= 8 * 2.0 ** -24 * mag).all())
    assert bool((got[mag == 0] == 0).all())
    hits = mag > 0
    assert int(hits.sum()) >= n // 2
    # the same data through gemm_x3 (16 mantissa bits an operand) is off by
    # far more: the bar above separates the two
    x3 = gemm_x3(a, b)
    torch.cuda.synchronize()
    rel3 = float(((x3.double() - exact).abs()[hits] / mag[hits]).max())
    assert rel3 > 64 * 2.0 ** -24, rel3


@pytest.mark.parametrize("m,n,k", [(1, 4, 4), (7, 64, 12), (130, 200, 68), (257, 129, 100), (64, 2560, 2560)])
def test_gemm_x6_against_float64(cuda, m, n, k):
    from engraft_ngram_amd.ple import gemm_x6
    _say(f"gemm_x6 m={m} n={n} k={k}")
    g = torch.Generator(device=cuda).manual_seed(m * 1000 + n + k)
    a = torch.randn(m, k, generator=g, device=cuda)
    b = torch.randn(n, k, generator=g, device=cuda) * 0.03
    _check_f32_bound(gemm_x6(a, b), (k + 31) // 32 * 32, a, b)


def test_gemm_x6_segments_groups_accumulate(cuda):
    """Two K segments, two column groups, accumulation into a given C, and
    the weights' planes kept between calls (cache_b)."""
    from engraft_ngram_amd.ple import gemm_x6
    _say("gemm_x6 two segments, two column groups, accumulate")
    g = torch.Generator(device=cuda).manual_seed(71)
    m, n, n2, k1, k2 = 200, 300, 96, 160, 96
    a1 = torch.randn(m, k1, generator=g, device=cuda)
    a2 = torch.randn(m, k2, generator=g, device=cuda)
    b1 = torch.randn(n, k1, generator=g, device=cuda) * 0.05
    b2 = torch.randn(n, k2, generator=g, device=cuda) * 0.05
    c1 = torch.randn(n2, k1, generator=g, device=cuda) * 0.05
    c2 = torch.randn(n2, k2, generator=g, device=cuda) * 0.05
    base = torch.randn(m, n, generator=g, device=cuda)
    base2 = torch.randn(m, n2, generator=g, device=cuda)
    out, out2 = base.clone(), base2.clone()
    gemm_x6(a1, b1, a2, b2, out=out, accumulate=True, cache_b=True, b_n2=c1, b2_n2=c2, out2=out2)
    _check_f32_bound(out, k1 + k2, a1, b1, a2, b2, base=base)
    _check_f32_bound(out2, k1 + k2, a1, c1, a2, c2, base=base2)
    again = gemm_x6(a1, b1, a2, b2, cache_b=True)
    torch.cuda.synchronize()
    assert torch.equal(again, gemm_x6(a1, b1, a2, b2))


@pytest.mark.parametrize("k_slices", [None, 5])
def test_gemm_x6_last_round_ranges(cuda, k_slices):
    """A ragged shape whose last round of tiles the library cuts into K ranges
    (or, with k_slices, every tile into equal K pieces).  One K segment: the
    hi / mid and hi / lo plane sets run as the two segments of one launch, so
    ranges and pieces cross from one plane set to the other."""
    from engraft_ngram_amd.ple import gemm_x6
    _say(f"gemm_x6 last round in K ranges, ragged, k_slices={k_slices}")
    g = torch.Generator(device=cuda).manual_seed(81)
    m, n, k = 1000, 18400, 3200
    a = torch.randn(m, k, generator=g, device=cuda)
    b = torch.randn(n, k, generator=g, device=cuda) * 0.05
    got = gemm_x6(a, b, k_slices=k_slices)
    _check_f32_bound(got, k, a, b)
    torch.cuda.synchronize()
    assert torch.equal(got, gemm_x6(a, b, k_slices=k_slices))


def test_gemm_x6_needs_three_planes(cuda):
    from engraft_ngram_amd.ple import SplitPlanes, gemm_x6
    a = torch.randn(8, 32, device=cuda)
    with pytest.raises(ValueError, match="three"):
        gemm_x6(SplitPlanes(a), a)
