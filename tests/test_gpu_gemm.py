"""eg_split_bf16 + eg_gemm_bf16x3 (the PLE projections' fp32 GEMM on the
bf16 matrix cores) against float64 products of the same fp32 operands.

Bar, elementwise: |C - C64| <= 2e-5 * (|A| |B|^T) + 1e-30.  The split keeps
16 of fp32's 24 mantissa bits per operand (hi + lo) and drops lo*lo, so each
product is within ~1.2e-5 of its exact value relative to |a b|, and the fp32
accumulation adds ulps of the running sum; a plain bf16 product (a missing lo
term) is off by ~4e-3 of |a b| and a wrong fragment layout by O(1), so either
fails the bar.  Shapes cover partial tiles in m, n and k, k below one
32-wide step, the two-segment form, two column groups, K slices and
accumulation, and the projections' real shape."""
from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _check(got, a, b, a2=None, b2=None, base=None):
    a64, b64 = a.double(), b.double()
    exp = a64 @ b64.T
    bound = a64.abs() @ b64.abs().T
    if a2 is not None:
        exp += a2.double() @ b2.double().T
        bound += a2.double().abs() @ b2.double().abs().T
    if base is not None:
        exp += base.double()
        bound += base.double().abs()
    err = (got.double() - exp).abs()
    worst = float((err / (bound + 1e-30)).max())
    assert bool((err <= 2e-5 * bound + 1e-30).all()), f"max err / bound {worst:.3e}"
    return worst


@pytest.mark.parametrize("m,n,k", [(1, 4, 4), (7, 64, 12), (130, 200, 68), (128, 128, 32), (257, 129, 100),
                                   (64, 2560, 2560)])
def test_gemm_x3_against_float64(cuda, m, n, k):
    from engraft_ngram_amd.ple import gemm_x3
    _say(f"gemm_x3 m={m} n={n} k={k}")
    g = torch.Generator(device=cuda).manual_seed(m * 1000 + n + k)
    a = torch.randn(m, k, generator=g, device=cuda)
    b = torch.randn(n, k, generator=g, device=cuda) * 0.03
    got = gemm_x3(a, b)
    torch.cuda.synchronize()
    _check(got, a, b)


def test_gemm_x3_two_segments_accumulate_and_strides(cuda):
    """d_emb = d_key w_key + d_value w_value as the backward calls it (B = the
    weights' transposes), then accumulated into an existing C; operands that
    are column slices of wider rows (leading dimension > k)."""
    from engraft_ngram_amd import _lib
    from engraft_ngram_amd.ple import gemm_x3
    _say("gemm_x3 two segments, accumulate, strided operands")
    g = torch.Generator(device=cuda).manual_seed(5)
    m, n, k1, k2 = 300, 192, 512, 128
    a1 = torch.randn(m, k1, generator=g, device=cuda)
    b1 = torch.randn(n, k1, generator=g, device=cuda) * 0.05
    a2 = torch.randn(m, k2, generator=g, device=cuda)
    b2 = torch.randn(n, k2, generator=g, device=cuda) * 0.05
    got = gemm_x3(a1, b1, a2, b2)
    _check(got, a1, b1, a2, b2)
    base = torch.randn(m, n, generator=g, device=cuda)
    acc = base.clone()
    gemm_x3(a1, b1, a2, b2, out=acc, accumulate=True)
    _check(acc, a1, b1, a2, b2, base=base)
    # leading dimensions wider than k (the planes of column slices), C wider than n
    wide_a = torch.randn(m, k1 + 64, generator=g, device=cuda)
    wide_b = torch.randn(n, k1 + 32, generator=g, device=cuda) * 0.05
    wide_c = torch.full((m, n + 16), 7.0, device=cuda)
    gemm_x3(wide_a[:, :k1], wide_b[:, :k1], out=wide_c[:, :n])
    torch.cuda.synchronize()
    _check(wide_c[:, :n], wide_a[:, :k1], wide_b[:, :k1])
    assert bool((wide_c[:, n:] == 7.0).all())  # columns past n untouched


def test_split_planes_exact(cuda):
    """hi = rne(x) and lo = rne(x - hi), zero padding to a multiple of 32; hi +
    lo within 2^-16 of x (relative)."""
    from engraft_ngram_amd.ple import SplitPlanes
    g = torch.Generator(device=cuda).manual_seed(3)
    x = torch.randn(37, 21, generator=g, device=cuda) * 10 ** torch.randint(-20, 20, (37, 21), generator=g,
                                                                             device=cuda).float()
    p = SplitPlanes(x)
    assert p.kp == 32 and p.hi.shape == (37, 32)
    hi = x.to(torch.bfloat16)
    lo = (x - hi.float()).to(torch.bfloat16)
    assert torch.equal(p.hi[:, :21].view(torch.int16), hi.view(torch.int16))
    assert torch.equal(p.lo[:, :21].view(torch.int16), lo.view(torch.int16))
    assert bool((p.hi[:, 21:].float() == 0).all()) and bool((p.lo[:, 21:].float() == 0).all())
    rel = ((p.hi[:, :21].double() + p.lo[:, :21].double() - x.double()).abs() / x.double().abs()).max()
    assert float(rel) <= 2.0 ** -16


def test_gemm_x3_projection_shape(cuda):
    """The forward's key projection at the real width (2560 -> 4 x 2560) on
    256 positions, and the result against torch's own fp32 GEMM."""
    from engraft_ngram_amd.ple import gemm_x3
    _say("gemm_x3 projection shape")
    g = torch.Generator(device=cuda).manual_seed(9)
    n = 2560
    emb = torch.randn(256, n, generator=g, device=cuda) * 0.1
    w = torch.randn(4 * n, n, generator=g, device=cuda) * n ** -0.5
    got = gemm_x3(emb, w)
    worst = _check(got, emb, w)
    ref32 = emb @ w.T
    torch.cuda.synchronize()
    worst32 = float(((ref32.double() - emb.double() @ w.double().T).abs()
                     / (emb.double().abs() @ w.double().abs().T)).max())
    _say(f"max err / bound: gemm_x3 {worst:.2e}, torch fp32 {worst32:.2e}")


@pytest.mark.parametrize("slices", [1, 3, 8])
def test_gemm_x3_column_groups_and_k_slices(cuda, slices):
    """key and value in one launch (two column groups over one A), and the
    backward's two K segments cut into K slices (summed in slice order: the
    result does not depend on the slice count beyond rounding, and repeats
    bit-identically)."""
    from engraft_ngram_amd.ple import gemm_x3
    _say(f"gemm_x3 column groups, k_slices={slices}")
    g = torch.Generator(device=cuda).manual_seed(11)
    m, k, n1, n2 = 200, 320, 384, 136
    a = torch.randn(m, k, generator=g, device=cuda)
    b1 = torch.randn(n1, k, generator=g, device=cuda) * 0.05
    bb = torch.randn(n2, k, generator=g, device=cuda) * 0.05
    o1, o2 = gemm_x3(a, b1, b_n2=bb, k_slices=slices)
    _check(o1, a, b1)
    _check(o2, a, bb)
    # two segments, one column group, sliced, accumulated
    a2 = torch.randn(m, 96, generator=g, device=cuda)
    b2 = torch.randn(n1, 96, generator=g, device=cuda) * 0.05
    base = torch.randn(m, n1, generator=g, device=cuda)
    acc = base.clone()
    gemm_x3(a, b1, a2, b2, out=acc, accumulate=True, k_slices=slices)
    _check(acc, a, b1, a2, b2, base=base)
    again = base.clone()
    gemm_x3(a, b1, a2, b2, out=again, accumulate=True, k_slices=slices)
    torch.cuda.synchronize()
    assert torch.equal(acc, again)


def test_gemm_x3_argument_errors(cuda):
    from engraft_ngram_amd import _lib
    hi = torch.zeros(8, 64, dtype=torch.bfloat16, device=cuda)
    c = torch.zeros(8, 8, device=cuda)
    ops = (_lib.EgGemmOperands * 2)()
    ops[0].a_hi = ops[0].a_lo = ops[0].b_hi = ops[0].b_lo = _lib.ptr(hi)
    ops[0].lda = ops[0].ldb = 64
    ops[0].k = 48
    with pytest.raises(ValueError, match="multiple of 32"):
        _lib.call("eg_gemm_bf16x3", ops, 1, 8, 8, 0, _lib.ptr(c), 8, None, 0, 0, 1, None, 0, _lib.stream_ptr(cuda))
    ops[0].k = 64  # two K steps: two slices need a workspace
    with pytest.raises(ValueError, match="workspace"):
        _lib.call("eg_gemm_bf16x3", ops, 1, 8, 8, 0, _lib.ptr(c), 8, None, 0, 0, 1 + 1, None, 0,
                  _lib.stream_ptr(cuda))
    # the kernel's 32-bit byte offsets: a plane of 4 GiB or more is refused
    # before anything is launched (only the leading dimension is large here)
    ops[0].lda = 1 << 31
    with pytest.raises(ValueError, match="4 GiB"):
        _lib.call("eg_gemm_bf16x3", ops, 1, 8, 8, 0, _lib.ptr(c), 8, None, 0, 0, 1, None, 0, _lib.stream_ptr(cuda))
