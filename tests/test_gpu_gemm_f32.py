"""eg_gemm_f32 (the PLE projections' GEMM in fp32 arithmetic on the fp32
matrix cores) against float64 products of the same fp32 operands.

Two bars.  Random data: |C - C64| <= (k + 2) 2^-24 (|A| |B|^T), the worst-case
bound of an fp32 sum of k fp32 products in any order; a wrong fragment layout,
a dropped K step or a lane half that reads the other half's k is off by O(1)
and fails it.  Exactness: with B a permutation scaled by powers of two, every
output is one product of an fp32 value with a power of two, exact in fp32, so
C must equal A's permuted, scaled columns bit for bit; operands rounded to
bf16 (or split into bf16 hi + lo planes: 16 of the 24 mantissa bits) anywhere
on the way fail it.  Shapes cover partial tiles in m and n, k below one
32-wide step and not a multiple of 32 (zero-padded copies), two K segments,
two column groups, K slices, accumulation, strided operands, and the
projections' real shape against torch's own fp32 matmul."""
from __future__ import annotations

import sys

import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


def _check(got, k, a, b, a2=None, b2=None, base=None):
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


@pytest.mark.parametrize("m,n,k", [(1, 4, 4), (7, 64, 12), (130, 200, 68), (128, 128, 32), (257, 129, 96),
                                   (64, 2560, 2560)])
def test_gemm_f32_against_float64(cuda, m, n, k):
    from engraft_ngram_amd.ple import gemm_f32
    _say(f"gemm_f32 m={m} n={n} k={k}")
    g = torch.Generator(device=cuda).manual_seed(m * 1000 + n + k)
    a = torch.randn(m, k, generator=g, device=cuda)
    b = torch.randn(n, k, generator=g, device=cuda) * 0.03
    got = gemm_f32(a, b)
    _check(got, (k + 31) // 32 * 32, a, b)


def _full_mantissa(rows, cols, g, dev):
    """fp32 values with all 24 significand bits random (bf16 keeps 8, hi + lo 16)."""
    mant = torch.randint(1 << 23, 1 << 24, (rows, cols), generator=g, device=dev).double()
    sign = torch.randint(0, 2, (rows, cols), generator=g, device=dev).double() * 2 - 1
    expo = torch.randint(-6, 6, (rows, cols), generator=g, device=dev).double()
    return (sign * mant * 2.0 ** (expo - 23)).float()


@pytest.mark.parametrize("m,n,k", [(96, 160, 64), (300, 136, 256)])
def test_gemm_f32_exact_products(cuda, m, n, k):
    """B = a permutation times powers of two: C[i, j] = A[i, p(j)] 2^e(j)
    exactly, in fp32; also through two column groups and two segments."""
    from engraft_ngram_amd.ple import gemm_f32
    _say(f"gemm_f32 exactness m={m} n={n} k={k}")
    g = torch.Generator(device=cuda).manual_seed(3 + m)
    a = _full_mantissa(m, k, g, cuda)
    perm = torch.randint(0, k, (n,), generator=g, device=cuda)
    scale = 2.0 ** torch.randint(-3, 4, (n,), generator=g, device=cuda).float()
    b = torch.zeros(n, k, device=cuda)
    b[torch.arange(n, device=cuda), perm] = scale
    exp = a[:, perm] * scale
    got = gemm_f32(a, b)
    torch.cuda.synchronize()
    assert torch.equal(got, exp)
    # the same through the second column group, and a second segment of zeros
    o1, o2 = gemm_f32(a, b, torch.zeros(m, 32, device=cuda), torch.zeros(n, 32, device=cuda),
                      b_n2=b.flip(0), b2_n2=torch.zeros(n, 32, device=cuda))
    torch.cuda.synchronize()
    assert torch.equal(o1, exp)
    assert torch.equal(o2, exp.flip(1))


def test_gemm_f32_two_segments_accumulate_and_strides(cuda):
    """d_emb = d_key w_key + d_value w_value as the backward calls it, then
    accumulated into an existing C; operands that are column slices of wider
    rows (leading dimension > k) and a C wider than n."""
    from engraft_ngram_amd.ple import gemm_f32
    _say("gemm_f32 two segments, accumulate, strided operands")
    g = torch.Generator(device=cuda).manual_seed(5)
    m, n, k1, k2 = 300, 192, 512, 128
    a1 = torch.randn(m, k1, generator=g, device=cuda)
    b1 = torch.randn(n, k1, generator=g, device=cuda) * 0.05
    a2 = torch.randn(m, k2, generator=g, device=cuda)
    b2 = torch.randn(n, k2, generator=g, device=cuda) * 0.05
    got = gemm_f32(a1, b1, a2, b2)
    _check(got, k1 + k2, a1, b1, a2, b2)
    base = torch.randn(m, n, generator=g, device=cuda)
    acc = base.clone()
    gemm_f32(a1, b1, a2, b2, out=acc, accumulate=True)
    _check(acc, k1 + k2 + 1, a1, b1, a2, b2, base=base)
    wide_a = torch.randn(m, k1 + 64, generator=g, device=cuda)
    wide_b = torch.randn(n, k1 + 32, generator=g, device=cuda) * 0.05
    wide_c = torch.full((m, n + 16), 7.0, device=cuda)
    gemm_f32(wide_a[:, :k1], wide_b[:, :k1], out=wide_c[:, :n])
    torch.cuda.synchronize()
    _check(wide_c[:, :n], k1, wide_a[:, :k1], wide_b[:, :k1])
    assert bool((wide_c[:, n:] == 7.0).all())  # columns past n untouched


@pytest.mark.parametrize("slices", [1, 3, 8])
def test_gemm_f32_column_groups_and_k_slices(cuda, slices):
    """key and value in one launch (two column groups over one A); two K
    segments cut into K slices, summed in slice order: repeats bit-identically."""
    from engraft_ngram_amd.ple import gemm_f32
    _say(f"gemm_f32 column groups, k_slices={slices}")
    g = torch.Generator(device=cuda).manual_seed(11)
    m, k, n1, n2 = 200, 320, 384, 136
    a = torch.randn(m, k, generator=g, device=cuda)
    b1 = torch.randn(n1, k, generator=g, device=cuda) * 0.05
    bb = torch.randn(n2, k, generator=g, device=cuda) * 0.05
    o1, o2 = gemm_f32(a, b1, b_n2=bb, k_slices=slices)
    _check(o1, k, a, b1)
    _check(o2, k, a, bb)
    a2 = torch.randn(m, 96, generator=g, device=cuda)
    b2 = torch.randn(n1, 96, generator=g, device=cuda) * 0.05
    base = torch.randn(m, n1, generator=g, device=cuda)
    acc = base.clone()
    gemm_f32(a, b1, a2, b2, out=acc, accumulate=True, k_slices=slices)
    _check(acc, k + 96 + slices, a, b1, a2, b2, base=base)
    again = base.clone()
    gemm_f32(a, b1, a2, b2, out=again, accumulate=True, k_slices=slices)
    torch.cuda.synchronize()
    assert torch.equal(acc, again)


def test_gemm_f32_projection_shape(cuda):
    """The forward's key projection at the real width (2560 -> 4 x 2560) on
    256 positions: within the fp32 bound, and no further from float64 than
    four times torch's own fp32 matmul on the same operands."""
    from engraft_ngram_amd.ple import gemm_f32
    _say("gemm_f32 projection shape")
    g = torch.Generator(device=cuda).manual_seed(9)
    n = 2560
    emb = torch.randn(256, n, generator=g, device=cuda) * 0.1
    w = torch.randn(4 * n, n, generator=g, device=cuda) * n ** -0.5
    got = gemm_f32(emb, w)
    worst = _check(got, n, emb, w)
    allow = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        ref32 = emb @ w.T
    finally:
        torch.backends.cuda.matmul.allow_tf32 = allow
    torch.cuda.synchronize()
    worst32 = float(((ref32.double() - emb.double() @ w.double().T).abs()
                     / (emb.double().abs() @ w.double().abs().T)).max())
    _say(f"max err / bound: gemm_f32 {worst:.2e}, torch fp32 {worst32:.2e}")
    assert worst <= 4 * worst32 + 1e-7


def test_gemm_f32_argument_errors(cuda):
    from engraft_ngram_amd import _lib
    x = torch.zeros(8, 64, device=cuda)
    c = torch.zeros(8, 8, device=cuda)
    ops = (_lib.EgGemmF32Operands * 2)()
    ops[0].a = ops[0].b = _lib.ptr(x)
    ops[0].lda = ops[0].ldb = 64
    ops[0].k = 48
    st = _lib.stream_ptr(cuda)
    with pytest.raises(ValueError, match="multiple of 32"):
        _lib.call("eg_gemm_f32", ops, 1, 8, 8, 0, _lib.ptr(c), 8, None, 0, 0, 1, None, 0, st)
    ops[0].k = 32
    ops[0].lda = 62
    with pytest.raises(ValueError, match="multiples of 4"):
        _lib.call("eg_gemm_f32", ops, 1, 8, 8, 0, _lib.ptr(c), 8, None, 0, 0, 1, None, 0, st)
    ops[0].lda = 64
    ops[0].k = 64  # two K steps: two slices need a workspace
    with pytest.raises(ValueError, match="workspace"):
        _lib.call("eg_gemm_f32", ops, 1, 8, 8, 0, _lib.ptr(c), 8, None, 0, 0, 2, None, 0, st)
    ops[0].a = _lib.ptr(x) + 4  # not 16-byte aligned
    with pytest.raises(ValueError, match="aligned"):
        _lib.call("eg_gemm_f32", ops, 1, 8, 8, 0, _lib.ptr(c), 8, None, 0, 0, 1, None, 0, st)


# (kind, m, n, k, plan on 256 CUs, workspace bytes of that plan).  fp32, one
# 256 x 256 tile a CU: 288 tiles, 32 of them in 256 ranges of 8 K steps (each
# inside one tile); 280 tiles, 24 in ranges of 9-10 of their 100 K steps (most
# ranges meet two tiles); 264 tiles of 16 K steps, too short for ranges, the 8
# past the first round in halves after 256 whole tiles.  bf16x3, the same
# tiles and plans: ranges inside one tile and ranges across two.  The ragged
# shapes' last row and column tiles lie partly outside C (the parts' sum is
# stored only inside it).
_LAST_ROUND = [
    ("f32", 1024, 18432, 2048, "ranges", 2 * 256 * 256 * 256 * 4),
    ("f32", 1024, 17920, 3200, "ranges", 2 * 256 * 256 * 256 * 4),
    ("f32", 1000, 18400, 3200, "ranges", 2 * 256 * 256 * 256 * 4),
    ("f32", 2048, 8448, 512, "halves", 8 * 2 * 256 * 256 * 4),
    ("bf16x3", 1024, 18432, 2048, "ranges", 2 * 256 * 256 * 256 * 4),
    ("bf16x3", 1024, 17920, 3200, "ranges", 2 * 256 * 256 * 256 * 4),
    ("bf16x3", 1000, 18400, 3200, "ranges", 2 * 256 * 256 * 256 * 4),
]


@pytest.mark.parametrize("kind,m,n,k,plan,ws_bytes", _LAST_ROUND, ids=[f"{c[0]}-{c[4]}-k{c[3]}" for c in _LAST_ROUND])
def test_gemm_last_round_in_pieces(cuda, kind, m, n, k, plan, ws_bytes):
    """Tile counts that leave the last round of workgroups mostly empty: the
    library's plan runs that round's tiles as K ranges or K pieces whose
    partial products are summed afterwards in K order.  Within the bar, equal
    to itself on a second call, refused with a workspace one byte short, and
    with accumulate on exactly twice the product."""
    from engraft_ngram_amd import _lib
    from engraft_ngram_amd.ple import gemm_f32, gemm_x3
    _say(f"gemm last round ({kind}, {plan}, m {m} n {n} k {k})")
    g = torch.Generator(device=cuda).manual_seed(21)
    a = torch.randn(m, k, generator=g, device=cuda)
    b = torch.randn(n, k, generator=g, device=cuda) * 0.05
    size_fn = "eg_gemm_f32_workspace_size" if kind == "f32" else "eg_gemm_workspace_size"
    need = int(getattr(_lib.load(), size_fn)(m, n, 0, k, 0))
    if torch.cuda.get_device_properties(cuda).multi_processor_count == 256:
        assert need > 0, "the mostly empty last round should be cut"
        if ws_bytes is not None:
            assert need == ws_bytes, f"workspace {need} B, the {plan} plan takes {ws_bytes} B"
    fn = gemm_f32 if kind == "f32" else gemm_x3
    got = fn(a, b)
    if kind == "f32":
        _check(got, k + 8, a, b)
    else:
        exp = a.double() @ b.double().T
        bound = a.double().abs() @ b.double().abs().T
        torch.cuda.synchronize()
        assert bool(((got.double() - exp).abs() <= 2e-5 * bound + 1e-30).all())
        del exp, bound
    again = fn(a, b)
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    if need > 0 and kind == "f32":
        ops = (_lib.EgGemmF32Operands * 2)()
        ops[0].a, ops[0].lda, ops[0].b, ops[0].ldb, ops[0].k = _lib.ptr(a), k, _lib.ptr(b), k, k
        ws = torch.empty(need // 4, device=cuda)
        out = torch.empty(m, n, device=cuda)
        with pytest.raises(ValueError, match="workspace"):
            _lib.call("eg_gemm_f32", ops, 1, m, n, 0, _lib.ptr(out), n, None, 0, 0, 0, _lib.ptr(ws), need - 1,
                      _lib.stream_ptr(cuda))
        _lib.call("eg_gemm_f32", ops, 1, m, n, 0, _lib.ptr(out), n, None, 0, 0, 0, _lib.ptr(ws), need,
                  _lib.stream_ptr(cuda))
        torch.cuda.synchronize()
        assert torch.equal(out, got)
        # accumulate: every output, whole tile or summed parts, adds the same
        # sum again, and doubling is exact
        _lib.call("eg_gemm_f32", ops, 1, m, n, 0, _lib.ptr(out), n, None, 0, 1, 0, _lib.ptr(ws), need,
                  _lib.stream_ptr(cuda))
        torch.cuda.synchronize()
        assert torch.equal(out, 2 * got)
