"""The PLE block that consumes the gathered rows, on the device: the drop-in
for ``PleWeights`` / ``ple_forward`` (``engraft/replica/layers.py:555-626``).

Forward:

* ``key = emb @ w_key^T`` and ``value = emb @ w_value^T`` in one launch: by
  default (``gemm="bf16x6"``) on the bf16 matrix cores with fp32 accuracy
  (``gemm_x6``: operands split into three bf16 planes, six products
  accumulated in fp32), with ``gemm="fp32"`` of the ``gemm_f32`` kernel on
  the fp32 matrix cores (fp32 products, as the reference's torch matmuls), or
  with ``gemm="bf16x3"`` of the ``gemm_x3`` kernel (hi + lo planes, three
  products: 16 mantissa bits per operand);
* ``eg_ple_gate``: per position and stream, the RMS norms of key and hidden,
  the score ``s``, the gate, ``gated = value * gate`` and its RMS norm;
* ``eg_ple_conv``: the dilated causal depthwise convolution over
  ``[history; normed]``, SiLU, and ``out = hidden + gated + conv``.

The result -- the output and the new history -- is differentiable in emb,
hidden, the history and the weights.  The backward runs
``eg_ple_conv_backward`` and ``eg_ple_gate_backward`` on the forward's saved
intermediates, then the projections' backward (one ``gemm_f32``, ``gemm_x3``
or ``gemm_x6`` call over two K segments); when weights need gradients, also the
two weight GEMMs (``gemm_f32`` with the positions as K) and
``eg_ple_weight_grads`` for the norm and convolution weights.  The
convolution takes 1..8 taps (the reference's blocks have 4; more raise
``ValueError``).  Only shapes beyond the HIP backward's limits (more than 4
streams, ``n_embd`` > 4096, a convolution reaching back more than 32 rows)
fall back to a recomputation of the block in torch elementwise operations
around ``gemm_f32`` products, differentiated by autograd.  An input that a
detached factor cuts off the output gets no gradient (None), as in the
reference's graph.  Either way the forward values are the HIP kernels'.
``detach_value`` / ``detach_gate`` change only the backward, as in the
reference.

``PleReplica`` (below) is the same block with its weights read from the model
GGUF, method for method as the reference's numpy replica.
"""
from __future__ import annotations

import dataclasses

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib


@dataclasses.dataclass
class PleWeights:
    """``engraft/replica/layers.py:555-562``."""

    w_key: torch.Tensor  # [hc*n_embd, n_embd]
    w_value: torch.Tensor  # [n_embd, n_embd]
    norm_key: torch.Tensor  # [hc*n_embd]
    norm_query: torch.Tensor  # [hc*n_embd]
    norm_conv: torch.Tensor  # [hc*n_embd]
    conv1d: torch.Tensor  # [hc*n_embd, K]


def _rms(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    return x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps) * w


class _GemmNT(torch.autograd.Function):
    """``a @ b.T`` on eg_gemm_f32, differentiable: ``d_a = d b`` and
    ``d_b = d^T a``, both on eg_gemm_f32 too."""

    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return gemm_f32(a.float(), b.float())

    @staticmethod
    def backward(ctx, d):
        a, b = ctx.saved_tensors
        d = d.float().contiguous()
        d_a = gemm_f32(d, b.float().T).to(a.dtype) if ctx.needs_input_grad[0] else None
        d_b = _weight_grad(d, a.float(), b).to(b.dtype) if ctx.needs_input_grad[1] else None
        return d_a, d_b


def _block_torch(emb, hidden, w_key, w_value, nk, nq, nc, conv, hist, eps, dil, detach_value, detach_gate):
    """The block as elementwise torch operations around ``gemm_f32`` products
    (the backward's recomputation beyond the HIP backward's limits): ``(out,
    new_hist)``."""
    t_len, hc, n = hidden.shape
    key = _rms(_GemmNT.apply(emb, w_key).reshape(t_len, hc, n), nk.reshape(hc, n), eps)
    query = _rms(hidden, nq.reshape(hc, n), eps)
    s = (key * query).sum(dim=-1) / (n ** 0.5)
    gate = torch.sigmoid(torch.sign(s) * torch.sqrt(torch.clamp(s.abs(), min=1e-6)))
    value = _GemmNT.apply(emb, w_value)
    g = gate.detach() if detach_gate else gate
    v = value.detach() if detach_value else value
    gated = v.unsqueeze(1) * g.unsqueeze(-1)
    normed = _rms(gated, nc.reshape(hc, n), eps).reshape(t_len, hc * n)
    full = torch.cat([hist.reshape(hist.shape[0], hc * n), normed], dim=0)
    taps = conv.shape[1]
    h0 = hist.shape[0]
    acc = torch.zeros_like(normed)
    for k in range(taps):
        back = (taps - 1 - k) * dil
        lo = max(0, back - h0)  # first position whose source row exists
        if lo < t_len:
            acc[lo:] = acc[lo:] + full[h0 + lo - back:h0 + t_len - back] * conv[:, k]
    out = hidden + gated + F.silu(acc).reshape(t_len, hc, n)
    hist_len = (taps - 1) * dil
    new_hist = full[-hist_len:] if hist_len > 0 else full[:0]
    return out, new_hist.reshape(-1, hc, n)


class _TransposedCache:
    """Row-major copies of the projection weights' transposes, kept between
    steps: the backward's ``d_emb = d @ w`` is ``gemm_x3(d, w^T)``, whose B
    operand is K-contiguous.  An entry is used only for the same tensor object
    (weak reference) at the same version counter, so a weight that is
    modified in place or freed and replaced is transposed again."""

    def __init__(self, size: int = 4):
        self._entries: list = []
        self._size = size

    def get(self, w: torch.Tensor) -> torch.Tensor:
        import weakref
        for ref, version, wt in self._entries:
            if ref() is w and version == w._version:
                return wt
        wt = w.T.contiguous()
        self._entries = [e for e in self._entries if e[0]() is not None][-(self._size - 1):]
        self._entries.append((weakref.ref(w), w._version, wt))
        return wt


_WT = _TransposedCache()


class SplitPlanes:
    """The bf16 hi / lo planes of an fp32 matrix ``[rows, cols]`` (``eg_split_bf16``),
    each ``[rows, kp]`` with ``kp`` = cols rounded up to 32, zero-padded.  With
    ``three=True`` (``eg_split_bf16x6``, the planes of :func:`gemm_x6`) ``lo``
    is the second plane rne(x - hi) and ``lo2`` the third, rne(x - hi - lo)."""

    def __init__(self, x: torch.Tensor, three: bool = False):
        if x.dim() != 2:
            raise ValueError("SplitPlanes: a 2-D matrix expected")
        x = x if x.dtype == torch.float32 else x.float()
        if x.stride(-1) != 1:
            x = x.contiguous()
        rows, cols = x.shape
        self.rows, self.cols, self.kp = rows, cols, (cols + 31) // 32 * 32
        self.hi = torch.empty((rows, self.kp), dtype=torch.bfloat16, device=x.device)
        self.lo = torch.empty_like(self.hi)
        self.lo2 = torch.empty_like(self.hi) if three else None
        if three:
            _lib.call("eg_split_bf16x6", _lib.ptr(x), rows, cols, max(x.stride(0), cols), _lib.ptr(self.hi),
                      _lib.ptr(self.lo), _lib.ptr(self.lo2), _lib.stream_ptr(x.device))
        else:
            _lib.call("eg_split_bf16", _lib.ptr(x), rows, cols, max(x.stride(0), cols), _lib.ptr(self.hi),
                      _lib.ptr(self.lo), _lib.stream_ptr(x.device))


def _empty_planes(rows: int, cols: int, device) -> "SplitPlanes":
    """Uninitialised planes of a [rows, cols] matrix, cols a multiple of 32 (no
    padding), for a kernel that writes them directly."""
    p = SplitPlanes.__new__(SplitPlanes)
    p.rows, p.cols, p.kp = rows, cols, cols
    p.hi = torch.empty((rows, cols), dtype=torch.bfloat16, device=device)
    p.lo = torch.empty_like(p.hi)
    return p


class _PlaneCache:
    """Split planes of weights, kept between steps: an entry is used only for
    the same tensor object (weak reference) at the same version counter."""

    def __init__(self, size: int = 8):
        self._entries: list = []
        self._size = size

    def get(self, w: torch.Tensor, three: bool = False) -> SplitPlanes:
        import weakref
        for ref, version, planes in self._entries:
            if ref() is w and version == w._version and (planes.lo2 is not None) == three:
                return planes
        planes = SplitPlanes(w, three=three)
        self._entries = [e for e in self._entries if e[0]() is not None][-(self._size - 1):]
        self._entries.append((weakref.ref(w), w._version, planes))
        return planes


_PLANES = _PlaneCache()


def _planes(x, cached: bool, three: bool = False) -> SplitPlanes:
    if isinstance(x, SplitPlanes):
        if three and x.lo2 is None:
            raise ValueError("gemm_x6 needs three-plane SplitPlanes (SplitPlanes(x, three=True))")
        return x
    return _PLANES.get(x, three) if cached else SplitPlanes(x, three=three)


def _gemm_workspace(m: int, n: int, n2: int, k: int, k_slices: int | None, dev, size_fn: str):
    """The K-slice argument for the GEMM entry points (0: the library plans the
    pieces of a partly filled last round) and the workspace that plan needs
    (``size_fn``: the entry point's workspace-size function)."""
    slices = 0 if k_slices is None else int(k_slices)
    if slices < 0:
        raise ValueError(f"k_slices must be >= 0, got {slices}")
    with torch.cuda.device(dev):
        ws_bytes = int(getattr(_lib.load(), size_fn)(m, n, n2, k, slices))
    if ws_bytes < 0:
        raise RuntimeError("eg_gemm_workspace_size: device query failed")
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=dev) if ws_bytes else None
    return slices, ws, ws_bytes


def gemm_x3(a, b, a2=None, b2=None, out: torch.Tensor | None = None, accumulate: bool = False,
            cache_b: bool = False, b_n2=None, b2_n2=None, out2: torch.Tensor | None = None,
            k_slices: int | None = None):
    """``a @ b.T (+ a2 @ b2.T)`` in fp32 on the bf16 matrix cores
    (``eg_gemm_bf16x3``: every operand split into bf16 hi + lo planes, three
    products accumulated in fp32; 16 mantissa bits per operand).  ``a [m, k]``, ``b [n, k]``, ``a2 [m, k2]``,
    ``b2 [n, k2]``: fp32 tensors on one device, or their ``SplitPlanes``;
    ``cache_b`` keeps the planes of the B operands between calls (weights).
    ``b_n2`` (and ``b2_n2`` with a second segment) ``[n2, k]`` add a second
    column group, ``a @ b_n2.T (+ a2 @ b2_n2.T)`` into ``out2``, in the same
    launch.  ``k_slices`` (default: the library's plan, which cuts the tiles
    of a partly filled last round of workgroups along K) cuts every 256 x 256
    tile into that many K pieces, summed in a fixed order.  Returns ``out`` (``[m, n]`` fp32,
    allocated when not given; added to when ``accumulate``), or ``(out,
    out2)`` with a second column group."""
    segs = [(_planes(a, False), _planes(b, cache_b), None if b_n2 is None else _planes(b_n2, cache_b))]
    if a2 is not None:
        segs.append((_planes(a2, False), _planes(b2, cache_b), None if b2_n2 is None else _planes(b2_n2, cache_b)))
    m, n = segs[0][0].rows, segs[0][1].rows
    n2 = 0 if segs[0][2] is None else segs[0][2].rows
    ops = (_lib.EgGemmOperands * 2)()
    k_tiles = 0
    for i, (pa, pb, pb2) in enumerate(segs):
        if pa.rows != m or pb.rows != n or pb.cols != pa.cols:
            raise ValueError(f"gemm_x3: segment {i}: a [m, k] and b [n, k] expected, got [{pa.rows}, {pa.cols}] "
                             f"and [{pb.rows}, {pb.cols}]")
        if (pb2 is None) != (n2 == 0) or (pb2 is not None and (pb2.rows != n2 or pb2.cols != pa.cols)):
            raise ValueError(f"gemm_x3: segment {i}: the second column group needs b [n2, k] in every segment")
        o = ops[i]
        o.a_hi, o.a_lo, o.lda = _lib.ptr(pa.hi), _lib.ptr(pa.lo), pa.kp
        o.b_hi, o.b_lo, o.ldb = _lib.ptr(pb.hi), _lib.ptr(pb.lo), pb.kp
        if pb2 is not None:
            o.b2_hi, o.b2_lo, o.ldb2 = _lib.ptr(pb2.hi), _lib.ptr(pb2.lo), pb2.kp
        o.k = pa.kp
        k_tiles += pa.kp // 32
    dev = segs[0][0].hi.device

    def _out(t, rows, cols, name):
        if t is None:
            if accumulate:
                raise ValueError(f"gemm_x3: accumulate needs {name}")
            return torch.empty((rows, cols), dtype=torch.float32, device=dev)
        if t.dtype != torch.float32 or t.shape != (rows, cols) or t.stride(1) != 1:
            raise ValueError(f"gemm_x3: {name} must be fp32 [{rows}, {cols}] with unit column stride")
        return t

    out = _out(out, m, n, "out")
    out2 = _out(out2, m, n2, "out2") if n2 else None
    slices, ws, ws_bytes = _gemm_workspace(m, n, n2, 32 * k_tiles, k_slices, dev, "eg_gemm_workspace_size")
    _lib.call("eg_gemm_bf16x3", ops, len(segs), m, n, n2, _lib.ptr(out), max(out.stride(0), n),
              _lib.ptr(out2), max(out2.stride(0), n2) if n2 else 0, int(accumulate), slices, _lib.ptr(ws),
              ws_bytes, _lib.stream_ptr(dev))
    return (out, out2) if n2 else out


def gemm_x6(a, b, a2=None, b2=None, out: torch.Tensor | None = None, accumulate: bool = False,
            cache_b: bool = False, b_n2=None, b2_n2=None, out2: torch.Tensor | None = None,
            k_slices: int | None = None):
    """:func:`gemm_x3`'s GEMM with fp32 accuracy on the bf16 matrix cores
    (``eg_gemm_bf16x6``): every operand split into three bf16 planes, hi + mid
    + lo keeping its 24 mantissa bits, and the six plane products above
    2^-23 of |a||b| accumulated in fp32 (one launch for one K segment, two
    for two).  Arguments, operands (fp32 tensors or three-plane
    ``SplitPlanes``) and result as :func:`gemm_x3`."""
    segs = [(_planes(a, False, True), _planes(b, cache_b, True),
             None if b_n2 is None else _planes(b_n2, cache_b, True))]
    if a2 is not None:
        segs.append((_planes(a2, False, True), _planes(b2, cache_b, True),
                     None if b2_n2 is None else _planes(b2_n2, cache_b, True)))
    m, n = segs[0][0].rows, segs[0][1].rows
    n2 = 0 if segs[0][2] is None else segs[0][2].rows
    hm, hl = (_lib.EgGemmOperands * 2)(), (_lib.EgGemmOperands * 2)()
    k_tiles = 0
    for i, (pa, pb, pb2) in enumerate(segs):
        if pa.rows != m or pb.rows != n or pb.cols != pa.cols:
            raise ValueError(f"gemm_x6: segment {i}: a [m, k] and b [n, k] expected, got [{pa.rows}, {pa.cols}] "
                             f"and [{pb.rows}, {pb.cols}]")
        if (pb2 is None) != (n2 == 0) or (pb2 is not None and (pb2.rows != n2 or pb2.cols != pa.cols)):
            raise ValueError(f"gemm_x6: segment {i}: the second column group needs b [n2, k] in every segment")
        for o, second in ((hm[i], "lo"), (hl[i], "lo2")):
            o.a_hi, o.a_lo, o.lda = _lib.ptr(pa.hi), _lib.ptr(getattr(pa, second)), pa.kp
            o.b_hi, o.b_lo, o.ldb = _lib.ptr(pb.hi), _lib.ptr(getattr(pb, second)), pb.kp
            if pb2 is not None:
                o.b2_hi, o.b2_lo, o.ldb2 = _lib.ptr(pb2.hi), _lib.ptr(getattr(pb2, second)), pb2.kp
            o.k = pa.kp
        k_tiles += pa.kp // 32
    dev = segs[0][0].hi.device

    def _out(t, rows, cols, name):
        if t is None:
            if accumulate:
                raise ValueError(f"gemm_x6: accumulate needs {name}")
            return torch.empty((rows, cols), dtype=torch.float32, device=dev)
        if t.dtype != torch.float32 or t.shape != (rows, cols) or t.stride(1) != 1:
            raise ValueError(f"gemm_x6: {name} must be fp32 [{rows}, {cols}] with unit column stride")
        return t

    out = _out(out, m, n, "out")
    out2 = _out(out2, m, n2, "out2") if n2 else None
    # one K segment runs as one launch over both plane sets: its plan covers 2 k steps
    k_plan = 32 * k_tiles * (2 if len(segs) == 1 else 1)
    slices, ws, ws_bytes = _gemm_workspace(m, n, n2, k_plan, k_slices, dev, "eg_gemm_workspace_size")
    _lib.call("eg_gemm_bf16x6", hm, hl, len(segs), m, n, n2, _lib.ptr(out), max(out.stride(0), n),
              _lib.ptr(out2), max(out2.stride(0), n2) if n2 else 0, int(accumulate), slices, _lib.ptr(ws),
              ws_bytes, _lib.stream_ptr(dev))
    return (out, out2) if n2 else out


def _f32_operand(x: torch.Tensor, kp: int) -> torch.Tensor:
    """``x [rows, k]`` fp32 as eg_gemm_f32 reads it: unit column stride, row
    stride a multiple of 4, 16-byte aligned, ``k`` a multiple of 32; otherwise
    a copy with the columns zero-padded to ``kp``."""
    if x.dtype != torch.float32:
        x = x.float()
    rows, cols = x.shape
    if (cols == kp and x.stride(1) == 1 and x.stride(0) % 4 == 0 and x.stride(0) >= cols
            and x.data_ptr() % 16 == 0):
        return x
    y = torch.zeros((rows, kp), dtype=torch.float32, device=x.device)
    y[:, :cols] = x
    return y


def gemm_f32(a, b, a2=None, b2=None, out: torch.Tensor | None = None, accumulate: bool = False,
             b_n2=None, b2_n2=None, out2: torch.Tensor | None = None, k_slices: int | None = None):
    """``a @ b.T (+ a2 @ b2.T)`` in fp32 arithmetic on the fp32 matrix cores
    (``eg_gemm_f32``): the products of an fp32 matmul, accumulated in fp32.
    Operands and the column groups, K segments and K slices as
    :func:`gemm_x3`, every operand an fp32 tensor (a ``k`` not a multiple of
    32 is zero-padded in a copy).  Returns ``out``, or ``(out, out2)`` with a
    second column group."""
    raw = [(a, b, b_n2)] + ([(a2, b2, b2_n2)] if a2 is not None else [])
    m, n = a.shape[0], b.shape[0]
    n2 = 0 if b_n2 is None else b_n2.shape[0]
    ops = (_lib.EgGemmF32Operands * 2)()
    keep = []
    k_tiles = 0
    for i, (xa, xb, xb2) in enumerate(raw):
        if xa.dim() != 2 or xb.dim() != 2 or xa.shape[0] != m or xb.shape[0] != n or xb.shape[1] != xa.shape[1]:
            raise ValueError(f"gemm_f32: segment {i}: a [m, k] and b [n, k] expected, got {list(xa.shape)} and "
                             f"{list(xb.shape)}")
        if (xb2 is None) != (n2 == 0) or (xb2 is not None and (xb2.dim() != 2 or xb2.shape[0] != n2
                                                                or xb2.shape[1] != xa.shape[1])):
            raise ValueError(f"gemm_f32: segment {i}: the second column group needs b [n2, k] in every segment")
        kp = (xa.shape[1] + 31) // 32 * 32
        ta, tb = _f32_operand(xa, kp), _f32_operand(xb, kp)
        tb2 = _f32_operand(xb2, kp) if xb2 is not None else None
        keep += [ta, tb, tb2]
        o = ops[i]
        o.a, o.lda, o.b, o.ldb = _lib.ptr(ta), ta.stride(0), _lib.ptr(tb), tb.stride(0)
        if tb2 is not None:
            o.b2, o.ldb2 = _lib.ptr(tb2), tb2.stride(0)
        o.k = kp
        k_tiles += kp // 32
    dev = a.device

    def _out(t, rows, cols, name):
        if t is None:
            if accumulate:
                raise ValueError(f"gemm_f32: accumulate needs {name}")
            return torch.empty((rows, cols), dtype=torch.float32, device=dev)
        if t.dtype != torch.float32 or t.shape != (rows, cols) or t.stride(1) != 1:
            raise ValueError(f"gemm_f32: {name} must be fp32 [{rows}, {cols}] with unit column stride")
        return t

    out = _out(out, m, n, "out")
    out2 = _out(out2, m, n2, "out2") if n2 else None
    slices, ws, ws_bytes = _gemm_workspace(m, n, n2, 32 * k_tiles, k_slices, dev, "eg_gemm_f32_workspace_size")
    _lib.call("eg_gemm_f32", ops, len(raw), m, n, n2, _lib.ptr(out), max(out.stride(0), n),
              _lib.ptr(out2), max(out2.stride(0), n2) if n2 else 0, int(accumulate), slices, _lib.ptr(ws),
              ws_bytes, _lib.stream_ptr(dev))
    return (out, out2) if n2 else out


WGRAD_MAX_TAPS = 8  # eg_ple_weight_grads' built tap counts (1..8)


def _weight_grad(d_y: torch.Tensor, x: torch.Tensor, w: torch.Tensor, gemm: str = "fp32") -> torch.Tensor:
    """``d_y^T x`` (``[out, T]`` x ``[T, in]``), the gradient of ``w`` in
    ``y = x w^T``, with the positions as K (both operands transposed into
    K-contiguous copies): on eg_gemm_f32, or with ``gemm="bf16x6"`` on
    eg_gemm_bf16x6 (the same fp32 accuracy; bf16x3's 16-bit operands are kept
    to the projections)."""
    if d_y.shape[0] == 0:
        return torch.zeros_like(w)
    if gemm == "bf16x6":
        return gemm_x6(d_y.T, x.T)
    return gemm_f32(d_y.T, x.T)


def _projection_backward(gemm: str, flat: list) -> torch.Tensor:
    """``d_emb = sum d_i w_i`` over the (d_i, w_i^T) pairs in ``flat``, on the
    forward's GEMM."""
    if gemm == "bf16x3":
        return gemm_x3(*flat, cache_b=True)
    if gemm == "bf16x6":
        return gemm_x6(*flat, cache_b=True)
    return gemm_f32(*flat)


def _native_backward_ok(hc: int, n: int, taps: int, dil: int, weights: bool = False) -> bool:
    """The HIP backward's built limits (eg_ple_gate_backward, eg_ple_conv_backward,
    and with ``weights`` eg_ple_weight_grads)."""
    return hc <= 4 and n <= 4096 and (taps - 1) * dil <= 32 and (not weights or taps <= WGRAD_MAX_TAPS)


class _PleFn(torch.autograd.Function):
    """Forward on the HIP kernels.  Backward: the HIP backward from the saved
    forward intermediates (the projections' GEMMs are not run again), with the
    weights' gradients when they are asked for; beyond the HIP kernels' limits,
    a torch recomputation of the block, differentiated by autograd."""

    @staticmethod
    def forward(ctx, emb, hidden, w_key, w_value, nk, nq, nc, conv, hist, eps, dil, detach_value, detach_gate,
                gemm):
        t_len, hc, n = hidden.shape
        dev = hidden.device
        f32 = dict(dtype=torch.float32, device=dev)
        emb32 = emb.to(**f32).contiguous()
        wk32 = w_key.to(**f32)
        wv32 = w_value.to(**f32)
        if gemm == "bf16x3":
            key, value = gemm_x3(SplitPlanes(emb32), wk32, cache_b=True, b_n2=wv32)
        elif gemm == "bf16x6":
            key, value = gemm_x6(SplitPlanes(emb32, three=True), wk32, cache_b=True, b_n2=wv32)
        else:
            key, value = gemm_f32(emb32, wk32, b_n2=wv32)
        hidden32 = hidden.to(**f32).contiguous()
        h0 = hist.shape[0]
        full = torch.empty((h0 + t_len, hc * n), **f32)
        if h0:
            full[:h0] = hist.reshape(h0, hc * n)
        s = torch.empty((t_len, hc), **f32)
        gate = torch.empty((t_len, hc), **f32)
        st = _lib.stream_ptr(dev)
        nk32, nq32, nc32 = (x.to(**f32).contiguous() for x in (nk, nq, nc))
        conv32 = conv.to(**f32).contiguous()
        taps = conv32.shape[1]
        native = any(ctx.needs_input_grad) and _native_backward_ok(hc, n, taps, int(dil),
                                                                   weights=any(ctx.needs_input_grad[2:8]))
        rstd = torch.empty((t_len, hc, 3), **f32) if native else None
        _lib.call("eg_ple_gate", _lib.ptr(key), _lib.ptr(value), _lib.ptr(hidden32), _lib.ptr(nk32), _lib.ptr(nq32),
                  _lib.ptr(nc32), t_len, hc, n, float(eps), _lib.ptr(full[h0:]), _lib.ptr(s), _lib.ptr(gate),
                  _lib.ptr(rstd), st)
        out = torch.empty((t_len, hc, n), **f32)
        pre = torch.empty((t_len, hc * n), **f32) if native else None  # kept for the backward's SiLU derivative
        _lib.call("eg_ple_conv", _lib.ptr(full), h0, t_len, hc, n, _lib.ptr(conv32), taps, int(dil), 0,
                  _lib.ptr(hidden32), _lib.ptr(value), _lib.ptr(gate), _lib.ptr(out), _lib.ptr(pre), st)
        hist_len = (taps - 1) * int(dil)
        new_hist = (full[-hist_len:] if hist_len > 0 else full[:0]).reshape(-1, hc, n).to(hidden.dtype).clone()
        ctx.native = native
        if native:
            # emb for the projection weights' gradients
            emb_w = emb32 if any(ctx.needs_input_grad[2:4]) else None
            ctx.save_for_backward(key, value, hidden32, full, s, gate, rstd, nk32, nq32, nc32, conv32, wk32, wv32, pre,
                                  emb_w)
            ctx.dtypes = (emb.dtype, hidden.dtype, hist.dtype)
            ctx.w_dtypes = tuple(x.dtype for x in (w_key, w_value, nk, nq, nc, conv))
            ctx.tail_rows = new_hist.shape[0]
        else:
            ctx.save_for_backward(emb, hidden, w_key, w_value, nk, nq, nc, conv, hist)
        ctx.cfg = (eps, dil, detach_value, detach_gate)
        ctx.gemm = gemm
        ctx.mark_non_differentiable(s, gate, value)
        return out.to(hidden.dtype), new_hist, s, gate, value

    @staticmethod
    def backward(ctx, d_out, d_hist, _d_s, _d_gate, _d_value):
        if ctx.native:
            return _PleFn._backward_native(ctx, d_out, d_hist)
        inputs = ctx.saved_tensors
        eps, dil, detach_value, detach_gate = ctx.cfg
        with torch.enable_grad():
            leaves = [x.detach().requires_grad_(need) for x, need in zip(inputs, ctx.needs_input_grad[:9])]
            out, new_hist = _block_torch(*leaves, eps, dil, detach_value, detach_gate)
            wrt = [x for x, need in zip(leaves, ctx.needs_input_grad[:9]) if need]
            outs, grads_in = [out], [d_out]
            if d_hist is not None and new_hist.numel():
                outs.append(new_hist)
                grads_in.append(d_hist)
            grads = iter(torch.autograd.grad(outs, wrt, grads_in, allow_unused=True) if wrt else [])
        # an input the detached graph does not reach keeps autograd's None, as
        # in the reference's own graph (its .grad stays None)
        res = [next(grads) if need else None for need in ctx.needs_input_grad[:9]]
        return (*res, None, None, None, None, None)

    @staticmethod
    def _backward_native(ctx, d_out, d_hist):
        key, value, hidden32, full, s, gate, rstd, nk32, nq32, nc32, conv32, wk32, wv32, pre, emb32 = ctx.saved_tensors
        _eps, dil, detach_value, detach_gate = ctx.cfg
        emb_dt, hidden_dt, hist_dt = ctx.dtypes
        t_len, hc, n = hidden32.shape
        c_dim = hc * n
        h0 = full.shape[0] - t_len
        dev = full.device
        f32 = dict(dtype=torch.float32, device=dev)
        st = _lib.stream_ptr(dev)
        need_emb, need_hidden, need_hist = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[8]
        d_out32 = d_out.to(**f32).contiguous()
        tail = ctx.tail_rows if (d_hist is not None and ctx.tail_rows > 0) else 0
        d_tail = d_hist.to(**f32).reshape(tail, c_dim).contiguous() if tail else None
        d_full = torch.empty((h0 + t_len, c_dim), **f32)
        _lib.call("eg_ple_conv_backward", _lib.ptr(full), h0, t_len, hc, n, _lib.ptr(conv32), conv32.shape[1],
                  int(dil), _lib.ptr(pre), _lib.ptr(d_out32), _lib.ptr(d_tail), tail, _lib.ptr(d_full), st)
        d_hidden = torch.empty((t_len, hc, n), **f32) if need_hidden else None
        need_w = ctx.needs_input_grad[2:8]
        if any(need_w):
            return _PleFn._backward_with_weights(ctx, d_out32, d_full, d_hidden)
        if ctx.gemm == "bf16x3" and n % 256 == 0:
            # d_key and d_value straight into the bf16 planes gemm_x3 takes
            pk = _empty_planes(t_len, c_dim, dev) if (need_emb and not detach_gate) else None
            pv = _empty_planes(t_len, n, dev) if (need_emb and not detach_value) else None
            if pk is not None or pv is not None or d_hidden is not None:
                _lib.call("eg_ple_gate_backward_planes", _lib.ptr(key), _lib.ptr(value), _lib.ptr(hidden32),
                          _lib.ptr(nk32), _lib.ptr(nq32), _lib.ptr(nc32), _lib.ptr(s), _lib.ptr(gate), _lib.ptr(rstd),
                          _lib.ptr(d_out32), _lib.ptr(d_full[h0:]), t_len, hc, n, int(bool(detach_value)),
                          int(bool(detach_gate)), _lib.ptr(pk.hi if pk else None), _lib.ptr(pk.lo if pk else None),
                          _lib.ptr(pv.hi if pv else None), _lib.ptr(pv.lo if pv else None), _lib.ptr(d_hidden), None,
                          st)
            d_emb = None
            if need_emb:
                # with both factors detached emb has no path to the output: None, as autograd gives
                parts = [(d, _WT.get(w)) for d, w in ((pk, wk32), (pv, wv32)) if d is not None]
                if parts:
                    d_emb = gemm_x3(*[x for part in parts for x in part], cache_b=True).to(emb_dt)
            d_hist_in = d_full[:h0].reshape(h0, hc, n).to(hist_dt) if need_hist else None
            return (d_emb, d_hidden.to(hidden_dt) if d_hidden is not None else None, None, None, None, None, None,
                    None, d_hist_in, None, None, None, None, None)
        d_key = torch.empty((t_len, c_dim), **f32) if (need_emb and not detach_gate) else None
        d_value = torch.empty((t_len, n), **f32) if (need_emb and not detach_value) else None
        if d_key is not None or d_value is not None or d_hidden is not None:
            _lib.call("eg_ple_gate_backward", _lib.ptr(key), _lib.ptr(value), _lib.ptr(hidden32), _lib.ptr(nk32),
                      _lib.ptr(nq32), _lib.ptr(nc32), _lib.ptr(s), _lib.ptr(gate), _lib.ptr(rstd), _lib.ptr(d_out32),
                      _lib.ptr(d_full[h0:]), t_len, hc, n, int(bool(detach_value)), int(bool(detach_gate)),
                      _lib.ptr(d_key), _lib.ptr(d_value), _lib.ptr(d_hidden), None, st)
        d_emb = None
        if need_emb:
            # the projections' backward, d_emb = d_key w_key + d_value w_value, as
            # products with the weights' transposes (kept between steps)
            parts = [(d, _WT.get(w)) for d, w in ((d_key, wk32), (d_value, wv32)) if d is not None]
            if parts:  # none: both factors detached, emb has no path to the output
                flat = [x for part in parts for x in part]
                d_emb = _projection_backward(ctx.gemm, flat).to(emb_dt)
        d_hist_in = d_full[:h0].reshape(h0, hc, n).to(hist_dt) if need_hist else None
        return (d_emb, d_hidden.to(hidden_dt) if d_hidden is not None else None, None, None, None, None, None, None,
                d_hist_in, None, None, None, None, None)


    @staticmethod
    def _backward_with_weights(ctx, d_out32, d_full, d_hidden):
        """The HIP backward with the weights' gradients too: the gate backward
        in fp32 (its d_key / d_value also feed the projection weights'
        gradients, and its score gradient d_s the norm weights'), the two
        weight GEMMs ``d_w_key = d_key^T emb`` and ``d_w_value = d_value^T emb``,
        and ``eg_ple_weight_grads`` for the norms and the convolution."""
        key, value, hidden32, full, s, gate, rstd, nk32, nq32, nc32, conv32, wk32, wv32, pre, emb32 = ctx.saved_tensors
        _eps, dil, detach_value, detach_gate = ctx.cfg
        emb_dt, hidden_dt, hist_dt = ctx.dtypes
        t_len, hc, n = hidden32.shape
        c_dim = hc * n
        h0 = full.shape[0] - t_len
        dev = full.device
        f32 = dict(dtype=torch.float32, device=dev)
        st = _lib.stream_ptr(dev)
        need = ctx.needs_input_grad
        need_emb, need_hist = need[0], need[8]
        need_wk, need_wv, need_nk, need_nq, need_nc, need_cv = need[2:8]
        d_key = torch.empty((t_len, c_dim), **f32) if ((need_emb or need_wk) and not detach_gate) else None
        d_value = torch.empty((t_len, n), **f32) if ((need_emb or need_wv) and not detach_value) else None
        d_s = torch.empty((t_len, hc), **f32)
        _lib.call("eg_ple_gate_backward", _lib.ptr(key), _lib.ptr(value), _lib.ptr(hidden32), _lib.ptr(nk32),
                  _lib.ptr(nq32), _lib.ptr(nc32), _lib.ptr(s), _lib.ptr(gate), _lib.ptr(rstd), _lib.ptr(d_out32),
                  _lib.ptr(d_full[h0:]), t_len, hc, n, int(bool(detach_value)), int(bool(detach_gate)),
                  _lib.ptr(d_key), _lib.ptr(d_value), _lib.ptr(d_hidden), _lib.ptr(d_s), st)
        d_emb = None
        if need_emb:
            parts = [(d, _WT.get(w)) for d, w in ((d_key, wk32), (d_value, wv32)) if d is not None]
            if parts:  # none: both factors detached, emb has no path to the output
                flat = [x for part in parts for x in part]
                d_emb = _projection_backward(ctx.gemm, flat).to(emb_dt)
        wdt = ctx.w_dtypes
        # the projection weights' gradients d_key^T emb and d_value^T emb on eg_gemm_f32
        # (K = the positions); a weight the detached factor cuts off keeps None
        d_wk = _weight_grad(d_key, emb32, wk32, ctx.gemm).to(wdt[0]) if (need_wk and d_key is not None) else None
        d_wv = _weight_grad(d_value, emb32, wv32, ctx.gemm).to(wdt[1]) if (need_wv and d_value is not None) else None
        if detach_gate:  # the gate's whole branch (key, its norm, the query norm) is detached
            need_nk = need_nq = False
        d_nk = d_nq = d_nc = d_cv = None
        if need_nk or need_nq or need_nc or need_cv:
            taps = conv32.shape[1]
            outs = [torch.zeros(c_dim, **f32) for _ in range(3)] + [torch.zeros((c_dim, taps), **f32)]
            if t_len > 0:
                ws_bytes = int(_lib.load().eg_ple_weight_grads_workspace_size(t_len, hc, n, taps))
                ws = torch.empty(max(ws_bytes // 4, 1), **f32)
                _lib.call("eg_ple_weight_grads", _lib.ptr(key), _lib.ptr(value), _lib.ptr(hidden32), _lib.ptr(gate),
                          _lib.ptr(rstd), _lib.ptr(d_s), _lib.ptr(nk32), _lib.ptr(nq32), _lib.ptr(d_out32),
                          _lib.ptr(d_full[h0:]), _lib.ptr(full), h0, _lib.ptr(pre), t_len, hc, n, taps, int(dil),
                          *[_lib.ptr(o) for o in outs], _lib.ptr(ws), ws_bytes, st)
            d_nk = outs[0].to(wdt[2]) if need_nk else None
            d_nq = outs[1].to(wdt[3]) if need_nq else None
            d_nc = outs[2].to(wdt[4]) if need_nc else None
            d_cv = outs[3].to(wdt[5]) if need_cv else None
        d_hist_in = d_full[:h0].reshape(h0, hc, n).to(hist_dt) if need_hist else None
        return (d_emb, d_hidden.to(hidden_dt) if d_hidden is not None else None, d_wk, d_wv, d_nk, d_nq, d_nc, d_cv,
                d_hist_in, None, None, None, None, None)


def ple_forward(emb: torch.Tensor, hidden: torch.Tensor, w: PleWeights, hist: torch.Tensor, hparams,
                diag: dict | None = None, detach_value: bool = False, detach_gate: bool = False,
                gemm: str = "bf16x6") -> tuple[torch.Tensor, torch.Tensor]:
    """``(hidden + gated + conv_out, new history)`` (``engraft/replica/layers.py:
    565-626``).  ``emb [T, n_embd]``, ``hidden [T, hc, n_embd]``, ``hist``
    ``[rows, hc, n_embd]`` (at most ``(K-1)*ple_ngram_size`` rows, empty at a
    sequence start); all on the device.  ``gemm`` picks the projections' GEMM:
    ``"bf16x6"``, the default (``gemm_x6``: the bf16 matrix cores with fp32
    accuracy, its error against float64 below both fp32 paths' and the
    fastest of the three at that accuracy), ``"fp32"`` (``gemm_f32``: fp32
    products on the fp32 matrix cores, the reference's torch matmul
    arithmetic) or ``"bf16x3"`` (``gemm_x3``: 16 mantissa bits per operand,
    about 1e-5 relative per projection, 1.7x faster than bf16x6)."""
    if gemm not in ("fp32", "bf16x3", "bf16x6"):
        raise ValueError(f"gemm must be 'fp32', 'bf16x3' or 'bf16x6', got {gemm!r}")
    hc = hparams.hc_mult
    n = hparams.n_embd
    eps = float(hparams.f_norm_rms_eps)
    dil = int(hparams.ple_ngram_size)
    if hidden.dim() != 3 or hidden.shape[1:] != (hc, n) or emb.shape != (hidden.shape[0], n):
        raise ValueError(f"emb [T, {n}] and hidden [T, {hc}, {n}] expected, got {tuple(emb.shape)}, "
                         f"{tuple(hidden.shape)}")
    hist = hist.reshape(-1, hc, n) if hist.numel() else hidden.new_zeros((0, hc, n))
    out, new_hist, s, gate, value = _PleFn.apply(emb, hidden, w.w_key, w.w_value, w.norm_key, w.norm_query,
                                                 w.norm_conv, w.conv1d, hist, eps, dil, detach_value, detach_gate,
                                                 gemm)
    if diag is not None:
        gated_norm = value.norm(dim=-1, keepdim=True) * gate.abs()
        diag["s"] = s.clone()
        diag["gate"] = gate.clone()
        diag["value_norm"] = value.norm(dim=-1).clone()
        diag["gated_norm"] = gated_norm.clone()
        diag["hidden_norm"] = hidden.detach().norm(dim=-1).clone()
    return out, new_hist


# ---------------------------------------------------------------------------------------------
# PleReplica (engraft/lens.py:221-415): the block with weights read from a model GGUF
# ---------------------------------------------------------------------------------------------

def _ple_tensor_types():
    from .ggufio import GGML_TYPE_F32, GGML_TYPE_Q8_0
    return {"ple_key": GGML_TYPE_Q8_0, "ple_value": GGML_TYPE_Q8_0, "ple_norm_key": GGML_TYPE_F32,
            "ple_norm_query": GGML_TYPE_F32, "ple_norm_conv": GGML_TYPE_F32, "ple_conv1d": GGML_TYPE_F32}


class PleReplica:
    """The PLE block of one layer on the device, method for method as
    ``engraft.lens.PleReplica`` (``engraft/lens.py:221-415``).

    Inputs are numpy arrays or tensors; results are f32 tensors on the device
    (the reference returns numpy: ``.cpu().numpy()`` gives the same layout).
    ``key``/``value`` are library GEMMs plus ``eg_ple_rms``; ``gate``,
    ``gated`` and ``ple_out`` run ``eg_ple_gate`` and ``eg_ple_conv``;
    ``conv_out`` runs ``eg_ple_rms`` and ``eg_ple_conv``; ``ple_out_at`` runs
    ``eg_ple_conv`` with one history shared by the batch.  The reference fixes
    4 streams of 2560 values, 4 taps and dilation 3; here the widths come from
    the tensors (``hc`` streams) and the dilation is a parameter.

    Attributes as the reference's: ``w_key [hc*n, n]``, ``w_value [n, n]``,
    ``norm_key``/``norm_query``/``norm_conv [hc, n]``, ``conv1d [hc, n, taps]``
    (in place: zeroing it switches the convolution off, as
    ``tests/test_lens.py:336-342`` does) and ``eps``."""

    def __init__(self, gguf_path, eps: float | None = None, *, device="cuda", hc: int = 4, dilation: int = 3,
                 layer: int = 1):
        from .ggufio import read_gguf, read_rms_eps, read_tensor_f32
        gf = read_gguf(gguf_path)
        types = _ple_tensor_types()
        ld = {k: read_tensor_f32(gf, f"blk.{layer}.{k}.weight", t) for k, t in types.items()}
        if eps is None:
            eps = read_rms_eps(gguf_path)
        self._setup(ld["ple_key"], ld["ple_value"], ld["ple_norm_key"], ld["ple_norm_query"], ld["ple_norm_conv"],
                    ld["ple_conv1d"], float(eps), hc, dilation, device)
        self.gguf_path = gguf_path

    @classmethod
    def from_weights(cls, w: PleWeights, eps: float, *, hc: int = 4, dilation: int = 3, device="cuda"):
        obj = cls.__new__(cls)
        obj._setup(w.w_key, w.w_value, w.norm_key, w.norm_query, w.norm_conv, w.conv1d, float(eps), hc, dilation,
                   device)
        obj.gguf_path = None
        return obj

    def _setup(self, w_key, w_value, nk, nq, nc, conv, eps, hc, dilation, device):
        f = lambda x: torch.as_tensor(x, dtype=torch.float32).to(device).contiguous()
        w_value = f(w_value)
        n = int(w_value.shape[0])
        if w_value.dim() != 2 or w_value.shape[1] != n:
            raise ValueError(f"ple_value: unexpected shape {tuple(w_value.shape)}")
        w_key = f(w_key)
        if tuple(w_key.shape) != (hc * n, n):
            raise ValueError(f"ple_key: unexpected shape {tuple(w_key.shape)}, expected {(hc * n, n)}")
        norms = []
        for name, arr in (("ple_norm_key", nk), ("ple_norm_query", nq), ("ple_norm_conv", nc)):
            a = f(arr)
            if a.numel() != hc * n:
                raise ValueError(f"{name}: unexpected shape {tuple(a.shape)}")
            norms.append(a.reshape(hc, n))
        conv = f(conv)
        if conv.dim() not in (2, 3) or conv.numel() % (hc * n) or not 1 <= conv.numel() // (hc * n) <= 8:
            raise ValueError(f"ple_conv1d: unexpected shape {tuple(conv.shape)}")
        self.hc, self.n_embd, self.dilation, self.eps = hc, n, int(dilation), float(eps)
        self.device = w_value.device
        self.w_key, self.w_value = w_key, w_value
        self.norm_key, self.norm_query, self.norm_conv = norms
        self.conv1d = conv.reshape(hc, n, -1)  # [stream, channel, tap], the kernel's [hc*n, taps] memory

    # ---- pieces ---------------------------------------------------------------------------
    def _in(self, x, *shape_tail) -> torch.Tensor:
        t = torch.as_tensor(x, dtype=torch.float32).to(self.device).contiguous()
        if tuple(t.shape[1:]) != shape_tail:
            raise ValueError(f"expected [T, {', '.join(map(str, shape_tail))}], got {tuple(t.shape)}")
        return t

    def _rms(self, x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
        out = torch.empty_like(x)
        _lib.call("eg_ple_rms", _lib.ptr(x), x.shape[0], self.hc, self.n_embd, _lib.ptr(weight), self.eps,
                  _lib.ptr(out), _lib.stream_ptr(self.device))
        return out

    def _gate_pass(self, emb: torch.Tensor, hidden: torch.Tensor):
        """value [T, n], normed [T, hc*n], s and gate [T, hc] (eg_ple_gate)."""
        t_len = emb.shape[0]
        key, value = gemm_f32(emb, self.w_key, b_n2=self.w_value)
        f32 = dict(dtype=torch.float32, device=self.device)
        normed = torch.empty((t_len, self.hc * self.n_embd), **f32)
        s = torch.empty((t_len, self.hc), **f32)
        gate = torch.empty((t_len, self.hc), **f32)
        _lib.call("eg_ple_gate", _lib.ptr(key), _lib.ptr(value), _lib.ptr(hidden), _lib.ptr(self.norm_key),
                  _lib.ptr(self.norm_query), _lib.ptr(self.norm_conv), t_len, self.hc, self.n_embd, self.eps,
                  _lib.ptr(normed), _lib.ptr(s), _lib.ptr(gate), None, _lib.stream_ptr(self.device))
        return value, normed, s, gate

    def _conv(self, full: torch.Tensor, hist_rows: int, n_pos: int, value=None, gate=None,
              shared: bool = False) -> torch.Tensor:
        out = torch.empty((n_pos, self.hc, self.n_embd), dtype=torch.float32, device=self.device)
        taps = self.conv1d.shape[2]
        _lib.call("eg_ple_conv", _lib.ptr(full), hist_rows, n_pos, self.hc, self.n_embd, _lib.ptr(self.conv1d), taps,
                  self.dilation, 1 if shared else 0, None, _lib.ptr(value), _lib.ptr(gate), _lib.ptr(out), None,
                  _lib.stream_ptr(self.device))
        return out

    # ---- the reference's methods ----------------------------------------------------------
    def key(self, emb) -> torch.Tensor:
        """``[T, n] -> [T, hc, n]``, RMS-normalised per stream (``lens.py:289-294``)."""
        emb = self._in(emb, self.n_embd)
        raw = gemm_f32(emb, self.w_key)
        return self._rms(raw, self.norm_key).reshape(-1, self.hc, self.n_embd)

    def value(self, emb) -> torch.Tensor:
        """``[T, n] -> [T, n]`` (``lens.py:296-299``)."""
        return gemm_f32(self._in(emb, self.n_embd), self.w_value)

    def gate(self, emb, hidden) -> torch.Tensor:
        """``[T, hc]`` (``lens.py:301-312``)."""
        return self._gate_pass(self._in(emb, self.n_embd), self._in(hidden, self.hc, self.n_embd))[3]

    def gated(self, emb, hidden) -> torch.Tensor:
        """``[T, hc, n]`` = value replicated over the streams x gate (``lens.py:314-318``)."""
        value, _, _, gate = self._gate_pass(self._in(emb, self.n_embd), self._in(hidden, self.hc, self.n_embd))
        return value[:, None, :] * gate[:, :, None]

    def conv_out(self, gated_seq) -> torch.Tensor:
        """norm_conv, the dilated causal convolution over zero history, SiLU
        (``lens.py:320-339``)."""
        g = self._in(gated_seq, self.hc, self.n_embd)
        normed = self._rms(g, self.norm_conv)
        return self._conv(normed, 0, g.shape[0])

    def ple_out(self, emb_seq, hidden_seq) -> torch.Tensor:
        """``gated + conv_out(gated)`` over a whole sequence (``lens.py:341-345``);
        the caller adds ``hidden``."""
        emb = self._in(emb_seq, self.n_embd)
        value, normed, _, gate = self._gate_pass(emb, self._in(hidden_seq, self.hc, self.n_embd))
        return self._conv(normed, 0, emb.shape[0], value, gate)

    def ple_out_at(self, emb_t, emb_seq, hidden_seq, t: int) -> torch.Tensor:
        """``[B, hc, n]``: ``ple_out[t]`` with ``emb_seq[t]`` replaced by each row of
        ``emb_t [B, n]``, the convolution history from the true sequence
        (``lens.py:347-385``)."""
        emb_t = self._in(emb_t, self.n_embd)
        emb_seq = self._in(emb_seq, self.n_embd)
        hidden_seq = self._in(hidden_seq, self.hc, self.n_embd)
        if not 0 <= t < emb_seq.shape[0]:
            raise ValueError(f"t={t} outside the sequence of {emb_seq.shape[0]} positions")
        b = emb_t.shape[0]
        h0 = min(t, (self.conv1d.shape[2] - 1) * self.dilation)
        hid_b = hidden_seq[t].expand(b, self.hc, self.n_embd).contiguous()
        value, normed_b, _, gate = self._gate_pass(emb_t, hid_b)
        if h0:
            normed_h = self._gate_pass(emb_seq[t - h0:t].contiguous(), hidden_seq[t - h0:t].contiguous())[1]
            full = torch.cat([normed_h, normed_b], dim=0)
        else:
            full = normed_b
        return self._conv(full, h0, b, value, gate, shared=True)

    def jacobian_out(self, emb_seq, hidden_seq, t: int, coords=None, step: float = 1e-3) -> torch.Tensor:
        """f64 ``[hc*n, n_coords]``: d ple_out[t] / d emb[t][coords] by central
        differences of ``ple_out_at``, 512 coordinates per batch
        (``lens.py:387-415``)."""
        emb_seq = self._in(emb_seq, self.n_embd)
        hidden_seq = self._in(hidden_seq, self.hc, self.n_embd)
        coords = torch.arange(self.n_embd) if coords is None else torch.as_tensor(np.asarray(coords),
                                                                                   dtype=torch.int64)
        coords = coords.to(self.device)
        jac = torch.empty((self.hc * self.n_embd, coords.numel()), dtype=torch.float64, device=self.device)
        for lo in range(0, coords.numel(), 512):
            idx = coords[lo:lo + 512]
            m = idx.numel()
            plus = emb_seq[t].expand(m, self.n_embd).clone()
            minus = plus.clone()
            r = torch.arange(m, device=self.device)
            plus[r, idx] += step
            minus[r, idx] -= step
            out = self.ple_out_at(torch.cat([plus, minus]), emb_seq, hidden_seq, t).reshape(2 * m, -1)
            jac[:, lo:lo + m] = ((out[:m].double() - out[m:].double()) / (2.0 * step)).T
        return jac
