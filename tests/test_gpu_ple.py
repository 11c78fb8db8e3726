"""GPU parity of the PLE block (ple_forward) against the torch fp32 oracle on
the CPU: the real dimensions (hc 4, n_embd 2560, 4 taps, dilation 3),
a sequence in two chunks with the history carried, and the gradient.

Bar (floating point, as the reference's own check of its two formulations,
tests/test_replica_layers.py:282): |out - oracle| <= 1e-4; history 1e-5;
gradients within 1e-4 relative of the largest entry.  With gemm="bf16x3" (the
projections on the bf16 matrix cores, 16 mantissa bits per operand: about 1e-5
relative per projection output) the output and gradient bars are the same and
the history, gate and score bars are 1e-4, 5e-5 and 1e-4 (measured: 2.1e-5,
7.8e-6 and 1.7e-5 on O(1)-O(5) values; the fp32 path: 3.6e-6, 5.1e-7, 1.4e-6).
With gemm="bf16x6" (three bf16 planes an operand, six products) the fp32
bars hold."""
from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

from oracle import ple as P
from tests.test_oracle_ple import ple_weights

pytestmark = pytest.mark.gpu


def _say(msg: str) -> None:
    print(f"[gpu-test] {msg}", file=sys.stderr, flush=True)


class _HP:
    hc_mult = 4
    n_embd = 2560
    f_norm_rms_eps = 1e-6
    ple_ngram_size = 3


def _dev_weights(w, dev):
    from engraft_ngram_amd.ple import PleWeights
    return PleWeights(**{k: v.to(dev) for k, v in w.items()})


# bf16x6 (three bf16 planes an operand, six products: fp32 accuracy) is held
# to the fp32 bars
_BARS = {"fp32": (1e-5, 1e-5, 1e-4), "bf16x3": (1e-4, 5e-5, 1e-4), "bf16x6": (1e-5, 1e-5, 1e-4)}  # history, gate, score


@pytest.mark.parametrize("gemm", ["fp32", "bf16x3", "bf16x6"])
def test_ple_forward_against_oracle(cuda, gemm):
    from engraft_ngram_amd import ple
    print(f"[gpu-test] ple_forward gemm={gemm}", file=sys.stderr, flush=True)
    bar_h, bar_g, bar_s = _BARS[gemm]
    hc, n, T = 4, 2560, 48
    w = ple_weights(hc, n, seed=3)
    wd = _dev_weights(w, cuda)
    g = torch.Generator().manual_seed(4)
    emb = torch.randn((T, n), generator=g) * 0.1
    hidden = torch.randn((T, hc, n), generator=g) * 0.1
    # two chunks, the history of the first fed to the second
    hist_c = torch.zeros(0, hc, n)
    hist_d = torch.zeros(0, hc, n, device=cuda)
    diag = {}
    for lo, hi in ((0, 30), (30, T)):
        exp, hist_c, s_c, gate_c = P.ple_forward(emb[lo:hi], hidden[lo:hi], w, hist_c, hc, n, 1e-6, 3)
        got, hist_d = ple.ple_forward(emb[lo:hi].to(cuda), hidden[lo:hi].to(cuda), wd, hist_d, _HP, diag=diag,
                                      gemm=gemm)
        err = (got.cpu() - exp).abs().max().item()
        assert err <= 1e-4, f"chunk [{lo},{hi}): max |diff| {err}"
        assert (hist_d.cpu() - hist_c).abs().max().item() <= bar_h
        assert (diag["gate"].cpu() - gate_c).abs().max().item() <= bar_g
        assert (diag["s"].cpu() - s_c).abs().max().item() <= bar_s
    assert hist_d.shape == (9, hc, n)


def test_ple_forward_gradient(cuda):
    """d(sum(out * R))/d(emb, hidden) against torch autograd of the oracle on the
    CPU; detach_gate keeps only the value path's share of the emb gradient."""
    from engraft_ngram_amd import ple
    hc, n, T = 4, 2560, 12
    w = ple_weights(hc, n, seed=5)
    wd = _dev_weights(w, cuda)
    g = torch.Generator().manual_seed(6)
    emb = torch.randn((T, n), generator=g) * 0.1
    hidden = torch.randn((T, hc, n), generator=g) * 0.1
    r = torch.randn((T, hc, n), generator=g)
    e_c = emb.clone().requires_grad_(True)
    h_c = hidden.clone().requires_grad_(True)
    out_c, _, _, _ = P.ple_forward(e_c, h_c, w, torch.zeros(0, hc, n), hc, n, 1e-6, 3)
    (out_c * r).sum().backward()
    e_d = emb.to(cuda).requires_grad_(True)
    h_d = hidden.to(cuda).requires_grad_(True)
    out_d, _ = ple.ple_forward(e_d, h_d, wd, torch.zeros(0, hc, n, device=cuda), _HP)
    (out_d * r.to(cuda)).sum().backward()
    for got, exp in ((e_d.grad, e_c.grad), (h_d.grad, h_c.grad)):
        scale = exp.abs().max().item()
        assert (got.cpu() - exp).abs().max().item() <= 1e-4 * scale
    # detach_gate: forward unchanged, the gate's share of the gradient removed
    e2 = emb.to(cuda).requires_grad_(True)
    out2, _ = ple.ple_forward(e2, hidden.to(cuda), wd, torch.zeros(0, hc, n, device=cuda), _HP, detach_gate=True)
    assert torch.equal(out2, out_d.detach())
    (out2 * r.to(cuda)).sum().backward()
    assert not torch.allclose(e2.grad, e_d.grad)


def test_ple_history_gradient_across_chunks(cuda):
    """The history returned by one chunk carries the gradient into the next, as
    the reference's differentiable ``new_hist`` (layers.py:623-626): the loss of
    chunk 2 reaches chunk 1's emb."""
    from engraft_ngram_amd import ple
    hc, n = 4, 2560
    w = ple_weights(hc, n, seed=8)
    wd = _dev_weights(w, cuda)
    g = torch.Generator().manual_seed(9)
    emb = torch.randn((14, n), generator=g) * 0.1
    hidden = torch.randn((14, hc, n), generator=g) * 0.1
    r = torch.randn((6, hc, n), generator=g)
    e_c = emb.clone().requires_grad_(True)
    _, h1, _, _ = P.ple_forward(e_c[:8], hidden[:8], w, torch.zeros(0, hc, n), hc, n, 1e-6, 3)
    out2, _, _, _ = P.ple_forward(e_c[8:], hidden[8:], w, h1, hc, n, 1e-6, 3)
    (out2 * r).sum().backward()
    e_d = emb.to(cuda).requires_grad_(True)
    hd = hidden.to(cuda)
    _, h1d = ple.ple_forward(e_d[:8], hd[:8], wd, torch.zeros(0, hc, n, device=cuda), _HP)
    out2d, _ = ple.ple_forward(e_d[8:], hd[8:], wd, h1d, _HP)
    (out2d * r.to(cuda)).sum().backward()
    scale = e_c.grad.abs().max().item()
    assert e_c.grad[:8].abs().max().item() > 0  # the first chunk does receive gradient
    assert (e_d.grad.cpu() - e_c.grad).abs().max().item() <= 1e-4 * scale


@pytest.mark.parametrize("dv,dg,gemm", [(False, False, "fp32"), (True, False, "fp32"), (False, True, "fp32"),
                                        (False, False, "bf16x3"), (True, False, "bf16x3"), (False, False, "bf16x6"),
                                        (False, False, None)])
def test_ple_native_backward_against_oracle(cuda, dv, dg, gemm):
    """The HIP backward (no weight gradients): d_emb, d_hidden and the incoming
    history's gradient, with a gradient on the returned history too, against
    autograd of the oracle on the CPU (T 40 after a 9-row history), for the
    plain block and with either factor of gated detached; the projections run
    on the library's GEMM of the chosen arithmetic (eg_gemm_f32,
    eg_gemm_bf16x3 or eg_gemm_bf16x6; None: ple_forward's default, bf16x6),
    key and value as one call and the backward's d_emb as one call over two K
    segments."""
    from engraft_ngram_amd import _lib, ple
    print(f"[gpu-test] ple native backward detach_value={dv} detach_gate={dg} gemm={gemm}", file=sys.stderr,
          flush=True)
    hc, n, T = 4, 2560, 40
    w = ple_weights(hc, n, seed=31)
    wd = _dev_weights(w, cuda)
    g = torch.Generator().manual_seed(32)
    emb = torch.randn((T, n), generator=g) * 0.1
    hidden = torch.randn((T, hc, n), generator=g) * 0.1
    hist = torch.randn((9, hc, n), generator=g) * 0.1
    r = torch.randn((T, hc, n), generator=g)
    rh = torch.randn((9, hc, n), generator=g)
    leaves_c = [x.clone().requires_grad_(True) for x in (emb, hidden, hist)]
    out_c, nh_c, _, _ = P.ple_forward(*leaves_c[:2], w, leaves_c[2], hc, n, 1e-6, 3, detach_value=dv, detach_gate=dg)
    ((out_c * r).sum() + (nh_c * rh).sum()).backward()
    leaves_d = [x.to(cuda).requires_grad_(True) for x in (emb, hidden, hist)]
    called = []
    real_call = _lib.call

    def spy(name, *args):
        called.append(name)
        return real_call(name, *args)

    _lib.call = spy
    try:
        kw = {} if gemm is None else {"gemm": gemm}
        out_d, nh_d = ple.ple_forward(leaves_d[0], leaves_d[1], wd, leaves_d[2], _HP, detach_value=dv,
                                      detach_gate=dg, **kw)
        ((out_d * r.to(cuda)).sum() + (nh_d * rh.to(cuda)).sum()).backward()
    finally:
        _lib.call = real_call
    gate_bwd = "eg_ple_gate_backward_planes" if gemm == "bf16x3" else "eg_ple_gate_backward"
    assert "eg_ple_conv_backward" in called and gate_bwd in called  # bf16x3: d_key, d_value written as planes
    mode = gemm or "bf16x6"
    entry = {"fp32": "eg_gemm_f32", "bf16x3": "eg_gemm_bf16x3", "bf16x6": "eg_gemm_bf16x6"}
    assert called.count(entry[mode]) == 2  # key + value in one call, then d_emb
    assert not any(entry[o] in called for o in entry if o != mode)
    for name, got, exp in zip(("emb", "hidden", "hist"), (x.grad for x in leaves_d), (x.grad for x in leaves_c)):
        scale = exp.abs().max().item()
        err = (got.cpu() - exp).abs().max().item()
        assert err <= 1e-4 * scale, f"d_{name}: {err} vs scale {scale}"


_WEIGHTS = ("w_key", "w_value", "norm_key", "norm_query", "norm_conv", "conv1d")


def _grad_close(got, exp, tol, name):
    """``got`` within ``tol`` of ``exp``'s largest entry; a gradient the
    oracle's autograd never reached (``None``) must be absent too (an
    optimizer skips a None gradient but steps a zero one)."""
    if exp is None:
        assert got is None, name
        return
    assert got is not None, name
    scale = max(exp.abs().max().item(), 1e-30)
    err = (got.detach().cpu().to(exp.dtype) - exp).abs().max().item()
    assert err <= tol * scale, f"{name}: {err / scale:.2e} of its largest entry"


@pytest.mark.parametrize("gemm,dv,dg", [("fp32", False, False), ("bf16x3", False, False), ("fp32", True, False),
                                        ("fp32", False, True), ("fp32", True, True), ("bf16x6", False, False)])
def test_ple_weight_gradients_native(cuda, gemm, dv, dg):
    """Every weight's gradient (w_key, w_value, the three norms, the conv taps)
    together with emb's, hidden's and the history's, from the HIP backward
    (eg_ple_gate_backward's d_s, the weight GEMMs, eg_ple_weight_grads)
    against autograd of the oracle on the CPU in float64: 150 positions after a 9-row
    history (three 64-position partial sums), a gradient on the new history
    too, with detach_value / detach_gate."""
    from engraft_ngram_amd import ple
    _say(f"PLE weight gradients {gemm} dv={dv} dg={dg}")
    hc, n, T, H = 4, 2560, 150, 9
    w = ple_weights(hc, n, seed=41)
    g = torch.Generator().manual_seed(42)
    emb = torch.randn((T, n), generator=g) * 0.1
    hidden = torch.randn((T, hc, n), generator=g) * 0.1
    hist = torch.randn((H, hc, n), generator=g) * 0.5
    r = torch.randn((T, hc, n), generator=g)
    rh = torch.randn((H, hc, n), generator=g)

    def oracle(dt, perm=None):
        # perm: the projections' K (emb's columns, the weights' columns) taken
        # in another order -- the same sums, another fp32 rounding
        wp = dict(w)
        ep = emb
        if perm is not None:
            ep = emb[:, perm]
            wp["w_key"], wp["w_value"] = w["w_key"][:, perm], w["w_value"][:, perm]
        wc = {k: v.clone().to(dt).requires_grad_(True) for k, v in wp.items()}
        xc = [x.clone().to(dt).requires_grad_(True) for x in (ep, hidden, hist)]
        out_c, nh_c, _, _ = P.ple_forward(*xc[:2], wc, xc[2], hc, n, 1e-6, 3, dv, dg)
        ((out_c * r.to(dt)).sum() + (nh_c * rh.to(dt)).sum()).backward()
        res = {"emb": xc[0].grad, "hidden": xc[1].grad, "hist": xc[2].grad, **{k: wc[k].grad for k in _WEIGHTS}}
        if perm is not None:
            inv = torch.argsort(perm)
            for k in ("emb", "w_key", "w_value"):
                if res[k] is not None:
                    res[k] = res[k][:, inv]
        return res

    ref64 = oracle(torch.float64)
    gp = torch.Generator().manual_seed(43)
    refs32 = [oracle(torch.float32)] + [oracle(torch.float32, torch.randperm(n, generator=gp)) for _ in range(2)]
    wd = ple.PleWeights(**{k: v.to(cuda).requires_grad_(True) for k, v in w.items()})
    xd = [x.to(cuda).requires_grad_(True) for x in (emb, hidden, hist)]
    out_d, nh_d = ple.ple_forward(xd[0], xd[1], wd, xd[2], _HP, detach_value=dv, detach_gate=dg, gemm=gemm)
    ((out_d * r.to(cuda)).sum() + (nh_d * rh.to(cuda)).sum()).backward()
    got = {"emb": xd[0].grad, "hidden": xd[1].grad, "hist": xd[2].grad, **{k: getattr(wd, k).grad for k in _WEIGHTS}}
    # Against the float64 oracle.  fp32 projections: 1e-4 of the largest
    # entry, or 3x the spread of fp32 oracles (the projections' K summed in
    # three orders) around float64 where that is larger.  The score's gradient
    # goes through the gate's 1/sqrt|s| derivative, which at a position with a
    # small |s| (150 positions reach |s| ~ 1.6e-3) amplifies the projections'
    # rounding: fp32 oracles land 2e-5 .. 2e-4 off float64 in the hidden,
    # w_key and key / query norm gradients, depending on the summation order
    # alone.  bf16x3 (16-bit mantissas in the projections): 2e-3.  bf16x6
    # (the projections and the weight GEMMs at fp32 accuracy): the fp32 bar.
    for name, exp in ref64.items():
        if exp is None:
            _grad_close(got[name], None, 0.0, name)
            continue
        scale = exp.abs().max().clamp_min(1e-300)
        spread = max(float((ref[name].double() - exp).abs().max() / scale) for ref in refs32)
        tol = max(3 * spread, 1e-4) if gemm in ("fp32", "bf16x6") else 2e-3
        _grad_close(got[name], exp, tol, name)


def test_ple_weight_gradients_recompute_path(cuda):
    """A convolution reaching back beyond the HIP backward's 32 rows (4 taps at
    dilation 12) goes through the torch recomputation of the block: the
    gradients of w_key, norm_conv and the taps, and of emb, against autograd
    of the oracle on the CPU."""
    from engraft_ngram_amd import ple

    class HP12(_HP):
        ple_ngram_size = 12

    hc, n, T = 4, 2560, 40
    w = ple_weights(hc, n, seed=41)
    g = torch.Generator().manual_seed(42)
    emb = torch.randn((T, n), generator=g) * 0.1
    hidden = torch.randn((T, hc, n), generator=g) * 0.1
    r = torch.randn((T, hc, n), generator=g)
    wc = {k: (v.clone().requires_grad_(k in ("w_key", "norm_conv", "conv1d"))) for k, v in w.items()}
    e_c = emb.clone().requires_grad_(True)
    out_c, _, _, _ = P.ple_forward(e_c, hidden, wc, torch.zeros(0, hc, n), hc, n, 1e-6, 12)
    (out_c * r).sum().backward()
    assert not ple._native_backward_ok(hc, n, 4, 12)
    wd = ple.PleWeights(**{k: v.to(cuda).requires_grad_(k in ("w_key", "norm_conv", "conv1d"))
                           for k, v in w.items()})
    e_d = emb.to(cuda).requires_grad_(True)
    out_d, _ = ple.ple_forward(e_d, hidden.to(cuda), wd, torch.zeros(0, hc, n, device=cuda), HP12)
    (out_d * r.to(cuda)).sum().backward()
    for got, exp in ((e_d.grad, e_c.grad), (wd.w_key.grad, wc["w_key"].grad), (wd.norm_conv.grad, wc["norm_conv"].grad),
                     (wd.conv1d.grad, wc["conv1d"].grad)):
        scale = exp.abs().max().item()
        assert (got.cpu() - exp).abs().max().item() <= 1e-4 * scale


def test_ple_nine_taps_rejected(cuda):
    """The convolution kernels are built for 1..8 taps (the reference's
    blocks have 4): nine taps are refused by the forward with a ValueError
    naming the taps, before any launch, whatever gradients are asked for;
    the backward's limit check agrees (no tap count above 8 reaches the
    weight-gradient kernel)."""
    from engraft_ngram_amd import ple

    class HP1(_HP):
        n_embd = 256
        ple_ngram_size = 1

    hc, n, T, taps = 4, 256, 40, 9
    g = torch.Generator().manual_seed(61)
    w = ple_weights(hc, n, taps=taps, seed=62)
    emb = torch.randn((T, n), generator=g) * 0.1
    hidden = torch.randn((T, hc, n), generator=g) * 0.1
    assert not ple._native_backward_ok(hc, n, taps, 1, weights=True)
    assert ple._native_backward_ok(hc, n, 8, 1, weights=True)
    for need in ((), ("conv1d", "norm_conv")):
        wd = ple.PleWeights(**{k: v.to(cuda).requires_grad_(k in need) for k, v in w.items()})
        with pytest.raises(ValueError, match="taps=9"):
            ple.ple_forward(emb.to(cuda), hidden.to(cuda), wd, torch.zeros(0, hc, n, device=cuda), HP1)


def test_conv_backward_stored_preactivation_equals_recompute(cuda):
    """eg_ple_conv_backward with the forward's stored pre-activation (what
    ple_forward's backward uses) and without it (recomputing the convolution
    from full): bit-identical, the forward and backward sum their taps in the
    same order."""
    from engraft_ngram_amd import _lib
    _say = lambda m: print(f"[gpu-test] {m}", file=sys.stderr, flush=True)
    _say("conv backward, stored pre-activation vs recompute")
    g = torch.Generator(device=cuda).manual_seed(51)
    hc, n, T, h0, taps, dil = 4, 256, 37, 9, 4, 3
    C = hc * n
    full = torch.randn(h0 + T, C, generator=g, device=cuda)
    conv = torch.randn(C, taps, generator=g, device=cuda) * 0.5
    hidden = torch.randn(T, C, generator=g, device=cuda)
    value = torch.randn(T, n, generator=g, device=cuda)
    gate = torch.rand(T, hc, generator=g, device=cuda)
    out = torch.empty(T, C, device=cuda)
    pre = torch.empty(T, C, device=cuda)
    st = _lib.stream_ptr(cuda)
    _lib.call("eg_ple_conv", _lib.ptr(full), h0, T, hc, n, _lib.ptr(conv), taps, dil, 0, _lib.ptr(hidden),
              _lib.ptr(value), _lib.ptr(gate), _lib.ptr(out), _lib.ptr(pre), st)
    d_out = torch.randn(T, C, generator=g, device=cuda)
    d_tail = torch.randn(9, C, generator=g, device=cuda)
    res = []
    for p in (pre, None):
        d_full = torch.empty(h0 + T, C, device=cuda)
        _lib.call("eg_ple_conv_backward", _lib.ptr(full), h0, T, hc, n, _lib.ptr(conv), taps, dil, _lib.ptr(p),
                  _lib.ptr(d_out), _lib.ptr(d_tail), 9, _lib.ptr(d_full), st)
        res.append(d_full)
    torch.cuda.synchronize()
    assert torch.equal(res[0], res[1])
    # the stored pre-activation is the convolution itself
    ref = torch.zeros(T, C, device=cuda, dtype=torch.float64)
    for k in range(taps):
        back = (taps - 1 - k) * dil
        ref += full[h0 - back:h0 + T - back].double() * conv[:, k].double()
    assert float((pre.double() - ref).abs().max()) <= 1e-5


@pytest.mark.parametrize("gemm", ["fp32", "bf16x3"])
def test_ple_forward_checkpointed_bit_identical(cuda, gemm):
    """As tests/test_seq.py:91-112 does for a whole layer: wrapping the block in
    torch.utils.checkpoint (the forward recomputed during the backward) changes
    nothing -- output, loss and the gradients of emb and hidden are torch.equal
    with and without it (every kernel on the path is deterministic)."""
    from torch.utils.checkpoint import checkpoint

    from engraft_ngram_amd import ple
    print(f"[gpu-test] ple_forward under checkpoint gemm={gemm}", file=sys.stderr, flush=True)
    hc, n, T = 4, 2560, 24
    w = ple_weights(hc, n, seed=61)
    wd = _dev_weights(w, cuda)
    g = torch.Generator().manual_seed(62)
    emb = (torch.randn((T, n), generator=g) * 0.1).to(cuda)
    hidden = (torch.randn((T, hc, n), generator=g) * 0.1).to(cuda)
    r = torch.randn((T, hc, n), generator=g).to(cuda)
    h0 = torch.zeros(0, hc, n, device=cuda)

    def block(e, h):
        return ple.ple_forward(e, h, wd, h0, _HP, gemm=gemm)[0]

    res = []
    for ckpt in (False, True):
        e = emb.clone().requires_grad_(True)
        h = hidden.clone().requires_grad_(True)
        out = checkpoint(block, e, h, use_reentrant=False) if ckpt else block(e, h)
        loss = (out * r).sum()
        loss.backward()
        res.append((out.detach(), loss.detach(), e.grad, h.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def _conv_pre(full, h0, T, hc, n, w, dil, dev):
    """eg_ple_conv's pre-activation (no hidden / value: out = silu(conv))."""
    from engraft_ngram_amd import _lib
    full = full.to(dev).contiguous()
    w = w.to(dev).contiguous()
    out = torch.empty((T, hc * n), device=dev)
    pre = torch.empty((T, hc * n), device=dev)
    _lib.call("eg_ple_conv", _lib.ptr(full), h0, T, hc, n, _lib.ptr(w), w.shape[1], dil, 0, None, None, None,
              _lib.ptr(out), _lib.ptr(pre), _lib.stream_ptr(dev))
    return out.cpu(), pre.cpu()


@pytest.mark.parametrize("taps,dil,h0", [(3, 2, 0), (3, 2, 3), (2, 5, 1), (6, 1, 2)])
def test_generic_conv_other_shapes_against_oracle(cuda, taps, dil, h0):
    """The generic convolution kernel (every tap count and dilation other than
    the model's 4 taps at dilation 3), with an empty, short or partial
    history, against the oracle's causal_depthwise_conv; out = silu(pre)."""
    hc, n, T = 2, 640, 70
    g = torch.Generator().manual_seed(60 + taps * 10 + dil)
    full = torch.randn((h0 + T, hc * n), generator=g)
    w = torch.randn((hc * n, taps), generator=g) * 0.5
    out, pre = _conv_pre(full, h0, T, hc, n, w, dil, cuda)
    exp = P.causal_depthwise_conv(full[h0:], full[:h0], w, dilation=dil)
    assert (pre - exp).abs().max().item() <= 1e-6 * max(exp.abs().max().item(), 1.0)
    assert (out - torch.nn.functional.silu(pre)).abs().max().item() <= 1e-6


def test_window_conv_equals_generic_conv(cuda):
    """The model's shape (4 taps, dilation 3) runs on the register-window
    kernel; the same convolution as 5 taps whose oldest tap is zero runs on the
    generic kernel.  Both give the same pre-activation."""
    hc, n, T, h0 = 4, 2560, 100, 9
    g = torch.Generator().manual_seed(71)
    full = torch.randn((h0 + T, hc * n), generator=g)
    w4 = torch.randn((hc * n, 4), generator=g) * 0.5
    w5 = torch.cat([torch.zeros((hc * n, 1)), w4], dim=1)
    _, pre4 = _conv_pre(full, h0, T, hc, n, w4, 3, cuda)
    _, pre5 = _conv_pre(full, h0, T, hc, n, w5, 3, cuda)
    assert (pre4 - pre5).abs().max().item() <= 1e-6 * pre4.abs().max().item()
