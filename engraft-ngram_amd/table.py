"""Device-resident n-gram (PLE) table: the drop-in for ``engraft.table``.

``DeviceTable`` is the table duck type every caller of the reference uses
(``PleTable``, ``engraft/table.py:40-144``; ``FakeTable``,
``engraft/testing/fake_table.py:23-76``): the attributes ``eos_token_id,
image_token_id, ngram_size, heads_per_ngram, layer_multipliers,
head_vocab_sizes, head_offsets, n_heads, heads`` and the methods
``read_rows_raw``, ``read_rows`` and ``ngram_addresses`` keep their names,
argument meaning, return types and errors.  The rows live in HBM in one merged
array indexed by global row id (``head_offsets[h] + local``), and every method
runs on the HIP library (``libengraft_ngram.so``): the hash, the gather and the
dequantisation never execute on the CPU.

Row formats (``fmt``): ``"iq4_nl"`` (the reference's real format, 90-byte rows
of 160 values), ``"q8_0"`` (int8 payload + fp16 scale per 32 values, split
layout), ``"bf16"``, ``"mxfp8"`` (e4m3 + e8m0 per 32 values, split layout),
``"f32"``.
"""
from __future__ import annotations

import ctypes
import dataclasses

import numpy as np
import torch

from . import _lib

# The reference's real table format (engraft/table.py:18-29).
ROW_LEN = 160
BLOCK_LEN = 32
BLOCKS_PER_ROW = ROW_LEN // BLOCK_LEN  # 5
BLOCK_BYTES = 18  # 2 (d, float16) + 16 (qs, nibble)
ROW_BYTES = BLOCKS_PER_ROW * BLOCK_BYTES  # 90

KVALUES_IQ4NL = np.array(
    [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113],
    dtype=np.float32,
)

MASK64 = (1 << 64) - 1
FORMATS = ("bf16", "q8_0", "mxfp8", "iq4_nl", "f32")


def _as_signed64(v: int) -> int:
    v &= MASK64
    return v - (1 << 64) if v >= (1 << 63) else v


def payload_shape(fmt: str, n_rows: int, dim: int) -> tuple[tuple, torch.dtype]:
    if fmt == "bf16":
        return (n_rows, dim), torch.bfloat16
    if fmt in ("q8_0", "mxfp8"):
        return (n_rows, dim), torch.uint8
    if fmt == "iq4_nl":
        return (n_rows, dim // BLOCK_LEN * BLOCK_BYTES), torch.uint8
    if fmt == "f32":
        return (n_rows, dim), torch.float32
    raise ValueError(f"unknown row format {fmt!r} (expected one of {FORMATS})")


def scales_shape(fmt: str, n_rows: int, dim: int) -> tuple[tuple, torch.dtype] | None:
    if fmt == "q8_0":
        return (n_rows, dim // BLOCK_LEN), torch.float16
    if fmt == "mxfp8":
        return (n_rows, dim // BLOCK_LEN), torch.uint8
    return None


def raw_row_bytes(fmt: str, dim: int) -> int:
    """Bytes of one row in its GGML-style interleaved wire form (``read_rows_raw``)."""
    nb = dim // BLOCK_LEN
    return {"bf16": 2 * dim, "q8_0": nb * 34, "mxfp8": nb * 33, "iq4_nl": nb * BLOCK_BYTES,
            "f32": 4 * dim}[fmt]


@dataclasses.dataclass(frozen=True)
class HeadInfo:
    """``engraft/table.py:32-37``; ``data_offset`` is the byte offset of the
    head's first row in the device payload."""

    head: int
    vocab_size: int
    offset: int
    data_offset: int


class RowStore:
    """Rows of one format in device memory (a table or an overlay's rows).

    IQ4_NL rows may sit in wider lines than their own 18-byte blocks: a
    payload ``[n_rows, stride]`` with ``stride`` above the row's bytes (an even
    count; ``padded_stride`` gives whole 128-byte lines) keeps every row inside
    one line, so that a random row read fetches one line instead of 1.7 on
    average; the bytes past the row are never read."""

    def __init__(self, fmt: str, dim: int, payload: torch.Tensor, scales: torch.Tensor | None = None):
        if fmt not in FORMATS:
            raise ValueError(f"unknown row format {fmt!r} (expected one of {FORMATS})")
        if dim <= 0 or dim % BLOCK_LEN:
            raise ValueError(f"dim={dim} must be a positive multiple of {BLOCK_LEN}")
        n_rows = int(payload.shape[0])
        shp, dt = payload_shape(fmt, n_rows, dim)
        padded = (fmt == "iq4_nl" and payload.dim() == 2 and payload.dtype == dt and payload.shape[1] > shp[1]
                  and payload.shape[1] % 2 == 0)
        if (tuple(payload.shape) != shp and not padded) or payload.dtype != dt:
            raise ValueError(f"{fmt} payload must be {dt} {shp} (IQ4_NL: or an even row stride above "
                             f"{shp[1]}), got {payload.dtype} {tuple(payload.shape)}")
        self.row_bytes = shp[1] * payload.element_size()  # one row's own bytes
        self.row_stride = int(payload.shape[1]) * payload.element_size() if padded else 0
        sshape = scales_shape(fmt, n_rows, dim)
        if sshape is not None:
            if scales is None or tuple(scales.shape) != sshape[0] or scales.dtype != sshape[1]:
                raise ValueError(f"{fmt} scales must be {sshape[1]} {sshape[0]}")
            if scales.device != payload.device:
                raise ValueError("payload and scales on different devices")
        if not payload.is_contiguous() or (scales is not None and not scales.is_contiguous()):
            raise ValueError("payload/scales must be contiguous")
        self.fmt = fmt
        self.dim = dim
        self.n_rows = n_rows
        self.payload = payload
        self.scales = scales if sshape is not None else None

    @property
    def device(self) -> torch.device:
        return self.payload.device

    def c_table(self) -> _lib.EgTable:
        t = _lib.EgTable()
        t.fmt = _lib.FMT_CODES[self.fmt]
        t.dim = self.dim
        t.n_rows = self.n_rows
        t.payload = _lib.ptr(self.payload)
        t.scales = _lib.ptr(self.scales)
        t.row_stride = self.row_stride
        return t

    @staticmethod
    def padded_stride(fmt: str, dim: int) -> int:
        """Bytes per row that keep each row of ``fmt`` in whole 128-byte lines
        (IQ4_NL; the other formats keep their own rows)."""
        shp, _ = payload_shape(fmt, 1, dim)
        return -(-shp[1] // 128) * 128 if fmt == "iq4_nl" else shp[1]

    @classmethod
    def empty(cls, fmt: str, n_rows: int, dim: int, device, row_stride: int | None = None) -> "RowStore":
        """``row_stride``: IQ4_NL bytes per row in memory (``padded_stride``
        for whole lines); None keeps the format's own rows."""
        shp, dt = payload_shape(fmt, n_rows, dim)
        if row_stride is not None and row_stride != shp[1]:
            if fmt != "iq4_nl":
                raise ValueError(f"{fmt} rows take no row_stride")
            shp = (n_rows, int(row_stride))
        payload = torch.empty(shp, dtype=dt, device=device)
        ss = scales_shape(fmt, n_rows, dim)
        scales = torch.empty(ss[0], dtype=ss[1], device=device) if ss is not None else None
        return cls(fmt, dim, payload, scales)

    def raw_rows(self, rows: torch.Tensor) -> np.ndarray:
        """GGML-style interleaved bytes of the given rows (host copy)."""
        rows = rows.to(device=self.device, dtype=torch.int64)
        p = self.payload.index_select(0, rows).view(torch.uint8).reshape(rows.numel(), -1)[:, :self.row_bytes]
        p = p.contiguous()
        if self.scales is None:
            return p.cpu().numpy()
        nb = self.dim // BLOCK_LEN
        s = self.scales.index_select(0, rows).contiguous().view(torch.uint8).reshape(rows.numel(), nb, -1)
        blocks = torch.cat([s, p.reshape(rows.numel(), nb, BLOCK_LEN)], dim=2)
        return blocks.reshape(rows.numel(), -1).cpu().numpy()


def hash_spec(*, eos_token_id, ngram_size, heads_per_ngram, layer_multipliers, head_vocab_sizes, head_offsets,
              head_multipliers_dev: torch.Tensor | None = None) -> _lib.EgHashSpec:
    n_heads = (ngram_size - 1) * heads_per_ngram
    if not 2 <= ngram_size <= _lib.EG_MAX_NGRAM:
        raise ValueError(f"ngram_size={ngram_size} outside [2, {_lib.EG_MAX_NGRAM}]")
    if len(head_vocab_sizes) != n_heads or len(head_offsets) != n_heads:
        raise ValueError(f"expected {n_heads} heads ((ngram_size-1)*heads_per_ngram), got "
                         f"{len(head_vocab_sizes)} sizes / {len(head_offsets)} offsets")
    if n_heads > _lib.EG_MAX_HEADS:
        raise ValueError(f"n_heads={n_heads} > {_lib.EG_MAX_HEADS}")
    if len(layer_multipliers) < ngram_size:
        raise ValueError(f"{len(layer_multipliers)} layer_multipliers < ngram_size={ngram_size}")
    s = _lib.EgHashSpec()
    s.eos_token_id = int(eos_token_id) & MASK64
    s.ngram_size = ngram_size
    s.heads_per_ngram = heads_per_ngram
    for j in range(min(len(layer_multipliers), _lib.EG_MAX_NGRAM)):
        s.layer_multipliers[j] = int(layer_multipliers[j]) & MASK64
    s.head_multipliers = _lib.ptr(head_multipliers_dev)
    for h in range(n_heads):
        s.head_vocab_sizes[h] = int(head_vocab_sizes[h])
        s.head_offsets[h] = int(head_offsets[h])
    return s


def _tokens_tensor(tokens, device) -> torch.Tensor:
    if isinstance(tokens, torch.Tensor):
        t = tokens.to(device=device, dtype=torch.int64)
    else:
        t = torch.as_tensor(np.asarray(tokens, dtype=np.int64), device=device)
    return t.reshape(-1).contiguous()


def _seg_start_tensor(seg_start, n: int, device) -> torch.Tensor | None:
    if seg_start is None:
        return None
    s = seg_start if isinstance(seg_start, torch.Tensor) else torch.as_tensor(np.asarray(seg_start))
    s = s.to(device=device, dtype=torch.int32).reshape(-1).contiguous()
    if s.numel() != n:
        raise ValueError(f"seg_start has {s.numel()} entries for {n} positions")
    return s


class DeviceTable:
    """A PLE table resident in HBM (see the module docstring)."""

    def __init__(self, rows: RowStore, *, eos_token_id: int, ngram_size: int, heads_per_ngram: int,
                 layer_multipliers, head_vocab_sizes, head_offsets, head_multipliers=None,
                 image_token_id: int = -1):
        self.store = rows
        self.fmt = rows.fmt
        self.row_len = rows.dim
        self.eos_token_id = int(eos_token_id)
        self.image_token_id = int(image_token_id)
        self.ngram_size = int(ngram_size)
        self.heads_per_ngram = int(heads_per_ngram)
        self.layer_multipliers = [int(m) for m in layer_multipliers]
        self.head_vocab_sizes = [int(v) for v in head_vocab_sizes]
        self.head_offsets = [int(o) for o in head_offsets]
        self.n_heads = len(self.head_vocab_sizes)
        self.head_multipliers = None if head_multipliers is None else [[int(m) for m in row]
                                                                         for row in head_multipliers]
        for h in range(self.n_heads):
            if self.head_offsets[h] + self.head_vocab_sizes[h] > rows.n_rows:
                raise ValueError(f"head {h}: rows [{self.head_offsets[h]}, "
                                 f"{self.head_offsets[h] + self.head_vocab_sizes[h]}) exceed the table's "
                                 f"{rows.n_rows} rows")
        rb = rows.payload.element_size() * int(np.prod(rows.payload.shape[1:]))  # bytes per row in memory
        self.heads = [HeadInfo(h, self.head_vocab_sizes[h], self.head_offsets[h], self.head_offsets[h] * rb)
                      for h in range(self.n_heads)]
        self._hm_dev = None
        if self.head_multipliers is not None:
            if len(self.head_multipliers) != self.n_heads or any(len(r) != self.ngram_size
                                                                 for r in self.head_multipliers):
                raise ValueError(f"head_multipliers must be [{self.n_heads}][{self.ngram_size}]")
            flat = [_as_signed64(m) for r in self.head_multipliers for m in r]
            self._hm_dev = torch.tensor(flat, dtype=torch.int64, device=rows.device)
        self._spec = hash_spec(eos_token_id=self.eos_token_id, ngram_size=self.ngram_size,
                               heads_per_ngram=self.heads_per_ngram, layer_multipliers=self.layer_multipliers,
                               head_vocab_sizes=self.head_vocab_sizes, head_offsets=self.head_offsets,
                               head_multipliers_dev=self._hm_dev)
        self._ctable = rows.c_table()

    # ---- properties -----------------------------------------------------------------------
    @property
    def device(self) -> torch.device:
        return self.store.device

    @property
    def n_rows(self) -> int:
        return self.store.n_rows

    @property
    def c_spec(self) -> _lib.EgHashSpec:
        return self._spec

    @property
    def c_table(self) -> _lib.EgTable:
        return self._ctable

    # ---- the reference's methods ------------------------------------------------------------
    def ngram_addresses(self, tokens) -> list[list[int]]:
        """For each position of ``tokens`` the ``n_heads`` local rows
        (``engraft/table.py:111-144``), hashed on the device."""
        n = len(tokens)
        if n == 0:
            return []
        return self.rows(tokens, global_ids=False).cpu().tolist()

    def read_rows_raw(self, h: int, start: int, n: int) -> np.ndarray:
        """``n`` raw rows of head ``h`` from local row ``start``, uint8
        ``[n, raw_row_bytes]`` (``engraft/table.py:90-104``; GGML block order:
        scale then values for the scaled formats)."""
        head = self.heads[h]
        assert 0 <= start and start + n <= head.vocab_size, (
            f"head {h}: requested rows [{start},{start+n}) outside [0,{head.vocab_size})"
        )
        rows = torch.arange(head.offset + start, head.offset + start + n, device=self.device)
        return self.store.raw_rows(rows)

    def read_rows(self, h: int, start: int, n: int) -> np.ndarray:
        """Dequantised rows, float32 ``[n, row_len]`` (``engraft/table.py:106-109``)."""
        head = self.heads[h]
        assert 0 <= start and start + n <= head.vocab_size, (
            f"head {h}: requested rows [{start},{start+n}) outside [0,{head.vocab_size})"
        )
        rows = torch.arange(head.offset + start, head.offset + start + n, device=self.device,
                            dtype=torch.int32)
        return self.gather(rows.reshape(-1, 1)).cpu().numpy().reshape(n, self.row_len)

    # ---- device-native entry points ---------------------------------------------------------
    def rows(self, tokens, seq_len: int | None = None, seg_start=None, global_ids: bool = True) -> torch.Tensor:
        """int32 ``[n, n_heads]`` row ids of every position of the flat ``tokens``."""
        tok = _tokens_tensor(tokens, self.device)
        n = tok.numel()
        out = torch.empty((n, self.n_heads), dtype=torch.int32, device=self.device)
        seg = _seg_start_tensor(seg_start, n, self.device)
        _lib.call("eg_hash_rows", ctypes.byref(self._spec), _lib.ptr(tok), n, int(seq_len or 0), _lib.ptr(seg),
                  1 if global_ids else 0, _lib.ptr(out), _lib.stream_ptr(self.device))
        return out

    def gather(self, rows: torch.Tensor, overlay=None) -> torch.Tensor:
        """f32 ``[n, k*row_len]`` dequantised rows for int32 global ids ``[n, k]``
        (overlay rows substituted when ``overlay`` is given)."""
        rows = rows.to(device=self.device, dtype=torch.int32)
        if rows.dim() == 1:
            rows = rows.reshape(-1, 1)
        rows = rows.contiguous()
        n, k = rows.shape
        out = torch.empty((n, k * self.row_len), dtype=torch.float32, device=self.device)
        ov = overlay.c_overlay() if overlay is not None else None
        _lib.call("eg_gather", ctypes.byref(self._ctable), ctypes.byref(ov) if ov is not None else None,
                  _lib.ptr(rows), n, k, _lib.ptr(out), _lib.stream_ptr(self.device))
        return out

    def forward(self, tokens, residual: torch.Tensor | None = None, *, out: torch.Tensor | None = None,
                overlay=None, seq_len: int | None = None, seg_start=None, return_rows: bool = False):
        """Fused hash -> gather -> dequant -> overlay -> residual add (one table layer)."""
        return forward([self], tokens, residual, out=out, overlays=[overlay], seq_len=seq_len,
                       seg_start=seg_start, return_rows=return_rows)

    # ---- construction -----------------------------------------------------------------------
    @classmethod
    def synthetic(cls, fmt: str, n_rows: int, dim: int, *, seed: int, sigma: float, eos_token_id: int,
                  ngram_size: int, heads_per_ngram: int, layer_multipliers, head_vocab_sizes, head_offsets,
                  head_multipliers=None, device="cuda", chunk_rows: int = 1 << 26) -> "DeviceTable":
        """Seeded synthetic table generated in place on the device (``eg_synth_table``)."""
        store = RowStore.empty(fmt, n_rows, dim, device)
        fill_synthetic(store, seed=seed, sigma=sigma, chunk_rows=chunk_rows)
        return cls(store, eos_token_id=eos_token_id, ngram_size=ngram_size, heads_per_ngram=heads_per_ngram,
                   layer_multipliers=layer_multipliers, head_vocab_sizes=head_vocab_sizes,
                   head_offsets=head_offsets, head_multipliers=head_multipliers)


class PleTable(DeviceTable):
    """The per-head IQ4_NL table of a Qwen4Exp GGUF file, loaded into HBM
    (``engraft/table.py:40-88``): hash parameters from the
    ``qwen4exp.ple.*`` metadata, head h's rows from tensor
    ``ple_ngram_embd.{h}.weight`` (IQ4_NL, shape ``[160, p_h]``) placed at
    global rows ``head_offsets[h] .. + p_h``.  The file is streamed in
    ``chunk_bytes`` stripes; same ``AssertionError``s as the reference.  A
    ``DeviceTable`` with the file's ``path``.

    ``pad_rows`` (default): each 90-byte row in a 128-byte line of its own
    (``RowStore.padded_stride``), 42 % more HBM (41 GB for the real table's
    320M rows) for one line per random row read instead of 1.7 on average."""

    def __init__(self, path, device=None, chunk_bytes: int = 1 << 28, pad_rows: bool = True):
        from pathlib import Path

        from .ggufio import GGML_TYPE_IQ4_NL, read_gguf

        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        g = read_gguf(path)
        f = g.fields
        eos = int(f["qwen4exp.ple.eos_token_id"])
        image = int(f["qwen4exp.ple.image_token_id"])
        ngram = int(f["qwen4exp.ple.ngram_size"])
        hpn = int(f["qwen4exp.ple.heads_per_ngram"])
        mults = [int(m) for m in f["qwen4exp.ple.layer_multipliers"]]
        vocab = [int(v) for v in f["qwen4exp.ple.head_vocab_sizes"]]
        offsets = [int(o) for o in f["qwen4exp.ple.head_offsets"]]
        n_rows = max(o + v for o, v in zip(offsets, vocab))
        stride = RowStore.padded_stride("iq4_nl", ROW_LEN) if pad_rows else ROW_BYTES
        store = RowStore.empty("iq4_nl", n_rows, ROW_LEN, dev, row_stride=stride)
        chunk_rows = max(1, chunk_bytes // ROW_BYTES)
        with open(Path(path), "rb") as fh:
            for h, (o, v) in enumerate(zip(offsets, vocab)):
                name = f"ple_ngram_embd.{h}.weight"
                t = g.tensors[name]
                assert t.ggml_type == GGML_TYPE_IQ4_NL, f"{name}: expected IQ4_NL, got {t.ggml_type}"
                assert int(t.shape[0]) == ROW_LEN, f"{name}: shape[0]={t.shape[0]} != {ROW_LEN}"
                assert int(t.shape[1]) == v, f"{name}: shape[1]={t.shape[1]} != head_vocab_sizes[{h}]={v}"
                fh.seek(t.data_offset)
                done = 0
                while done < v:  # whole rows a stripe
                    k = min(chunk_rows, v - done)
                    buf = np.frombuffer(fh.read(k * ROW_BYTES), dtype=np.uint8)
                    if buf.size != k * ROW_BYTES:
                        raise ValueError(f"{path}: {name} is truncated")
                    dst = store.payload[o + done:o + done + k, :ROW_BYTES]
                    dst.copy_(torch.from_numpy(buf.reshape(k, ROW_BYTES).copy()))
                    done += k
        super().__init__(store, eos_token_id=eos, ngram_size=ngram, heads_per_ngram=hpn, layer_multipliers=mults,
                         head_vocab_sizes=vocab, head_offsets=offsets, image_token_id=image)
        self.path = Path(path)


def quantile_table(sigma: float) -> np.ndarray:
    """16,384 normal quantiles ``f32(sigma * Phi^-1((i + 0.5) / 16384))``."""
    import statistics

    nd = statistics.NormalDist(0.0, 1.0)
    q = np.array([nd.inv_cdf((i + 0.5) / 16384.0) for i in range(16384)], dtype=np.float64)
    return (q * sigma).astype(np.float32)


def fill_synthetic(store: RowStore, *, seed: int, sigma: float, row0: int = 0, n_rows: int | None = None,
                   chunk_rows: int = 1 << 26) -> None:
    q = torch.as_tensor(quantile_table(sigma), device=store.device)
    t = store.c_table()
    end = store.n_rows if n_rows is None else row0 + n_rows
    st = _lib.stream_ptr(store.device)
    for r in range(row0, end, chunk_rows):
        _lib.call("eg_synth_table", ctypes.byref(t), int(seed) & MASK64, _lib.ptr(q), r, min(chunk_rows, end - r),
                  st)
    torch.cuda.current_stream(store.device).synchronize()  # q is freed on return


class PreparedForward:
    """One fused-forward call with every argument validated and translated to
    the C ABI once; calling it only launches (``eg_forward`` on the current
    stream, or ``stream``).  Used by ``forward`` and by launch-bound loops
    (benchmark, decode), including under HIP graph capture."""

    def __init__(self, tables: list[DeviceTable], tokens, residual: torch.Tensor | None = None, *,
                 out: torch.Tensor | None = None, overlays=None, seq_len: int | None = None, seg_start=None,
                 return_rows: bool = False, decode_ctx: int | None = None, return_slot_vars: bool = False):
        if not 1 <= len(tables) <= _lib.EG_MAX_LAYERS:
            raise ValueError(f"{len(tables)} table layers (1..{_lib.EG_MAX_LAYERS} supported)")
        t0 = tables[0]
        dev = t0.device
        tok = _tokens_tensor(tokens, dev)
        n = tok.numel()
        if decode_ctx is not None:
            if decode_ctx < 1 or n % decode_ctx != 0:
                raise ValueError(f"{n} tokens are not [n_seq, {decode_ctx}]")
            if seq_len is not None or seg_start is not None:
                raise ValueError("decode: every sequence is its own segment (no seq_len / seg_start)")
            n //= decode_ctx
        w = t0.n_heads * t0.row_len
        if residual is not None:
            if residual.dtype != torch.bfloat16 or residual.device != dev:
                raise ValueError("residual must be a bf16 tensor on the table's device")
            if residual.numel() != n * w or not residual.is_contiguous():
                raise ValueError(f"residual must be contiguous with {n}x{w} elements")
            if out is None:
                out = torch.empty_like(residual)
        elif out is None:
            out = torch.empty((n, w), dtype=torch.float32, device=dev)
        want = torch.bfloat16 if residual is not None else torch.float32
        if out.dtype != want or out.numel() != n * w or not out.is_contiguous() or out.device != dev:
            raise ValueError(f"out must be a contiguous {want} tensor with {n}x{w} elements")
        seg = _seg_start_tensor(seg_start, n, dev)
        nl = len(tables)
        self._specs = (_lib.EgHashSpec * nl)(*[t.c_spec for t in tables])
        self._ctabs = (_lib.EgTable * nl)(*[t.c_table for t in tables])
        self._ovs = None
        self._overlays = overlays
        if overlays is not None and any(o is not None for o in overlays):
            self._ovs = (_lib.EgOverlay * nl)(*[(o.c_overlay() if o is not None else _lib.EgOverlay())
                                                for o in overlays])
        self.rows = torch.empty((nl, n, t0.n_heads), dtype=torch.int32, device=dev) if return_rows else None
        # return_slot_vars: the overlay row each slot read (-1: base table), eg_forward_slots
        self.slot_vars = None
        if return_slot_vars:
            if decode_ctx is not None:
                raise ValueError("slot variables are written by eg_forward_slots, not the decode step")
            self.slot_vars = torch.empty((nl, n, t0.n_heads), dtype=torch.int32, device=dev)
        self.out = out
        self._keep = (tables, tok, residual, seg)
        if self.slot_vars is not None:
            self._fn = _lib.load().eg_forward_slots
            self._args = (nl, self._specs, self._ctabs, self._ovs, _lib.ptr(tok), n, int(seq_len or 0),
                          _lib.ptr(seg), _lib.ptr(residual), _lib.ptr(out), _lib.ptr(self.rows),
                          _lib.ptr(self.slot_vars))
        elif decode_ctx is None:
            self._fn = _lib.load().eg_forward
            self._args = (nl, self._specs, self._ctabs, self._ovs, _lib.ptr(tok), n, int(seq_len or 0),
                          _lib.ptr(seg), _lib.ptr(residual), _lib.ptr(out), _lib.ptr(self.rows))
        else:
            self._fn = _lib.load().eg_forward_decode
            self._args = (nl, self._specs, self._ctabs, self._ovs, _lib.ptr(tok), n, int(decode_ctx),
                          _lib.ptr(residual), _lib.ptr(out), _lib.ptr(self.rows))
        self._decode = decode_ctx is not None
        self.device = dev
        self.n_positions = n

    def __call__(self, stream: int | None = None) -> None:
        st = stream if stream is not None else _lib.stream_ptr(self.device)
        rc = self._fn(*self._args, st)
        if rc != _lib.EG_OK:
            _lib.check(rc)

    def timed(self, start_event: int, stop_event: int, stream: int | None = None) -> None:
        """The same launch through ``eg_forward_timed``: the two hipEvent_t
        handles receive the kernel dispatch's own start / end timestamps."""
        if self._decode or self.slot_vars is not None:
            raise ValueError("timed launches are for eg_forward")
        st = stream if stream is not None else _lib.stream_ptr(self.device)
        rc = _lib.load().eg_forward_timed(*self._args, start_event, stop_event, st)
        if rc != _lib.EG_OK:
            _lib.check(rc)


def forward(tables: list[DeviceTable], tokens, residual: torch.Tensor | None = None, *,
            out: torch.Tensor | None = None, overlays=None, seq_len: int | None = None, seg_start=None,
            return_rows: bool = False):
    """Fused forward over 1-2 table layers with equal ``n_heads`` and ``row_len``:
    ``out = bf16(f32(residual) + emb_0 + emb_1)`` with a bf16 residual, or the
    f32 embedding sum without one.  Returns ``out`` (and int32 row ids
    ``[n_layers, n, n_heads]`` with ``return_rows``)."""
    call = PreparedForward(tables, tokens, residual, out=out, overlays=overlays, seq_len=seq_len,
                           seg_start=seg_start, return_rows=return_rows)
    call()
    return (call.out, call.rows) if return_rows else call.out


class PreparedForwardRows:
    """``eg_forward_rows`` with its arguments marshalled once: the forward's
    residual add from row ids already known (int32 ``[n_layers, n, n_heads]``,
    the layout ``forward(..., return_rows=True)`` returns)."""

    def __init__(self, tables: list[DeviceTable], rows: torch.Tensor, residual: torch.Tensor, *,
                 out: torch.Tensor | None = None, overlays=None):
        if not 1 <= len(tables) <= _lib.EG_MAX_LAYERS:
            raise ValueError(f"{len(tables)} table layers (1..{_lib.EG_MAX_LAYERS} supported)")
        t0 = tables[0]
        dev = t0.device
        nl = len(tables)
        if rows.dtype != torch.int32 or rows.device != dev or not rows.is_contiguous():
            raise ValueError("rows must be a contiguous int32 tensor on the table's device")
        if rows.dim() == 2:
            rows = rows.unsqueeze(0)
        if rows.dim() != 3 or rows.shape[0] != nl or rows.shape[2] != t0.n_heads:
            raise ValueError(f"rows must be [{nl}, n, {t0.n_heads}]")
        n = int(rows.shape[1])
        w = t0.n_heads * t0.row_len
        if residual.dtype != torch.bfloat16 or residual.device != dev or residual.numel() != n * w \
                or not residual.is_contiguous():
            raise ValueError(f"residual must be a contiguous bf16 tensor with {n}x{w} elements on {dev}")
        if out is None:
            out = torch.empty_like(residual)
        if out.dtype != torch.bfloat16 or out.numel() != n * w or not out.is_contiguous() or out.device != dev:
            raise ValueError(f"out must be a contiguous bf16 tensor with {n}x{w} elements")
        self._ctabs = (_lib.EgTable * nl)(*[t.c_table for t in tables])
        self._ovs = None
        if overlays is not None and any(o is not None for o in overlays):
            self._ovs = (_lib.EgOverlay * nl)(*[(o.c_overlay() if o is not None else _lib.EgOverlay())
                                                for o in overlays])
        self.out = out
        self._keep = (tables, rows, residual, overlays)
        self._fn = _lib.load().eg_forward_rows
        self._args = (nl, self._ctabs, self._ovs, _lib.ptr(rows), n, t0.n_heads, _lib.ptr(residual), _lib.ptr(out))
        self.device = dev

    def __call__(self, stream: int | None = None) -> None:
        st = stream if stream is not None else _lib.stream_ptr(self.device)
        rc = self._fn(*self._args, st)
        if rc != _lib.EG_OK:
            _lib.check(rc)


def forward_rows(tables: list[DeviceTable], rows: torch.Tensor, residual: torch.Tensor, *,
                 out: torch.Tensor | None = None, overlays=None) -> torch.Tensor:
    """The residual add of ``forward`` from known row ids (``eg_forward_rows``)."""
    call = PreparedForwardRows(tables, rows, residual, out=out, overlays=overlays)
    call()
    return call.out


def stream_copy(src: torch.Tensor, dst: torch.Tensor) -> None:
    """``dst[:] = src`` by the library's streaming copy kernel (``eg_stream_copy``):
    the streaming ceiling the forward's roofline is read against."""
    nbytes = src.numel() * src.element_size()
    if dst.numel() * dst.element_size() != nbytes or not (src.is_contiguous() and dst.is_contiguous()):
        raise ValueError("src and dst must be contiguous with the same number of bytes")
    _lib.call("eg_stream_copy", _lib.ptr(src), _lib.ptr(dst), nbytes, _lib.stream_ptr(src.device))


def forward_decode(tables: list[DeviceTable], tokens, residual: torch.Tensor | None = None, *,
                   out: torch.Tensor | None = None, overlays=None, return_rows: bool = False):
    """One decode step: ``tokens`` int ``[n_seq, ctx]`` (each sequence's last
    ``ctx`` tokens, the new one last), ``residual`` bf16 ``[n_seq, W]``: the
    embedding of every sequence's new position added into its residual
    (overlays resolved per id).  Returns ``out`` (and the row ids)."""
    tok = tokens if isinstance(tokens, torch.Tensor) else torch.as_tensor(np.asarray(tokens, dtype=np.int64))
    if tok.dim() != 2:
        raise ValueError("decode tokens must be [n_seq, ctx]")
    call = PreparedForward(tables, tok, residual, out=out, overlays=overlays, return_rows=return_rows,
                           decode_ctx=int(tok.shape[1]))
    call()
    return (call.out, call.rows) if return_rows else call.out


def dequant_iq4nl(raw) -> np.ndarray:
    """``engraft/table.py:147-169`` on the device: uint8 ``[n, 18*nb]`` ->
    float32 ``[n, 32*nb]``."""
    raw_np = np.ascontiguousarray(np.asarray(raw, dtype=np.uint8))
    n, nbytes = raw_np.shape
    if nbytes % BLOCK_BYTES:
        raise ValueError(f"IQ4_NL rows must be a multiple of {BLOCK_BYTES} bytes, got {nbytes}")
    dim = nbytes // BLOCK_BYTES * BLOCK_LEN
    if n == 0:
        return np.zeros((0, dim), dtype=np.float32)
    dev = torch.device("cuda", torch.cuda.current_device())
    store = RowStore("iq4_nl", dim, torch.as_tensor(raw_np, device=dev))
    rows = torch.arange(n, dtype=torch.int32, device=dev).reshape(n, 1)
    out = torch.empty((n, dim), dtype=torch.float32, device=dev)
    ct = store.c_table()
    _lib.call("eg_gather", ctypes.byref(ct), None, _lib.ptr(rows), n, 1, _lib.ptr(out), _lib.stream_ptr(dev))
    return out.cpu().numpy()


def row_is_zero(raw) -> np.ndarray:
    """``engraft/table.py:172-183``: True iff every block's fp16 scale bit
    pattern is 0x0000 (-0.0 counts as non-zero).  Bit test on the device."""
    raw_np = np.ascontiguousarray(np.asarray(raw, dtype=np.uint8))
    n, nbytes = raw_np.shape
    dev = torch.device("cuda", torch.cuda.current_device())
    t = torch.as_tensor(raw_np, device=dev).reshape(n, nbytes // BLOCK_BYTES, BLOCK_BYTES)
    return ((t[:, :, 0] == 0) & (t[:, :, 1] == 0)).all(dim=1).cpu().numpy()
