"""MI355X-native Engram/PLE n-gram table path (import name ``engraft_ngram_amd``).

Drop-in for the table path of fulvian/engraft-ngram: the n-gram row hash, the
gather + dequantisation of block-quantised table rows, their add into the
residual stream, and the descent backward (deterministic sparse gradient
scatter + Adam + requantisation on the touched overlay rows).  Host code is
Python on PyTorch-ROCm; every stage runs in hand-written gfx950 HIP kernels
behind the C ABI of ``include/engraft_ngram.h`` (``libengraft_ngram.so``);
``OverlayEmb``'s differentiable gather is a C++ autograd function over two of
those entry points (``_eg_autograd.so``, host code built beside the library).

Modules mirror the reference's:
  table       -- ``engraft.table``            (DeviceTable = PleTable duck type)
  lens        -- ``engraft.lens``             (.pleo, local_to_global, RowSet)
  seq         -- ``engraft.replica.seq``      OverlayEmb, ple_true_emb, the
                                               sequence seam, exclusive_rows_at_position
  overlay     -- the device overlay (sorted ids + rows) the forward resolves per id
  descent     -- ``engraft.replica.distill``  row vars + the optimizer step
  dequant     -- ``engraft.replica.dequant``  wire-form row dequantisation
  pack        -- ``engraft.replica.pack``     segments
  damage      -- ``engraft.damage``           vectorized ngram_rows / scan_hits
  overlay_sum -- ``engraft.replica.overlay_sum`` the overlay merge
  ple         -- ``engraft.replica.layers``   ple_forward / PleWeights, ``engraft.lens`` PleReplica
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
