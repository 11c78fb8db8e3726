"""CPU oracle for the Engram/PLE n-gram table path.

TEST INFRASTRUCTURE ONLY.  This package is the checker, never the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product path (``engraft-ngram_amd/``) never
imports it and fails loudly when its HIP library is missing.

Modules (each function cites the reference ``file:line`` it restates):

* ``oracle.hash``     -- the n-gram row hash: literal scalar restatement of
  ``engraft/table.py:111-144`` and a vectorized numpy-uint64 restatement of
  ``engraft/damage.py:68-104`` generalised to any ``ngram_size`` and to
  segment starts (``engraft/replica/seq.py:392-399``).
* ``oracle.formats``  -- row formats: bf16, Q8_0 (split), MXFP8 (split),
  IQ4_NL; dequantisation (``engraft/table.py:147-183``,
  ``engraft/replica/dequant.py:77-93``) and the requantisation rule.
* ``oracle.synth``    -- the seeded synthetic table / token generators that the
  device generator must reproduce bit for bit.
* ``oracle.forward``  -- gather + overlay substitution + residual add
  (``engraft/lens.py:126-136``, ``engraft/replica/model.py:473-495``,
  ``engraft/replica/seq.py:372-444``).
* ``oracle.backward`` -- the sparse gradient scatter and the optimizer step
  (``engraft/replica/seq.py:433-441`` autograd, ``engraft/descend_corpus.py:
  785-790, 921-947``).
* ``oracle.overlay_emb`` -- ``OverlayEmb.build`` / ``ple_true_emb`` per
  position (``engraft/replica/seq.py:185-234, 372-444``,
  ``engraft/replica/model.py:473-495``).
* ``oracle.damage``   -- the damage plan's corpus scan (``engraft/damage.py:
  107-224``).
* ``oracle.cpu_baseline`` -- the vectorized CPU forward timed beside the GPU
  by ``bench.py`` (numpy hash, torch gather / dequant / add).

Pinning status of every function is listed in the header of its module.
"""
