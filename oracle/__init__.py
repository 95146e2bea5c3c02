"""ORACLE — CPU restatement of the reference's gated-mixture Linear path.

This package is TEST INFRASTRUCTURE.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker or as the timed CPU baseline.  The product
(``voodoo_quant`` on top of ``libvoodoo_hip.so``) never imports, links or runs
anything here.

Contents and what pins each part (reference files cited relative to the
reference checkout):

* ``dequant_ref.c`` / :mod:`oracle.cdequant` — scalar C restatement of ggml's
  ``dequantize_row_{q8_0,q2_K,q3_K,q4_K,q5_K,q6_K}`` in ggml's loop order.
  Pinned by (a) the golden vectors of the reference's own torch decoders
  (``voodoo_quant/layers.py:62-213``; Q8_0/Q4_K/Q5_K/Q6_K) under
  ``tests/golden/``, (b) the closed-form field values of :mod:`oracle.blocks`
  (all six formats), (c) hand-computed special blocks.  Q2_K/Q3_K have no
  reference text: against ggml itself they are **parity unpinned**.
* :mod:`oracle.blocks` — structured block packers (fields -> bytes) and the
  closed-form value of every weight from its fields; random valid blocks.
* :mod:`oracle.mixture` — fp32/fp64 torch restatement of
  ``_MixedWeightFunction`` (``voodoo_quant/layers.py:336-363``), ``F.linear``
  and its backward, the temperature softmax (``layers.py:1342-1375``), the
  budget (``layers.py:1537-1557``) and the trainer's anneal / size loss /
  optimizer (``training/trainer.py:199-203, 2378-2379, 2577-2616``).  Pinned
  by finite differences in float64, the softmax-Jacobian identity ported from
  ``tests/test_ptqr.py:161-172`` and linearity checks.
"""

from oracle.cdequant import oracle_dequant, oracle_dequant_parallel, load_oracle_lib  # noqa: F401
