"""CPU restatement of the reference's gated dense and paged sparse attention.

TEST INFRASTRUCTURE ONLY. This package is the checker that the HIP kernels in
``exploration_amd`` are compared against. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it; the product path never does, and it never stands in for a missing
HIP library.

Every function follows the reference (zhjerry25/Exploration, package ``st``)
and cites the file:line it restates. The arithmetic is stock torch on CPU
tensors in float64 or float32 (the reference's own eager path is torch too).

Pinning (each function is checked by something other than a retyped formula,
see ``tests/test_oracle.py``):

* ``dense.loop_attention``     brute force per row; cross-checked with
  ``dense.eager_attention`` (vectorised) and ``dense.forward_stats``
  (flash-style statistics), with closed forms: plain causal softmax when no
  remote block exists, padding rows are zero, the block-mass gate on
  constant-score blocks reduces to M_j^2 / Z_R weights.
* ``dense.eager_attention``    gradcheck in float64 (the reference's
  tests/test_attention.py:65-73 case) and the cases of
  tests/test_attention.py:48-63.
* ``dense.backward_explicit``  equals autograd of ``eager_attention`` in
  float64 on the same cases.
* ``sparse.*``                 topk >= visible blocks equals the dense
  operator (tests/test_attention.py:75-86 cases), brute-force
  logsumexp for scores and log Z_R, planted blocks give a known selection.
"""
