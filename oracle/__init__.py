"""CPU oracle for the Boltz-2 pair-representation hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker.  The product package (``boltz_lumi_amd``) never imports it and never
falls back to it.

Contents
--------
``boltz_ref``  fp32 restatement of the upstream Boltz 2.2.1 modules that
               lauritsf/boltz-lumi patches (same class names, parameter names
               and shapes, so state dicts move between the oracle and real
               Boltz modules).
``mixed``      the same math with Boltz's bf16-mixed (autocast) rounding points
               made explicit, used to report how far Boltz's own bf16 path
               sits from fp32.
``brute``      fp64 pure-Python loop versions for tiny sizes; they pin the
               vectorised restatement.

Pinning status (each function's pin lives in ``tests/test_oracle_pins.py``):

* LayerNorm, Linear, sigmoid, SiLU, softmax: textbook routines, checked against
  ``torch.nn.functional`` and fp64 loops.
* TriangleMultiplication{Outgoing,Incoming}: fp64 loops, the reference's own
  operand layout (permute + bmm, ``multiplication.py:105-122``), the
  outgoing/incoming transpose identity, zero-mask closed form, permutation
  equivariance.
* TriangleAttention{,EndingNode}: fp64 loops, the reference's softmax test
  recipe (``tests/test_triangle_softmax.py:38-47``), fully-masked-row closed
  form, N=1 closed form, ending = transpose(starting(transpose)).
* Transition: fp64 loops, zero-``fc3`` closed form, the reference's chunked
  variant equals the plain one.
* AdaLN / ConditionedTransitionBlock / SwiGLU: fp64 loops, zero-weight closed
  forms, the reference epilogue formulas (``diffusion_hip.cu:14-27``).
* AttentionPairBias: fp64 loops (math restated from ``pair_bias.py:21-36``).
* PairformerLayer: composition order and the fp32 s-stack are **parity
  unpinned** (only an import of upstream Boltz could pin them; the reference
  corroborates them at ``multiplication.py:59``, ``triangle.py:113`` and
  ``adapters.py:39-45``).  Its sub-blocks are pinned as above.
"""
