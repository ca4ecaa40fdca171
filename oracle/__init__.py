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
* AttentionPairBias with the bias given directly (diffusion transformers,
  separate key rows, multiplicity): fp64 loops (``brute.attention_pair_bias_keys``).
* PairformerLayer: branch isolation (every pair branch but one silenced gives
  ``z + branch(z)`` of the fp64 loop module), chained branches (the second
  reads the z the first updated), the sequence stack on the updated z by fp64
  loops, and the sequence stack in fp32 under bf16 autocast.  The op order
  itself is a restatement of upstream (only an import of upstream Boltz could
  show it); the reference corroborates it at ``multiplication.py:59``,
  ``triangle.py:113`` and ``adapters.py:39-45``.
* PairformerNoSeqLayer: bit-identical to the PairformerLayer pair stack.
* DiffusionTransformerLayer: attention silenced gives ``a + transition(a, s)``;
  transition silenced gives ``a + sigmoid(gate(s)) * attention(adaln(a, s))``
  (with multiplicity); ``to_keys`` gathers keys and key mask alike (windows
  written out by hand); upstream's output-gate initialisation.

bf16-mixed reference: the GPU tests run these fp32 modules under
``torch.autocast("cuda", dtype=torch.bfloat16)`` as upstream Boltz's own
bf16-mixed inference path (its linears and matmuls autocast the same way; the
Pairformer sequence stack disables autocast, as upstream does).
"""
