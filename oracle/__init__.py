"""CPU oracle for the Pairformer pair-stack hot path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference equations of the pair-stack ops on the CPU so
that the HIP kernels of ``foldforge_amd`` can be checked against them. It is the
checker, never the thing measured or shipped: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import
it. No module under ``foldforge_amd`` imports, calls or links anything here.

Modules
-------
``pairstack``  fp32 / fp64 PyTorch-CPU restatement of every op of the block
               (LayerNorm, triangle multiplication outgoing/incoming, triangle
               attention starting/ending, pair transition, attention with pair
               bias, single transition, the sequential block and the trunk).
``brute``      pure-Python fp64 loop restatements for tiny shapes, written from
               the equations independently of ``pairstack``; they pin it.
``params``     seeded random-init parameter sets in the engine's state_dict
               names (the init convention of the reference's block tests).

Pinning status (what each ``pairstack`` function is checked against, in
``tests/test_oracle.py``):

* ``layer_norm``            closed form (fp64 mean / variance) and
                            ``torch.nn.functional.layer_norm``.
* ``triangle_multiplication`` brute-force triple loop (``brute``), the
                            outgoing/incoming transpose identity, mask zeros.
* ``triangle_attention``    brute-force softmax loops (``brute``),
                            ``scaled_dot_product_attention`` math backend,
                            softmax shift invariance, key-mask exactness, large
                            logits, the transposed-bias start/end identity.
* ``transition``            brute-force loops and the closed-form SwiGLU.
* ``attention_pair_bias``   brute-force loops.
* ``pairformer_block``      composition of the pinned ops (checked against the
                            op-by-op brute force on a tiny block).

Conventions the reference leaves open (engine ``pytorch`` backend outputs at
padded positions are not pinned by any reference test, which compare valid
pairs only): padded query rows are computed like valid rows under the key mask;
a batch element with no valid key at all gets a zero attention output. Both are
stated here and enforced identically by the HIP kernels.
"""
