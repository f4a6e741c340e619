"""CPU oracle for the Pairformer pair-stack hot path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference equations of the pair-stack ops on the CPU so
that the HIP kernels of ``foldforge_amd`` can be checked against them. It is the
checker, never the thing measured or shipped: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` import
it. No module under ``foldforge_amd`` imports, calls or links anything here.

Modules
-------
``pairstack``  fp32 / fp64 PyTorch-CPU restatement of every op of the path
               (LayerNorm, LayerNorm + linear, SwiGLU FFN, triangle
               multiplication outgoing/incoming and its length-divided form,
               triangle attention starting/ending in every lineage's bias and
               output form, pair transition, attention with pair bias, MSA
               pair-weighted averaging, outer product mean in its plain and
               grouped forms, the sequential and parallel block).
``brute``      pure-Python fp64 loop restatements for tiny shapes, written from
               the equations independently of ``pairstack``; they pin it.
``released``   the same ops on the released (dense AF3-family) parameter layouts
               (interleaved projections, ``transition1`` chunking, the outer
               product's ``output_w``), restated independently of ``pairstack``;
               it pins the released-to-engine conversion.

Pinning status (what each function is checked against, in ``tests/test_oracle.py``
and ``tests/test_released.py``):

* ``layer_norm``            closed form (fp64 mean / variance) and
                            ``torch.nn.functional.layer_norm``.
* ``layer_norm_linear``, ``swiglu_ffn``  element loops; ``swiglu_ffn(LN(x))`` equals
                            the transition without its norm.
* ``triangle_multiplication`` brute-force triple loop (``brute``), the
                            outgoing/incoming transpose identity, mask zeros,
                            golden fixtures; the length-divided form against
                            loops with their own length count.
* ``triangle_attention``    brute-force softmax loops (``brute``),
                            ``scaled_dot_product_attention`` math backend,
                            softmax shift invariance, key-mask exactness, large
                            logits, the transposed-bias start/end identity, the
                            untransposed and dual output forms' closed forms.
* ``transition``            brute-force loops and the closed-form SwiGLU.
* ``attention_pair_bias``   brute-force loops (with and without an extra bias).
* ``msa_pair_weighted_averaging``  brute-force loops; zero logits give the plain
                            mean over valid keys; MSA-row permutation.
* ``outer_product_mean``    brute-force loops for every form; repeated MSA rows,
                            a masked extra row, a single-row closed form.
* ``pairformer_block``      composition of the pinned ops (checked against the
                            op-by-op brute force on a tiny block); the parallel
                            schedule equals the sum of the ops' updates.
* ``released``              the converted engine modules on the ``pytorch``
                            backend match it (2e-5 per op, 1e-4 per block).

Conventions the reference leaves open (engine ``pytorch`` backend outputs at
padded positions are not pinned by any reference test, which compare valid
pairs only): padded query rows are computed like valid rows under the key mask;
a batch element with no valid key at all gets a zero attention output. Both are
stated here and enforced identically by the HIP kernels.
"""
