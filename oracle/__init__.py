"""CPU oracle for the TinyTransformer inference hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference computes on the path the HIP library
replaces.  It exists to CHECK the product, never to BE the product:

* only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
  it, and only as the checker (or, in ``bench.py``, as the timed CPU baseline);
* ``mdlarc_scale_amd`` (the product) never imports it and has no CPU fallback: its GPU path fails
  loudly when the HIP library is missing.

Contents
--------
``reference_path``  floating-point model path in torch on the CPU (fp32 by default, fp64 for the
                    closed-form checks): RMSNorm, 3D RoPE, SwiGLU, masked causal attention with the
                    zero-output rule for fully-masked rows, ``forward``, ``prefill``,
                    ``decode_step``, ``generate_output`` (bug-compatible ``lengths-1`` index),
                    ``GridState`` and ``derive_initial_state``.
``data_format``     token format, 3D positions, dihedral transforms and colour permutations in
                    plain Python / numpy.
``augment``         the augmentation caller ``predict_with_augmentations`` (batched chunk loop and
                    sequential loop, greedy) on ``reference_path``.

How each function is pinned (the tests that would catch a dropped term, wrong sign or index)
------------------------------------------------------------------------------------------------
* ``rmsnorm``            fp64 closed form on hand-built rows (constant rows, scaling invariance)
                         and the reference's end-to-end golden logits.
* ``rope3d_tables`` / ``apply_rope3d``
                         closed-form invariants: pairwise-norm preservation, identity at (0,0,0),
                         relative-position property per axis, y=z=0 reduces to textbook
                         interleaved 1D RoPE on dims 0-19, clamping (100,100,100)==(31,31,7);
                         plus the golden logits.
* ``swiglu``             fp64 closed form silu(a)=a/(1+e^-a) on hand-picked values.
* ``attention``          brute force per query in fp64 against an explicit allowed-key list;
                         fully-masked rows give 0.
* ``forward`` / ``prefill`` / ``decode_step`` / ``generate_output``
                         golden vectors written by ``tests/golden/make_golden.py`` from the
                         reference itself (left-padded ragged batch, per-step logits, decode
                         positions, stop-on-END), plus incremental == teacher-forced forward.
* ``apply_logit_constraints`` / ``generate_output(constraints=...)``
                         bit-exact against the reference's own ``_apply_logit_constraints`` on
                         nine cases covering every branch (tests/golden/constraints.npz, written
                         by make_golden.py), and a planted mistake that the fixture catches.
* ``augment.predict_with_augmentations``
                         token for token against the reference's own runs
                         (tests/golden/augment_micro.npz): chunk sizes 16 and 5, the sequential
                         loop, constraints on and off, two micro models; decoded grids too.
* ``GridState`` / ``derive_initial_state``
                         golden traces from the reference, and equality with
                         ``data_format.compute_positions_3d`` on whole token streams.
* ``data_format``        the reference's own known-answer tests (tests/test_data.py:97-317) and
                         the golden colour-permutation table.
"""
