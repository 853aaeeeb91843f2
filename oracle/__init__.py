"""CPU oracle for the Mamba-3 SISO hot path -- TEST INFRASTRUCTURE ONLY.

Nothing in the shipped package imports this directory. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it, and only
as the checker (or, for the baseline, as the thing timed on the host cores) -- never
as a compute path of the product.

`siso_oracle` restates the reference's pure-JAX maths (``mamba3_pallas/reference.py``,
``layout.py``, ``layer.py``, ``siso.py``, ``kernel_bwd.py``'s epilogue) in plain torch on
the CPU, in float64 or float32. Gradients come from torch autograd of the chunked
restatement, as the reference takes ``jax.grad`` of ``siso_chunked``
(``tests.py:595-606``).

How each function is pinned (none is checked only by retyping its own formula):

* ``siso_recurrent`` -- against golden vectors produced by the reference's own
  ``torch_ref.mamba3_siso_ref`` (upstream's three-term step reference, interleaved
  layout) through the de-interleave permutation; and the closed-form rotation-parity
  answer ``y_t = (-1)^parity`` (``tests.py:451-513``).
* ``siso_chunked`` -- equal to ``siso_recurrent`` in float64 to ~1e-10 (the trapezoid
  collapse, ``reference.py:104-131``; the reference measured 1.2e-8); segment
  chaining invariance (``tests.py:653-726``); the parity known answer.
* gradients (autograd of ``siso_chunked``) -- central finite differences in float64.
* ``siso_step`` -- one step equals one token of the golden recurrence; a chain of
  steps equals one chunked prefill call (``tests.py:734-877``).
* ``preprocess`` -- closed forms (softplus, heavy-tail at both signs, sigmoid, the
  ``t+1`` shift of ``scale``, wrap of ``phi`` into ``[0, 2*pi)``) and the golden vectors.
* ``layer_forward`` -- against golden vectors of the reference's
  ``torch_ref.Mamba3SISOTorch`` forward (in_proj split order, BCNorm, C-is-query /
  B-is-key, biases, D skip, gate) through ``convert``'s permutation.
* rope / permutation helpers -- ``perm(interleaved_rope(u)) == halfsplit_rope(perm(u))``
  exactly, and ``rope_dphi`` against a finite difference of the rotation angle.
"""
