"""oracle: CPU restatements of the reference's normalization / row-reduction
goldens.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the CPU
baseline, as the timed CPU path).  The product path (``dslperfgap_amd``) never
imports it and has no CPU fallback.

Modules
-------
pytorch_impl
    The six unified-API functions of ViperBench/<kernel>/pytorch_impl.py,
    restated on CPU torch (fp32 arithmetic, the reference's own formulas).
    This is what the reference's test.py compares a backend against.
numpy_ref
    Independent float64 numpy closed forms of the same functions, used to pin
    ``pytorch_impl`` (tests/test_oracle_pins.py).
ce_loops
    Pure-Python per-(row, column block) loops following the reference's Triton
    program (ViperBench/cross_entropy/triton_impl.py:33-75, 98-120), for tiny
    inputs; pins the vectorized CE restatement.

Pinning (what checks each function; see tests/test_oracle_pins.py):
  layer_norm      numpy fp64 closed form; mean-0 / variance invariants; all-equal
                  rows -> bias; torch F.layer_norm in fp64
  rms_norm        numpy fp64 closed form; scale invariance y(c*x) = y(x);
                  hand-computed 1x4 known answer
  softmax         numpy fp64; rows sum to 1; shift invariance; uniform on
                  all-equal rows; 2-element closed form (logistic)
  log_softmax     numpy fp64; x - logsumexp(x); exp sums to 1; dim != -1 via
                  transposition identity
  logsumexp       numpy fp64; lse(x + c) = lse(x) + c; lse of N equal values
                  = v + log N; torch edge values (+inf, -inf, NaN rows)
  cross_entropy   ce_loops brute force (all reference test.py configs and more);
                  F.cross_entropy (reduction none, label_smoothing) for one
                  block; vocab-parallel SPLIT identity: logsumexp over block
                  lse + sum of SPLIT block losses = F.cross_entropy; z-loss
                  closed form; ignored rows; class_start shift
  cross_entropy_bwd  ce_loops brute force; torch.autograd of
                  F.cross_entropy(+ z-loss term) for one block
  mean_reduction  numpy fp64 over one and several dims, keepdim; the dtype
                  argument casts before reducing (bf16 in, fp32 out)
  max_reduction / argmax  hand-computed known answers (ties -> first index,
                  NaN is the largest value, all -inf rows -> 0, +inf ties);
                  numpy first-occurrence argmax over every dim
The reference itself ships no golden vectors or fixtures for this path, and its
Python was not imported or run: every function above is pinned by the checks
listed, none is "parity unpinned".
"""
