"""CPU oracle for the Kernel-DeltaNet prefill path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm (jatin-yadav-acad/kernel-deltanet) on the CPU so that
the HIP kernels can be checked against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker or the timed CPU
baseline -- never as the thing measured or shipped.  The product package (``kernel-deltanet_amd``)
never imports it and has no CPU fallback.

Modules
  lift  -- seeded Rademacher tables, the explicit projection Omega, the plain FWHT and the cosine
           feature lift (reference kernels/fwht.py:25-131).
  scan  -- the float64 token recurrence that defines the delta rule (reference
           tests/test_fused_kernel.py:33-67, kernels/kernel_deltanet_fused.py:288-300) and an op-for-op
           torch CPU restatement of the chunked WY scan (reference kernels/fused_kernel_deltanet.py:47-155).

How each function is pinned (see tests/test_oracle_*.py):
  make_projection   torch.manual_seed(42) uniform stream (known values), Sylvester H vs scipy.linalg.hadamard,
                    Omega_m^T Omega_m = 4096 I, Omega columns vs butterfly construction, bit table vs signs.
  fwht_rows         explicit H products, involution H(Hx) = n x, brute force on tiny inputs.
  lift              ||phi_hat|| = 1, closed form on basis vectors (x = 0 -> cos(b)), Omega-vs-butterfly
                    projection, float32/float64 agreement.
  token_recurrence  brute-force dense-matrix products on tiny inputs, beta = 0 / orthonormal-key
                    overwrite closed forms, contractivity.
  chunked_forward   equals token_recurrence to 1e-12 in float64 for every chunk size, with and without
                    decay and initial state; reference carry-algebra pin (tests/test_inter_woodbury.py:14-84).
  factored_lift     ||phi|| = 1; closed form at x = 0 (cos(b1), cos(b2) halves); with both halves of x and
                    both projections equal it is the single lift divided by sqrt(2) (to the 1e-7 and 1e-8
                    epsilons); the seed-42 and seed-1042 tables are make_projection's (pinned above).
  rff_features      with renorm and the seed-42 projection equals lift (pinned above); closed form at x = 0.
  rkhs_features     ||phi|| = 1 exactly; phi(x).phi(y) = mean cos(sqrt(2 gamma) Omega (x - y)) (the
                    cos/sin pairing); gamma scaling at x and sqrt(gamma) x.
  linear_recurrence explicit double sum y_t = sum_{j<t} beta_j (prod lambda) (phi_q(t).phi_k(j)) v_j;
                    equals token_recurrence when the keys are mutually orthogonal (the erasure term
                    S_{t-1} phi_k(t) then vanishes), and differs from it otherwise.
  linear_chunked    equals linear_recurrence to 1e-12 for several chunk sizes and ragged T (the reference's
                    own acceptance check, tests/test_parallel_vs_recurrent.py:19-51).
  token_recurrence_torch / delta_rule_torch (the gradient oracle of the backward pass)
                    forward equals token_recurrence / delta_rule to 1e-12; torch.autograd.gradcheck
                    (central finite differences, float64) of every input -- q, k, v, beta, lambda, S_0 --
                    through the lift and the recurrence (pattern tests/test_fused_chunk_kernel.py:54-72).
"""
