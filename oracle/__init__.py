"""The oracle: CPU restatements of the reference's Sinkhorn, used ONLY as a checker.

TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and
only to check or to time the reference's CPU path; the product (trainium-sinkhorn_amd/trnopt) never imports
it and has no fallback to it.

Modules
  reference.py  -- the reference's plain-PyTorch Sinkhorn (src/trnopt/sinkhorn.py:108-119, 131-167, 211-403),
                   restated on the CPU in float64 or float32. The parity target of the HIP path, and (float32,
                   all host cores) the CPU baseline of bench.py.
  brute.py      -- independent float64 checks: full-cost-matrix log-domain Sinkhorn with scipy logsumexp
                   (tests/test_sinkhorn.py:54-71 of the reference, extended with the reference's initial g and
                   eps schedules), wot's scaling-form iteration (tests/test_sinkhorn.py:186-205), and the
                   row-LSE / half-step kernel known-answer formulas (examples/nki_sinkhorn_check.py:22-35, 60-73).
  data.py       -- seeded input generators for the benchmark configurations.

How each function is pinned (tests/test_oracle.py):
  reference.sinkhorn_ref, float64 -- the reference's published float64 cost 0.8971549234175153 at 20
      iterations (results/sinkhorn_trn1.2xlarge_2026-10-30.csv:5, mixture clouds 10k x 10k d 64, eps 0.05);
      iterate-by-iterate equality with brute.sinkhorn_dense (no shifted potentials, no padding, dense C) for
      balanced / unbalanced / targets / eps_start / stages / blocks; plans against the converged brute force
      and wot's scaling form; row sums == a exactly after an f update.
  reference.sinkhorn_ref, float32 -- within float32 rounding of the float64 run; the published float32 costs
      of the same problem (0.8971549341961733 torch, 0.8971549319624892 NKI; csv:5,10) to the float32 level
      (test_published_float32_cost_10k).
  reference.eps_schedule -- its closed form eps_start decay^k (strictly above eps, capped at max_iters) and the
      stage override (test_eps_schedule_closed_form), for the oracle and the product alike.
  brute.* -- closed forms and special cases (m = 1, identical columns, translation of the potentials,
      comparison against scipy on random inputs), and mutation tests that plant a wrong sign / index in the
      oracle and require a pin to fail.
  Iteration counts of staged / unbalanced runs where a check lands within rounding of a threshold: parity
      unpinned beyond the brute-force iterate equality (the reference was not run to produce fixtures).
"""
