"""CPU oracle for the selective-scan hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in float64 on the CPU, the arithmetic of the reference's
selective scan so the HIP engine can be checked against it.  It is the checker,
never the thing measured or shipped: only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` may import it.  The product package
(``ssm_scan``) never imports anything from here and has no CPU fallback.

Modules
  scan_ref     numpy fp64 restatement: discretize, the four scan algorithms, the
               selective scan forward/backward with D skip and SiLU gate, the
               recurrent decode step, the causal depthwise conv, and the integer
               planning functions.
  c_oracle     ctypes binding of ssm_oracle.c (fp64 sequential scan + adjoint,
               OpenMP over channels) for sizes where numpy loops are too slow.
  cpu_chunked  torch-CPU restatement of the reference CPU path (SelectiveScanFn
               over scan_chunked), used as bench.py's cpu_baseline.

How each function is pinned (tests/test_oracle_*.py):
  discretize          closed forms; dense matrix-exponential ZOH (scipy expm);
                      RK4 integration of the ODE; Euler/bilinear -> ZOH as dt -> 0.
  scan_*              pure-Python scalar brute force; all algorithms agree with the
                      sequential loop incl. ragged chunks and extreme decays.
  selective_scan_fwd  scalar brute-force loop with math.exp/expm1; torch fp64.
  selective_scan_bwd  torch.autograd (fp64) through an independent textbook loop;
                      central finite differences on tiny shapes.  Its optional term
                      magnitudes (mag=True) equal the C oracle's for ddelta, bound
                      their values, equal |value| for one-term elements and add over
                      batch rows.
  ssm_step            decode step == one column of the full forward.
  conv1d_causal       torch.nn.functional.conv1d (fp64).
  plan functions      closed forms over exhaustive integer ranges; committed table.
  C oracle            equals the numpy oracle to 1e-12.
  all of the above    reproduce the committed vectors (tests/golden/vectors.npz) from
                      their stored inputs.
No function of the oracle is left "parity unpinned".
"""
