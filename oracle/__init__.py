"""CPU oracle for the TTC-Net batched receding-horizon LQR solve.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package (``ttc-net_amd/``)
may import, call, link or execute anything under ``oracle/``.  The only
permitted users are ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` -- and there only as the *checker* or as
the timed CPU baseline, never as the thing measured on the GPU.

Contents
--------
``lqr64``    fp64 numpy restatement of the reference ``riccati`` forward and of
             the ``kkt`` implicit-differentiation backward, chained through the
             discount expansion (ground truth for every parity test).
``dense_qp`` fp64 torch brute-force dense QP over all controls; independent of
             any Riccati recursion, differentiable by autograd.  Pins ``lqr64``.
``ref_torch`` op-for-op torch restatement of the reference ``direct_lqr_solve``
             (``riccati``) and ``kkt_lqr_solve`` (``kkt``), including their fp32
             casts; used as the CPU baseline and to report the reference
             algorithm's own error against fp64.
``layer_ref`` torch restatement of the ``TTCLayer`` front-end / back-end around
             the solver call (random-init weights, configs 1-5).
``inputs``   seeded synthetic input generators (solver-level and layer-level).

Pinning status of every function is listed in each module's header.
"""
