"""TEST INFRASTRUCTURE ONLY -- the CPU oracle the HIP path is checked against.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker (or, for the baseline,
as the timed CPU path); the product in ``gm-attention_amd/`` never imports it.

* :mod:`oracle.eager` -- a float64 PyTorch restatement of the reference's
  pure-PyTorch (eager) path at the fused ops' boundary, each function citing
  the reference file:line it follows; gradients come from autograd.
* :mod:`oracle.sphere` -- numpy brute force for neighbourhoods and
  Clenshaw-Curtis weights from Chebyshev moments.
* :mod:`oracle.ref` -- ``oracle/_ref/libgmref.so``: the reference's own
  header-only CPU arithmetic (``nn/fused/attention.h``, ``factored.h``)
  compiled by ``oracle/Makefile`` from ``oracle/ref_driver.cpp``.

Each function is pinned by the CPU tests ``tests/test_oracle_*.py``: the
reference's own known answers, the compiled reference, closed forms, finite
differences or gauge equivariance.
"""
