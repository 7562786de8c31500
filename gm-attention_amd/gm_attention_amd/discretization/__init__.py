"""Sphere discretization: grids, tangent frames, CSR neighbourhoods and
per-edge geometry (the reference's ``gm_attention.discretization``)."""
