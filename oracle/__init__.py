"""CPU oracle for the Mamba-1 selective scan — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may
import this package, and only as the checker / the reported CPU baseline. The
product path (``jax-mambas_amd/mamba_amd``) never imports it and fails loudly when
the HIP library is missing.

Modules:
  * ``scan64``   — float64 numpy restatement of the reference's sequential
                   recurrence (forward) and its hand-derived adjoint (backward),
                   including the fused extras (delta bias, softplus, D skip,
                   silu(z) gate, initial / last state, variable lengths).
  * ``assoc_torch`` — torch CPU restatement of the reference's pure-JAX
                   ``selective_scan_reference`` (odd/even associative scan over a
                   materialised (B, L, D, N) tensor); used as the CPU baseline and as an
                   independent formulation the sequential oracle is checked against.
  * ``mamba1_torch`` — torch restatement of the reference's Mamba-1 S6 / block / stacked
                   model in its (B, L, features) layout, for checking the channel-major
                   model of the product end to end.
"""
