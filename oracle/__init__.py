"""CPU oracle for the CyFA attention hot path -- TEST INFRASTRUCTURE ONLY.

This package restates the reference algorithm (Chyxx/CyFA-Jittor v0.1.2) on the
CPU in plain PyTorch so that the HIP path can be checked against it. It is the
checker, never the thing measured or shipped: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product package (``cyfa-jittor_amd/cyclic_flow_attention``) never
imports anything from here and fails loudly when its HIP library is missing.

Modules:
    cyfa_oracle   -- ops-level math (basis, phase, write vector, ScalarGatedLA in
                     chunkwise and recurrent form, slot readout, chunk_cyfa,
                     fused_recurrent_cyfa), in "exact" (float64, no intermediate
                     rounding) and "mirror" (float32 with bfloat16 rounding at the
                     reference's rounding points) modes.
    model_oracle  -- the layer / block / causal-LM plumbing around the op
                     (projections, short convolution, gates, gated RMSNorm,
                     SwiGLU MLP), used for layer and model parity.
    relative_time -- the README's relative-time recurrence with dense slot
                     transports, an independent formulation used to pin the
                     two-pass absolute-clock math.

Every function of the oracle is pinned by at least one check in
``tests/test_oracle_*.py`` (closed forms, brute force on tiny inputs, library
routines, invariants); see the table in the top of each test module.
"""
