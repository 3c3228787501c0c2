"""CPU oracle for the BudgetFormer hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm for
  * budgeted query-centric edge construction (``edge_table``), and
  * sparse edge attention forward/backward (``sparse_attention``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import it, and only as the checker / the timed CPU baseline. The
product path (``budgetformer_amd``) never imports it and fails loudly when the
HIP library is missing.

Pinning status (what each function is checked against) is listed in the
header of each module.
"""
