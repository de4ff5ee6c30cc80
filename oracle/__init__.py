"""CPU oracle for the PKDA recurrence -- test infrastructure, never the product.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg import this package.  The product package ``delta_feedback_experiment_amd``
fails loudly when its HIP library is missing instead of falling back here.
"""
