"""CPU oracle of the ADana-family optimizer step: test infrastructure only.

Used by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as the
checker; the product package ``adana_amd`` never imports it.
"""
