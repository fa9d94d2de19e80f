"""CPU oracle of the packed complex-phase linear path (test infrastructure).

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg; the product under rpfq-review_amd/ never imports it.
"""
