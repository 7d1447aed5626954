"""CPU oracle of the reference MoE block arithmetic — test infrastructure only.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg; the product (pb_amd, libpbmoe.so) never uses it.
"""
