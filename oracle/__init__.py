"""CPU oracle of the fused QKV + QK-Norm + RoPE path -- test infrastructure only.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg; the shipped package (mqk) never uses it.
"""
