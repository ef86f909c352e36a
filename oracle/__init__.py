"""CPU oracle of the multi-LoRA linear — test infrastructure only.

Importable by tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg;
never by the product package.
"""
