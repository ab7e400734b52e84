"""CPU oracle of the tiered KV-cache arithmetic: test infrastructure only (what the kernels are compared with, never the product).
Importable only from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg."""
