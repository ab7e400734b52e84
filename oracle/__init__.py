"""CPU oracle of the tiered KV-cache arithmetic: test infrastructure only (the checker, never the product).
Importable only from tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg."""
