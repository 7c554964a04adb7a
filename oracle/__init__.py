"""CPU oracle (test infrastructure only): a NumPy restatement of the reference algorithm used
as the checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg. The product
package ssa_amd never imports it."""
