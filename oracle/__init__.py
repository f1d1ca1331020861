"""ORACLE: CPU restatements of the reference's int8 graph semantics (test infrastructure only).

semantics.py / interp.py restate anvil/semantics.py, xf.golden and anvil/interp/graph.py in numpy; scalar_oracle.c
restates the same ops as per-element C loops. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
use this package, as the checker or the timed CPU baseline; the product path never imports it.
"""
