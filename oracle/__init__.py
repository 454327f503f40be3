"""CPU oracle of the int8 hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and
only as the checker. The product package (torch_xdna) never imports it.
"""
