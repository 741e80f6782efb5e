"""Parity oracle -- TEST INFRASTRUCTURE ONLY.

CPU restatements of the reference's hot-path arithmetic used as the checker in
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.  Nothing in
the product package (molnex_amd) imports, links or calls anything here.

Parity status of each function is stated in its module docstring.
"""
