"""CPU oracle of the attention operator: TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker.
The product (supra2-img-web_amd/) never imports it.
"""
