"""CPU oracle of Ferrum's KV-cache path: TEST INFRASTRUCTURE, never the product.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg.
"""
