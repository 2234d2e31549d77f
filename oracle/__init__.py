"""CPU oracle of the FlashDP hot path -- test infrastructure, not product code.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg.  The product path (flashdp4review_amd) never imports it.
"""
