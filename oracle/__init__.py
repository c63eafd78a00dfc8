"""CPU oracle of the packed ragged LayerSkip-Llama forward and its EESD step glue.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, where it is the parity reference or the timed CPU baseline -- never by the product path.
"""
