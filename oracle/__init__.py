"""CPU oracle of the Bonsai/Qwen3 decode path -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, and only as the checker or the timed CPU baseline.  Nothing in the
product package (nnzap_amd) imports it.
"""
