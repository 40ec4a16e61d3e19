"""The oracle: a CPU restatement of the needle-cs quantized decode path.

TEST INFRASTRUCTURE ONLY.  Loaded by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the parity checker; the product
(needle_cs_amd/) never imports it.
"""
