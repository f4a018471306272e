"""CPU oracle for the lgml ragged decode/prefill path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py import this package, and only as the checker
(or the CPU baseline). The shipped library (lgml_amd/) never imports it.
"""
