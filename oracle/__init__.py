"""CPU oracle for the W8A8 path -- TEST INFRASTRUCTURE ONLY.

Used by tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py as
the checker / baseline; the product (fish-audio-cpp_amd/) never imports it.
"""
