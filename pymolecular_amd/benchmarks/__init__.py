"""The reference's benchmark drivers (test_speedup.py, test_mem.py) on the HIP layer."""
