"""Measurement support: analytic traffic model, the benchmark configurations, timing.

Mirrors the reference's kernels/benchmarks (roofline.py, throughput.py) with
MI355X figures in place of the H100 ones.
"""
