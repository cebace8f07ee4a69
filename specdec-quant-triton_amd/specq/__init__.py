"""Host-side runtime of the MI355X quantized verification kernels.

_lib       ctypes binding of libspecq.so (include/specq.h)
workspace  per-device scratch for the split reductions
plan       device plan buffer for one-graph-for-every-shape replay
timing     event-based benchmarking with an Infinity-Cache flush
gen        seeded synthetic inputs for the benchmark configurations
"""
