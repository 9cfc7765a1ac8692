"""CPU oracle for the ncnn Convolution / DepthWise / InnerProduct / int8 path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
product library never imports or calls anything here.
"""
