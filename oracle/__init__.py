"""CPU oracle for the W4A16 hot path -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import anything here, and only as the checker or the timed CPU baseline.
"""
