"""CPU oracle for the KudaCuda gfx950 decode path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import anything from this package, and only as the checker / CPU baseline.
"""
