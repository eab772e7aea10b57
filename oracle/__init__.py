"""CPU oracle of the reference's training-step hot path.

TEST INFRASTRUCTURE ONLY (see oracle/oracle.cpp): the checker that the HIP
product path is compared against.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import it.
"""
