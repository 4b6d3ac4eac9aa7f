"""CPU oracle of the fused-MoE path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import anything here. The product package (flaggems_sglang) never does, and
its ops raise instead of falling back to the CPU.
"""
