"""CPU oracle for the W4A8 MoE layer -- TEST INFRASTRUCTURE ONLY.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, and there only as the checker / the timed CPU baseline.
The product (q36_amd, libq36moe.so) never imports or calls it.
"""
