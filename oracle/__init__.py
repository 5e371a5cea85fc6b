"""CPU oracle of Realm's quantized compute path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py may
import this package.  The product (realm_amd/) never does.
"""
