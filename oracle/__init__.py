"""CPU restatement of esp's llama-family decoder (TEST INFRASTRUCTURE).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker / reported CPU baseline.
"""
