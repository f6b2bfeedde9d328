"""CPU oracle for the reduction / scan path — test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker or as the timed CPU baseline; the product
package hephaestus_amd never does.
"""
