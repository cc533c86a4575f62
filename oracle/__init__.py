"""CPU oracle for the joyomni_ops hot path — TEST INFRASTRUCTURE ONLY.

Restates on the CPU what the reference computes for each op of
deploy/joyomni_ops (each function cites the reference file:line it follows).
It is the checker, never the product: only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg import it; joyai-video-edit_amd/joyomni_ops never
does. ops.py holds the torch-on-CPU restatements; fp8_ref.c (built by build.py,
loaded by fp8ref.py) is an independent C restatement of the e4m3fn encoding and
of the per-token / per-group quantization rule. tests/test_oracle.py pins each
function against something independent of it.
"""
