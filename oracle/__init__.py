"""CPU oracle of the dotsnote FP8 sparse-MLA path. TEST INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() as the checker and by bench.py's cpu_baseline leg, never by the product package.

spmla_ref.py: numpy restatement of each function on the path (with the reference file:line it follows);
e4m3.c: an independent C e4m3fn encoder (nearest-value search), built into oracle/_build/ by build.py here.
cpu_port.py: the float32 torch-CPU restatement timed as the CPU baseline.
Parity status of each function (what pins it) is listed in spmla_ref.PINS; none is left unpinned.
"""
