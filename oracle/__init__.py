"""CPU oracle -- TEST INFRASTRUCTURE ONLY.

A plain restatement, on the CPU, of the reference's algorithm for the hot path
(attention forward, the SiLU MLP, the staged naive pipeline, and the tile
semantics of grammar programs), used only as the checker in tests/, in
__graft_entry__.smoke() and as bench.py's cpu_baseline leg. Nothing in the
product package imports it; the GPU path never routes through it.

Every function cites the reference file:line it follows. See each module's
header for which checks pin it.
"""
