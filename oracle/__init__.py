"""CPU oracle for the fused-MoE hot path.

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, as the checker. The tinyserve_amd package never imports it.

- oracle.moe_oracle: torch-CPU restatement of the reference's plain-PyTorch MoE path
  (serve.py:933-996 moe_reference, serve.py:1089-1096 router) and a numpy restatement of
  moe_align_block_size (tinykernels.py:1070-1190).
- oracle.c_oracle: ctypes bindings of moe_oracle.c (bit-exact router and align restatements).
"""
