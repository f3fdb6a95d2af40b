"""CPU oracle for the fused kernel layer — TEST INFRASTRUCTURE ONLY.

A restatement, in plain torch CPU ops with fp32 arithmetic, of TrainScale's
math for RMSNorm, RoPE and vocabulary cross-entropy (reference paths in each
function's docstring, relative to data_pipeline/trainer/). It is the checker
for the gfx950 kernels and the CPU baseline that bench.py times. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it; the
product package never does.

Pinning (tests/test_oracle.py): every function here is checked against an
independent float64 formulation (numpy closed forms, complex-number rotation,
scipy logsumexp, torch.autograd on the float64 forward, finite differences)
and against the committed golden vectors in tests/golden/. TrainScale's own
tests hold no golden vectors for this path.
"""
from .ops import *  # noqa: F401,F403
