"""CPU oracle for the MSDA operator -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or, in bench.py, as the CPU
baseline that is timed beside the GPU).  The product path
(msda-triton_amd/) never imports it and has no CPU fallback.

Contents (msda_reference.py), each restating a function of the reference
roulbac/msda-triton:
  msda_reference          per-level F.grid_sample      tests/reference_impls.py:12-45
  msda_naive              float64 loops                tests/reference_impls.py:48-87
  msda_backward_analytic  flat-index hand gradients    labs/solutions/lab07.py:12-104
  run_reference(_fp32)    CPU upcast protocol          tests/test_msda.py:80-93
  msda_fused_reference    front-end + operator         labs/solutions/lab00.py:201-208
  run_fused_reference     its CPU upcast protocol (fwd + 4 gradients)
and (projection_reference.py) the layer's projections either side:
  projection_reference            nn.Linear (+ masked rows)  labs/solutions/lab00.py:199-208
  projection_backward_reference   its gradients
Every function is pinned by tests/test_oracle.py, tests/test_oracle_fused.py
and tests/test_oracle_projection.py (naive vs grid_sample in float64, closed
forms, gradcheck, adjoint identity, torch's linear in float64,
planted-mistake checks).
"""

from .msda_reference import (  # noqa: F401
    level_start_index_of,
    msda_backward_analytic,
    msda_fused_reference,
    msda_naive,
    msda_reference,
    run_fused_reference,
    run_reference,
    run_reference_fp32,
)
from .projection_reference import (  # noqa: F401
    projection_backward_reference,
    projection_reference,
)
