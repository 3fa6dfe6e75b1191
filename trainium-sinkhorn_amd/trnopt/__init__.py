"""trnopt for AMD Instinct MI355X: entropic optimal transport (log-domain Sinkhorn) with a fused HIP half-step.

Drop-in for the reference package's public surface (src/trnopt/__init__.py): Backend, SinkhornOptions,
SinkhornResult, sinkhorn, transport_plan. Backend.preset("rocm") with kernel="auto" or "hip" selects the
hand-written gfx950 kernels in hip_sinkhorn.py. plan_marginals and pull_back (trnopt.plan) evaluate a result's
plan without forming it.
"""

from .backend import Backend
from .sinkhorn import SinkhornOptions, SinkhornResult, sinkhorn, transport_plan
from .plan import plan_marginals, pull_back

__all__ = ["Backend", "SinkhornOptions", "SinkhornResult", "sinkhorn", "transport_plan", "plan_marginals",
           "pull_back"]
