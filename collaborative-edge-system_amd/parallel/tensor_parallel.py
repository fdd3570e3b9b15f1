"""``collab_infer.parallel.tensor_parallel`` for this path: the fused column-parallel
projection (collab_infer/parallel/tensor_parallel.py:264-313) on one device, computed by the
gfx950 GEMM, plus the fused gate/up projection with its activation."""

from ..projection import FusedColumnParallelLinear, fused_linear, linear, linear_gated  # noqa: F401

__all__ = ["FusedColumnParallelLinear", "fused_linear", "linear", "linear_gated"]
