"""MI355X (gfx950) DASH sparse attention: HIP kernels behind the reference's
Python interfaces (DashAttention, the inference router and the fused gather
attention)."""

__all__ = ["ops", "workloads"]
