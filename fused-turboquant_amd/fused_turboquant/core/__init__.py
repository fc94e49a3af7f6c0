"""Host-side mirror of the reference's ``fused_turboquant.core`` API."""
