"""ViperBench/max_reduction: HIP backend (hip_impl)."""
