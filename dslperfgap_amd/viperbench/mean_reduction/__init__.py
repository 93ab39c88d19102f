"""ViperBench/mean_reduction: HIP backend (hip_impl)."""
