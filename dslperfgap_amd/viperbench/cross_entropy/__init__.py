"""ViperBench/cross_entropy: HIP backend (hip_impl)."""
