"""ViperBench/argmax: HIP backend (hip_impl)."""
