"""ViperBench/softmax: HIP backend (hip_impl)."""
