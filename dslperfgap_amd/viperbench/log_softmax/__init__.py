"""ViperBench/log_softmax: HIP backend (hip_impl)."""
