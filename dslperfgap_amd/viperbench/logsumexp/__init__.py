"""ViperBench/logsumexp: HIP backend (hip_impl)."""
