"""ViperBench/rms_norm: HIP backend (hip_impl)."""
