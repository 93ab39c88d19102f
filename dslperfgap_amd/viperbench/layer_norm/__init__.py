"""ViperBench/layer_norm: HIP backend (hip_impl)."""
