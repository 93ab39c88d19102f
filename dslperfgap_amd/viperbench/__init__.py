"""Drop-in `hip_impl` modules, one per ViperBench kernel directory."""
