"""dslperfgap_amd: a gfx950 (MI355X) HIP backend for ViperBench's normalization /
row-reduction family (layer_norm, rms_norm, softmax, log_softmax, logsumexp,
cross_entropy).

The drop-in modules live at ``dslperfgap_amd/viperbench/<kernel>/hip_impl.py``
and export the reference's per-kernel function signatures; they call the
hand-written HIP kernels of ``libvbhip.so`` through its C ABI
(``include/vbhip.h``).
"""
__version__ = "0.1.0"
