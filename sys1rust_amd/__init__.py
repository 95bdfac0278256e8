"""sys1rust_amd: an MI355X (gfx950) backend for sys1rust's decision model.

The compute path is libsys1hip.so (hand-written HIP kernels behind the C ABI of
include/sys1hip.h); this package holds its Python binding (`backend.HipBackend`), the synthetic
workloads, the answer decode and the build script.
"""
from .backend import BackendOutput, HipBackend, S1Error, synth_checkpoint  # noqa: F401
