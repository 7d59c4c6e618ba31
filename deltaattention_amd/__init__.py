"""MI355X-native (gfx950) DeltaAttention prefill path.

Hand-written HIP kernels behind the C ABI of include/deltaattn.h (libdeltaattn.so):
anchor selection, fused index/pack/counts, the two-phase compressed GQA flash prefill
and the dense flash prefill used as the control.  ``ops`` is the torch-tensor API;
``flashAttention``, ``tritonModules``, ``deltaFlashAttention`` keep the reference's
module and kernel names for drop-in use.
"""
from ._native import DeltaAttnError, NativeLibraryError, lib  # noqa: F401

__version__ = "0.1.0"
