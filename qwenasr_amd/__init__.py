"""qwenasr_amd -- MI355X (gfx950) kernels for QwenASR's per-layer fused path.

* ``qwenasr_amd.kernels``  -- host mirror of ``qwen_asr::kernels`` over device tensors
* ``qwenasr_amd._lib``     -- ctypes binding of the C-ABI (include/qasr.h)
* ``qwenasr_amd.build``    -- hipcc build recipe for ``libqasr_hip.so`` / ``.a``
* ``qwenasr_amd.qint8``    -- ``.qint8`` weight files: reader, device upload (``QuantFile``)
* ``qwenasr_amd.decoder``  -- the INT8 decode step and prefill assembled from the entry points
"""
from ._lib import LIB_PATH, QasrError, QasrLibraryMissing, lib, version  # noqa: F401

__all__ = ["LIB_PATH", "QasrError", "QasrLibraryMissing", "lib", "version"]
