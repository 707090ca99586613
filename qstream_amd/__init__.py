"""qstream_amd: MI355X (gfx950) backend for QStream's quantized matvec path.

* ``qstream_amd.qsf_hip``    ctypes mirror of libqsf_hip (include/qsf_hip.h)
* ``qstream_amd.qsf_format`` QSF block/outlier/MXFP4 payload writer
* ``qstream_amd.build``      in-tree build of libqsf_hip.so (gfx950)
"""
__all__ = ["qsf_hip", "qsf_format", "build"]
