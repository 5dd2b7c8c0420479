"""MI355X (gfx950) HIP backend for the qppocr-kernels operator set.

Modules:
  _lib   ctypes binding of libqppocr_hip.so (include/qppocr_hip.h)
  ops    operator API mirroring qppocr-kernels (conv2d, sgemm, softmax_last_dim, ...)
  nets   det / rec graphs of the synthetic workloads and HipSession (DeviceSession)
  build  compiles csrc/*.hip for gfx950
"""
__all__ = ["ops", "nets", "build"]
