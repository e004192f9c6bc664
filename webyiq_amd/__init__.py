"""MI355X-native (gfx950) int4 x int8 linear-layer path of webyIQ.

Hand-written HIP kernels behind a C ABI (include/webyiq_q4q8.h), built in-tree
into libwebyiq_q4q8.so by webyiq_amd.build:
  per-token int8 activation quantiser, decode GEMV (M <= 8), prefill GEMM on
  int8 MFMA, lm_head GEMV with fused argmax.
webyiq_amd.ops is the host-side operator API (names of the reference's
Builder::quant / gemv / gemm / matmul / head_ops) over torch device tensors.
"""
from . import _lib  # noqa: F401

__all__ = ["ops", "build"]
