"""sihc_hip: SiHC hyper-connection read/write path on MI355X (gfx950) HIP kernels.

Modules
  sublayer_kernels   drop-in for the reference's sihc/models/sihc/sublayer_kernels.py
                     (`sihc::` custom ops: read, write, weight grad, triangular)
  blockwise_kernels  drop-in for the reference's block-wise adapters
  event_ops          per-event fused write+read (literal schedule) with autograd
  indexed            spatially indexed (int32 state index) gather/scatter and read/write
  launch             tensor-level launchers over the C ABI (include/sihc_hip.h)
"""
from ._lib import LIB_PATH, lib  # noqa: F401
from .sublayer_kernels import sublayer_read, sublayer_triangular, sublayer_write  # noqa: F401
from .event_ops import event_write_read, literal_stage  # noqa: F401

__all__ = ["LIB_PATH", "lib", "sublayer_read", "sublayer_write", "sublayer_triangular",
           "event_write_read", "literal_stage"]
