"""MI355X-native streaming sparse INT4 MLP (gfx950 HIP) behind LeanStream's
ComputeBackend / ExecDesc / ready-queue contracts.

The compute path is libleanstream_hip.so (built in-tree from leanstream_amd/csrc);
this package is its Python binding for tests and benchmarks.
"""
from . import synth
from ._native import LIBRARY_PATH, library
from .backend import (MODE_AUTO, MODE_BATCH_COMPAT, MODE_PROGRESSIVE, STATUS_BAD_DESCRIPTOR, STATUS_QUEUE_ERROR,
                      STATUS_TIMEOUT, Mapped, NativeBackend, ReadyQueue, quantize_io_load, rank_groups)

__all__ = ["synth", "library", "LIBRARY_PATH", "Mapped", "NativeBackend", "ReadyQueue", "rank_groups",
           "quantize_io_load", "MODE_AUTO", "MODE_BATCH_COMPAT", "MODE_PROGRESSIVE", "STATUS_TIMEOUT",
           "STATUS_QUEUE_ERROR", "STATUS_BAD_DESCRIPTOR"]
