"""MI355X-native (gfx950) MOGT scan operator.

Public surface:
  - ``mogt_amd.ops``: ``diag_scan``, ``coupled_rank_scan`` (torch.ops.mogt.*).
Native code lives in ``mogt_amd/csrc`` (HIP, C ABI declared in
``include/mogt_scan.h``) and is built in-tree into ``mogt_amd/lib``.
"""
from . import _lib, ops  # noqa: F401
from .ops import coupled_rank_scan, dense_scan, diag_scan  # noqa: F401

__all__ = ["diag_scan", "coupled_rank_scan"]
