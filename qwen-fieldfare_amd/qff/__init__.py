"""Python host side of the MI355X attention hot path.

Mirrors the reference's per-layer dispatch (the encoder blocks inside
QwenQ4ActiveExpertStreamingRunner.forwardToken) over the C ABI in
include/qff/qff.h, loaded from the in-tree libqff_hip.so with ctypes.
torch supplies device memory and streams; the library does the compute and
fails loudly (QffError) when it is missing or a call is rejected. There is no
fallback path.
"""
from ._lib import (BF16, F16, F32, LIB_PATH, QffError, lib)  # noqa: F401
from . import checkpoint  # noqa: F401
from .ops import (Context, deltanet_decode, deltanet_prefill, gqa_decode,  # noqa: F401
                  gqa_prefill, q4_dequant, q4_matmul, q4_matmul_parts, q4_norm_matmul_parts,
                  q8_dequant, router_top8)
