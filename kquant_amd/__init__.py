"""kquant_amd: MI355X-native block-scaled quantization hot path of kquant.

Drop-in modules mirroring kquant's API:
  kquant_amd.io.mxfp4         <- kquant/io/mxfp4.py
  kquant_amd.mxfp8            <- kquant/mxfp8.py
  kquant_amd.mxfp4            MXFP4 quantizer (absent from kquant)
  kquant_amd.constants        <- kquant/constants.py (format block)

Every compute call runs a HIP kernel of libkquant_amd.so (C ABI in
include/kquant_amd.h) on the GPU.
"""

from . import constants  # noqa: F401

__all__ = ["constants"]
