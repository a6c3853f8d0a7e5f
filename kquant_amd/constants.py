"""Format constants of the MX codec (kquant/constants.py:64-75).

compressed-tensors "mxfp4-pack-quantized":
  weight_packed: uint8 [out, in/2], two E2M1 codes per byte, low nibble first
  weight_scale:  uint8 [out, in/32], E8M0 (value = 2^(byte - 127)), K-blocks
"""

MXFP4_BLOCK = 32
E8M0_BIAS = 127
# E2M1 code -> value; codes 8..15 are the negated mirror (8 == -0).
E2M1_LUT = (
    0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
)
MXFP4_BITS_EFFECTIVE = 4.25  # 4b code + 8b scale / 32
E2M1_MAX = 6.0
