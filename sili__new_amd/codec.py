"""Host-side FP4 E2M1 codec (numpy), for building inputs on the host.

Same bit rules as the device codec (csrc/common.hpp) and the reference's
fp4quant.hpp:68-121: code 8 decodes to NaN, encoding rounds to nearest with
ties away from zero, saturates at 6, maps NaN and |v| < 0.25 to code 0.
"""
from __future__ import annotations

import numpy as np


def fp4_encode_np(v: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(v, dtype=np.float32).view(np.uint32)
    a = bits & np.uint32(0x7FFFFFFF)
    r = np.minimum(a + np.uint32(1 << 21), np.uint32(0x40C00000))
    hi = ((((r >> np.uint32(23)) & np.uint32(0xFF)) - np.uint32(126)) << np.uint32(1)) | ((r >> np.uint32(22)) & np.uint32(1))
    mag = np.where(a < 0x3E800000, 0, np.where(a < 0x3F400000, 1, np.where(a < 0x3F800000, 2, hi))).astype(np.uint32)
    mag = np.where(a > 0x7F800000, 0, mag)
    code = np.where(mag == 0, 0, ((bits >> np.uint32(31)) << np.uint32(3)) | mag)
    return code.astype(np.uint8)


def fp4_decode_np(code: np.ndarray) -> np.ndarray:
    c = np.asarray(code, dtype=np.uint32) & np.uint32(0xF)
    s, e, m = (c >> 3) & 1, (c >> 1) & 3, c & 1
    normal = (s << 31) | ((e + 126) << 23) | (m << 22)
    special = np.where(m == 1, np.uint32(0x3F000000) | (s << 31), np.where(s == 1, np.uint32(0x7FC00000), np.uint32(0)))
    return np.where(e == 0, special, normal).astype(np.uint32).view(np.float32)
