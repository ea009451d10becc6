"""Host-side weight formats and load transforms for the quantised decode path.

Q1 ("Q1_0_g128", nnmetal/src/metal.zig:227-335):
  * codes: row-major [M x K] bit matrix, 32 columns per little-endian uint32
    word, bit i of word j <-> column 32*j + i (LSB first; the byte view is the
    same as nnmetal/src/shaders/compute.metal:1654-1671).
  * scales: one float16 per ``group_size`` consecutive weights of a row,
    index ``row * K/gs + col/gs``.
  * dequant: ``bit ? +s : -s``.  MLX stores an affine (scale, bias) pair;
    the load transform keeps ``s = f16(f32(scale) / 2)`` and drops the bias
    (nnmetal/src/model.zig:911-960, :1058-1070).  That is exact only when
    ``bias == -scale/2``; :func:`q1_affine_to_symmetric` checks it.

Q4 ("Q4_MLX", nnmetal/src/metal.zig:337-469):
  * codes: row-major [M x K] 4-bit unsigned nibbles, 8 per uint32 word,
    nibble i of word j <-> column 8*j + i at bits [4i, 4i+3]
    (nnmetal/src/shaders/q4mv_bf16_specialized.metal:24-27).
  * scales, biases: one 16-bit value per group; the reference stores raw
    BF16 and truncates f16/f32 checkpoint values to BF16 at load
    (nnmetal/src/model.zig:1169-1220).  This build also accepts float16
    scales/biases unchanged (``scale_dtype`` in the weight descriptor).
  * dequant: ``s * nibble + b``.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

DT_F32 = 0
DT_F16 = 1
DT_BF16 = 2


@dataclass
class QWeight:
    """Host copy of one quantised matrix (the reference's PackedBuffer/Q4Buffer)."""

    bits: int            # 1 or 4
    M: int
    K: int
    group_size: int
    codes: np.ndarray    # uint32 [M, K*bits/32]
    scales: np.ndarray   # uint16 raw (f16 or bf16 bits) [M, K/gs]
    biases: np.ndarray | None  # uint16 raw [M, K/gs] (Q4 only)
    scale_dtype: int     # DT_F16 or DT_BF16

    @property
    def nbytes(self) -> int:
        n = self.codes.nbytes + self.scales.nbytes
        if self.biases is not None:
            n += self.biases.nbytes
        return n


def pack_q1(bits: np.ndarray) -> np.ndarray:
    """bool/uint8 [M, K] -> uint32 [M, K/32], LSB-first."""
    bits = np.asarray(bits, dtype=np.uint8)
    M, K = bits.shape
    assert K % 32 == 0
    by = np.packbits(bits.reshape(M, K // 8, 8), axis=-1, bitorder="little")
    return np.ascontiguousarray(by.reshape(M, K // 8)).view("<u4").reshape(M, K // 32)


def unpack_q1(codes: np.ndarray, K: int) -> np.ndarray:
    codes = np.ascontiguousarray(codes, dtype="<u4")
    M = codes.shape[0]
    by = codes.view(np.uint8).reshape(M, K // 8)
    return np.unpackbits(by, axis=-1, bitorder="little").reshape(M, K)


def pack_q4(nibbles: np.ndarray) -> np.ndarray:
    """uint8 [M, K] values 0..15 -> uint32 [M, K/8], nibble i at bits 4i."""
    nib = np.asarray(nibbles, dtype=np.uint32)
    M, K = nib.shape
    assert K % 8 == 0
    nib = nib.reshape(M, K // 8, 8)
    shifts = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    return np.bitwise_or.reduce(nib << shifts, axis=-1).astype(np.uint32)


def unpack_q4(codes: np.ndarray, K: int) -> np.ndarray:
    codes = np.asarray(codes, dtype=np.uint32)
    M = codes.shape[0]
    shifts = (np.arange(8, dtype=np.uint32) * 4)[None, None, :]
    return ((codes[:, :, None] >> shifts) & np.uint32(0xF)).astype(np.uint8).reshape(M, K)


def f16_bits(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, dtype=np.float16).view(np.uint16)


def q1_affine_to_symmetric(scale_f16: np.ndarray, bias_f16: np.ndarray | None,
                           check: bool = True) -> np.ndarray:
    """MLX affine 1-bit (scale, bias) -> symmetric half scale, as f16 bits.

    Follows nnmetal/src/model.zig:1058-1070 (``f16(f32(s) / 2)``).  With
    ``check`` the function refuses groups whose bias is not exactly
    ``-scale/2``, the only case in which dropping the bias is lossless.
    """
    s = np.asarray(scale_f16, dtype=np.float16)
    half = (s.astype(np.float32) / np.float32(2.0)).astype(np.float16)
    if check and bias_f16 is not None:
        b = np.asarray(bias_f16, dtype=np.float16)
        if not np.array_equal(b.astype(np.float32), -half.astype(np.float32)):
            raise ValueError("Q1 affine->symmetric: bias != -scale/2 for some group")
    return half.view(np.uint16)


def to_bf16_truncate(x_f16_or_f32: np.ndarray) -> np.ndarray:
    """The reference's copyRawBF16 for f16/f32 sources: widen to f32 and keep
    the upper 16 bits (truncation), nnmetal/src/model.zig:1191-1215."""
    f = np.asarray(x_f16_or_f32).astype(np.float32)
    return (f.view(np.uint32) >> np.uint32(16)).astype(np.uint16)
