"""The group-128 int4 interchange format and its dequant-GEMV, restated. TEST ONLY.

Format (reference ``kernels/tiled_gemv.py:242-288``, ``kernels/quantised_linear.py:193-207``):

* ``packed`` is uint8 ``[K/2, N]`` (K-major). Byte ``[j, n]`` holds ``k = j`` in its low
  nibble and ``k = j + K/2`` in its high nibble; nibbles are stored offset by 8.
* ``scale`` is ``[K/group, N]``. The reference stores fp32; the synthetic configs draw bf16.
  ``(nibble - 8) * scale`` is exact in fp32 either way (4-bit x 8/24-bit products).
* ``group = 128`` when ``K % 256 == 0`` else ``K / 2``.

The head/linear expression (reference ``kernels/visible_int4_head.py:187-199``)::

    W = bf16( (nibble - 8) * scale )            # rounded to bf16 BEFORE the product
    y = bf16( x.float() @ W.float() )           # fp32 accumulation, one final rounding
"""

from __future__ import annotations

import numpy as np
import torch

__all__ = [
    "bf16_bits_from_f32",
    "dequant_gemv",
    "dequant_gemv_variant",
    "dequantise_int4_k_major",
    "dequantise_int4_k_major_np",
    "f32_from_bf16_bits",
    "group_size_for",
    "quantise_int4_k_major",
]


def group_size_for(k: int) -> int:
    """Reference ``kernels/quantised_linear.py:193-207``."""
    if k % 2:
        raise ValueError(f"int4 packing needs an even K, got {k}")
    group = 128 if k % 256 == 0 else k // 2
    if group & (group - 1):
        raise ValueError(f"group {group} for K={k} is not a power of two")
    return group


# -- bit-level bf16 (numpy), an independent restatement of round-to-nearest-even ----------


def bf16_bits_from_f32(values: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest, ties to even (finite inputs)."""
    bits = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    lsb = (bits >> 16) & 1
    rounded = (bits + 0x7FFF + lsb) >> 16
    return rounded.astype(np.uint16)


def f32_from_bf16_bits(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def dequantise_int4_k_major_np(packed: np.ndarray, scale_bits: np.ndarray, group: int) -> np.ndarray:
    """``bf16((nibble - 8) * scale)`` as bf16 bit patterns ``[K, N]``, by integer arithmetic.

    ``scale_bits`` are bf16 bit patterns ``[K/group, N]``. Written without torch so that it
    pins the torch expression below rather than repeating it.
    """
    half, n = packed.shape
    k = 2 * half
    low = (packed & 0x0F).astype(np.int32) - 8
    high = (packed >> 4).astype(np.int32) - 8
    q = np.concatenate((low, high), axis=0)  # [K, N]: row j is k=j, row j+K/2 is k=j+K/2
    s = f32_from_bf16_bits(scale_bits)  # [K/group, N]
    s_full = np.repeat(s, group, axis=0)  # [K, N]
    product = q.astype(np.float32) * s_full  # exact: |q| <= 8, s has 8 significant bits
    return bf16_bits_from_f32(product).reshape(k, n)


# -- the torch expressions the reference uses ---------------------------------------------


def dequantise_int4_k_major(packed: torch.Tensor, scale: torch.Tensor, group_size: int) -> torch.Tensor:
    """``[K, N]`` fp32 weight (reference ``kernels/tiled_gemv.py:281-288``)."""
    half, n = packed.shape
    k = 2 * half
    nibbles = torch.cat((packed & 0x0F, packed >> 4), dim=0).to(torch.int16) - 8
    grouped = nibbles.float().reshape(k // group_size, group_size, n)
    return (grouped * scale.float().unsqueeze(1)).reshape(k, n)


def dequant_gemv(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, group_size: int) -> torch.Tensor:
    """``torch_dequant_gemv_int4`` (reference ``kernels/visible_int4_head.py:187-199``).

    ``x`` is ``[..., K]`` in the activation dtype; the result is ``[..., N]`` in that dtype.
    """
    k = packed.shape[0] * 2
    n = packed.shape[1]
    rows = x.reshape(-1, k)
    weight = dequantise_int4_k_major(packed, scale, group_size).to(x.dtype)
    out = rows.float() @ weight.float()
    return out.to(x.dtype).reshape(*x.shape[:-1], n)


def dequant_gemv_variant(x: torch.Tensor, packed: torch.Tensor, scale: torch.Tensor, group_size: int, *,
                         round_weights: bool = True, accumulate: torch.dtype = torch.float32) -> torch.Tensor:
    """``dequant_gemv`` with one of its two arithmetic choices changed, for measuring how far a
    model's outputs move under a change of that size (not a restatement of the reference):

    * ``accumulate=torch.float64``: the same bf16 weights, summed in float64 -- any fp32
      implementation differs from the reference by at most a summation-order change;
    * ``round_weights=False``: ``(nibble - 8) * scale`` kept exact (no bf16 rounding of the
      weight before the product), the arithmetic of a kernel that applies each group's scale
      once to an integer dot product.
    """
    k = packed.shape[0] * 2
    n = packed.shape[1]
    rows = x.reshape(-1, k)
    weight = dequantise_int4_k_major(packed, scale, group_size)
    if round_weights:
        weight = weight.to(x.dtype)
    out = rows.to(accumulate) @ weight.to(accumulate)
    return out.to(x.dtype).reshape(*x.shape[:-1], n)


def quantise_int4_k_major(weight: torch.Tensor, scale_dtype: torch.dtype = torch.bfloat16):
    """Symmetric int4 of an ``[N, K]`` weight into the K-major format.

    Reference ``kernels/tiled_gemv.py:242-278`` (scale = group amax / 7, round, clamp to
    [-7, 7], store q + 8). With ``scale_dtype=bfloat16`` the scale is rounded to bf16
    first and q is computed against the rounded scale, so the stored pair is self-consistent.
    Returns ``(packed [K/2, N] uint8, scale [K/group, N], group)``.
    """
    n, k = weight.shape
    group = group_size_for(k)
    half = k // 2
    blocks = weight.detach().float().reshape(n, k // group, group)
    s = blocks.abs().amax(dim=2) / 7.0
    s = torch.where(s > 0, s, torch.ones_like(s)).to(scale_dtype)
    q = torch.round(blocks / s.float().unsqueeze(2)).clamp_(-7, 7).to(torch.int16).reshape(n, k)
    low = (q[:, :half] + 8).to(torch.uint8)
    high = (q[:, half:] + 8).to(torch.uint8)
    packed = (low | (high << 4)).t().contiguous()
    return packed, s.t().contiguous(), group
