"""Blockwise absmax quantisation of optimizer state on the GPU.

Same layout and results as the reference's helpers
(came_pytorch/blockwise_quantization.py:11-42 for the allocators,
:66-82 / :112-124 for quantize / dequantize): flat row-major blocks of
``block_size`` elements, one fp32 absmax per block (``0 -> 1``), int8 codes
with Q = 127 (signed) or uint8 codes with Q = 255 (unsigned),
``code = clamp(round_half_even((x / absmax) * Q))`` and
``x = code * (absmax / Q)``.  The arithmetic runs in libcame8
(``came8_quantize_blockwise`` / ``came8_dequantize_blockwise``).
"""
from __future__ import annotations

import math

import torch

from . import _lib

SIGNED_QMAX = 127.0
UNSIGNED_QMAX = 255.0


def num_blocks(numel: int, block_size: int) -> int:
    """At least one block, even for an empty tensor (blockwise_quantization.py:11-14)."""
    if block_size <= 0:
        raise ValueError(f"block_size must be > 0, got {block_size}")
    return max(1, math.ceil(numel / block_size))


def init_qstate(shape, *, device, signed: bool, block_size: int):
    """Zero codes and unit absmax (blockwise_quantization.py:17-27)."""
    qdtype = torch.int8 if signed else torch.uint8
    q = torch.zeros(shape, device=device, dtype=qdtype)
    absmax = torch.ones((num_blocks(q.numel(), block_size),), device=device, dtype=torch.float32)
    return q, absmax


def init_batched_qstate(shape, *, batch_size: int, device, signed: bool, block_size: int):
    """``batch_size`` stacked states, blocks counted per item (blockwise_quantization.py:30-42)."""
    qdtype = torch.int8 if signed else torch.uint8
    q = torch.zeros((batch_size, *shape), device=device, dtype=qdtype)
    per_item_blocks = num_blocks(math.prod(shape), block_size)
    absmax = torch.ones((batch_size, per_item_blocks), device=device, dtype=torch.float32)
    return q, absmax


def _require_cuda(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{what}: came_amd runs on the GPU; got a {t.device} tensor")


def quantize_blockwise(tensor: torch.Tensor, *, signed: bool, block_size: int):
    """Return ``(codes shaped like tensor, absmax[num_blocks])`` computed by libcame8."""
    _require_cuda(tensor, "quantize_blockwise")
    lib = _lib.load()
    flat = tensor.detach().reshape(-1).to(torch.float32).contiguous()
    nb = num_blocks(flat.numel(), block_size)
    q = torch.empty(flat.numel(), device=flat.device, dtype=torch.int8 if signed else torch.uint8)
    absmax = torch.empty(nb, device=flat.device, dtype=torch.float32)
    with torch.cuda.device(flat.device):
        stream = torch.cuda.current_stream(flat.device).cuda_stream
        _lib.check(
            lib.came8_quantize_blockwise(flat.data_ptr(), flat.numel(), int(bool(signed)), int(block_size),
                                         q.data_ptr(), absmax.data_ptr(), stream),
            "came8_quantize_blockwise",
        )
    return q.view(tensor.shape), absmax


def dequantize_blockwise(q: torch.Tensor, absmax: torch.Tensor, *, signed: bool, block_size: int,
                         dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """``q * (absmax / Q)`` per element, shaped like ``q``."""
    _require_cuda(q, "dequantize_blockwise")
    lib = _lib.load()
    qc = q.contiguous()
    ac = absmax.to(torch.float32).contiguous()
    if ac.numel() < num_blocks(qc.numel(), block_size):
        raise ValueError("absmax has fewer entries than the number of blocks")
    out = torch.empty(qc.shape, device=qc.device, dtype=torch.float32)
    with torch.cuda.device(qc.device):
        stream = torch.cuda.current_stream(qc.device).cuda_stream
        _lib.check(
            lib.came8_dequantize_blockwise(qc.data_ptr(), ac.data_ptr(), qc.numel(), int(bool(signed)),
                                           int(block_size), out.data_ptr(), stream),
            "came8_dequantize_blockwise",
        )
    return out.to(dtype)
