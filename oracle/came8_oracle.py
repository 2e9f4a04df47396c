"""CPU oracle for the CAME 8-bit optimizer step -- TEST INFRASTRUCTURE ONLY.

This module is the checker that the HIP kernels in ``came_amd`` are compared
against.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it.  The product path (``came_amd``) never
imports, calls or falls back to anything here.

It restates, op for op on CPU torch tensors, the arithmetic of the reference's
pure-PyTorch CPU path:

* blockwise absmax quantisation   -- reference ``came_pytorch/blockwise_quantization.py:11-42,66-82,112-124``
* the full8bit state layout       -- reference ``came_pytorch/CAME8bitFull.py:748-788,919-923``
  (CPU branch; ``CAME8bitMemory.py:390-447`` uses the same shapes)
* one full8bit parameter step     -- reference ``came_pytorch/CAME8bitFull.py:939-1075`` (CPU branch)
* the fp32-state CAMECUDA step    -- reference ``came_pytorch/CAMECUDA.py:275-326`` (generic branch)
* the 8bit2d step (16x16-tile momentum) -- reference CUDA kernels, ``came_cuda/csrc/came_kernels.cu``
  (see ``came8bit2d_step``; parity unpinned against the reference, which cannot run here)

The op sequence is kept identical to the reference because the point of the
oracle is bit-level agreement with it: each rounding step (``mul_`` then
``add_(alpha=)`` which torch CPU evaluates as one fused multiply-add, true
division, ``rsqrt`` = correctly rounded ``1/sqrt``, round-half-even) is the
same one the reference performs.  The oracle is pinned by
``tests/golden/*.npz`` (vectors written by importing the reference's CPU path,
see ``tests/golden/make_golden.py``) and by closed-form tests in
``tests/test_oracle_closed_form.py``.
"""
from __future__ import annotations

import math
from typing import Dict

import numpy as np

import torch

SIGNED_QMAX = 127.0
UNSIGNED_QMAX = 255.0


# --------------------------------------------------------------------------
# blockwise quantisation  (reference blockwise_quantization.py)
# --------------------------------------------------------------------------
def num_blocks(numel: int, block_size: int) -> int:
    """Reference blockwise_quantization.py:11-14 (at least one block, even when empty)."""
    if block_size <= 0:
        raise ValueError(f"block_size must be > 0, got {block_size}")
    return max(1, math.ceil(numel / block_size))


def quantize_blockwise(x: torch.Tensor, *, signed: bool, block_size: int):
    """Reference blockwise_quantization.py:66-82.

    Flat row-major blocks of ``block_size``; the tail block is zero padded
    (so an unsigned block's max includes 0).  ``absmax == 0 -> 1``.
    ``q = clamp(round_half_even((x / absmax) * Q))`` with Q = 127 (int8) or 255 (uint8).
    """
    flat = x.detach().reshape(-1).to(torch.float32)
    nb = num_blocks(flat.numel(), block_size)
    buf = torch.zeros(nb * block_size, dtype=torch.float32)
    buf[: flat.numel()] = flat
    blocks = buf.view(nb, block_size)
    if signed:
        amax = blocks.abs().amax(dim=1)
        qmax, lo, qdtype = SIGNED_QMAX, -SIGNED_QMAX, torch.int8
    else:
        amax = blocks.amax(dim=1)
        qmax, lo, qdtype = UNSIGNED_QMAX, 0.0, torch.uint8
    amax = torch.where(amax > 0, amax, torch.ones_like(amax))
    scaled = (blocks / amax.unsqueeze(1)) * qmax
    q = torch.round(scaled).clamp(lo, qmax).to(qdtype)
    return q.reshape(-1)[: flat.numel()].view_as(x), amax


def dequantize_blockwise(q: torch.Tensor, absmax: torch.Tensor, *, signed: bool, block_size: int) -> torch.Tensor:
    """Reference blockwise_quantization.py:112-124: ``q * (absmax / Q)`` per element."""
    qf = q.reshape(-1).to(torch.float32)
    step = absmax.repeat_interleave(block_size)[: qf.numel()] / (SIGNED_QMAX if signed else UNSIGNED_QMAX)
    return (qf * step).view_as(q)


def quantize_items(x: torch.Tensor, items: int, *, signed: bool, block_size: int):
    """quantize_blockwise restarted at each of ``items`` equal consecutive parts of ``x`` (the per-matrix
    blocks of the reference's CUDA N-D layout, CAME8bitFull.py:790-829, which quantises with
    init_batched_qstate's (batch, n) shapes, blockwise_quantization.py:30-42): every part zero padded to
    whole blocks of its own.  Returns the codes (shape of x) and the scales [items][blocks per part]."""
    parts = x.detach().reshape(items, -1).to(torch.float32)
    n = parts.shape[1]
    nb = num_blocks(n, block_size)
    buf = torch.zeros(items, nb * block_size, dtype=torch.float32)
    buf[:, :n] = parts
    blocks = buf.view(items, nb, block_size)
    if signed:
        amax = blocks.abs().amax(dim=2)
        qmax, lo, qdtype = SIGNED_QMAX, -SIGNED_QMAX, torch.int8
    else:
        amax = blocks.amax(dim=2)
        qmax, lo, qdtype = UNSIGNED_QMAX, 0.0, torch.uint8
    amax = torch.where(amax > 0, amax, torch.ones_like(amax))
    scaled = (blocks / amax.unsqueeze(2)) * qmax
    q = torch.round(scaled).clamp(lo, qmax).to(qdtype)
    return q.reshape(items, -1)[:, :n].reshape(x.shape), amax


def dequantize_items(q: torch.Tensor, absmax: torch.Tensor, items: int, *, signed: bool,
                     block_size: int) -> torch.Tensor:
    """dequantize_blockwise of each of ``items`` consecutive parts with its own scales [items][blocks]."""
    parts = q.reshape(items, -1).to(torch.float32)
    n = parts.shape[1]
    step = absmax.reshape(items, -1).repeat_interleave(block_size, dim=1)[:, :n] / (
        SIGNED_QMAX if signed else UNSIGNED_QMAX)
    return (parts * step).reshape(q.shape)


def is_per_matrix(st: Dict[str, object]) -> bool:
    """The reference CUDA N-D path's per-matrix layout (flags of CAME8bitFull.py:783-785)."""
    return bool(st.get("_cuda_factored_nd_ext_path", False) or st.get("_cuda_factored_nd_chunked_ext_path", False))


# --------------------------------------------------------------------------
# state layout (reference CAME8bitFull._init_state, CPU branch)
# --------------------------------------------------------------------------
def init_full8bit_state(shape, block_size: int = 256, per_matrix: bool = False) -> Dict[str, object]:
    """Reference CAME8bitFull.py:748-788,919-923 (CPU branch) and blockwise_quantization.py:17-42.

    ``per_matrix`` (N-D shapes, ndim >= 3): the reference CUDA N-D path's layout instead
    (CAME8bitFull.py:790-829): scales per matrix, ``exp_avg_absmax`` [P][ceil(R*C/B)], row codes
    [2P][R] with scales [2P][ceil(R/B)], column codes [2P][C] with scales [2P][ceil(C/B)], its
    routing flags and shape keys (its fp32 scratch buffers are left out)."""
    shape = tuple(int(s) for s in shape)
    if per_matrix and len(shape) >= 3:
        P, R, C = math.prod(shape[:-2]), shape[-2], shape[-1]
        st = {"step": 0, "_mode": "full8bit", "RMS": 0}
        st["exp_avg_q"] = torch.zeros(shape, dtype=torch.int8)
        st["exp_avg_absmax"] = torch.ones((P, num_blocks(R * C, block_size)), dtype=torch.float32)
        st["factored"] = True
        st["factored_row_q"] = torch.zeros((2 * P, R), dtype=torch.uint8)
        st["factored_row_absmax"] = torch.ones((2 * P, num_blocks(R, block_size)), dtype=torch.float32)
        st["factored_col_q"] = torch.zeros((2 * P, C), dtype=torch.uint8)
        st["factored_col_absmax"] = torch.ones((2 * P, num_blocks(C, block_size)), dtype=torch.float32)
        st.update(_cuda_factored_fastpath=True, _cuda_factored_nd_ext_path=True,
                  _cuda_factored_nd_chunked_ext_path=False, _cuda_factored_ext_path=True,
                  prefix_batch=P, matrix_rows=R, matrix_cols=C)
        return st
    numel = math.prod(shape)
    st: Dict[str, object] = {"step": 0, "_mode": "full8bit", "RMS": 0}
    st["exp_avg_q"] = torch.zeros(shape, dtype=torch.int8)
    st["exp_avg_absmax"] = torch.ones(num_blocks(numel, block_size), dtype=torch.float32)
    factored = len(shape) >= 2
    st["factored"] = factored
    if factored:
        row_shape = shape[:-1]
        col_shape = shape[:-2] + shape[-1:]
        st["factored_row_q"] = torch.zeros((2,) + row_shape, dtype=torch.uint8)
        st["factored_row_absmax"] = torch.ones((2, num_blocks(math.prod(row_shape), block_size)), dtype=torch.float32)
        st["factored_col_q"] = torch.zeros((2,) + col_shape, dtype=torch.uint8)
        st["factored_col_absmax"] = torch.ones((2, num_blocks(math.prod(col_shape), block_size)), dtype=torch.float32)
        # the CUDA routing flags, all False on CPU (CAME8bitFull.py:783-787)
        for k in ("_cuda_factored_fastpath", "_cuda_factored_nd_ext_path", "_cuda_factored_nd_chunked_ext_path",
                  "_cuda_factored_ext_path"):
            st[k] = False
    else:
        st["exp_avg_sq_q"] = torch.zeros(shape, dtype=torch.uint8)
        st["exp_avg_sq_absmax"] = torch.ones(num_blocks(numel, block_size), dtype=torch.float32)
        st["_cuda_nonfactored_fastpath"] = False  # CAME8bitFull.py:921
    return st


def _approx_sq_grad(row: torch.Tensor, col: torch.Tensor) -> torch.Tensor:
    """Reference CAME8bitFull.py:124-128.

    NB: ``col.unsqueeze(-2).clamp_min_`` clamps the caller's column state in
    place (it is a view), so the stored/quantised column state is clamped to
    >= 1e-30; the row state is not.
    """
    rmean = row.mean(dim=-1, keepdim=True).clamp_min_(1e-30)
    r = (row / rmean).rsqrt_().unsqueeze(-1)
    c = col.unsqueeze(-2).clamp_min_(1e-30).rsqrt()
    return torch.mul(r, c)


def _rms(t: torch.Tensor) -> torch.Tensor:
    """Reference CAME8bitFull.py:121-122."""
    return t.norm(2) / (t.numel() ** 0.5)


@torch.no_grad()
def full8bit_step(p: torch.Tensor, grad: torch.Tensor, st: Dict[str, object], *, beta1: float, beta2: float,
                  beta3: float, eps0: float, eps1: float, lr: float, clip_threshold: float,
                  weight_decay: float, block_size: int, capture: Dict[str, torch.Tensor] | None = None,
                  exact_norm: bool = False, fp16_update: bool = False) -> None:
    """One CPU full8bit step on parameter ``p`` (in place) and state ``st`` (in place).

    Follows reference CAME8bitFull.py:962-966 (step/RMS bookkeeping) and
    :1006-1075 (the arithmetic), in the same operation order.  If ``capture``
    is a dict it receives the fp32 states just before they are requantised
    (keys ``exp_avg``, ``sq_row``/``sq_col``/``res_row``/``res_col`` or ``sq``)
    and the clip divisor; capturing does not change any result.

    ``capture`` also receives the clipped update (``update``) and, for factored
    tensors, the residual factor the momentum is scaled by (``res_factor``).

    ``exact_norm=True`` replaces the reference's float32 ``norm(2)`` (whose
    accumulation error reaches ~1e-4 relative on multi-million-element
    tensors) by sqrt of the fp64 sum of squares rounded to float32: the
    library's opt-in exactly rounded clip (CAME8_FLAG_EXACT_NORM).  Every
    other operation is unchanged.

    ``fp16_update=True`` is the reference's fp16-update CUDA variant for
    unfactored tensors (came_kernels.cu:1068-1122,1546-1601): the norm is that
    of the fp32 update, and the momentum takes the update rounded to fp16 (round
    to nearest even) before the clip division.
    """
    st["step"] += 1
    st["RMS"] = _rms(p)
    if grad.dtype in (torch.float16, torch.bfloat16):
        grad = grad.float()
    bs = block_size
    factored = st["factored"]
    # the reference CUDA N-D path's per-matrix blocks (is_per_matrix): the same arithmetic, each of the P
    # matrices quantised in blocks of its own (items); one item is the flat layout
    pm = factored and is_per_matrix(st) and p.dim() >= 3
    P = math.prod(p.shape[:-2]) if pm else 1

    def deq(q, a, signed, items):
        if pm:
            return dequantize_items(q, a, items, signed=signed, block_size=bs)
        return dequantize_blockwise(q, a, signed=signed, block_size=bs)

    def quant(x, signed, items):
        if pm:
            return quantize_items(x, items, signed=signed, block_size=bs)
        return quantize_blockwise(x, signed=signed, block_size=bs)

    m = deq(st["exp_avg_q"], st["exp_avg_absmax"], True, P)
    upd = (grad ** 2) + eps0
    if factored:
        # [0]: the second moment, [1]: the residual (per-matrix: [2P][n] stored, the same element order)
        rq, ra = st["factored_row_q"].view(2, -1), st["factored_row_absmax"].view(2, -1)
        cq, ca = st["factored_col_q"].view(2, -1), st["factored_col_absmax"].view(2, -1)
        row_shape, col_shape = p.shape[:-1], p.shape[:-2] + p.shape[-1:]
        sq_row = deq(rq[0], ra[0], False, P).view(row_shape)
        sq_col = deq(cq[0], ca[0], False, P).view(col_shape)
        sq_row.mul_(beta2).add_(upd.mean(dim=-1), alpha=1.0 - beta2)
        sq_col.mul_(beta2).add_(upd.mean(dim=-2), alpha=1.0 - beta2)
        upd = _approx_sq_grad(sq_row, sq_col)
        upd.mul_(grad)
    else:
        sq = dequantize_blockwise(st["exp_avg_sq_q"], st["exp_avg_sq_absmax"], signed=False, block_size=bs)
        sq.mul_(beta2).add_(upd, alpha=1.0 - beta2)
        upd = sq.clamp_min_(1e-30).rsqrt().mul_(grad)

    if exact_norm:
        norm = torch.tensor(math.sqrt(float((upd.double() ** 2).sum())), dtype=torch.float32)
        rms = norm / (upd.numel() ** 0.5)
    else:
        rms = _rms(upd)
    clipv = (rms / clip_threshold).clamp_(min=1.0)
    if fp16_update and not factored:
        upd = upd.half().float()
    upd.div_(clipv)
    if capture is not None:
        capture["update"] = upd.clone()
    m.mul_(beta1).add_(upd, alpha=1.0 - beta1)
    res = (upd - m) ** 2 + eps1
    if factored:
        res_row = deq(rq[1], ra[1], False, P).view(row_shape)
        res_col = deq(cq[1], ca[1], False, P).view(col_shape)
        res_row.mul_(beta3).add_(res.mean(dim=-1), alpha=1.0 - beta3)
        res_col.mul_(beta3).add_(res.mean(dim=-2), alpha=1.0 - beta3)
        step_dir = _approx_sq_grad(res_row, res_col)
        if capture is not None:
            capture["res_factor"] = step_dir.clone()
        step_dir.mul_(m)
    else:
        step_dir = m.clone()

    if weight_decay != 0.0:
        p.add_(p, alpha=-weight_decay * lr)
    p.add_(step_dir, alpha=-lr)

    if capture is not None:
        capture["clip"] = clipv.clone()
        capture["exp_avg"] = m.clone()
        if factored:
            capture.update(sq_row=sq_row.clone(), sq_col=sq_col.clone(), res_row=res_row.clone(),
                           res_col=res_col.clone())
        else:
            capture["sq"] = sq.clone()
    q, a = quant(m, True, P)
    st["exp_avg_q"].copy_(q)
    st["exp_avg_absmax"].copy_(a.view_as(st["exp_avg_absmax"]))
    if factored:
        for k, (row, col) in enumerate(((sq_row, sq_col), (res_row, res_col))):
            q, a = quant(row, False, P)
            rq[k].copy_(q.reshape(-1))
            ra[k].copy_(a.reshape(-1))
            q, a = quant(col, False, P)
            cq[k].copy_(q.reshape(-1))
            ca[k].copy_(a.reshape(-1))
    else:
        q, a = quantize_blockwise(sq, signed=False, block_size=bs)
        st["exp_avg_sq_q"].copy_(q)
        st["exp_avg_sq_absmax"].copy_(a)


# --------------------------------------------------------------------------
# fp32-state step (reference CAMECUDA._step_param_generic)
# --------------------------------------------------------------------------
def init_fp32_state(shape) -> Dict[str, object]:
    """Reference CAMECUDA.py:83-103 (state keys of the fp32-state mode)."""
    shape = tuple(int(s) for s in shape)
    st: Dict[str, object] = {"step": 0, "_mode": "cudafp", "factored": len(shape) >= 2}
    st["exp_avg"] = torch.zeros(shape, dtype=torch.float32)
    if st["factored"]:
        st["exp_avg_sq_row"] = torch.zeros(shape[:-1], dtype=torch.float32)
        st["exp_avg_sq_col"] = torch.zeros(shape[:-2] + shape[-1:], dtype=torch.float32)
        st["exp_avg_res_row"] = torch.zeros(shape[:-1], dtype=torch.float32)
        st["exp_avg_res_col"] = torch.zeros(shape[:-2] + shape[-1:], dtype=torch.float32)
    else:
        st["exp_avg_sq"] = torch.zeros(shape, dtype=torch.float32)
    st["_cuda_fp_factored_fastpath"] = False  # CAMECUDA.py:117-118, False on CPU
    st["_cuda_fp_nonfactored_fastpath"] = False
    return st


@torch.no_grad()
def fp32_state_step(p: torch.Tensor, grad: torch.Tensor, st: Dict[str, object], *, beta1: float, beta2: float,
                    beta3: float, eps0: float, eps1: float, lr: float, clip_threshold: float,
                    weight_decay: float, capture: Dict[str, torch.Tensor] | None = None) -> None:
    """Reference CAMECUDA.py:275-326 (generic fp32-state step), same op order.  ``capture``, if a
    dict, receives the clip divisor under "clip"."""
    st["step"] += 1
    if grad.dtype in (torch.float16, torch.bfloat16):
        grad = grad.float()
    m = st["exp_avg"]
    upd = (grad ** 2) + eps0
    if st["factored"]:
        row, col = st["exp_avg_sq_row"], st["exp_avg_sq_col"]
        row.mul_(beta2).add_(upd.mean(dim=-1), alpha=1.0 - beta2)
        col.mul_(beta2).add_(upd.mean(dim=-2), alpha=1.0 - beta2)
        upd = _approx_sq_grad(row, col)
        upd.mul_(grad)
    else:
        sq = st["exp_avg_sq"]
        sq.mul_(beta2).add_(upd, alpha=1.0 - beta2)
        upd = sq.clamp_min_(1e-30).rsqrt().mul_(grad)
    clipv = (_rms(upd) / clip_threshold).clamp_(min=1.0)
    if capture is not None:
        capture["clip"] = clipv.clone()
    upd.div_(clipv)
    m.mul_(beta1).add_(upd, alpha=1.0 - beta1)
    if st["factored"]:
        rrow, rcol = st["exp_avg_res_row"], st["exp_avg_res_col"]
        res = (upd - m) ** 2 + eps1
        rrow.mul_(beta3).add_(res.mean(dim=-1), alpha=1.0 - beta3)
        rcol.mul_(beta3).add_(res.mean(dim=-2), alpha=1.0 - beta3)
        step_dir = _approx_sq_grad(rrow, rcol).mul_(m)
    else:
        step_dir = m
    if weight_decay != 0.0:
        p.add_(p, alpha=-weight_decay * lr)
    p.add_(step_dir, alpha=-lr)


# --------------------------------------------------------------------------
# 8bit2d step (reference CAME8bit2D / the CUDA 2-D path of CAME8bit)
# --------------------------------------------------------------------------
# The reference's 8bit2d step exists only as CUDA kernels (came_cuda/csrc/came_kernels.cu:
# kUpdateSqRowQuantized :60-96, kUpdateSqColQuantizedFinalize :198-243, kFinalizeQuantizedRFactor
# :298-333, kSumUpdateSq :595-619, kUpdateExpAvgQuantAndResSumsTiled :2584-2684,
# kUpdateResRowQuantized :2685-2707, kReduceRow/ColTilePartials :2708-2741,
# kUpdateResColQuantizedFinalize :2742-2780, kParamUpdateTiled :3333-3367; launch order
# :3598-4040).  This is a CPU restatement written from that source, with its float32 operation
# order; PARITY UNPINNED against the reference itself (it cannot run here): its reductions are
# CUB block sums and float atomics of unfixed order, its rsqrtf is not correctly rounded and its
# compiler may contract multiply-adds.  Here: sums in a fixed order (sequential where the kernel is
# sequential), correctly rounded 1/sqrt, no contraction except the final parameter write (a fused
# multiply-add, as torch's add_(alpha=) and the GPU both do), and the update-RMS sum in fp64.
TILE_2D = 16


def init_8bit2d_state(shape, block_size: int = 256) -> Dict[str, object]:
    """Reference came8bit2d_state.py:33-75, persistent part (the scratch tensors it also allocates are
    listed in SCRATCH_8BIT2D_KEYS)."""
    rows, cols = (int(s) for s in shape)
    tr, tc = math.ceil(rows / TILE_2D), math.ceil(cols / TILE_2D)
    st: Dict[str, object] = {"_mode": "8bit2d"}
    st["exp_avg_q"] = torch.zeros((rows, cols), dtype=torch.int8)
    st["exp_avg_absmax"] = torch.zeros(tr * tc, dtype=torch.float32)  # 0: "no momentum yet"
    for k, n in (("exp_avg_sq_row", rows), ("exp_avg_sq_col", cols), ("exp_avg_res_row", rows),
                 ("exp_avg_res_col", cols)):
        st[k + "_q"] = torch.zeros(n, dtype=torch.uint8)
        st[k + "_absmax"] = torch.ones(num_blocks(n, block_size), dtype=torch.float32)
    st.update(rows=rows, cols=cols, tile_rows=tr, tile_cols=tc, num_tiles=tr * tc)
    return st


SCRATCH_8BIT2D_KEYS = ("r_factor", "c_factor", "r_res_factor", "c_res_factor", "res_row_sum", "res_col_sum",
                       "res_row_partial", "res_col_partial", "sum_sq_row", "sum_update", "sum_update_partial",
                       "sum_res_row")


def _f32(x) -> np.float32:
    return np.float32(x)


def _quant_inv(x: torch.Tensor, absmax: torch.Tensor, signed: bool) -> torch.Tensor:
    """came_kernels.cu:833-847: rint((x * (1 / absmax)) * Q), clamped; each product rounded."""
    inv = (torch.ones_like(absmax) / absmax)
    qmax = SIGNED_QMAX if signed else UNSIGNED_QMAX
    q = torch.round((x * inv) * qmax).clamp(-qmax if signed else 0.0, qmax)
    return q.to(torch.int8 if signed else torch.uint8)


def _block_fix(v: torch.Tensor, block_size: int) -> torch.Tensor:
    """Per flat block of ``v`` (>= 0 values): max over the block, 0 -> 1; one value per element."""
    n = v.numel()
    nb = num_blocks(n, block_size)
    buf = torch.zeros(nb * block_size, dtype=torch.float32)
    buf[:n] = v
    a = buf.view(nb, block_size).amax(dim=1)
    a = torch.where(a > 0, a, torch.ones_like(a))
    return a


def _ema_f32(old: torch.Tensor, mean: torch.Tensor, beta: float) -> torch.Tensor:
    """(old * beta) + ((1.0f - beta) * mean) in float32, unfused (came_kernels.cu:91, 229, 2701, 2764)."""
    b = _f32(beta)
    a = _f32(1.0) - b
    return (old * float(b)) + (mean * float(a))


def _rsqrt(x: torch.Tensor) -> torch.Tensor:
    return torch.ones_like(x) / torch.sqrt(x)


@torch.no_grad()
def came8bit2d_step(p: torch.Tensor, grad: torch.Tensor, st: Dict[str, object], *, beta1: float, beta2: float,
                    beta3: float, eps0: float, eps1: float, lr: float, clip_threshold: float, weight_decay: float,
                    block_size: int = 256, capture: Dict[str, torch.Tensor] | None = None) -> None:
    """One 8bit2d step on a 2-D parameter ``p`` (in place) and state ``st`` (in place)."""
    rows, cols = p.shape
    bs = block_size
    g = grad.float()
    U = (g * g) + float(_f32(eps0))
    # row second moment (kUpdateSqRowQuantized)
    old_r = dequantize_blockwise(st["exp_avg_sq_row_q"], st["exp_avg_sq_row_absmax"], signed=False, block_size=bs)
    row_mean = U.sum(dim=1) / float(cols)
    upd_r = _ema_f32(old_r, row_mean, beta2)
    sum_sq_row = upd_r.sum()
    # column second moment, summed row after row (kUpdateSqColQuantizedFinalize)
    col_acc = torch.zeros(cols, dtype=torch.float32)
    for i in range(rows):
        col_acc = col_acc + U[i]
    old_c = dequantize_blockwise(st["exp_avg_sq_col_q"], st["exp_avg_sq_col_absmax"], signed=False, block_size=bs)
    upd_c = _ema_f32(old_c, col_acc / float(rows), beta2)
    ca = _block_fix(upd_c, bs)
    st["exp_avg_sq_col_absmax"].copy_(ca)
    st["exp_avg_sq_col_q"].copy_(_quant_inv(upd_c, ca.repeat_interleave(bs)[:cols], signed=False))
    c = _rsqrt(upd_c)
    # row factors (kFinalizeQuantizedRFactor)
    ra = _block_fix(upd_r, bs)
    st["exp_avg_sq_row_absmax"].copy_(ra)
    st["exp_avg_sq_row_q"].copy_(_quant_inv(upd_r, ra.repeat_interleave(bs)[:rows], signed=False))
    mean = sum_sq_row / float(rows)
    mean = mean if float(mean) > 0 else torch.tensor(1.0)
    r = _rsqrt(upd_r / mean)
    # update RMS (kSumUpdateSq; the sum in fp64 here) and clip
    u0 = (g * r[:, None]) * c[None, :]
    sum_update = _f32(float((u0.double() ** 2).sum()))
    rms = np.sqrt(_f32(sum_update / _f32(rows * cols)), dtype=np.float32)
    clip = max(_f32(1.0), _f32(rms / _f32(clip_threshold)))
    upd = u0 / float(clip)
    # momentum in 16x16 tiles (kUpdateExpAvgQuantAndResSumsTiled)
    tr, tc = st["tile_rows"], st["tile_cols"]
    tile = (torch.arange(rows)[:, None] // TILE_2D) * tc + (torch.arange(cols)[None, :] // TILE_2D)
    old_am = st["exp_avg_absmax"][tile]
    m_old = torch.where(old_am > 0, st["exp_avg_q"].float() * (old_am / SIGNED_QMAX), torch.zeros(()))
    b1 = _f32(beta1)
    m_new = (m_old * float(b1)) + (upd * float(_f32(1.0) - b1))
    diff = upd - m_new
    res = (diff * diff) + float(_f32(eps1))
    am = torch.zeros(tr * tc, dtype=torch.float32).scatter_reduce(0, tile.reshape(-1), m_new.abs().reshape(-1),
                                                                   reduce="amax", include_self=True)
    am = torch.where(am > 0, am, torch.ones_like(am))
    st["exp_avg_absmax"].copy_(am)
    q_new = _quant_inv(m_new, am[tile], signed=True)
    st["exp_avg_q"].copy_(q_new)
    # residual sums: 16 elements of a tile in order, then tiles in order (kReduceRow/ColTilePartials)
    pad_r, pad_c = tr * TILE_2D, tc * TILE_2D
    rp = torch.zeros(pad_r, pad_c)
    rp[:rows, :cols] = res
    row_part = torch.zeros(pad_r, tc)
    col_part = torch.zeros(tr, pad_c)
    for j in range(TILE_2D):
        row_part = row_part + rp.view(pad_r, tc, TILE_2D)[:, :, j]
        col_part = col_part + rp.view(tr, TILE_2D, pad_c)[:, j, :]
    res_row_sum = torch.zeros(pad_r)
    for tx in range(tc):
        res_row_sum = res_row_sum + row_part[:, tx]
    res_col_sum = torch.zeros(pad_c)
    for ty in range(tr):
        res_col_sum = res_col_sum + col_part[ty]
    res_row_sum, res_col_sum = res_row_sum[:rows], res_col_sum[:cols]
    # multiplicative weight decay, rounded to the parameter type
    if weight_decay != 0.0:
        fac = _f32(1.0) - _f32(lr) * _f32(weight_decay)
        p.copy_((p.float() * float(fac)).to(p.dtype))
    # residual factors (kUpdateResRowQuantized, kUpdateResColQuantizedFinalize, kFinalizeQuantizedRFactor)
    old_rr = dequantize_blockwise(st["exp_avg_res_row_q"], st["exp_avg_res_row_absmax"], signed=False, block_size=bs)
    upd_rr = _ema_f32(old_rr, res_row_sum / float(cols), beta3)
    sum_res_row = upd_rr.sum()
    old_rc = dequantize_blockwise(st["exp_avg_res_col_q"], st["exp_avg_res_col_absmax"], signed=False, block_size=bs)
    upd_rc = _ema_f32(old_rc, res_col_sum / float(rows), beta3)
    cra = _block_fix(upd_rc, bs)
    st["exp_avg_res_col_absmax"].copy_(cra)
    st["exp_avg_res_col_q"].copy_(_quant_inv(upd_rc, cra.repeat_interleave(bs)[:cols], signed=False))
    cr = _rsqrt(upd_rc)
    rra = _block_fix(upd_rr, bs)
    st["exp_avg_res_row_absmax"].copy_(rra)
    st["exp_avg_res_row_q"].copy_(_quant_inv(upd_rr, rra.repeat_interleave(bs)[:rows], signed=False))
    rmean = sum_res_row / float(rows)
    rmean = rmean if float(rmean) > 0 else torch.tensor(1.0)
    rr = _rsqrt(upd_rr / rmean)
    # parameter write from the requantised momentum (kParamUpdateTiled): p - lr * ((m * rr) * cr), fused
    m_q = q_new.float() * (am[tile] / SIGNED_QMAX)
    update2 = (m_q * rr[:, None]) * cr[None, :]
    pf = p.float()
    pf.add_(update2, alpha=-lr)
    p.copy_(pf.to(p.dtype))
    if capture is not None:
        capture.update(clip=torch.tensor(float(clip)), exp_avg=m_new.clone(), sq_row=upd_r.clone(),
                       sq_col=upd_c.clone(), res_row=upd_rr.clone(), res_col=upd_rc.clone(), update=upd.clone(),
                       res_factor=rr[:, None] * cr[None, :])
