"""Conversions between the optimizer-state layouts of the reference's CAME optimizers.

The reference keeps the state of one parameter in one of these layouts, named by ``state["_mode"]``:

  ``full8bit``  int8 momentum and uint8 row/column states in flat row-major blocks
                (came_pytorch/CAME8bitFull.py:748-788, CPU branch; CAME8bitMemory.py:390-447).
                On its CUDA path an N-D tensor (N >= 3) may instead be blocked per matrix: every one of
                the prod(shape[:-2]) matrices has blocks of its own, and the row/column states are
                (2*prefix, n) batches (CAME8bitFull.py:790-829, views :188-229; flagged by
                ``_cuda_factored_nd_ext_path`` / ``_cuda_factored_nd_chunked_ext_path``).
  ``8bit2d``    int8 momentum quantised per 16x16 tile, uint8 row/column states in flat blocks
                (came_pytorch/came8bit2d_state.py:33-75).
  ``cudafp``    fp32 states (came_pytorch/CAMECUDA.py:83-104).

The reference re-initialises a state whose ``_mode`` is not its optimizer's own
(CAME8bit.py:757-759), so a checkpoint written by its CUDA path (8bit2d states for 2-D
parameters, per-matrix blocks for N-D ones) loses its momentum, or fails a block count check,
in an optimizer that keeps flat blocks.  ``convert_state`` carries a state across instead: it
dequantises every stored quantity to fp32 and requantises it in the target layout, with the
target layout's own formulas.  Row and column states whose blocks coincide in both layouts are
copied code for code; everything else takes one quantisation step, like any optimizer step.

These are one-off tensor operations at checkpoint load, on whatever device the state lives.
"""
from __future__ import annotations

import math

import torch

from .blockwise_quantization import num_blocks

MODES = ("full8bit", "8bit2d", "cudafp")
_TILE = 16
_QS, _QU = 127.0, 255.0


# ------------------------------------------------------------------------------- block arithmetic
def _deq_blocks(q: torch.Tensor, absmax: torch.Tensor, *, signed: bool, block_size: int, items: int = 1):
    """Blockwise dequantisation of `items` equal runs of codes, each blocked from its own start:
    ``code * (absmax / Q)``, the scale rounded first (blockwise_quantization.py:112-124).  The number
    of scales must be the block count of that block size (a state read with another block size
    would come out scaled wrongly)."""
    qmax = _QS if signed else _QU
    n = q.numel() // max(items, 1)
    nb = num_blocks(n, block_size)
    if absmax.numel() != items * nb:
        raise ValueError(f"{absmax.numel()} block scales for {items} x {n} codes: not the layout of block size "
                         f"{block_size} ({items * nb} scales)")
    codes = q.reshape(items, n).to(torch.float32)
    scale = (absmax.reshape(items, -1)[:, :nb].to(torch.float32) / qmax)
    scale = scale.repeat_interleave(block_size, dim=1)[:, :n]
    return (codes * scale).reshape(q.shape)


def _quant_blocks(x: torch.Tensor, *, signed: bool, block_size: int, items: int = 1):
    """Blockwise quantisation of `items` equal runs (blockwise_quantization.py:66-82): flat blocks,
    zero-padded tail, absmax (signed: of |x|; unsigned: of x) with 0 -> 1,
    ``clamp(round_half_even((x / absmax) * Q))``.  Returns (codes shaped like x, absmax [items, nb])."""
    qmax = _QS if signed else _QU
    n = x.numel() // max(items, 1)
    nb = num_blocks(n, block_size)
    flat = torch.zeros((items, nb * block_size), dtype=torch.float32, device=x.device)
    flat[:, :n] = x.reshape(items, n).to(torch.float32)
    blocks = flat.view(items, nb, block_size)
    absmax = (blocks.abs() if signed else blocks).amax(dim=2)
    absmax = torch.where(absmax == 0, torch.ones_like(absmax), absmax)
    codes = torch.round((blocks / absmax.unsqueeze(2)) * qmax)
    codes = codes.clamp(-qmax, qmax) if signed else codes.clamp(0.0, qmax)
    codes = codes.reshape(items, nb * block_size)[:, :n].to(torch.int8 if signed else torch.uint8)
    return codes.reshape(x.shape), absmax


def _tiles(rows: int, cols: int):
    return math.ceil(rows / _TILE), math.ceil(cols / _TILE)


def _deq_tiles(q: torch.Tensor, absmax: torch.Tensor) -> torch.Tensor:
    """8bit2d momentum: ``code * (absmax_tile / 127)`` (came_kernels.cu:829-831), tile (ty, tx) at
    ty * tile_cols + tx; a tile whose absmax is 0 holds no momentum yet."""
    rows, cols = q.shape
    tr, tc = _tiles(rows, cols)
    scale = (absmax.reshape(tr, tc).to(torch.float32) / _QS)
    scale = scale.repeat_interleave(_TILE, 0).repeat_interleave(_TILE, 1)[:rows, :cols]
    return q.to(torch.float32) * scale


def _quant_tiles(x: torch.Tensor):
    """8bit2d momentum quantisation (came_kernels.cu:833-837): per 16x16 tile absmax = max |x|, codes
    ``clamp(rint((x * (1/absmax)) * 127))``; an all-zero tile keeps absmax 0 and zero codes."""
    rows, cols = x.shape
    tr, tc = _tiles(rows, cols)
    pad = torch.zeros((tr * _TILE, tc * _TILE), dtype=torch.float32, device=x.device)
    pad[:rows, :cols] = x.to(torch.float32)
    t = pad.view(tr, _TILE, tc, _TILE)
    absmax = t.abs().amax(dim=(1, 3))
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    inv = inv.repeat_interleave(_TILE, 0).repeat_interleave(_TILE, 1)
    codes = torch.round((pad * inv) * _QS).clamp(-_QS, _QS)
    return codes[:rows, :cols].to(torch.int8).contiguous(), absmax.reshape(-1).contiguous()


# ------------------------------------------------------------------------------------ layouts
def _is_nd_batched(state: dict) -> bool:
    return bool(state.get("_cuda_factored_nd_ext_path", False) or state.get("_cuda_factored_nd_chunked_ext_path", False))


def layout_of(state: dict) -> str:
    """``_mode`` of a state, with ``"full8bit-nd"`` for the reference CUDA path's per-matrix blocks;
    ``""`` for an empty state."""
    mode = state.get("_mode", "")
    if mode == "full8bit" and _is_nd_batched(state):
        return "full8bit-nd"
    return mode


def _shapes(shape):
    shape = tuple(int(s) for s in shape)
    return shape[:-1], shape[:-2] + shape[-1:]


def state_values(state: dict, shape, block_size: int = 256) -> dict:
    """The fp32 values a state holds: ``exp_avg`` [shape] and either the factored row/column states
    ``sq_row``, ``res_row`` [shape[:-1]], ``sq_col``, ``res_col`` [shape[:-2] + shape[-1:]] or, for
    1-D tensors, ``sq`` [shape]; plus ``step`` (0 where the layout keeps none)."""
    shape = tuple(int(s) for s in shape)
    mode = layout_of(state)
    out = {"step": int(state.get("step", 0) or 0)}
    factored = len(shape) >= 2
    row_shape, col_shape = _shapes(shape) if factored else ((), ())
    if mode == "cudafp":
        out["exp_avg"] = state["exp_avg"].to(torch.float32).reshape(shape)
        if factored:
            for k in ("sq_row", "res_row", "sq_col", "res_col"):
                out[k] = state[f"exp_avg_{k}"].to(torch.float32).reshape(row_shape if "row" in k else col_shape)
        else:
            out["sq"] = state["exp_avg_sq"].to(torch.float32).reshape(shape)
        return out
    if mode == "8bit2d":
        if len(shape) != 2:
            raise ValueError(f"an 8bit2d state belongs to a 2-D parameter, got shape {shape}")
        out["exp_avg"] = _deq_tiles(state["exp_avg_q"].reshape(shape), state["exp_avg_absmax"])
        for k in ("sq_row", "res_row", "sq_col", "res_col"):
            out[k] = _deq_blocks(state[f"exp_avg_{k}_q"], state[f"exp_avg_{k}_absmax"], signed=False,
                                 block_size=256)
        return out
    if mode in ("full8bit", "full8bit-nd", "8bit1d"):  # 8bit1d: CAME8bit's 1-D states, full8bit's keys
        nd = mode == "full8bit-nd"
        prefix = math.prod(shape[:-2]) if factored else 1
        items = prefix if nd else 1
        out["exp_avg"] = _deq_blocks(state["exp_avg_q"].reshape(shape), state["exp_avg_absmax"], signed=True,
                                     block_size=block_size, items=items)
        if factored:
            rq, ra = state["factored_row_q"], state["factored_row_absmax"]
            cq, ca = state["factored_col_q"], state["factored_col_absmax"]
            rows = _deq_blocks(rq, ra, signed=False, block_size=block_size, items=2 * items).reshape(2, -1)
            cols = _deq_blocks(cq, ca, signed=False, block_size=block_size, items=2 * items).reshape(2, -1)
            out["sq_row"], out["res_row"] = rows[0].reshape(row_shape), rows[1].reshape(row_shape)
            out["sq_col"], out["res_col"] = cols[0].reshape(col_shape), cols[1].reshape(col_shape)
        else:
            out["sq"] = _deq_blocks(state["exp_avg_sq_q"].reshape(shape), state["exp_avg_sq_absmax"], signed=False,
                                    block_size=block_size)
        return out
    raise ValueError(f"unknown optimizer state layout {mode!r}")


def full8bit_state(values: dict, shape, block_size: int = 256) -> dict:
    """A full8bit state in flat blocks with the keys of CAME8bitFull's CPU branch
    (CAME8bitFull.py:748-788, 919-923), quantising `values` (see ``state_values``)."""
    shape = tuple(int(s) for s in shape)
    st = {"step": int(values.get("step", 0)), "_mode": "full8bit", "RMS": 0}
    st["exp_avg_q"], am = _quant_blocks(values["exp_avg"].reshape(shape), signed=True, block_size=block_size)
    st["exp_avg_absmax"] = am.reshape(-1)
    factored = len(shape) >= 2
    st["factored"] = factored
    if factored:
        row_shape, col_shape = _shapes(shape)
        for name, a, b, sh in (("row", "sq_row", "res_row", row_shape), ("col", "sq_col", "res_col", col_shape)):
            stacked = torch.stack([values[a].reshape(sh), values[b].reshape(sh)])
            st[f"factored_{name}_q"], st[f"factored_{name}_absmax"] = _quant_blocks(
                stacked, signed=False, block_size=block_size, items=2)
    else:
        st["exp_avg_sq_q"], am = _quant_blocks(values["sq"].reshape(shape), signed=False, block_size=block_size)
        st["exp_avg_sq_absmax"] = am.reshape(-1)
    return st


def cudafp_state(values: dict, shape) -> dict:
    """A CAMECUDA fp32 state (CAMECUDA.py:83-104) holding `values`."""
    shape = tuple(int(s) for s in shape)
    st = {"step": int(values.get("step", 0)), "_mode": "cudafp", "factored": len(shape) >= 2,
          "exp_avg": values["exp_avg"].reshape(shape).to(torch.float32).clone()}
    if st["factored"]:
        for k in ("sq_row", "res_row", "sq_col", "res_col"):
            st[f"exp_avg_{k}"] = values[k].to(torch.float32).clone()
    else:
        st["exp_avg_sq"] = values["sq"].reshape(shape).to(torch.float32).clone()
    return st


def state_8bit2d_tensors(values: dict, shape) -> dict:
    """The persistent tensors of an 8bit2d state (came8bit2d_state.py:40-56) holding `values`; the
    caller adds the layout's scratch tensors and shape keys."""
    shape = tuple(int(s) for s in shape)
    if len(shape) != 2:
        raise ValueError(f"the 8bit2d layout holds 2-D parameters only, got shape {shape}")
    st = {"_mode": "8bit2d"}
    st["exp_avg_q"], st["exp_avg_absmax"] = _quant_tiles(values["exp_avg"].reshape(shape))
    for k in ("sq_row", "res_row", "sq_col", "res_col"):
        q, am = _quant_blocks(values[k].reshape(-1), signed=False, block_size=256)
        st[f"exp_avg_{k}_q"], st[f"exp_avg_{k}_absmax"] = q, am.reshape(-1)
    return st


def _copy_flat_rowcol(src: dict, dst: dict, shape, block_size: int, to_2d: bool) -> None:
    """Row/column states of a 2-D parameter are flat uint8 blocks of the same size in the full8bit and
    8bit2d layouts (for block size 256): carry their codes and scales over unchanged."""
    if block_size != 256 or len(shape) != 2:
        return
    for i, (rk, ck) in enumerate((("sq_row", "sq_col"), ("res_row", "res_col"))):
        if to_2d:
            dst[f"exp_avg_{rk}_q"] = src["factored_row_q"][i].reshape(-1).clone()
            dst[f"exp_avg_{rk}_absmax"] = src["factored_row_absmax"][i].reshape(-1).clone()
            dst[f"exp_avg_{ck}_q"] = src["factored_col_q"][i].reshape(-1).clone()
            dst[f"exp_avg_{ck}_absmax"] = src["factored_col_absmax"][i].reshape(-1).clone()
        else:
            dst["factored_row_q"][i].copy_(src[f"exp_avg_{rk}_q"].reshape(-1))
            dst["factored_row_absmax"][i].copy_(src[f"exp_avg_{rk}_absmax"].reshape(-1))
            dst["factored_col_q"][i].copy_(src[f"exp_avg_{ck}_q"].reshape(-1))
            dst["factored_col_absmax"][i].copy_(src[f"exp_avg_{ck}_absmax"].reshape(-1))


def convert_state(state: dict, shape, to_mode: str, block_size: int = 256) -> dict:
    """A new state of layout `to_mode` ("full8bit" in flat blocks, "8bit2d" or "cudafp") holding what
    `state` holds.  For the 8bit2d target the result has the persistent tensors only."""
    if to_mode not in MODES:
        raise ValueError(f"to_mode must be one of {MODES}, got {to_mode!r}")
    src = layout_of(state)
    vals = state_values(state, shape, block_size)
    if to_mode == "cudafp":
        return cudafp_state(vals, shape)
    if to_mode == "full8bit":
        out = full8bit_state(vals, shape, block_size)
        if src == "8bit2d":
            _copy_flat_rowcol(state, out, tuple(shape), block_size, to_2d=False)
        return out
    out = state_8bit2d_tensors(vals, shape)
    if src == "full8bit":
        _copy_flat_rowcol(state, out, tuple(shape), block_size, to_2d=True)
    return out
