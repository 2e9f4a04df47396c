"""Layout conversions of optimizer state (came_amd.state_layout), on the CPU.

The fixtures are built with the oracle's blockwise quantiser (pinned to the reference's golden
vectors) and brute-force tile loops, so a wrong block origin, a transposed tile index or a
swapped row/column state fails here."""
import math

import numpy as np
import pytest
import torch

from came_amd import state_layout as SL
from oracle import came8_oracle as orc


def _rand(shape, seed, scale=1.0):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)) * scale


def _nd_batched_state(shape, B, seed):
    """A full8bit state in the reference CUDA N-D layout (CAME8bitFull.py:790-829): every matrix of
    the prefix blocked from its own start, row/column states as (2*prefix, n) batches."""
    P, R, C = math.prod(shape[:-2]), shape[-2], shape[-1]
    m = _rand(shape, seed, 1e-3)
    rows = _rand((2, P, R), seed + 1).abs()
    cols = _rand((2, P, C), seed + 2).abs()
    qs, am = zip(*(orc.quantize_blockwise(m.reshape(P, R * C)[i], signed=True, block_size=B) for i in range(P)))
    rq, ra = zip(*(orc.quantize_blockwise(rows.reshape(2 * P, R)[i], signed=False, block_size=B) for i in range(2 * P)))
    cq, ca = zip(*(orc.quantize_blockwise(cols.reshape(2 * P, C)[i], signed=False, block_size=B) for i in range(2 * P)))
    st = {"step": 4, "_mode": "full8bit", "factored": True, "_cuda_factored_nd_ext_path": True,
          "prefix_batch": P, "matrix_rows": R, "matrix_cols": C,
          "exp_avg_q": torch.stack(qs).reshape(shape), "exp_avg_absmax": torch.stack(am),
          "factored_row_q": torch.stack(rq), "factored_row_absmax": torch.stack(ra),
          "factored_col_q": torch.stack(cq), "factored_col_absmax": torch.stack(ca)}
    expect = {
        "exp_avg": torch.stack([orc.dequantize_blockwise(q, a, signed=True, block_size=B)
                                for q, a in zip(qs, am)]).reshape(shape),
        "rows": torch.stack([orc.dequantize_blockwise(q, a, signed=False, block_size=B)
                             for q, a in zip(rq, ra)]).reshape(2, P, R),
        "cols": torch.stack([orc.dequantize_blockwise(q, a, signed=False, block_size=B)
                             for q, a in zip(cq, ca)]).reshape(2, P, C),
    }
    return st, expect


@pytest.mark.parametrize("shape,B", [((3, 5, 7), 16), ((2, 3, 40, 9), 64), ((4, 33, 8), 256)])
def test_nd_batched_values_match_per_matrix_dequantisation(shape, B):
    st, ex = _nd_batched_state(shape, B, seed=1)
    assert SL.layout_of(st) == "full8bit-nd"
    v = SL.state_values(st, shape, B)
    P = math.prod(shape[:-2])
    assert torch.equal(v["exp_avg"], ex["exp_avg"])
    assert torch.equal(v["sq_row"], ex["rows"][0].reshape(shape[:-1]))
    assert torch.equal(v["res_row"], ex["rows"][1].reshape(shape[:-1]))
    assert torch.equal(v["sq_col"], ex["cols"][0].reshape(shape[:-2] + shape[-1:]))
    assert torch.equal(v["res_col"], ex["cols"][1].reshape(shape[:-2] + shape[-1:]))
    assert v["step"] == 4 and P > 1


@pytest.mark.parametrize("shape,B", [((3, 5, 7), 16), ((2, 3, 40, 9), 64)])
def test_nd_batched_to_flat_blocks_requantises_with_the_reference_formula(shape, B):
    st, ex = _nd_batched_state(shape, B, seed=2)
    out = SL.convert_state(st, shape, "full8bit", B)
    assert out["_mode"] == "full8bit" and out["step"] == 4 and out["factored"]
    # flat blocks over the whole tensor, quantised as the reference quantises
    q, a = orc.quantize_blockwise(ex["exp_avg"], signed=True, block_size=B)
    assert torch.equal(out["exp_avg_q"], q.reshape(shape)) and torch.equal(out["exp_avg_absmax"], a)
    for name, key in (("rows", "factored_row"), ("cols", "factored_col")):
        for i in range(2):
            q, a = orc.quantize_blockwise(ex[name][i].reshape(-1), signed=False, block_size=B)
            assert torch.equal(out[f"{key}_q"][i].reshape(-1), q) and torch.equal(out[f"{key}_absmax"][i], a)
    # the layout the optimizer allocates
    ref = orc.init_full8bit_state(shape, B)
    for k in ("exp_avg_q", "exp_avg_absmax", "factored_row_q", "factored_row_absmax", "factored_col_q",
              "factored_col_absmax"):
        assert out[k].shape == ref[k].shape and out[k].dtype == ref[k].dtype, k


def _tile_state(rows, cols, seed, zero_tile=None):
    """An 8bit2d momentum built by brute force: absmax per 16x16 tile, codes rint((x * (1/a)) * 127)."""
    x = _rand((rows, cols), seed, 1e-2)
    tr, tc = math.ceil(rows / 16), math.ceil(cols / 16)
    if zero_tile is not None:
        ty, tx = zero_tile
        x[ty * 16:(ty + 1) * 16, tx * 16:(tx + 1) * 16] = 0.0
    q = np.zeros((rows, cols), np.int8)
    am = np.zeros(tr * tc, np.float32)
    xn = x.numpy()
    for ty in range(tr):
        for tx in range(tc):
            blk = xn[ty * 16:(ty + 1) * 16, tx * 16:(tx + 1) * 16]
            a = np.float32(np.abs(blk).max())
            am[ty * tc + tx] = a
            if a > 0:
                inv = np.float32(1.0) / a
                q[ty * 16:(ty + 1) * 16, tx * 16:(tx + 1) * 16] = np.clip(
                    np.rint((blk * inv).astype(np.float32) * np.float32(127)), -127, 127)
    return x, torch.from_numpy(q), torch.from_numpy(am)


def _state_2d(rows, cols, seed, zero_tile=None):
    x, q, am = _tile_state(rows, cols, seed, zero_tile)
    st = {"_mode": "8bit2d", "exp_avg_q": q, "exp_avg_absmax": am}
    for i, (k, n) in enumerate((("sq_row", rows), ("sq_col", cols), ("res_row", rows), ("res_col", cols))):
        st[f"exp_avg_{k}_q"], st[f"exp_avg_{k}_absmax"] = orc.quantize_blockwise(
            _rand((n,), seed + 10 + i).abs(), signed=False, block_size=256)
    return x, st


def test_8bit2d_values_are_tile_dequantisation():
    rows, cols = 37, 50  # ragged tiles on both edges
    x, st = _state_2d(rows, cols, seed=3, zero_tile=(1, 2))
    v = SL.state_values(st, (rows, cols))
    tc = math.ceil(cols / 16)
    q, am = st["exp_avg_q"].numpy(), st["exp_avg_absmax"].numpy()
    for i in (0, 15, 16, 36):
        for j in (0, 17, 33, 49):
            scale = np.float32(am[(i // 16) * tc + j // 16]) / np.float32(127)
            assert v["exp_avg"][i, j].item() == np.float32(np.float32(q[i, j]) * scale)
    assert float(v["exp_avg"][16:32, 32:48].abs().sum()) == 0.0  # the zero tile
    assert (v["exp_avg"] - x).abs().max().item() <= st["exp_avg_absmax"].max().item() / 127 / 2 * 1.001
    sq_row = orc.dequantize_blockwise(st["exp_avg_sq_row_q"], st["exp_avg_sq_row_absmax"], signed=False,
                                      block_size=256)
    assert torch.equal(v["sq_row"], sq_row)


def test_8bit2d_to_full8bit_and_back():
    rows, cols = 40, 300
    x, st = _state_2d(rows, cols, seed=4, zero_tile=(0, 0))
    full = SL.convert_state(st, (rows, cols), "full8bit", 256)
    # row / column states move code for code (same flat blocks in both layouts)
    assert torch.equal(full["factored_row_q"][0], st["exp_avg_sq_row_q"])
    assert torch.equal(full["factored_row_q"][1], st["exp_avg_res_row_q"])
    assert torch.equal(full["factored_col_absmax"][1], st["exp_avg_res_col_absmax"])
    # the momentum takes one requantisation into flat 256-blocks: within half a step of those blocks
    m2d = SL.state_values(st, (rows, cols))["exp_avg"]
    mf = orc.dequantize_blockwise(full["exp_avg_q"], full["exp_avg_absmax"], signed=True, block_size=256)
    step = full["exp_avg_absmax"].repeat_interleave(256)[: rows * cols].reshape(rows, cols) / 127
    assert ((mf - m2d).abs() <= step / 2 * 1.0001).all()
    assert full["step"] == 0 and full["RMS"] == 0
    back = SL.convert_state(full, (rows, cols), "8bit2d", 256)
    assert torch.equal(back["exp_avg_sq_col_q"], st["exp_avg_sq_col_q"])
    mb = SL.state_values(back, (rows, cols))["exp_avg"]
    assert ((mb - mf).abs() <= back["exp_avg_absmax"].max() / 127 / 2 * 1.0001).all()
    assert back["exp_avg_absmax"][0].item() == 0.0  # the zero tile stays a tile without momentum


def test_fp32_states_round_trip_within_half_a_quantisation_step():
    shape = (6, 70)
    vals = {"step": 7, "exp_avg": _rand(shape, 5, 1e-3), "sq_row": _rand((6,), 6).abs(),
            "res_row": _rand((6,), 7).abs(), "sq_col": _rand((70,), 8).abs(), "res_col": _rand((70,), 9).abs()}
    fp = SL.cudafp_state(vals, shape)
    assert SL.layout_of(fp) == "cudafp"
    q8 = SL.convert_state(fp, shape, "full8bit", 64)
    back = SL.state_values(q8, shape, 64)
    assert back["step"] == 7
    for k in ("exp_avg", "sq_row", "res_row", "sq_col", "res_col"):
        a = vals[k].reshape(-1)
        blocks = math.ceil(a.numel() / 64)
        amax = torch.zeros(blocks * 64)
        amax[: a.numel()] = a.abs()
        half = amax.view(blocks, 64).amax(1).repeat_interleave(64)[: a.numel()] / (127 if k == "exp_avg" else 255) / 2
        assert ((back[k].reshape(-1) - a).abs() <= half * 1.0001 + 1e-12).all(), k
    fp2 = SL.convert_state(q8, shape, "cudafp", 64)
    assert torch.equal(fp2["exp_avg"], back["exp_avg"]) and fp2["step"] == 7
    with pytest.raises(ValueError, match="block size"):  # read with the wrong block size
        SL.convert_state(q8, shape, "cudafp", 256)


def test_one_dimensional_states():
    st = orc.init_full8bit_state((300,), 64)
    st["exp_avg_q"], st["exp_avg_absmax"] = orc.quantize_blockwise(_rand((300,), 11), signed=True, block_size=64)
    st["exp_avg_sq_q"], st["exp_avg_sq_absmax"] = orc.quantize_blockwise(_rand((300,), 12).abs(), signed=False,
                                                                          block_size=64)
    fp = SL.convert_state(st, (300,), "cudafp", 64)
    assert not fp["factored"] and fp["exp_avg_sq"].shape == (300,)
    back = SL.convert_state(fp, (300,), "full8bit", 64)
    assert torch.equal(back["exp_avg_q"], st["exp_avg_q"])
    assert torch.equal(back["exp_avg_sq_q"], st["exp_avg_sq_q"])
    with pytest.raises(ValueError):
        SL.convert_state(st, (300,), "8bit2d", 64)
    with pytest.raises(ValueError):
        SL.convert_state(st, (300,), "nonsense", 64)
