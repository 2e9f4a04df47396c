"""The oracle's per-matrix layout (the reference CUDA N-D path's blocks, CAME8bitFull.py:790-842), pinned
without the reference (its CUDA path cannot run here):

  * where the block size divides every period (R*C, R, C) the per-matrix blocks are the flat ones, so the
    step must equal the flat step bit for bit from the same (reshaped) state;
  * the requantised states against brute force: every block of every matrix, its scale the maximum over
    exactly that block's elements of the pre-quantisation values (oracle capture), its codes
    round_half_even(x / scale * Q);
  * with the clip inactive, a per-matrix step of a (P, R, C) tensor is P flat steps of (R, C) matrices
    (each matrix's blocks, states and row mean are its own in both), bit for bit.
"""
import math

import pytest
import torch

from oracle import came8_oracle as orc

HP = dict(beta1=0.9, beta2=0.999, beta3=0.9999, eps0=1e-30, eps1=1e-16, lr=1e-3, clip_threshold=1.0,
          weight_decay=1e-2)


def _run_steps(shape, B, per_matrix, steps=3, seed=0, st=None):
    gen = torch.Generator().manual_seed(seed)
    p = torch.randn(shape, generator=gen) * 0.02
    st = orc.init_full8bit_state(shape, B, per_matrix=per_matrix) if st is None else st
    caps = []
    for _ in range(steps):
        g = torch.randn(shape, generator=gen) * 1e-3
        cap = {}
        orc.full8bit_step(p, g, st, capture=cap, block_size=B, **HP)
        caps.append(cap)
    return p, st, caps


@pytest.mark.parametrize("shape,B", [((3, 64, 32), 32), ((2, 2, 256, 512), 256), ((4, 16, 16), 16)])
def test_per_matrix_equals_flat_where_blocks_coincide(shape, B):
    pa, sa, _ = _run_steps(shape, B, per_matrix=True)
    pb, sb, _ = _run_steps(shape, B, per_matrix=False)
    assert torch.equal(pa, pb)
    for k in ("exp_avg_q", "exp_avg_absmax", "factored_row_q", "factored_row_absmax", "factored_col_q",
              "factored_col_absmax"):
        assert torch.equal(sa[k].reshape(-1), sb[k].reshape(-1)), k


def _check_blocks(values, q, absmax, items, B, signed):
    """values [items * n] fp32 before quantisation; q codes; absmax [items][blocks]: brute force."""
    Q = 127 if signed else 255
    v = values.reshape(items, -1)
    qq = q.reshape(items, -1).to(torch.int32)
    a = absmax.reshape(items, -1)
    n = v.shape[1]
    for i in range(items):
        for b in range(math.ceil(n / B)):
            blk = v[i, b * B:(b + 1) * B]
            mx = blk.abs().max() if signed else torch.clamp(blk.max(), min=0.0)  # zero padding joins
            if len(blk) < B and not signed:
                mx = torch.clamp(mx, min=0.0)
            want = mx.item() if mx.item() > 0 else 1.0
            assert a[i, b].item() == want, (i, b)
            codes = torch.round((blk / a[i, b]) * Q).clamp(-Q if signed else 0, Q).to(torch.int32)
            assert torch.equal(qq[i, b * B:(b + 1) * B], codes), (i, b)


@pytest.mark.parametrize("shape,B", [((3, 40, 24), 64), ((2, 5, 33, 7), 16), ((4, 10, 10), 256), ((2, 3, 5), 4)])
def test_per_matrix_blocks_brute_force(shape, B):
    p, st, caps = _run_steps(shape, B, per_matrix=True, steps=2)
    cap = caps[-1]
    P = math.prod(shape[:-2])
    _check_blocks(cap["exp_avg"], st["exp_avg_q"], st["exp_avg_absmax"], P, B, True)
    rq, ra = st["factored_row_q"].view(2, -1), st["factored_row_absmax"].view(2, -1)
    cq, ca = st["factored_col_q"].view(2, -1), st["factored_col_absmax"].view(2, -1)
    for k, (row, col) in enumerate((("sq_row", "sq_col"), ("res_row", "res_col"))):
        _check_blocks(cap[row].reshape(-1), rq[k], ra[k], P, B, False)
        _check_blocks(cap[col].reshape(-1), cq[k], ca[k], P, B, False)
    # the layout is the reference's: per-matrix scale arrays
    assert st["exp_avg_absmax"].shape == (P, math.ceil(shape[-2] * shape[-1] / B))
    assert st["factored_row_absmax"].shape == (2 * P, math.ceil(shape[-2] / B))
    assert st["factored_col_absmax"].shape == (2 * P, math.ceil(shape[-1] / B))


@pytest.mark.parametrize("shape,B", [((3, 40, 24), 64), ((2, 5, 33, 7), 16), ((4, 100, 100), 256), ((2, 3, 5), 4)])
def test_per_matrix_step_is_independent_flat_steps_of_its_matrices(shape, B):
    """With the clip inactive (clip_threshold 1e30: the divisor is 1), a per-matrix step of a (P, R, C)
    tensor is P flat steps of (R, C) matrices -- each matrix's blocks, row states, column states and row
    mean are its own in both -- so parameters and every state match bit for bit over three steps.  (With
    the clip active the whole tensor shares one divisor, as in the flat layout.)"""
    P, R, C = math.prod(shape[:-2]), shape[-2], shape[-1]
    hp = dict(HP, clip_threshold=1e30)
    gen = torch.Generator().manual_seed(5)
    p = torch.randn(shape, generator=gen) * 0.02
    st = orc.init_full8bit_state(shape, B, per_matrix=True)
    mats = [p.reshape(P, R, C)[i].clone() for i in range(P)]
    sts = [orc.init_full8bit_state((R, C), B) for _ in range(P)]
    for _ in range(3):
        g = torch.randn(shape, generator=gen) * 1e-3
        orc.full8bit_step(p, g, st, block_size=B, **hp)
        for i in range(P):
            orc.full8bit_step(mats[i], g.reshape(P, R, C)[i], sts[i], block_size=B, **hp)
    assert torch.equal(p.reshape(P, R, C), torch.stack(mats))
    assert torch.equal(st["exp_avg_q"].reshape(P, R, C), torch.stack([s["exp_avg_q"] for s in sts]))
    assert torch.equal(st["exp_avg_absmax"], torch.stack([s["exp_avg_absmax"] for s in sts]))
    for key in ("row", "col"):
        q = st[f"factored_{key}_q"].view(2, P, -1)
        a = st[f"factored_{key}_absmax"].view(2, P, -1)
        for j in (0, 1):
            assert torch.equal(q[j], torch.stack([s[f"factored_{key}_q"][j] for s in sts])), (key, j)
            assert torch.equal(a[j], torch.stack([s[f"factored_{key}_absmax"][j] for s in sts])), (key, j)
