"""Checks that pin the CPU restatement of the 8bit2d step (oracle.came8bit2d_step), which has no runnable
reference here: closed forms, invariants and brute force, each chosen so that a plausible slip (a
transposed tile index, a dropped absmax guard, additive instead of multiplicative weight decay, the
exact instead of the requantised momentum in the parameter write) fails one of them."""
import math

import numpy as np
import pytest
import torch

from oracle import came8_oracle as orc

HP = dict(beta1=0.9, beta2=0.999, beta3=0.9999, eps0=1e-30, eps1=1e-16, lr=2e-4, clip_threshold=1.0,
          weight_decay=0.0)


def test_state_layout_matches_reference_init():
    """came8bit2d_state.py:33-75: int8 codes shaped like p, one fp32 absmax per 16x16 tile starting at 0,
    four uint8 row/col states with fp32 block scales starting at 1, and the tile geometry."""
    st = orc.init_8bit2d_state((37, 50), 256)
    assert st["_mode"] == "8bit2d" and "step" not in st
    assert st["exp_avg_q"].dtype == torch.int8 and tuple(st["exp_avg_q"].shape) == (37, 50)
    assert st["exp_avg_absmax"].dtype == torch.float32 and st["exp_avg_absmax"].numel() == 3 * 4
    assert float(st["exp_avg_absmax"].abs().sum()) == 0.0
    for k, n in (("exp_avg_sq_row", 37), ("exp_avg_sq_col", 50), ("exp_avg_res_row", 37), ("exp_avg_res_col", 50)):
        assert st[k + "_q"].dtype == torch.uint8 and st[k + "_q"].numel() == n
        assert torch.equal(st[k + "_absmax"], torch.ones(1))
    assert (st["rows"], st["cols"], st["tile_rows"], st["tile_cols"], st["num_tiles"]) == (37, 50, 3, 4, 12)


def test_first_step_constant_magnitude_closed_form():
    """|g| = s everywhere: r = 1, c = 1/(s sqrt(a2)), so |u| = 1/sqrt(a2) before the clip and 1 after;
    m = (1 - b1) u = +-0.1 in every tile, stored as codes +-127 with tile absmax 0.1."""
    gen = torch.Generator().manual_seed(0)
    sign = torch.where(torch.rand(40, 48, generator=gen) < 0.5, -1.0, 1.0)
    g = 3e-3 * sign
    st = orc.init_8bit2d_state((40, 48))
    cap = {}
    orc.came8bit2d_step(torch.zeros(40, 48), g, st, capture=cap, **HP)
    a2 = float(np.float32(1.0) - np.float32(0.999))
    assert abs(float(cap["clip"]) * math.sqrt(a2) - 1.0) < 1e-5
    assert torch.equal(st["exp_avg_q"], (127 * sign).to(torch.int8))
    assert torch.allclose(st["exp_avg_absmax"], torch.full((3 * 3,), 0.1), rtol=1e-6)


def test_zero_grads_give_exact_multiplicative_weight_decay():
    """g = 0: the momentum stays 0 (tile absmax 0 -> 1, codes 0), so p <- round(p * (1 - lr*wd)) and the
    parameter write adds exactly 0 -- multiplicative, not p + (-lr*wd)*p."""
    gen = torch.Generator().manual_seed(1)
    for dt in (torch.float32, torch.bfloat16):
        p = (torch.randn(33, 20, generator=gen) * 0.02).to(dt)
        p0 = p.clone()
        st = orc.init_8bit2d_state((33, 20))
        orc.came8bit2d_step(p, torch.zeros(33, 20, dtype=dt), st, **dict(HP, weight_decay=0.1, lr=1e-2))
        fac = np.float32(1.0) - np.float32(1e-2) * np.float32(0.1)
        assert torch.equal(p, (p0.float() * float(fac)).to(dt))
        assert int(st["exp_avg_q"].abs().sum()) == 0
        assert torch.equal(st["exp_avg_absmax"], torch.ones_like(st["exp_avg_absmax"]))


def test_zero_absmax_guard_ignores_stale_codes():
    """A tile whose absmax is 0 contributes no old momentum, whatever its codes say."""
    gen = torch.Generator().manual_seed(2)
    g = torch.randn(20, 36, generator=gen) * 1e-3
    a = orc.init_8bit2d_state((20, 36))
    b = orc.init_8bit2d_state((20, 36))
    b["exp_avg_q"].copy_(torch.randint(-127, 128, (20, 36), generator=gen).to(torch.int8))
    pa, pb = torch.zeros(20, 36), torch.zeros(20, 36)
    orc.came8bit2d_step(pa, g, a, **HP)
    orc.came8bit2d_step(pb, g, b, **HP)
    assert torch.equal(pa, pb) and torch.equal(a["exp_avg_q"], b["exp_avg_q"])


@pytest.mark.parametrize("shape", [(17, 33), (16, 16), (5, 70), (64, 3)])
def test_tile_absmax_brute_force(shape):
    gen = torch.Generator().manual_seed(3)
    st = orc.init_8bit2d_state(shape)
    cap = {}
    for _ in range(2):
        orc.came8bit2d_step(torch.zeros(shape), torch.randn(shape, generator=gen) * 1e-3, st, capture=cap, **HP)
    m = cap["exp_avg"]
    R, C = shape
    tc = math.ceil(C / 16)
    for ty in range(math.ceil(R / 16)):
        for tx in range(tc):
            blk = m[ty * 16:(ty + 1) * 16, tx * 16:(tx + 1) * 16]
            want = float(blk.abs().max()) or 1.0
            assert float(st["exp_avg_absmax"][ty * tc + tx]) == want, (ty, tx)


def test_residual_states_match_direct_means():
    """Step 1 from zero states: res_row = a3 * mean over columns of (u - m)^2 + eps1, res_col likewise over
    rows, against an fp64 recomputation from the captured update and momentum."""
    gen = torch.Generator().manual_seed(4)
    shape = (19, 45)
    st = orc.init_8bit2d_state(shape)
    cap = {}
    orc.came8bit2d_step(torch.zeros(shape), torch.randn(shape, generator=gen) * 1e-3, st, capture=cap, **HP)
    res = (cap["update"].double() - cap["exp_avg"].double()) ** 2 + 1e-16
    a3 = float(np.float32(1.0) - np.float32(0.9999))
    assert torch.allclose(cap["res_row"].double(), a3 * res.mean(dim=1), rtol=1e-5)
    assert torch.allclose(cap["res_col"].double(), a3 * res.mean(dim=0), rtol=1e-5)


def test_parameter_write_uses_requantised_momentum():
    """With wd = 0 the parameter moves by -lr * (m_q * rr) * cr where m_q is the dequantised NEW code,
    not the exact momentum: on a step where quantisation error is visible the two differ."""
    gen = torch.Generator().manual_seed(5)
    shape = (16, 32)
    st = orc.init_8bit2d_state(shape)
    p = torch.zeros(shape)
    cap = {}
    orc.came8bit2d_step(p, torch.randn(shape, generator=gen) * 1e-3, st, capture=cap, **dict(HP, lr=1.0))
    tile = (torch.arange(16)[:, None] // 16) * 2 + (torch.arange(32)[None, :] // 16)
    m_q = st["exp_avg_q"].double() * (st["exp_avg_absmax"][tile].double() / 127)
    # the direction of -p is m_q scaled per row and column: its ratio to m_q is rank one
    ratio = (-p.double()) / m_q
    ok = m_q != 0
    rk = ratio[ok].reshape(-1)
    assert float((rk.max() - rk.min()) / rk.mean()) > 1e-6  # rr_i * cr_j vary
    rr_cr = ratio[:, :1] * ratio[:1, :] / ratio[0, 0]
    assert torch.allclose(ratio[ok], rr_cr[ok], rtol=1e-5)
    # the exact momentum does not give a rank-one ratio: the write did not use it
    exact = (-p.double()) / cap["exp_avg"].double()
    fit = exact[:, :1] * exact[:1, :] / exact[0, 0]
    assert float(((exact - fit)[ok] / fit[ok]).abs().max()) > 1e-4
