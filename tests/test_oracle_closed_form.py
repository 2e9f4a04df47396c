"""Closed-form and invariant checks that pin the CPU oracle where the golden vectors leave it open.

Each test is chosen so that a plausible slip in the oracle (a dropped term, a swapped beta, a wrong
axis of a mean, a missing clamp, round-half-away instead of half-even) fails it.
"""
import math

import numpy as np
import pytest
import torch

from oracle import came8_oracle as orc

HP = dict(beta1=0.9, beta2=0.999, beta3=0.9999, eps0=1e-30, eps1=1e-16, lr=2e-4, clip_threshold=1.0,
          weight_decay=0.0, block_size=256)


# ------------------------------------------------------------------ blockwise quantisation
@pytest.mark.parametrize("signed", [True, False])
def test_quantize_brute_force_every_code(signed):
    """Every code value round-trips exactly through an absmax of Q (scale 1); half-way points round to even."""
    Q = 127 if signed else 255
    codes = torch.arange(-Q if signed else 0, Q + 1, dtype=torch.float32)
    x = torch.cat([codes, codes[:-1] + 0.5])  # integers and exact half-way points
    x[0] = -Q if signed else 0.0
    x = torch.cat([x, torch.tensor([float(Q)])])  # absmax = Q -> scale exactly 1
    q, a = orc.quantize_blockwise(x, signed=signed, block_size=x.numel())
    assert a.item() == Q
    expect = torch.round(x)  # torch.round is half-to-even
    assert torch.equal(q.to(torch.float32), expect)
    halves = x[codes.numel():-1]
    assert torch.equal(q[codes.numel():-1].to(torch.float32) % 2, torch.zeros_like(halves))  # even
    d = orc.dequantize_blockwise(q, a, signed=signed, block_size=x.numel())
    assert torch.equal(d[: codes.numel()], codes)


def test_quantize_zero_block_tail_and_unsigned_padding():
    x = torch.zeros(600)
    x[300:] = torch.linspace(-1, 1, 300)
    q, a = orc.quantize_blockwise(x, signed=True, block_size=256)
    assert a.tolist()[0] == 1.0  # all-zero block -> 1
    assert q[:256].abs().sum() == 0
    assert a.numel() == 3
    # unsigned: a partial tail block of negative values has max(padding 0) = 0 -> absmax 1
    qu, au = orc.quantize_blockwise(-torch.ones(257), signed=False, block_size=256)
    assert au.tolist() == [1.0, 1.0] and int(qu.max()) == 0


def test_dequantize_is_code_times_rounded_scale():
    q = torch.tensor([1, -3, 127, -127], dtype=torch.int8)
    a = torch.tensor([3.3], dtype=torch.float32)
    d = orc.dequantize_blockwise(q, a, signed=True, block_size=4)
    scale = np.float32(np.float32(3.3) / np.float32(127.0))
    assert d.tolist() == [float(np.float32(v * scale)) for v in (1, -3, 127, -127)]


# ------------------------------------------------------------------ one step from the initial state
def test_first_step_unfactored_closed_form():
    """Step 1, 1-D: v = (1-b2)(g^2+eps0); u = g/sqrt(v) = sign(g)/sqrt(1-b2) for constant |g|;
    rms = 1/sqrt(1-b2) > 1 so the clip gives |u| = 1; m = (1-b1) u; p -= lr * m."""
    n = 512
    g = torch.full((n,), 3e-3)
    g[::2] = -3e-3
    p = torch.zeros(n)
    st = orc.init_full8bit_state((n,))
    cap = {}
    orc.full8bit_step(p, g, st, capture=cap, **HP)
    v = (1 - 0.999) * (3e-3 ** 2)
    assert torch.allclose(cap["sq"], torch.full((n,), v), rtol=1e-6)
    assert abs(cap["clip"].item() - 1 / math.sqrt(1 - 0.999)) < 1e-4
    assert torch.allclose(cap["exp_avg"], torch.sign(g) * 0.1, rtol=1e-6)
    assert torch.allclose(p, -2e-4 * torch.sign(g) * 0.1, rtol=1e-6)


def test_first_step_factored_rank_one_closed_form():
    """Step 1 on a rank-one |g| = a_i * b_j: R_i = (1-b2) a_i^2 mean(b^2), C_j = (1-b2) b_j^2 mean(a^2),
    r_i c_j g_ij = sign(g_ij) * sqrt(mean(a^2)... ) -> |u| constant, so after the clip |u| = 1 everywhere."""
    a = torch.linspace(0.5, 2.0, 48)
    b = torch.linspace(1.0, 3.0, 80)
    sign = torch.where(torch.rand(48, 80, generator=torch.Generator().manual_seed(0)) < 0.5, -1.0, 1.0)
    g = 1e-3 * a[:, None] * b[None, :] * sign
    p = torch.zeros(48, 80)
    st = orc.init_full8bit_state((48, 80))
    cap = {}
    orc.full8bit_step(p, g, st, capture=cap, **HP)
    R = (1 - 0.999) * (1e-6 * a ** 2 * (b ** 2).mean())
    C = (1 - 0.999) * (1e-6 * b ** 2 * (a ** 2).mean())
    assert torch.allclose(cap["sq_row"], R, rtol=1e-5)
    assert torch.allclose(cap["sq_col"], C, rtol=1e-5)
    assert torch.allclose(cap["exp_avg"].abs(), torch.full((48, 80), 0.1), rtol=1e-5)
    assert torch.equal(torch.sign(cap["exp_avg"]), sign)


def test_beta1_zero_momentum_is_update_and_residual_is_eps():
    """b1 = 0: m = u exactly, so res = eps1 everywhere and the residual factors are uniform."""
    gen = torch.Generator().manual_seed(1)
    g = torch.randn(32, 40, generator=gen) * 1e-3
    st = orc.init_full8bit_state((32, 40))
    cap = {}
    hp = dict(HP, beta1=0.0)
    p = torch.zeros(32, 40)
    orc.full8bit_step(p, g, st, capture=cap, **hp)
    rr = cap["res_row"]
    assert torch.allclose(rr, torch.full_like(rr, (1 - 0.9999) * 1e-16), rtol=1e-5)


def test_zero_grads_give_pure_weight_decay():
    gen = torch.Generator().manual_seed(2)
    p = torch.randn(20, 30, generator=gen) * 0.02
    p0 = p.clone()
    st = orc.init_full8bit_state((20, 30))
    orc.full8bit_step(p, torch.zeros(20, 30), st, **dict(HP, weight_decay=0.1, lr=1e-2))
    alpha = np.float32(-0.1 * 1e-2)
    expect = torch.from_numpy((p0.double().numpy() * float(alpha) + p0.double().numpy()).astype(np.float32))
    assert torch.equal(p, expect)


def test_block_size_one_matches_fp32_state_came():
    """block_size = 1: every state element is its own block, so quantisation is exact up to the
    rounding of (x/|x|)*Q*(|x|/Q); the 8-bit step must then track the fp32-state CAME step."""
    gen = torch.Generator().manual_seed(3)
    shapes = [(24, 36), (50,)]
    for s in shapes:
        p8 = torch.randn(s, generator=gen) * 0.02
        p32 = p8.clone()
        st8 = orc.init_full8bit_state(s, 1)
        st32 = orc.init_fp32_state(s)
        for _ in range(5):
            g = torch.randn(s, generator=gen) * 1e-3
            orc.full8bit_step(p8, g, st8, **dict(HP, block_size=1, weight_decay=1e-2))
            hp32 = {k: v for k, v in HP.items() if k != "block_size"}
            orc.fp32_state_step(p32, g, st32, **dict(hp32, weight_decay=1e-2))
        assert torch.allclose(p8, p32, rtol=1e-5, atol=1e-8), s


# ------------------------------------------------------------------ the reference's norm
def _fma32(a, b, c):
    """float32 fma(a, b, c) rounded once (round to nearest even), elementwise.  a*b is exact in float64;
    TwoSum gives s + e == a*b + c exactly; s rounded to float32 is the fused result unless s sits exactly
    on a float32 midpoint, where the sign of e decides (e == 0: a true tie, which the cast breaks to even)."""
    a, b, c = (np.asarray(v, dtype=np.float32) for v in (a, b, c))
    p = a.astype(np.float64) * b.astype(np.float64)
    c64 = c.astype(np.float64)
    s = p + c64
    bb = s - p
    e = (p - (s - bb)) + (c64 - bb)
    r = s.astype(np.float32)
    r64 = r.astype(np.float64)
    up = np.where(s > r64, np.float32(np.inf), np.float32(-np.inf)).astype(np.float32)
    toward = np.nextafter(r, up)
    nb64 = toward.astype(np.float64)
    at_mid = (s != r64) & (s == (r64 + nb64) / 2)
    go = at_mid & (e != 0) & ((e > 0) == (nb64 > r64))
    return np.where(go, toward, r).astype(np.float32)


def _norm_reference_order(x: np.ndarray) -> np.float32:
    """torch's CPU float32 norm(2) order: 8 interleaved fused multiply-add accumulators over the first
    n - n%8 elements; their left-to-right sum; then, when four or more elements remain, four rounded
    squares added one at a time; then the last n%4 elements as fused multiply-adds; sqrt (rounded
    once: a float64 sqrt of a float32 rounds correctly to float32)."""
    x = x.reshape(-1).astype(np.float32)
    n = x.size
    main = n - n % 8
    acc = np.zeros(8, dtype=np.float32)
    for row in x[:main].reshape(-1, 8):
        acc = _fma32(row, row, acc)
    b = np.float32(acc[0])
    for j in range(1, 8):
        b = np.float32(b + acc[j])
    d = main
    if n - d >= 4:
        for d in range(d, d + 4):
            b = np.float32(b + np.float32(x[d] * x[d]))
        d += 1
    for d in range(d, n):
        b = _fma32(x[d], x[d], b)
    return np.float32(math.sqrt(np.float64(b)))


def test_fma32_against_fractions():
    """The float32 fma used by the replica against exact rational arithmetic, on values built to land the
    float64 sum on float32 midpoints (where a float64-then-float32 rounding goes wrong)."""
    from fractions import Fraction
    rng = np.random.default_rng(5)

    def rn32(fr):
        f = np.float32(float(fr))
        best = None
        for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
            dist = abs(Fraction(float(c)) - fr)
            if best is None or dist < best[0] or (dist == best[0] and int(np.array(c).view(np.uint32)) & 1 == 0):
                best = (dist, c)
        return best[1]

    hits_mid = 0
    for i in range(3000):
        if i % 2:  # generic operands
            a = np.float32(rng.standard_normal() * 10.0 ** rng.uniform(-3, 3))
            b = np.float32(rng.standard_normal() * 10.0 ** rng.uniform(-3, 3))
            c = np.float32(rng.standard_normal() * 10.0 ** rng.uniform(-3, 3))
        else:  # c with an odd last bit and a*b = half an ulp of c minus 2^-46 of it: the float64 sum is the
            # midpoint, the exact sum lies just inside, and ties-to-even on the float64 value goes the wrong way
            E = 2 * int(rng.integers(-20, 20))
            k = 2 * int(rng.integers(0, 2 ** 21)) + 1
            sign = 1.0 if rng.uniform() < 0.5 else -1.0
            c = np.float32(sign * (1 + k * 2.0 ** -23) * 2.0 ** E)
            a = np.float32(2.0 ** (E // 2 - 12) * (1 + 2.0 ** -23))
            b = np.float32(sign * 2.0 ** (E // 2 - 12) * (1 - 2.0 ** -23))
        want = rn32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))
        s64 = np.float64(a) * np.float64(b) + np.float64(c)
        hits_mid += np.float32(s64) != want
        assert _fma32(a, b, c) == want, (a, b, c)
    assert hits_mid > 0  # the draws include cases a float64 intermediate would get wrong


@pytest.mark.parametrize("n", list(range(1, 24)) + [255, 1000, 4099])
def test_reference_norm_order_replica(n):
    """The summation order the GPU's default clip reproduces equals torch.norm bit for bit, over a few
    hundred draws per length (the tail rules for n % 8 in 1..7 each decide a few percent of draws)."""
    rng = np.random.default_rng(n)
    draws = 300 if n < 24 else 20
    for i in range(draws):
        if i % 2:
            x = (rng.standard_normal(n) * rng.uniform(0.1, 100)).astype(np.float32)
        else:  # wide dynamic range within a draw
            x = (rng.standard_normal(n) * 10.0 ** rng.uniform(-6, 3, n)).astype(np.float32)
        assert np.float32(torch.from_numpy(x).norm(2).item()) == _norm_reference_order(x), (n, i)


def test_reference_norm_tail_rules_are_load_bearing():
    """The replica with a separately rounded tail, or with the four-element block fused, misses torch.norm
    on some draws: each rule of the tail is pinned, not just tolerated."""
    rng = np.random.default_rng(99)

    def variant(x, block_fused, tail_fused):
        n = x.size
        b = np.float32(0)
        d = 0
        if n >= 4 and n < 8:
            for d in range(4):
                b = _fma32(x[d], x[d], b) if block_fused else np.float32(b + np.float32(x[d] * x[d]))
            d = 4
        for d in range(d, n):
            b = _fma32(x[d], x[d], b) if tail_fused else np.float32(b + np.float32(x[d] * x[d]))
        return np.float32(math.sqrt(np.float64(b)))

    miss_block = miss_tail = 0
    for n in (2, 3, 5, 6, 7):
        for _ in range(300):
            x = (rng.standard_normal(n) * rng.uniform(0.1, 100)).astype(np.float32)
            t = np.float32(torch.from_numpy(x).norm(2).item())
            assert t == variant(x, False, True)
            miss_tail += t != variant(x, False, False)
            miss_block += n >= 5 and t != variant(x, True, True)
    assert miss_tail > 0 and miss_block > 0


def test_reference_norm_error_on_c1_and_exact_norm_variant():
    """The reference's float32 norm of a C1-sized update is off the exact one by ~1e-4 relative (which is
    why the library replays its order rather than computing the exact value)."""
    gen = torch.Generator().manual_seed(0)
    g = torch.randn(2048, 2048, generator=gen) * 1e-3
    u = g * 30.0
    exact = math.sqrt(math.fsum(float(v) ** 2 for v in u.double().reshape(-1).tolist()))
    ref = u.norm(2).item()
    assert 1e-6 < abs(ref / exact - 1) < 5e-4


def _exact_clip(u: torch.Tensor, thr: float) -> float:
    """max(RN32(sqrt(sum u^2)) / RN32(sqrt(n)) / thr, 1) with the sum exactly rounded (math.fsum) and
    each float32 operation rounded as torch rounds it."""
    s = math.fsum(float(v) ** 2 for v in u.double().reshape(-1).tolist())
    norm = np.float32(math.sqrt(s))
    rms = np.float32(norm / np.float32(u.numel() ** 0.5))
    q = np.float32(rms / np.float32(thr))
    return float(max(q, np.float32(1.0)))


@pytest.mark.parametrize("case", ["const4096", "const_ragged", "heavy", "rank_one"])
def test_exact_norm_branch_clip(case):
    """The oracle's exact_norm=True clip against math.fsum, bit for bit, on updates built so that the
    oracle's step-1 update u is known: 1-D tensors at step 1 have u = g / sqrt((1-b2)(g^2+eps0)) elementwise
    (recomputed here exactly as the oracle forms it), and for constant |g| every |u| is equal, so the
    norm is |u| sqrt(n) (n = 4096: sqrt exact).  A dropped square, a wrong count or a float32 sum would
    fail these (the C1-size test above shows the float32 sum is off by far more than an ulp)."""
    gen = torch.Generator().manual_seed(7)
    n = {"const4096": 4096, "const_ragged": 4099, "heavy": 200_003, "rank_one": 4096}[case]
    if case.startswith("const") or case == "rank_one":
        g = torch.full((n,), 3e-4) * torch.where(torch.rand(n, generator=gen) < 0.5, -1.0, 1.0)
    else:
        g = torch.randn(n, generator=gen) / torch.rand(n, generator=gen).clamp_min(1e-3) * 1e-3
    hp = dict(HP, clip_threshold=1e-3)
    st = orc.init_full8bit_state((n,))
    cap = {}
    orc.full8bit_step(torch.zeros(n), g.clone(), st, capture=cap, exact_norm=True, **hp)
    # the update exactly as the oracle forms it at step 1 (zero state)
    sq = (g * g + hp["eps0"]) * (1.0 - hp["beta2"])
    u = sq.clamp_min(1e-30).rsqrt() * g
    want = _exact_clip(u, hp["clip_threshold"])
    assert float(cap["clip"]) == want, (case, float(cap["clip"]), want)
    if case == "const4096":
        absu = float(u.abs()[0])
        assert float(np.float32(np.float32(absu * 64.0) / np.float32(64.0))) == float(np.float32(absu))
        assert all(float(v) == absu for v in u.abs()[:50])


def test_first_step_fp16_update_closed_form():
    """Step 1, 1-D, the fp16-update branch: v = (1-b2)(g^2+eps0), u = g/sqrt(v) (eps0 = 1e-6, about g^2,
    so that |u| varies); the clip is the RMS of the fp32 u (threshold 0.5, so active and not a power
    of two); the momentum takes u rounded to fp16 before the division: m = (1-b1) * fp16(u) / clip.
    Computed here in fp64 with numpy's fp16 rounding; elements whose u lies within 1e-6 of an fp16
    rounding tie are left out.  Rounding after the division, rounding the norm's input, or not
    rounding at all each miss by up to 2^-11."""
    gen = torch.Generator().manual_seed(7)
    n = 4096
    g = torch.randn(n, generator=gen) * 1e-3 * torch.exp(torch.randn(n, generator=gen))
    hp = dict(HP, clip_threshold=0.5, eps0=1e-6)
    p = torch.zeros(n)
    st = orc.init_full8bit_state((n,))
    cap = {}
    orc.full8bit_step(p, g, st, capture=cap, fp16_update=True, **hp)
    g64 = g.double().numpy()
    v = (1 - 0.999) * (g64 ** 2 + 1e-6)
    u = g64 / np.sqrt(v)
    clip = max(np.sqrt(np.mean(u ** 2)) / 0.5, 1.0)
    assert abs(cap["clip"].item() / clip - 1) < 1e-6
    u16 = u.astype(np.float16).astype(np.float64)
    # distance of u from an fp16 rounding tie, relative
    ulp = np.abs(np.spacing(u.astype(np.float16)).astype(np.float64))
    frac = np.abs(u - u16) / ulp
    keep = np.abs(frac - 0.5) > 1e-6 * np.abs(u) / ulp + 1e-3
    m = (1 - 0.9) * u16 / clip
    got = cap["exp_avg"].double().numpy()
    assert keep.mean() > 0.99
    assert np.allclose(got[keep], m[keep], rtol=2e-6, atol=0), np.abs(got[keep] / m[keep] - 1).max()
    m32 = (1 - 0.9) * u / clip  # without the rounding: visibly different
    assert np.abs(got / m32 - 1).max() > 1e-4
