"""GPU: the clip divisor of the default step against the reference's.

The reference divides the update by max(u.norm(2) / sqrt(N) / clip_threshold, 1)
(came_pytorch/CAME8bitFull.py:121-122,1032), where torch's CPU norm sums fp32 squares as eight
serial fused-multiply-add chains; at these sizes the chains drift from the exact norm by up to ~1%
(32000 x 4096), so only a replay of those chains gives the reference's value.  The library replays
them in parallel (came_amd/csrc/came8_norm.h); these tests read its divisors back
(came8_read_clip) and compare them with the oracle's, which calls torch.norm itself.

Bit for bit wherever the update u itself is the reference's bit for bit: 1-D tensors (u is
elementwise), and matrices whose gradients make the row and column factors exact in any summation
order ("latin": magnitudes 2^-(10+l) with l = (a_i + b_j) mod 4 and a, b balanced, so every row and
every column holds the same multiset of powers of two, and the row count is a power of two).  Other
matrices: within 4 fp32 ulps, because the GPU forms the row/column means in fp64 rounded once while
torch rounds along the way, so u can differ from the reference's by an ulp; the drift-regime test
also checks that the exactly rounded norm misses the reference by far more than that.

A clip threshold of 1e-6 keeps the divisor active (rms / threshold > 1), so that every bit of the
norm reaches it.  Step 2 starts from the oracle's state (teacher-forced), so both sides norm the
same update.
"""
import math

import pytest
import torch

from oracle import came8_oracle as orc
from tests import parity as P

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import came_amd._lib as L
    L.load()
    torch.set_num_threads(8)
    yield


def _grad(gen, shape, kind, dtype):
    n = math.prod(shape)
    if kind == "normal":
        g = torch.randn(n, generator=gen) * 1e-3
    elif kind == "const":
        g = torch.full((n,), 1e-3)
    elif kind == "sparse":
        g = torch.zeros(n)
        k = max(1, n // 97)
        g[torch.randint(0, n, (k,), generator=gen)] = torch.randn(k, generator=gen)
    elif kind == "heavy":
        return P.heavy_grad(gen, shape, dtype)
    elif kind == "latin":
        R, C = shape
        a = torch.arange(R) % 4
        b = torch.arange(C) % 4
        a = a[torch.randperm(R, generator=gen)]
        b = b[torch.randperm(C, generator=gen)]
        l = (a.reshape(-1, 1) + b.reshape(1, -1)) % 4
        sign = torch.where(torch.rand(R, C, generator=gen) < 0.5, -1.0, 1.0)
        return (sign * torch.pow(2.0, -(10 + l).double()).float()).to(dtype)
    elif kind == "scaled":  # rows of very different scales
        g = torch.randn(shape, generator=gen) * torch.logspace(-6, 0, shape[0]).reshape(-1, *([1] * (len(shape) - 1)))
    else:
        raise ValueError(kind)
    return g.reshape(shape).to(dtype)


def _ulps(a: float, b: float) -> int:
    ia = torch.tensor([a], dtype=torch.float32).view(torch.int32).item()
    ib = torch.tensor([b], dtype=torch.float32).view(torch.int32).item()
    return abs(ia - ib)


def _run(cls_name, cases, steps=2, max_ulps=0, check_exact_gap=False, seed=1234, **hp_kw):
    import came_amd
    gen = torch.Generator().manual_seed(seed)
    shapes = [c[0] for c in cases]
    dts = [c[2] for c in cases]
    params = [(torch.randn(s, generator=gen) * 0.02).to(dt) for s, dt in zip(shapes, dts)]
    grads = [[_grad(gen, s, kind, dt) for s, kind, dt in cases] for _ in range(steps)]
    hp = dict(lr=2e-4, weight_decay=1e-2, clip_threshold=1e-6)
    hp.update(hp_kw)
    ohp = P.oracle_hp(hp)
    ps = [torch.nn.Parameter(p.clone().to(DEV)) for p in params]
    opt = getattr(came_amd, cls_name)(ps, **hp)
    fp32 = cls_name == "CAMECUDA"
    refs = [p.clone() for p in params]
    sts = [(orc.init_fp32_state(p.shape) if fp32 else orc.init_full8bit_state(p.shape, ohp["block_size"]))
           for p in refs]
    for s in range(steps):
        with torch.no_grad():  # teacher forcing: the GPU starts from the oracle's state
            for p, r, st in zip(ps, refs, sts):
                p.data.copy_(r.to(DEV))
                gst = opt.state[p]
                for k, v in gst.items():
                    if isinstance(v, torch.Tensor) and k in st and isinstance(st[k], torch.Tensor) and v.shape == st[k].shape:
                        v.copy_(st[k].to(DEV))
        for p, g in zip(ps, grads[s]):
            p.grad = g.to(DEV)
        opt.step()
        got = opt.last_clip_divisors()
        for i, (r, g, st) in enumerate(zip(refs, grads[s], sts)):
            ex = None
            if check_exact_gap:  # the exactly rounded norm on the same inputs (the oracle's opt-in branch)
                cap2 = {}
                st2 = {k: (v.clone() if isinstance(v, torch.Tensor) else v) for k, v in st.items()}
                orc.full8bit_step(r.clone(), g, st2, capture=cap2, exact_norm=True, **ohp)
                ex = float(cap2["clip"])
            cap = {}
            if fp32:
                orc.fp32_state_step(r, g, st, capture=cap, **{k: v for k, v in ohp.items() if k != "block_size"})
            else:
                orc.full8bit_step(r, g, st, capture=cap, **ohp)
            want = float(cap["clip"])
            have = got[ps[i]]
            assert want > 1.0, f"case {cases[i]}: the clip is not active"
            exact = cases[i][1] == "latin" or len(cases[i][0]) == 1
            tol = 0 if exact else max_ulps
            d = _ulps(have, want)
            print(f"[norm] {cls_name} step {s + 1} {cases[i]}: clip {have!r} vs {want!r}: {d} ulps"
                  + ("" if ex is None else f"; exactly rounded norm: {_ulps(ex, want)} ulps"), flush=True)
            assert d <= tol, (f"{cls_name} step {s + 1} case {cases[i]}: clip {have!r} != reference {want!r} "
                              f"({d} ulps; {(have - want) / want:.3e} relative; allowed {tol})")
            if ex is not None:
                assert _ulps(ex, want) > 100, f"{cases[i]}: the exactly rounded norm is as close as the replay"


F32, BF16 = torch.float32, torch.bfloat16

ONE_D = [((n,), "normal", F32) for n in (1, 7, 8, 9, 63, 4095, 4096, 4097, 8193, 100003)] + [
    ((1_000_000,), "const", F32), ((300_001,), "sparse", F32), ((250_000,), "heavy", BF16)]


def test_norm_one_d():
    _run("CAME8bit", ONE_D)


# Every tail length N % 8 = 1..7, short and long: torch adds the tail after the eight chains as a block of
# four separately rounded squares (when four or more remain) and then fused multiply-adds; each rule
# decides the last bit in a few percent of draws, so several seeds are needed to see a wrong rule.
TAILS = [((n,), "normal", F32) for n in (2, 3, 4, 5, 6, 7, 12, 13, 14, 15, 17, 4097, 4098, 4099, 4100, 4101,
                                         4102, 4103)]


@pytest.mark.parametrize("seed", range(6))
def test_norm_one_d_tails(seed):
    _run("CAME8bit", TAILS, seed=seed)


MATRICES = [((2048, 2048), "latin", F32), ((256, 4096), "latin", BF16), ((64, 1000), "latin", F32),
            ((2048, 2048), "normal", F32), ((64, 20000), "normal", BF16), ((1000, 3), "normal", F32),
            ((3, 50257), "heavy", F32), ((4097, 129), "normal", BF16), ((777, 1024), "sparse", BF16),
            ((512, 4096), "scaled", BF16), ((320, 320, 3, 3), "normal", F32), ((1280, 640, 1, 1), "heavy", F32),
            ((5, 7, 1), "normal", F32)]


def test_norm_matrices():
    _run("CAME8bit", MATRICES, max_ulps=4)


# Row widths at the edges of the record kernels' forms: the LDS-staged kernel takes rows of 128 to 16384
# columns (whole 8-element chunks) or 128 to 16376 (other rows, which read 8 factors past the row);
# narrower and wider rows take the per-segment kernel.  Latin matrices (widths a multiple of 4) are bit
# exact; the odd widths within 4 ulps.
ROW_WIDTHS = [((256, 124), "latin", F32), ((256, 128), "latin", BF16), ((256, 132), "latin", F32),
              ((64, 16372), "latin", BF16), ((64, 16380), "latin", F32), ((64, 16384), "latin", BF16),
              ((64, 16388), "latin", F32), ((128, 16375), "normal", F32), ((512, 129), "normal", BF16)]


def test_norm_row_widths():
    _run("CAME8bit", ROW_WIDTHS, max_ulps=4)


def test_norm_large_matrices_drift_regime():
    """Chains of millions of elements, where the reference's norm is far from the exact one."""
    _run("CAME8bit", [((8192, 4096), "latin", BF16), ((2048, 11008), "latin", BF16), ((4096, 11008), "normal", BF16)],
         steps=1, max_ulps=4, check_exact_gap=True)


def test_norm_memory_and_camecuda():
    _run("CAME8bitMemory", [((256, 5460), "latin", BF16), ((300, 5461), "normal", BF16), ((2048,), "normal", BF16)],
         max_ulps=4, betas=(0.9, 0.95, 0.995))
    _run("CAMECUDA", [((256, 5460), "latin", BF16), ((300, 5461), "normal", BF16), ((2048,), "normal", F32),
                      ((33, 4, 4), "heavy", F32)], max_ulps=4)


# Time bound of the walk on tie-dense chains: every replayed segment costs a load of its elements and
# factors (at most 6 us, under contention) and every wavefront round at most 0.8 us (a round's scan,
# ballot and lane reads are one dependent chain of about 2000 cycles: 14.5 ms measured for this input,
# 18.7 ms allowed); the counts are the replay rules' on this input (tests.parity.TIE_REPLAYS_MAX /
# TIE_ROUNDS_MAX, pinned on the CPU).
WALK_US_PER_REPLAY, WALK_US_PER_ROUND, WALK_MS_FIXED = 6.0, 0.8, 0.5


def test_norm_walk_on_tie_dense_chains_is_bounded():
    """A 2048 x 4096 bf16 matrix whose update under power-of-two factors puts a rounding tie in about
    half of every chain's segments (1058 of 2048 replayed, against ~16 for Gaussian data): the divisor is
    the reference's bit for bit, and the walk's time stays within the bound its replay and round counts
    give.  A Gaussian matrix of the same shape from the zero state (factors that are not powers of two,
    so an update of 24 significant bits) is timed beside it."""
    import came_amd
    from came_amd import _lib
    gen = torch.Generator().manual_seed(P.TIE_SEED)
    g = P.tie_dense_grad(gen, P.TIE_SHAPE)
    p0 = (torch.randn(P.TIE_SHAPE, generator=gen) * 0.02).to(torch.bfloat16)
    hp = dict(lr=2e-4, weight_decay=0.0, betas=P.TIE_DENSE_BETAS, clip_threshold=1e-6)
    walk = {}
    for kind in ("normal", "tie-dense"):
        grad = g if kind == "tie-dense" else (torch.randn(P.TIE_SHAPE, generator=gen) * 1e-5).to(torch.bfloat16)
        ps = [torch.nn.Parameter(p0.clone().to(DEV))]
        opt = came_amd.CAME8bit(ps, **hp)
        ps[0].grad = grad.to(DEV)
        opt.prime_for_cuda_graph()  # creates the state
        st = orc.init_full8bit_state(P.TIE_SHAPE)
        if kind == "tie-dense":
            P.tie_dense_state(opt.state[ps[0]])
            P.tie_dense_state(st)
        torch.cuda.synchronize()
        _lib.profile_enable(True)
        _lib.profile_read(reset=True)
        opt.step()
        torch.cuda.synchronize()
        phases = _lib.profile_read(reset=True)
        _lib.profile_enable(False)
        walk[kind] = phases["norm_walk"][1]
        cap = {}
        orc.full8bit_step(p0.clone(), grad, st, capture=cap, **P.oracle_hp(hp))
        have, want = opt.last_clip_divisors()[ps[0]], float(cap["clip"])
        print(f"[walk] {kind}: {walk[kind]:.3f} ms; clip {have!r} vs {want!r}", flush=True)
        # exact factors make u the reference's bit for bit; the Gaussian case's factors may differ by an ulp
        assert _ulps(have, want) <= (0 if kind == "tie-dense" else 4), f"{kind}: clip {have!r} != reference {want!r}"
    bound = (P.TIE_REPLAYS_MAX * WALK_US_PER_REPLAY + P.TIE_ROUNDS_MAX * WALK_US_PER_ROUND) / 1e3 + WALK_MS_FIXED
    assert walk["tie-dense"] <= bound, f"tie-dense walk {walk['tie-dense']:.3f} ms > bound {bound:.3f} ms"
