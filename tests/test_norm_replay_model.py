"""CPU check of the parallel replay of torch's fp32 norm chains (came_amd/csrc/came8_norm.h): a C model of
its rules (tests/native/norm_replay_model.c), segment records and the wavefront replay of a segment, must
equal the serial chain s = fma(x, x, s) bit for bit on adversarial inputs (constant values that stall the chain, values with few significant bits that make
rounding ties, zeros, outliers, squares that are subnormal (some exact half-units of the subnormal grid)
or overflow, NaN, rows of very different scales), whatever the binade estimates (exact, 1% off, 50% off), and replay few segments when the
estimates are good."""
import ctypes
import os
import shutil
import subprocess
import zlib

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("gcc not available")
    out = str(tmp_path_factory.mktemp("replay") / "model.so")
    subprocess.run([cc, "-O2", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC", "-o", out,
                    os.path.join(HERE, "native", "norm_replay_model.c"), "-lm"], check=True)
    so = ctypes.CDLL(out)
    so.chain_serial.restype = ctypes.c_float
    so.chain_serial.argtypes = [ctypes.c_void_p, ctypes.c_int64]
    so.chain_replay.restype = ctypes.c_float
    so.chain_replay.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int64)]
    so.chain_replay_stats.restype = ctypes.c_float
    so.chain_replay_stats.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                      ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]
    so.chain_serial_from.restype = ctypes.c_float
    so.chain_serial_from.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_float]
    so.segment_replay.restype = ctypes.c_float
    so.segment_replay.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.POINTER(ctypes.c_int64)]
    return so


def _inputs(kind, n, rng):
    scale = float(np.exp(rng.uniform(-25, 25)))
    if kind == "normal":
        x = rng.standard_normal(n) * scale
    elif kind == "const":
        x = np.full(n, scale)
    elif kind == "fewbits":
        x = np.ldexp(np.floor(rng.uniform(0, 16, n)), rng.integers(0, 6, n))
    elif kind == "zeros":
        x = np.where(rng.uniform(size=n) < 0.3, 0.0, rng.standard_normal(n) * scale)
    elif kind == "outliers":
        x = rng.standard_normal(n) * scale * np.where(rng.uniform(size=n) < 0.01, 1e3, 1.0)
    elif kind == "subnormal":
        x = rng.standard_normal(n) * 1e-25
    elif kind == "overflow":
        x = rng.standard_normal(n) * 1e18
    elif kind == "nan":
        x = rng.standard_normal(n)
        x[n // 2] = np.nan
    elif kind == "subties":  # squares (2k+1)^2 * 2^-150: half-units of the subnormal grid, so every one a tie
        x = np.ldexp(rng.choice([0.0, 1.0, 3.0, 5.0, 7.0], n), -75) * rng.choice([-1.0, 1.0], n)
    elif kind == "halfunits":  # a chain of one unit (2^-149, odd), then only 0 and +-2^-75: squares of half a unit
        x = np.ldexp(rng.choice([0.0, 1.0, -1.0], n), -75)
        x[: min(n, 512)] = 0.0
        x[min(n, 512) - 1] = np.ldexp(1.5, -75)  # (1.5 * 2^-75)^2 = 1.125 units: the chain becomes 1 unit
    elif kind == "blocks":
        x = np.where((np.arange(n) // 1000) % 2 == 0, 0.0, rng.standard_normal(n) * scale)
    else:
        raise ValueError(kind)
    return x.astype(np.float32)


KINDS = ["normal", "const", "fewbits", "zeros", "outliers", "subnormal", "subties", "halfunits", "overflow", "nan", "blocks"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("noise", [0.0, 0.01, 0.5])
def test_replay_equals_serial_chain(lib, kind, noise):
    rng = np.random.default_rng(zlib.crc32(f"{kind}/{noise}".encode()))
    for n in (1, 7, 511, 512, 513, 4097, int(rng.integers(10_000, 300_000)), 1_000_003):
        if kind in ("subties", "halfunits") and n > 5000:  # a chain that stays subnormal replays every element alone
            continue
        x = _inputs(kind, n, rng)
        nseg = (n + 511) // 512
        exact = np.concatenate([[0.0], np.cumsum(x.astype(np.float64) ** 2)])[::512][:nseg]
        est = (exact * (1.0 + noise * (rng.uniform(size=nseg) - 0.5))).astype(np.float64)
        est = np.ascontiguousarray(est)
        rep = ctypes.c_int64(0)
        a = lib.chain_serial(x.ctypes.data, n)
        b = lib.chain_replay(x.ctypes.data, n, est.ctypes.data, ctypes.byref(rep))
        assert np.float32(a).tobytes() == np.float32(b).tobytes(), (kind, noise, n, a, b)


def test_replays_are_few_on_realistic_chains(lib):
    """16.4 M chain elements of u ~ N(0, 30^2) (a 32000 x 4096 matrix's chain), exact estimates: the
    chain's start, one replay per binade crossing and a few ties."""
    rng = np.random.default_rng(0)
    n = 16_384_000
    x = (rng.standard_normal(n) * 30).astype(np.float32)
    nseg = (n + 511) // 512
    est = np.ascontiguousarray(np.concatenate([[0.0], np.cumsum(x.astype(np.float64) ** 2)])[::512][:nseg])
    rep = ctypes.c_int64(0)
    a = lib.chain_serial(x.ctypes.data, n)
    b = lib.chain_replay(x.ctypes.data, n, est.ctypes.data, ctypes.byref(rep))
    assert np.float32(a).tobytes() == np.float32(b).tobytes()
    assert rep.value < 60, rep.value


def test_replays_on_tie_dense_chains(lib):
    """The tie-dense matrix of the GPU walk test (tests.parity.tie_dense_grad under power-of-two factors):
    the oracle's first step with that state has factors r_i = 1 and c_j = 1/8 exactly, so u = g / 8; each
    of its eight chains (1 M elements, 2048 segments) replays about half of its segments, against 16 for
    a Gaussian chain of the same length, and the counts are the ones the GPU test bounds its time by."""
    import torch
    from oracle import came8_oracle as orc
    from tests import parity as P
    gen = torch.Generator().manual_seed(P.TIE_SEED)
    g = P.tie_dense_grad(gen, P.TIE_SHAPE)
    st = orc.init_full8bit_state(P.TIE_SHAPE)
    P.tie_dense_state(st)
    cap = {}
    hp = P.oracle_hp(dict(lr=2e-4, weight_decay=0.0, betas=P.TIE_DENSE_BETAS, clip_threshold=1e-6))
    orc.full8bit_step(torch.zeros(P.TIE_SHAPE, dtype=torch.bfloat16), g, st, capture=cap, **hp)
    assert bool((cap["sq_row"] == 127.5).all()) and bool((cap["sq_col"] == 64.0).all())
    u = (g.float() * 0.125).reshape(-1).numpy()
    reps, rounds = [], []
    for c in range(8):
        x = np.ascontiguousarray(u[c::8])
        n = x.size
        nseg = (n + 511) // 512
        est = np.ascontiguousarray(np.concatenate([[0.0], np.cumsum(x.astype(np.float64) ** 2)])[::512][:nseg])
        rep, rnd = ctypes.c_int64(0), ctypes.c_int64(0)
        a = lib.chain_serial(x.ctypes.data, n)
        b = lib.chain_replay_stats(x.ctypes.data, n, est.ctypes.data, ctypes.byref(rep), ctypes.byref(rnd))
        assert np.float32(a).tobytes() == np.float32(b).tobytes()
        assert rep.value >= 0.4 * nseg, f"chain {c}: {rep.value} of {nseg} segments replayed: not tie-dense"
        reps.append(rep.value)
        rounds.append(rnd.value)
    assert (max(reps), max(rounds)) == (P.TIE_REPLAYS_MAX, P.TIE_ROUNDS_MAX), (reps, rounds)


def _starts(rng):
    """Chain values a replay may start from: zero, subnormals, values at and next to binade edges,
    random normals, the largest float, +inf and NaN."""
    edges = [np.float32(2.0) ** int(e) for e in rng.integers(-126, 127, 12)]
    near = [np.nextafter(e, np.float32(0)) for e in edges] + [np.nextafter(e, np.float32(np.inf)) for e in edges]
    rand = list(np.exp(rng.uniform(-80, 80, 12)).astype(np.float32))
    # the unit-2^-149 range [0, 2^-125): odd and even multiples of the unit, subnormal and normal
    low = list(np.array([1, 2, 3, 0x7FFFFF, 0x800000, 0x800001, 0xFFFFFE, 0xFFFFFF], np.uint32).view(np.float32))
    return ([np.float32(0.0), np.float32(3e-39), np.float32(3.4e38), np.float32(np.inf), np.float32(np.nan)]
            + low + edges + near + rand)


@pytest.mark.parametrize("kind", KINDS)
def test_segment_replay_from_any_start(lib, kind):
    """One segment (up to 512 chain elements) replayed in wavefront rounds from every kind of start value
    equals the serial fmaf loop from that value.  For finite starts the elements are also rescaled so
    that their squares are 2^-k of the start (k in [0, 12]): increments of a few units, where half-unit
    ties and binade crossings concentrate."""
    rng = np.random.default_rng(zlib.crc32(kind.encode()))
    for s0 in _starts(rng):
        for cnt in (1, 2, 8, 9, 63, 64, 65, 300, 511, 512):
            for near in (False, True):
                x = _inputs(kind, cnt, rng)
                if near:
                    if not (np.isfinite(s0) and s0 > 0):
                        continue
                    top = float(np.nanmax(np.abs(x))) if np.isfinite(x).any() else 0.0
                    if not top > 0 or not np.isfinite(top):
                        continue
                    x = (x.astype(np.float64) / top * np.sqrt(float(s0)) * 2.0 ** -rng.uniform(0, 6)).astype(np.float32)
                x = np.ascontiguousarray(x)
                rounds = ctypes.c_int64(0)
                want = lib.chain_serial_from(x.ctypes.data, cnt, float(s0))
                got = lib.segment_replay(x.ctypes.data, cnt, float(s0), ctypes.byref(rounds))
                same = np.float32(got).tobytes() == np.float32(want).tobytes() or (np.isnan(got) and np.isnan(want))
                assert same, (kind, float(s0), cnt, near, got, want)
