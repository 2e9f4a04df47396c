"""CPU check of the parallel replay of torch's fp32 norm chains (came_amd/csrc/came8_norm.h): a C model of
its rules (tests/native/norm_replay_model.c) must equal the serial chain s = fma(x, x, s) bit for bit on
adversarial inputs (constant values that stall the chain, values with few significant bits that make
rounding ties, zeros, outliers, squares that are subnormal or overflow, NaN, rows of very different
scales), whatever the binade estimates (exact, 1% off, 50% off), and replay few segments when the
estimates are good."""
import ctypes
import os
import shutil
import subprocess

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
    elif kind == "blocks":
        x = np.where((np.arange(n) // 1000) % 2 == 0, 0.0, rng.standard_normal(n) * scale)
    else:
        raise ValueError(kind)
    return x.astype(np.float32)


KINDS = ["normal", "const", "fewbits", "zeros", "outliers", "subnormal", "overflow", "nan", "blocks"]


@pytest.mark.parametrize("kind", KINDS)
@pytest.mark.parametrize("noise", [0.0, 0.01, 0.5])
def test_replay_equals_serial_chain(lib, kind, noise):
    rng = np.random.default_rng(hash((kind, noise)) % 2**32)
    for n in (1, 7, 511, 512, 513, 4097, int(rng.integers(10_000, 300_000)), 1_000_003):
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
