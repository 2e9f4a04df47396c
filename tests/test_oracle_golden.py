"""Pin the CPU oracle against golden vectors written from the reference's own CPU path.

The fixtures come from ``tests/golden/make_golden.py`` (reference
``came_pytorch/CAME8bitFull.py:1006-1075`` driven through ``CAME8bitFull``,
``CAME8bit`` and ``CAME8bitMemory`` on CPU tensors).  The oracle replays the
same inputs with the same torch thread count; agreement is required to be
bit-exact for parameters, int8/uint8 codes and fp32 absmax scales.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from oracle import came8_oracle as orc

DEFAULTS = dict(lr=None, eps=(1e-30, 1e-16), clip_threshold=1.0, betas=(0.9, 0.999, 0.9999),
                weight_decay=0.0, block_size=256)


def _hp(hp):
    h = dict(DEFAULTS)
    h.update(hp)
    b1, b2, b3 = h["betas"]
    return dict(beta1=b1, beta2=b2, beta3=b3, eps0=h["eps"][0], eps1=h["eps"][1], lr=h["lr"],
                clip_threshold=h["clip_threshold"], weight_decay=h["weight_decay"], block_size=h["block_size"])


def _to_torch(arr, dtype):
    t = torch.from_numpy(np.array(arr))
    if dtype == torch.bfloat16:
        t = t.view(torch.bfloat16)
    return t


def _as_np(t):
    t = t.detach()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.numpy()


@pytest.fixture(scope="module")
def small(golden_dir):
    z = np.load(os.path.join(golden_dir, "golden_small.npz"))
    meta = json.loads(str(z["meta_json"]))
    return z, meta


@pytest.fixture(autouse=True)
def _threads():
    old = torch.get_num_threads()
    torch.set_num_threads(4)
    yield
    torch.set_num_threads(old)


CASES = ["full_ragged_fp32", "came8bit_heavy_fp32", "memory_bf16", "full_zero_grads", "came8bit_bs64_clip"]


@pytest.mark.parametrize("case", CASES)
def test_oracle_matches_reference_bit_exact(small, case):
    z, meta = small
    m = meta[case]
    dtype = getattr(torch, m["dtype"])
    hp = _hp(m["hp"])
    shapes = [tuple(s) for s in m["shapes"]]
    params = [_to_torch(z[f"{case}/p0/{i}"], dtype).clone() for i in range(len(shapes))]
    states = [orc.init_full8bit_state(s, hp["block_size"]) for s in shapes]
    for step in range(1, m["steps"] + 1):
        for i in range(len(shapes)):
            g = _to_torch(z[f"{case}/g{step}/{i}"], dtype)
            orc.full8bit_step(params[i], g, states[i], **hp)
        if step in (1, m["steps"]):
            for i in range(len(shapes)):
                np.testing.assert_array_equal(_as_np(params[i]), z[f"{case}/p{step}/{i}"],
                                              err_msg=f"{case} step {step} param {i} {shapes[i]}")
                for k, v in states[i].items():
                    key = f"{case}/s{step}/{i}/{k}"
                    if isinstance(v, torch.Tensor) and key in z:
                        np.testing.assert_array_equal(_as_np(v), z[key], err_msg=key)
                assert int(z[f"{case}/s{step}/{i}/step"]) == states[i]["step"]


def test_oracle_c1_digest(golden_dir):
    """Config 1 (2048x2048 fp32 + 2048 bias, CAME8bit, 10 steps): every state tensor bit-identical."""
    z = np.load(os.path.join(golden_dir, "golden_c1_digest.npz"))
    digests = json.loads(str(z["c1/digests_json"]))
    gen = torch.Generator().manual_seed(0)
    w = torch.randn(2048, 2048, generator=gen) * 0.02
    b = torch.randn(2048, generator=gen) * 0.02
    params = [w, b]
    hp = _hp(dict(lr=2e-4, weight_decay=1e-2))
    states = [orc.init_full8bit_state(p.shape) for p in params]
    for step in range(1, 11):
        g2 = torch.Generator().manual_seed(1 + step)
        gw = torch.randn(2048, 2048, generator=g2) * 1e-3
        gb = torch.randn(2048, generator=g2) * 1e-3
        for p, g, st in zip(params, (gw, gb), states):
            orc.full8bit_step(p, g, st, **hp)
        if step in (1, 10):
            for i, (p, st) in enumerate(zip(params, states)):
                h = hashlib.sha256(p.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()
                assert h == digests[f"s{step}/p{i}"], f"param {i} step {step}"
                for k, v in st.items():
                    key = f"s{step}/p{i}/{k}"
                    if key in digests:
                        hv = hashlib.sha256(v.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()
                        assert hv == digests[key], key


CAMECUDA_CASES = ["cudafp_ragged_fp32", "cudafp_heavy_bf16", "cudafp_clip_fp32"]


@pytest.mark.parametrize("case", CAMECUDA_CASES)
def test_fp32_state_oracle_matches_reference_camecuda(golden_dir, case):
    """oracle.fp32_state_step against the reference's CAMECUDA on CPU tensors (its fp32-state
    _step_param_generic, CAMECUDA.py:275-326; golden_camecuda.npz from make_golden.py --camecuda):
    parameters and every fp32 state bit-exact after steps 1 and 10, ragged shapes, fp32 and bf16."""
    z = np.load(os.path.join(golden_dir, "golden_camecuda.npz"))
    m = json.loads(str(z["meta_json"]))[case]
    dtype = getattr(torch, m["dtype"])
    hp = _hp(m["hp"])
    hp.pop("block_size")
    shapes = [tuple(s) for s in m["shapes"]]
    params = [_to_torch(z[f"{case}/p0/{i}"], dtype).clone() for i in range(len(shapes))]
    states = [orc.init_fp32_state(s) for s in shapes]
    for step in range(1, m["steps"] + 1):
        for i in range(len(shapes)):
            g = _to_torch(z[f"{case}/g{step}/{i}"], dtype)
            orc.fp32_state_step(params[i], g, states[i], **hp)
        if step in (1, m["steps"]):
            for i in range(len(shapes)):
                np.testing.assert_array_equal(_as_np(params[i]), z[f"{case}/p{step}/{i}"],
                                              err_msg=f"{case} step {step} param {i} {shapes[i]}")
                n = 0
                for k, v in states[i].items():
                    key = f"{case}/s{step}/{i}/{k}"
                    if isinstance(v, torch.Tensor) and key in z:
                        np.testing.assert_array_equal(_as_np(v), z[key], err_msg=key)
                        n += 1
                assert n == (5 if states[i]["factored"] else 2), f"{case} {shapes[i]}: {n} states compared"
                assert int(z[f"{case}/s{step}/{i}/step"]) == states[i]["step"]
