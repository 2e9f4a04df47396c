"""The ragged stress configuration (c5) at full size on the GPU: 500 tensors
(bench.ragged_shapes: 1-D lengths 1..4097, 1000x3, 3x50257, 4097x129, conv weights 320x320x3x3 and
1280x640x1x1, 245 matrices up to 5000x5000 with no dimension a multiple of 64; 1.52 G elements),
heavy-tailed gradients with 10% exact zeros and +-1e3 outliers (bench.heavy_grad), stepped by
CAME8bitFull in one multi-tensor launch per phase.

Two steps over all 500 tensors.  Checked against the CPU oracle, teacher-forced (each checked
tensor's parameter and state are set from the oracle before the step), with the tolerances of
tests/test_gpu_parity.py: every 1-D tensor, the named 2-D and conv shapes, and the smallest random
matrices, bounded to what the oracle steps in seconds.  Every tensor, checked or not, is held to
what the blockwise quantiser fixes whatever the values: in each block the largest code magnitude is
the full scale (127 signed, 255 unsigned) -- its element divided by the block's absmax is exactly
1 -- or the block is all zero codes under absmax 1, and every state and parameter is finite.
"""
import math

import pytest
import torch

import bench
from oracle import came8_oracle as orc
from tests import parity as P
from tests.test_gpu_parity import _tight_step_check

pytestmark = pytest.mark.gpu

HP = dict(lr=2e-4, weight_decay=1e-2)
N_RANDOM_CHECKED = 8


def _checked(shapes):
    fixed = {(1000, 3), (3, 50257), (4097, 129), (320, 320, 3, 3), (1280, 640, 1, 1)}
    idx = [i for i, s in enumerate(shapes) if len(s) == 1 or s in fixed]
    rand2d = sorted((i for i, s in enumerate(shapes) if len(s) == 2 and s not in fixed),
                    key=lambda i: math.prod(shapes[i]))
    return sorted(idx + rand2d[:N_RANDOM_CHECKED])


def _block_full_scale(q, absmax, B, qmax):
    """Per block: max |code| is qmax, or the block holds only zero codes and its absmax is 1."""
    flat = q.reshape(-1).to(torch.int32).abs()
    nb = absmax.numel()
    pad = torch.zeros(nb * B, dtype=torch.int32, device=flat.device)
    pad[: flat.numel()] = flat
    mx = pad.view(nb, B).amax(1)
    ok = (mx == qmax) | ((mx == 0) & (absmax.reshape(-1) == 1.0))
    return bool(ok.all()), int((~ok).sum())


def test_ragged_500_full_size_vs_oracle():
    import came_amd
    from came_amd import _lib
    _lib.load()
    shapes = bench.ragged_shapes()
    assert len(shapes) == 500
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(5)
    ps = [torch.nn.Parameter(torch.randn(s, device=dev, generator=gen).mul_(0.02)) for s in shapes]
    opt = came_amd.CAME8bitFull(ps, **HP)
    chk = _checked(shapes)
    refs = {i: ps[i].detach().cpu().clone() for i in chk}
    sts = {i: orc.init_full8bit_state(shapes[i], 256) for i in chk}
    ohp = P.oracle_hp(HP)
    check = _tight_step_check("C5 full size")
    for step in range(2):
        grads = [bench.heavy_grad(s, gen, torch.float32, device=dev) for s in shapes]
        with torch.no_grad():
            for i in chk:
                ps[i].data.copy_(refs[i].to(dev))
                gst = opt.state[ps[i]]
                for k in P.STATE_KEYS:
                    if len(gst) and k in sts[i]:
                        gst[k].copy_(sts[i][k].to(dev))
        for p, g in zip(ps, grads):
            p.grad = g
        opt.step()
        torch.cuda.synchronize()
        print(f"[c5] step {step + 1}: GPU step over {len(shapes)} tensors done; oracle on {len(chk)}", flush=True)
        for i in chk:
            g = grads[i].cpu()
            before = refs[i].double()
            cap = {}
            orc.full8bit_step(refs[i], g, sts[i], capture=cap, exact_norm=False, **ohp)
            check(step + 1, i, ps[i].data, refs[i], opt.state[ps[i]], sts[i], (refs[i].double() - before).abs(), cap)
        # what the quantiser fixes, on every tensor
        bad = []
        for i, (p, s) in enumerate(zip(ps, shapes)):
            st = opt.state[p]
            assert torch.isfinite(p.data).all(), f"tensor {i} {s}: non-finite parameter"
            ok, n = _block_full_scale(st["exp_avg_q"], st["exp_avg_absmax"], 256, 127)
            if not ok:
                bad.append((i, s, "exp_avg", n))
            pairs = ([("factored_row", 0), ("factored_row", 1), ("factored_col", 0), ("factored_col", 1)]
                     if st["factored"] else [("exp_avg_sq", None)])
            for key, j in pairs:
                q = st[f"{key}_q"] if j is None else st[f"{key}_q"][j]
                a = st[f"{key}_absmax"] if j is None else st[f"{key}_absmax"][j]
                assert torch.isfinite(a).all(), f"tensor {i} {s}: non-finite {key} scale"
                ok, n = _block_full_scale(q, a, 256, 255)
                if not ok:
                    bad.append((i, s, key, j, n))
        assert not bad, f"blocks without a full-scale code: {bad[:5]}"
