"""The BASELINE workloads C2, C3 and C4 at full size on the GPU, in the library's default mode (the
reference's float32 clip norm).

  c2  GPT-2 Medium shapes, fp32, CAME8bit (292 tensors, 355 M parameters)
  c3  Llama-1B-style shapes, bf16, CAME8bitMemory, betas (0.9, 0.95, 0.995) (219 tensors, 1.34 G)
  c4  Llama-7B shapes, bf16, CAME8bit (291 tensors, 6.74 G): the headline workload

Each config takes bench.py's own construction (bench.CONFIGS: shapes, dtypes, hyperparameters and
gradient scale) and two steps over all its tensors in one optimizer, so every launch variant the
workload selects runs at its real size: the 32000 x 4096 embedding and lm_head bands, the 11008-wide
512-thread pass variants, the 5461-wide rows, the norm's LDS-staged and row-crossing segment kernels.
A representative subset is checked against the CPU oracle, teacher-forced (each checked tensor's
parameter and state are set from the oracle before each step), with the tolerances of
tests/test_gpu_parity.py.  Every tensor is held to what the blockwise quantiser fixes whatever the
values (a full-scale code in every block, or an all-zero block under absmax 1) and to finiteness.
"""
import math

import pytest
import torch

import bench
from oracle import came8_oracle as orc
from tests import parity as P
from tests.test_gpu_c5 import _block_full_scale
from tests.test_gpu_parity import _tight_step_check

pytestmark = pytest.mark.gpu

# the tensors checked against the oracle: the first occurrence of each named shape (and the last
# one for the 32000-row embedding / lm_head pair)
SUBSETS = {
    "c2": [(50257, 1024), (1024, 1024), (3072, 1024), (1024, 4096), (3072,), (1024,)],
    "c3": [(32000, 2048), (5461, 2048), (2048, 5461), (2048, 2048), (2048,)],
    "c4": [(32000, 4096), (11008, 4096), (4096, 11008), (4096, 4096), (4096,)],
}


def _subset(name, shapes):
    want = SUBSETS[name]
    idx = [shapes.index(s) for s in want]
    if name in ("c3", "c4"):  # the lm_head: the last 32000-row matrix
        idx.append(len(shapes) - 1 - shapes[::-1].index(want[0]))
    return sorted(set(idx))


def _f32_bits(v: float) -> int:
    return torch.tensor([v], dtype=torch.float32).view(torch.int32).item()


def _full_scale_checks(opt, ps, shapes, block):
    bad = []
    for i, (p, s) in enumerate(zip(ps, shapes)):
        st = opt.state[p]
        assert torch.isfinite(p.data).all(), f"tensor {i} {s}: non-finite parameter"
        assert torch.isfinite(st["exp_avg_absmax"]).all(), f"tensor {i} {s}: non-finite momentum scale"
        ok, n = _block_full_scale(st["exp_avg_q"], st["exp_avg_absmax"], block, 127)
        if not ok:
            bad.append((i, s, "exp_avg", n))
        pairs = ([("factored_row", 0), ("factored_row", 1), ("factored_col", 0), ("factored_col", 1)]
                 if st["factored"] else [("exp_avg_sq", None)])
        for key, j in pairs:
            q = st[f"{key}_q"] if j is None else st[f"{key}_q"][j]
            a = st[f"{key}_absmax"] if j is None else st[f"{key}_absmax"][j]
            assert torch.isfinite(a).all(), f"tensor {i} {s}: non-finite {key} scale"
            ok, n = _block_full_scale(q, a, block, 255)
            if not ok:
                bad.append((i, s, key, j, n))
    assert not bad, f"blocks without a full-scale code: {bad[:5]}"


@pytest.mark.parametrize("name", ["c2", "c3", "c4"])
def test_baseline_config_full_size_vs_oracle(name):
    import came_amd
    from came_amd import _lib
    _lib.load()
    label, shapes_fn, pdt, gdt, gstd, cls_name, hp = bench.CONFIGS[name]
    shapes = shapes_fn()
    stds = bench.grad_stds(gstd, len(shapes))  # c2: a per-tensor scale, log-uniform in [1e-5, 1e-2]
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(17)
    ps = [torch.nn.Parameter(torch.randn(s, device=dev, generator=gen).mul_(0.02).to(pdt)) for s in shapes]
    opt = getattr(came_amd, cls_name)(ps, **hp)
    assert not opt.exact_norm, "the default mode is the reference's float32 clip norm"
    chk = _subset(name, shapes)
    block = opt.param_groups[0]["block_size"]
    refs = {i: ps[i].detach().cpu().clone() for i in chk}
    sts = {i: orc.init_full8bit_state(shapes[i], block) for i in chk}
    ohp = P.oracle_hp(hp)
    check = _tight_step_check(f"{name} full size")
    n_el = sum(math.prod(s) for s in shapes)
    print(f"[{name}] {label}: {len(shapes)} tensors, {n_el} elements; checked {[shapes[i] for i in chk]}", flush=True)
    for step in range(2):
        grads = [torch.randn(s, device=dev, generator=gen).mul_(std).to(gdt) for s, std in zip(shapes, stds)]
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
        print(f"[{name}] step {step + 1}: GPU step over {len(shapes)} tensors done", flush=True)
        for i in chk:
            g = grads[i].cpu()
            before = refs[i].double()
            cap = {}
            orc.full8bit_step(refs[i], g, sts[i], capture=cap, **ohp)
            check(step + 1, i, ps[i].data, refs[i], opt.state[ps[i]], sts[i], (refs[i].double() - before).abs(), cap)
            # the clip divisor: the reference's float32 norm replayed; u itself may differ by an ulp
            # where the row / column means round differently, hence a few ulps (tests/test_gpu_norm.py)
            have, want = opt.last_clip_divisors()[ps[i]], float(cap["clip"])
            d = abs(_f32_bits(have) - _f32_bits(want))
            assert d <= 4, f"{name} step {step + 1} tensor {i}: clip {have!r} vs {want!r} ({d} ulps)"
        print(f"[{name}] step {step + 1}: {len(chk)} tensors match the oracle", flush=True)
        del grads
        _full_scale_checks(opt, ps, shapes, block)


# Free-running over 10 steps: the lm_head (32000 rows), the MLP matrices (11008 / 5461 wide and tall),
# a square attention matrix and a norm weight, free-running against the oracle from the same initial
# parameters while the GPU steps the whole workload.
FREE = {
    "c3": [(5461, 2048), (2048, 5461), (2048, 2048), (2048,)],
    "c4": [(11008, 4096), (4096, 11008), (4096, 4096), (4096,)],
}


def _bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """The bf16 spacing at |x| (x holds bf16 values), as float64."""
    a = x.abs().to(torch.bfloat16)
    return (torch.nextafter(a, torch.full_like(a, float("inf"))) - a).double()


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_baseline_config_free_running_ten_steps(name):
    """north_star's bar at the headline shapes, free-running: the GPU steps the whole workload 10 times
    and the oracle steps the checked tensors alongside from the same initial parameters.

    Step 1 (both sides start from the same state): every differing code one apart and at a rounding tie
    of the reference's value, parameters within 1 bf16 ulp (the teacher-forced bar).  Every step: at most
    2e-3 of the momentum codes apart, and every parameter's difference explained by the step itself --
    at most the difference carried from the step before (scaled by the weight decay), plus one bf16 ulp
    per rounding of the step (the weight decay's and the update's: torch's fp32 means and the fp64 means
    here can part u by an fp32 ulp, which flips a bf16 rounding now and then), plus 1e-5 relative, plus
    twice the drift that codes apart at earlier ties allow it (parity.DriftBound).  After 10 steps at
    least 99.99% of the parameters within 1 ulp of the oracle's, block scales as in the C1 free-running
    test."""
    import came_amd
    from came_amd import _lib
    _lib.load()
    label, shapes_fn, pdt, gdt, gstd, cls_name, hp = bench.CONFIGS[name]
    assert pdt == torch.bfloat16
    shapes = shapes_fn()
    stds = bench.grad_stds(gstd, len(shapes))
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev).manual_seed(29)
    ps = [torch.nn.Parameter(torch.randn(s, device=dev, generator=gen).mul_(0.02).to(pdt)) for s in shapes]
    opt = getattr(came_amd, cls_name)(ps, **hp)
    chk = sorted([shapes.index(s) for s in FREE[name]] + [len(shapes) - 1])  # + the lm_head
    ohp = P.oracle_hp(hp)
    decay = abs(1.0 - ohp["lr"] * ohp["weight_decay"])
    roundings = 2 if ohp["weight_decay"] else 1
    refs = {i: ps[i].detach().cpu().clone() for i in chk}
    sts = {i: orc.init_full8bit_state(shapes[i], ohp["block_size"]) for i in chk}
    bounds = {i: P.DriftBound(shapes[i], len(shapes[i]) >= 2, ohp) for i in chk}
    prev_d = {i: torch.zeros(shapes[i], dtype=torch.float64) for i in chk}
    prev_dp = {i: torch.zeros(shapes[i], dtype=torch.float64) for i in chk}
    prev_gp = {i: refs[i].clone() for i in chk}
    tight = _tight_step_check(f"{name} free step 1")
    print(f"[{name} free] {len(shapes)} tensors on the GPU; oracle alongside for {[shapes[i] for i in chk]}", flush=True)
    for step in range(1, 11):
        grads = [torch.randn(s, device=dev, generator=gen).mul_(std).to(gdt) for s, std in zip(shapes, stds)]
        for p, g in zip(ps, grads):
            p.grad = g
        opt.step()
        torch.cuda.synchronize()
        for i in chk:
            g = grads[i].cpu()
            before = refs[i].double()
            # the weight decay rounds at the magnitude before the step: its ulp can be twice the final one
            ulp_before = torch.maximum(_bf16_ulp(refs[i]), _bf16_ulp(prev_gp[i])) if step > 1 else _bf16_ulp(refs[i])
            cap = {}
            orc.full8bit_step(refs[i], g, sts[i], capture=cap, **ohp)
            mv = (refs[i].double() - before).abs()
            gst = opt.state[ps[i]]
            bounds[i].update(gst, sts[i], cap)
            where = f"{name} free-running step {step} tensor {i} {shapes[i]}"
            if step == 1:
                tight(step, i, ps[i].data, refs[i], gst, sts[i], mv, cap)
            # after step 1 the sides step from states that differ where codes came out one apart at ties;
            # such a difference is carried (beta1 * one code step) and can meet another tie, so codes may
            # part by more than one; the parameter bound accounts for the exact differences
            apart = {k: P.code_mismatch(gst[k], sts[i][k]) for k in P.STATE_KEYS if k in sts[i] and k.endswith("_q")}
            assert apart["exp_avg_q"][0] <= 2e-3, f"{where}: {apart['exp_avg_q'][0]:.3e} of the momentum codes differ"
            inc = bounds[i].D - prev_d[i] * decay  # this step's drift allowance
            prev_d[i] = bounds[i].D.clone()
            gp, rp = ps[i].data.cpu(), refs[i]
            dp = (gp.double() - rp.double()).abs()
            ulp = torch.maximum(_bf16_ulp(rp), _bf16_ulp(gp))
            rms = rp.double().pow(2).mean().sqrt().item()
            allow = (decay * prev_dp[i] + roundings * torch.maximum(ulp, ulp_before)
                     + 1e-5 * (rp.double().abs() + mv + 1e-2 * rms) + 2.0 * inc)
            bad = dp > allow
            if bool(bad.any()):
                k = int((dp - allow).argmax())
                raise AssertionError(
                    f"{where}: {int(bad.sum())} parameters beyond what the step explains; worst element {k}: "
                    f"gpu {gp.reshape(-1)[k].item()!r} ref {rp.reshape(-1)[k].item()!r} before {before.reshape(-1)[k].item()!r} "
                    f"|dp| {dp.reshape(-1)[k].item():.3e} carried {prev_dp[i].reshape(-1)[k].item():.3e} "
                    f"ulp {ulp.reshape(-1)[k].item():.3e}/{ulp_before.reshape(-1)[k].item():.3e} "
                    f"drift {inc.reshape(-1)[k].item():.3e} allowed {allow.reshape(-1)[k].item():.3e}")
            prev_dp[i] = dp
            prev_gp[i] = gp.clone()
            far = float((dp > ulp).double().mean())
            print(f"[{name} free] {where}: codes apart (fraction, max) {apart}; params beyond 1 ulp {far:.2e}",
                  flush=True)
        del grads
    for i in chk:
        where = f"{name} free-running 10 steps tensor {i} {shapes[i]}"
        far = float((prev_dp[i] > torch.maximum(_bf16_ulp(refs[i]), _bf16_ulp(ps[i].data.cpu()))).double().mean())
        assert far <= 1e-4, f"{where}: {far:.3e} of the parameters more than 1 ulp from the oracle's"
        ga, ra = opt.state[ps[i]]["exp_avg_absmax"].cpu().double(), sts[i]["exp_avg_absmax"].double()
        off = ((ga - ra).abs() / ra > 1e-5).double().mean().item()
        print(f"[{name} free] {where}: {far:.2e} of the parameters beyond 1 ulp; "
              f"{off:.2e} of the block scales beyond 1e-5", flush=True)
        assert off <= 1e-2, f"{where}: {off:.3e} of the block scales differ by more than 1e-5"
