"""GPU: the reference's fp16-update variant for unfactored tensors (CAME8_FLAG_FP16_UPDATE;
came_pytorch/came_cuda/csrc/came_kernels.cu:1068-1122,1546-1601, selected by
CAME8bitFull(cuda_nonfactored_use_fp16_update=True), CAME8bit's repeated_fp16_pairmin mode, and always
by the reference's CUDA CAME8bitMemory for 1-D tensors, CAME8bitMemory.py:524-557).

  * Against the oracle's fp16_update branch, teacher-forced over three steps, with the tolerances of
    tests/test_gpu_parity.py: 1-D tensors of ragged lengths, fp32 and bf16, block sizes 256 (vector
    passes) and 100 (the per-block pass), heavy-tailed gradients.
  * Lossy by a stated amount against the fp32 update: from the same state, a step moves each
    element's momentum by (1 - beta1) * u / clip with u rounded to fp16 instead, so the parameters
    of the two variants part by at most lr * (1 - beta1) * |u / clip| * 2^-11 (half an fp16 ulp,
    relative) plus the usual 1e-5 relative.
  * Matrices are unaffected: with the flag set they step bit for bit as without it.
  * CAME8bit chooses per tensor, as the reference routes each 1-D tensor (CAME8_TENSOR_FP16_UPDATE):
    seven kwarg combinations over one tensor set that exercises every route.
"""
import pytest
import torch

import came_amd
from oracle import came8_oracle as orc
from tests import parity as P
from tests.test_gpu_parity import _tight_step_check

pytestmark = pytest.mark.gpu

SHAPES = [(1,), (3,), (255,), (256,), (4097,), (100003,), (2048,)]


def _run(dtype, block, steps=3):
    dt = getattr(torch, dtype)
    params = P.make_params(SHAPES, dt, seed=71 + block)
    gen = torch.Generator().manual_seed(73 + block)
    grads = [[P.heavy_grad(gen, s, dt) for s in SHAPES] for _ in range(steps)]
    hp = dict(lr=1e-3, weight_decay=1e-2, block_size=block)
    ohp = P.oracle_hp(hp)
    ps = [torch.nn.Parameter(p.clone().cuda()) for p in params]
    opt = came_amd.CAME8bitFull(ps, cuda_nonfactored_use_fp16_update=True, **hp)
    refs = [p.clone() for p in params]
    sts = [orc.init_full8bit_state(p.shape, block) for p in refs]
    check = _tight_step_check(f"fp16 update {dtype} B={block}", block=block)
    for s in range(steps):
        with torch.no_grad():
            for p, r, st in zip(ps, refs, sts):
                p.data.copy_(r.cuda())
                gst = opt.state[p]
                for k in P.STATE_KEYS:
                    if len(gst) and k in st:
                        gst[k].copy_(st[k].cuda())
        for p, g in zip(ps, grads[s]):
            p.grad = g.cuda()
        opt.step()
        torch.cuda.synchronize()
        for i, (r, g, st) in enumerate(zip(refs, grads[s], sts)):
            before = r.double()
            cap = {}
            orc.full8bit_step(r, g, st, capture=cap, fp16_update=True, **ohp)
            check(s + 1, i, ps[i].data, r, opt.state[ps[i]], st, (r.double() - before).abs(), cap)


@pytest.mark.parametrize("block", [256, 100])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_fp16_update_vs_oracle(dtype, block):
    _run(dtype, block)


def test_fp16_update_is_lossy_by_half_an_fp16_ulp():
    params = P.make_params(SHAPES, torch.float32, seed=81)
    gen = torch.Generator().manual_seed(83)
    grads = [P.heavy_grad(gen, s, torch.float32) for s in SHAPES]
    hp = dict(lr=1e-3, weight_decay=1e-2)
    ohp = P.oracle_hp(hp)
    out = {}
    for fp16 in (False, True):
        ps = [torch.nn.Parameter(p.clone().cuda()) for p in params]
        opt = came_amd.CAME8bitFull(ps, cuda_nonfactored_use_fp16_update=fp16, **hp)
        for p, g in zip(ps, grads):
            p.grad = g.cuda()
        opt.step()
        torch.cuda.synchronize()
        out[fp16] = [p.data.cpu() for p in ps]
    for i, (p0, g) in enumerate(zip(params, grads)):
        cap = {}
        orc.full8bit_step(p0.clone(), g, orc.init_full8bit_state(p0.shape), capture=cap, **ohp)
        u = cap["update"].double().abs()  # u / clip of the fp32 variant
        allow = hp["lr"] * (1 - ohp["beta1"]) * u * 2.0 ** -11 + 1e-5 * (p0.double().abs() + 1e-2)
        d = (out[True][i].double() - out[False][i].double()).abs()
        assert bool((d <= allow).all()), f"tensor {i} {SHAPES[i]}: the variants part by {d.max().item():.3e}"
        if p0.numel() >= 256:  # the rounding is visible: some elements differ
            assert bool((d > 0).any()), f"tensor {i} {SHAPES[i]}: the fp16 update changed nothing"


def test_fp16_update_leaves_matrices_alone():
    shapes = [(64, 2048), (33, 5461), (3, 40, 96)]
    params = P.make_params(shapes, torch.bfloat16, seed=91)
    gen = torch.Generator().manual_seed(93)
    grads = [P.heavy_grad(gen, s, torch.bfloat16) for s in shapes]
    out = {}
    for fp16 in (False, True):
        ps = [torch.nn.Parameter(p.clone().cuda()) for p in params]
        opt = came_amd.CAME8bitFull(ps, lr=1e-3, weight_decay=1e-2, cuda_nonfactored_use_fp16_update=fp16)
        for _ in range(2):
            for p, g in zip(ps, grads):
                p.grad = g.cuda()
            opt.step()
        torch.cuda.synchronize()
        out[fp16] = ([p.data.cpu() for p in ps], [opt.state[p]["exp_avg_q"].cpu() for p in ps])
    for a, b in zip(out[False][0] + out[False][1], out[True][0] + out[True][1]):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b)


# ------------------------------------------------------------------ CAME8bit's per-tensor selection
# The reference's CAME8bit takes the fp16-update kernels for a 1-D tensor only on some of its routes
# (CAME8bit.py:224-245, 441-529, 712-891); which ones depends on the kwargs and on the tensor's bucket
# (device, dtype, length) within the group.  Tensors: a bucket of five 2048-long vectors (batched range
# [1024, 65536], bucket >= 4), a bucket of two 4096-long ones (below the minimum bucket), lengths outside the
# range (512, 100003), a non-contiguous gradient (the reference's generic path) and a matrix.
SEL_SHAPES = [(2048,)] * 5 + [(4096,)] * 2 + [(512,), (100003,), (3000,), (64, 96)]
NONCONTIG = 9  # index of the tensor whose gradient is a strided view
SEL_CASES = {
    "default": ({}, [False] * 11),
    "batched_fp16_alone": ({"cuda_1d_batched_use_fp16_update": True}, [False] * 11),
    "batched_no_multitensor": ({"prefer_cuda_1d_batched_fast_path": True, "cuda_1d_batched_use_fp16_update": True},
                               [False] * 11),
    "multitensor_fp16": ({"prefer_cuda_1d_batched_fast_path": True, "prefer_cuda_1d_multitensor_fast_path": True,
                          "cuda_1d_batched_use_fp16_update": True}, [True] * 5 + [False] * 6),
    "nonfactored_fp16": ({"cuda_nonfactored_use_fp16_update": True}, [True] * 9 + [False, False]),
    "multitensor_fp32_rest_fp16": ({"prefer_cuda_1d_batched_fast_path": True,
                                    "prefer_cuda_1d_multitensor_fast_path": True,
                                    "cuda_nonfactored_use_fp16_update": True}, [False] * 5 + [True] * 4 + [False] * 2),
    "repeated_fp16_pairmin": ({"cuda_1d_runtime_mode": "repeated_fp16_pairmin"}, [True] * 9 + [False, False]),
}


@pytest.mark.filterwarnings("ignore::RuntimeWarning")
@pytest.mark.parametrize("case", sorted(SEL_CASES))
def test_came8bit_fp16_update_selection_per_tensor(case):
    kw, want = SEL_CASES[case]
    params = P.make_params(SEL_SHAPES, torch.float32, seed=101)
    gen = torch.Generator().manual_seed(103)
    grads = [P.heavy_grad(gen, s, torch.float32) for s in SEL_SHAPES]
    hp = dict(lr=1e-3, weight_decay=1e-2)
    ohp = P.oracle_hp(hp)
    ps = [torch.nn.Parameter(p.clone().cuda()) for p in params]
    opt = came_amd.CAME8bit(ps, **hp, **kw)
    for i, (p, g) in enumerate(zip(ps, grads)):
        if i == NONCONTIG:
            wide = torch.zeros(2 * g.numel(), device="cuda")
            wide[::2] = g.cuda()
            p.grad = wide[::2]
            assert not p.grad.is_contiguous()
        else:
            p.grad = g.cuda()
    opt.step()
    torch.cuda.synchronize()
    check = _tight_step_check(f"CAME8bit {case}")
    for i, (p0, g) in enumerate(zip(params, grads)):
        outs = {}
        for fp16 in (False, True):
            r, st, cap = p0.clone(), orc.init_full8bit_state(p0.shape), {}
            orc.full8bit_step(r, g, st, capture=cap, fp16_update=fp16, **ohp)
            outs[fp16] = (r, st, cap)
        r, st, cap = outs[want[i]]
        check(1, i, ps[i].data, r, opt.state[ps[i]], st, (r.double() - p0.double()).abs(), cap)
        if p0.dim() == 1 and p0.numel() >= 2048:  # the choice is visible: nearer the expected variant
            gp = ps[i].data.cpu().double()
            d_want = (gp - outs[want[i]][0].double()).abs().max().item()
            d_other = (gp - outs[not want[i]][0].double()).abs().max().item()
            assert d_want < d_other, f"{case} tensor {i} {SEL_SHAPES[i]}: fp16 update {not want[i]} fits better"
