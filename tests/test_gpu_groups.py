"""Several param groups in one optimizer: each group is stepped by its own library call with its own
hyper-parameters and block size, and keeps a workspace (launch plan) of its own.  The result must
equal, bit for bit, separate single-group optimizers stepped with the same gradients."""
import pytest
import torch

import came_amd
from tests import parity as P

pytestmark = pytest.mark.gpu

DECAY = [(96, 200), (64, 2048), (3, 5, 7)]
NO_DECAY = [(200,), (2048,), (33, 130)]


@pytest.mark.parametrize("cls_name", ["CAME8bit", "CAME8bitFull", "CAMECUDA"])
def test_param_groups_step_like_separate_optimizers(cls_name):
    cls = getattr(came_amd, cls_name)
    dt = torch.bfloat16
    pa0 = P.make_params(DECAY, dt, seed=1)
    pb0 = P.make_params(NO_DECAY, dt, seed=2)
    ha = dict(lr=2e-4, weight_decay=1e-2, betas=(0.9, 0.999, 0.9999))
    hb = dict(lr=5e-4, weight_decay=0.0, betas=(0.8, 0.99, 0.999))
    if cls_name != "CAMECUDA":
        hb["block_size"] = 64
    gen = torch.Generator().manual_seed(3)
    steps = 4
    grads = [[(torch.randn(s, generator=gen) * 1e-3).to(dt).cuda() for s in DECAY + NO_DECAY] for _ in range(steps)]

    pa = [torch.nn.Parameter(p.clone().cuda()) for p in pa0]
    pb = [torch.nn.Parameter(p.clone().cuda()) for p in pb0]
    opt = cls([dict(params=pa, **ha), dict(params=pb, **hb)], lr=1e-3)
    sa = [torch.nn.Parameter(p.clone().cuda()) for p in pa0]
    sb = [torch.nn.Parameter(p.clone().cuda()) for p in pb0]
    oa, ob = cls(sa, **ha), cls(sb, **hb)
    for step in range(steps):
        for p, g in zip(pa + pb, grads[step]):
            p.grad = g
        for p, g in zip(sa + sb, grads[step]):
            p.grad = g
        opt.step()
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    assert len(opt._came8_workspaces) == 2
    for i, (a, b) in enumerate(zip(pa + pb, sa + sb)):
        where = f"{cls_name} tensor {i} {tuple(a.shape)}"
        assert torch.equal(a.data, b.data), f"{where}: parameters differ"
        st, su = opt.state[a], (oa if i < len(pa) else ob).state[b]
        for k, v in st.items():
            if isinstance(v, torch.Tensor):
                assert torch.equal(v, su[k]), f"{where}: state {k} differs"
