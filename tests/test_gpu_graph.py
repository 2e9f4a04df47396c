"""The step under HIP graph capture (the reference's `prime_for_cuda_graph` / `cuda_graph_compatible`,
CAME8bit.py:672-693, CAME8bit2D.py:52-72): once a first eager step has created the states, the
workspace and its uploaded launch plan, `came8_step` issues kernel launches only (no allocation, no
copy, no memset, no host synchronisation), so `opt.step()` can be captured and replayed.

Each replay is checked bit for bit against an eager optimizer stepped with the same gradients, with
the program's own eager work (gradient copies, the eager step, a synchronisation) between replays.
"""
import pytest
import torch

import came_amd
from tests import parity as P
from tests import test_gpu_8bit2d as T2

pytestmark = pytest.mark.gpu

SHAPES = [(96, 200), (200,), (3, 5, 7), (64, 2048), (20, 8, 1, 1)]


def _keys(state):
    """The state tensors the step writes (the 8bit2d layout also keeps the reference's scratch
    tensors, allocated uninitialised and left unwritten here)."""
    if state.get("_mode") == "8bit2d":
        return list(T2.PERSIST)
    return sorted(k for k, v in state.items() if isinstance(v, torch.Tensor))


@pytest.mark.parametrize("cls_name,dtype", [("CAME8bit", torch.bfloat16), ("CAME8bitFull", torch.float32),
                                            ("CAME8bit2D", torch.bfloat16), ("CAMECUDA", torch.bfloat16)])
def test_captured_step_replays_like_eager(cls_name, dtype):
    shapes = [s for s in SHAPES if len(s) == 2] if cls_name == "CAME8bit2D" else SHAPES
    cls = getattr(came_amd, cls_name)
    params0 = P.make_params(shapes, dtype, seed=3)
    gen = torch.Generator().manual_seed(4)
    steps = 5
    grads = [[(torch.randn(s, generator=gen) * 1e-3).to(dtype).cuda() for s in shapes] for _ in range(steps)]
    hp = dict(lr=2e-4, weight_decay=1e-2)

    pe = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
    oe = cls(pe, **hp)
    pg = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
    og = cls(pg, **hp)
    static = [torch.zeros_like(p) for p in pg]
    for p, g in zip(pg, static):
        p.grad = g

    # first step eagerly on both: states, workspace and launch plan
    for p, g in zip(pe, grads[0]):
        p.grad = g
    oe.step()
    for sg, g in zip(static, grads[0]):
        sg.copy_(g)
    og.step()
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        og.step()
    torch.cuda.synchronize()

    for step in range(1, steps):
        for p, g in zip(pe, grads[step]):
            p.grad = g
        oe.step()
        for sg, g in zip(static, grads[step]):
            sg.copy_(g)
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pe, pg)):
            where = f"{cls_name} replay {step} tensor {i} {tuple(a.shape)}"
            assert torch.equal(a.data, b.data), f"{where}: parameters differ"
            sa, sb = oe.state[a], og.state[b]
            for k in _keys(sa):
                assert torch.equal(sa[k], sb[k]), f"{where}: state {k} differs"


@pytest.mark.parametrize("cls_name,dtype", [("CAME8bit", torch.bfloat16), ("CAME8bit2D", torch.bfloat16)])
def test_primed_capture_without_eager_step(cls_name, dtype):
    """prime_for_cuda_graph creates the states and uploads the launch plan, so the very first step can
    be captured: its replays equal an eager optimizer's steps bit for bit."""
    shapes = [s for s in SHAPES if len(s) == 2] if cls_name == "CAME8bit2D" else SHAPES
    cls = getattr(came_amd, cls_name)
    params0 = P.make_params(shapes, dtype, seed=5)
    gen = torch.Generator().manual_seed(6)
    steps = 4
    grads = [[(torch.randn(s, generator=gen) * 1e-3).to(dtype).cuda() for s in shapes] for _ in range(steps)]
    hp = dict(lr=2e-4, weight_decay=1e-2)
    pe = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
    oe = cls(pe, **hp)
    pg = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
    og = cls(pg, **hp)
    static = [torch.zeros_like(p) for p in pg]
    for p, g in zip(pg, static):
        p.grad = g
    og.prime_for_cuda_graph()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        og.step()
    torch.cuda.synchronize()
    for step in range(steps):
        for p, g in zip(pe, grads[step]):
            p.grad = g
        oe.step()
        for sg, g in zip(static, grads[step]):
            sg.copy_(g)
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pe, pg)):
            where = f"{cls_name} primed replay {step} tensor {i} {tuple(a.shape)}"
            assert torch.equal(a.data, b.data), f"{where}: parameters differ"
            for k in _keys(oe.state[a]):
                assert torch.equal(oe.state[a][k], og.state[b][k]), f"{where}: state {k} differs"


def test_capture_without_plan_fails_cleanly():
    """A capture that would have to build the launch plan (no eager step, no priming) fails with the
    library's message instead of recording a host-to-device copy into the graph.  (States created
    inside a capture would be filled by captured kernels that never run: they are created first.)"""
    shapes = [(64, 96), (96,)]
    ps = [torch.nn.Parameter(p.cuda()) for p in P.make_params(shapes, torch.float32, seed=8)]
    opt = came_amd.CAME8bit(ps, lr=1e-3)
    for p in ps:
        p.grad = torch.randn_like(p) * 1e-3
        opt._prepare_param(p, 256)  # the states exist (created and filled outside the capture); the plan does not
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError):
        with torch.cuda.graph(graph):
            opt.step()
    torch.cuda.synchronize()
    # the optimizer and the device are usable afterwards
    opt.step()
    torch.cuda.synchronize()
    assert all(torch.isfinite(p).all() for p in ps)
