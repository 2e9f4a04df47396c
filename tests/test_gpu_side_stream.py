"""The side stream of a pass with many kernel launches: came8_step spreads a pass of four or more launches
(band variants of several row widths, the tiny-matrix and 1-D kernels) over the caller's stream and a side
stream, while came8_step_static keeps every launch on the caller's stream.  Both must step the same
tensors to the same bits, on two steps in a row and on a second, different tensor list."""
import ctypes

import pytest
import torch

import came_amd
from came_amd import _lib
from tests import parity as P

pytestmark = pytest.mark.gpu

# row widths that take different pass-1/pass-2 variants (4096-, 11008-, 5461-wide, ragged, one chunk),
# plus a tiny N-D tensor and 1-D tensors: at least four launches in passes 1 and 2
SHAPES = [(48, 4096), (20, 11008), (33, 5461), (40, 100), (64, 64), (3, 5, 7), (2048,), (17,)]
SHAPES_2 = [(16, 11008), (30, 2000), (5, 3, 3), (64, 128), (1000,)]


def _static_step(opt, params):
    group = opt.param_groups[0]
    items = []
    for p in params:
        state, grad = opt._prepare_param(p, opt._group_block_size(group))
        opt._count_step(state)
        items.append((p, state, grad))
    descs, keep, copyback = opt._descriptors(items)
    hp = opt._group_hparams(group)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.came8_step_static(descs, len(items), ctypes.byref(hp), stream), "came8_step_static")
    assert not copyback


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_side_stream_step_matches_one_stream(dtype):
    gen = torch.Generator().manual_seed(5)
    for call, shapes in enumerate((SHAPES, SHAPES_2)):
        params0 = P.make_params(shapes, dtype, seed=30 + call)
        pa = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
        pb = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
        oa = came_amd.CAME8bit(pa, lr=2e-4, weight_decay=1e-2)
        ob = came_amd.CAME8bit(pb, lr=2e-4, weight_decay=1e-2)
        for step in range(2):
            grads = [P.heavy_grad(gen, s, dtype).cuda() for s in shapes]
            for p, q, g in zip(pa, pb, grads):
                p.grad = g
                q.grad = g.clone()
            if step == 0:
                oa.prime_for_cuda_graph()
                ob.prime_for_cuda_graph()
            oa.step()
            _static_step(ob, pb)
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(pa, pb)):
                where = f"call {call} step {step + 1} tensor {i} {tuple(a.shape)}"
                assert torch.equal(a.data, b.data), f"{where}: parameters differ"
                for k, v in oa.state[a].items():
                    if torch.is_tensor(v):
                        assert torch.equal(v, ob.state[b][k]), f"{where}: state {k} differs"


def test_side_streams_are_bounded_across_caller_streams():
    """A caller stepping on many streams in turn: at most 16 idle side streams are kept (the least recently
    used released after its work completes), and every step still matches the one-stream static entry."""
    lib = _lib.load()
    params0 = P.make_params(SHAPES, torch.float32, seed=77)
    pa = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
    pb = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
    oa = came_amd.CAME8bit(pa, lr=2e-4, weight_decay=1e-2)
    ob = came_amd.CAME8bit(pb, lr=2e-4, weight_decay=1e-2)
    gen = torch.Generator().manual_seed(79)
    streams = [torch.cuda.Stream() for _ in range(40)]  # default priority
    most = 0
    for k, s in enumerate(streams):
        grads = [P.heavy_grad(gen, sh, torch.float32).cuda() for sh in SHAPES]
        for p, q, g in zip(pa, pb, grads):
            p.grad = g
            q.grad = g.clone()
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            oa.step()
        s.synchronize()
        _static_step(ob, pb)
        torch.cuda.synchronize()
        most = max(most, lib.came8_side_stream_count())
        for i, (a, b) in enumerate(zip(pa, pb)):
            assert torch.equal(a.data, b.data), f"stream {k} tensor {i}: parameters differ"
    assert lib.came8_side_stream_count() <= 16, lib.came8_side_stream_count()
    assert most <= 17, most  # the 16 idle ones and at most the one a step was using


# The long-chain group: a matrix whose clip-norm chain is at least 8192 segments of 4096 elements and
# more than twice as long as the others', holding at most 60% of the factored elements.  An eager
# came8_step walks it, takes its clip and runs its pass 2 on the side stream while the other tensors do
# the same on the caller's stream; under graph capture everything stays on one stream in pass order.
LONG_SHAPES = [(8200, 4096), (2048, 4096), (1000, 11008), (2048, 4096), (4096,), (3, 5, 7)]


def test_long_chain_group_matches_one_stream():
    dtype = torch.bfloat16
    params0 = P.make_params(LONG_SHAPES, dtype, seed=41)
    gen = torch.Generator(device="cuda").manual_seed(43)
    hp = dict(lr=2e-4, weight_decay=1e-2)
    pe = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
    pg = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
    oe = came_amd.CAME8bit(pe, **hp)
    og = came_amd.CAME8bit(pg, **hp)
    static = [torch.zeros_like(p) for p in pg]
    for p, g in zip(pg, static):
        p.grad = g
    og.prime_for_cuda_graph()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        og.step()
    torch.cuda.synchronize()
    for step in range(3):
        grads = [(torch.randn(s, generator=gen, device="cuda") * 1e-3).to(dtype) for s in LONG_SHAPES]
        for p, sg, g in zip(pe, static, grads):
            p.grad = g
            sg.copy_(g)
        oe.step()
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pe, pg)):
            where = f"step {step + 1} tensor {i} {tuple(a.shape)}"
            assert torch.equal(a.data, b.data), f"{where}: parameters differ"
            for k, v in oe.state[a].items():
                if torch.is_tensor(v):
                    assert torch.equal(v, og.state[b][k]), f"{where}: state {k} differs"
