"""came8_step_static (the entry point that allocates nothing; its workspace is a static array in the
library) against came8_step with a caller workspace: the same tensors stepped through each end bit for
bit identical, on two calls in a row, the second over a smaller tensor list.  Both optimizers' states are
created by prime_for_cuda_graph (no step), so they start alike."""
import ctypes

import pytest
import torch

import came_amd
from came_amd import _lib
from tests import parity as P

pytestmark = pytest.mark.gpu


def _static_step(opt, params):
    """One step of `opt` over `params` through came8_step_static (the C ABI), with the optimizer's own
    descriptors and hyper-parameters."""
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
def test_static_scratch_step_matches_workspace_step(dtype):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    shapes_1 = [(1024, 2048), (2048,), (3, 5, 7), (129, 4097), (33,)]
    shapes_2 = [(256, 512), (100,)]  # the second call: a smaller input
    gen = torch.Generator().manual_seed(11)
    for call, shapes in enumerate((shapes_1, shapes_2)):
        params0 = P.make_params(shapes, dtype, seed=20 + call)
        grads = [(torch.randn(s, generator=gen) * 1e-3).to(dtype).cuda() for s in shapes]
        pa = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
        pb = [torch.nn.Parameter(p.clone().cuda()) for p in params0]
        oa = came_amd.CAME8bit(pa, lr=2e-4, weight_decay=1e-2)
        ob = came_amd.CAME8bit(pb, lr=2e-4, weight_decay=1e-2)
        for p, q, g in zip(pa, pb, grads):
            p.grad = g
            q.grad = g.clone()
        oa.prime_for_cuda_graph()
        ob.prime_for_cuda_graph()
        for _ in range(2):  # two steps each, the second from the first's state
            oa.step()
            _static_step(ob, pb)
            torch.cuda.synchronize()
            for i, (a, b) in enumerate(zip(pa, pb)):
                where = f"call {call} tensor {i} {tuple(a.shape)}"
                assert torch.equal(a.data, b.data), f"{where}: parameters differ"
                for k, v in oa.state[a].items():
                    if isinstance(v, torch.Tensor):
                        assert torch.equal(v, ob.state[b][k]), f"{where}: state {k} differs"


def test_static_scratch_rejects_oversized_lists():
    """A tensor list whose workspace exceeds the static scratch fails with the library's message (and
    touches nothing); the rows of one matrix are doubled until the workspace the device sizes for it
    exceeds 32 MiB."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = _lib.load()
    rows = 4096
    while True:
        p = torch.nn.Parameter(torch.zeros(rows, 4096, device="cuda", dtype=torch.bfloat16))
        p.grad = torch.zeros_like(p)
        opt = came_amd.CAME8bit([p], lr=1e-3)
        opt.prime_for_cuda_graph()
        group = opt.param_groups[0]
        state, grad = opt._prepare_param(p, 256)
        descs, keep, _ = opt._descriptors([(p, state, grad)])
        need = ctypes.c_size_t(0)
        _lib.check(lib.came8_workspace_size(descs, 1, 256, ctypes.byref(need)), "came8_workspace_size")
        if need.value > (32 << 20) or rows >= 65536:
            break
        rows *= 2
    assert need.value > (32 << 20)
    before = p.data.clone()
    with pytest.raises(RuntimeError, match="static scratch holds"):
        _static_step(opt, [p])
    torch.cuda.synchronize()
    assert torch.equal(p.data, before)
