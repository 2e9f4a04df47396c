"""Checkpoints across state layouts on the GPU: a state dict saved in one of the reference's layouts
loads into an optimizer that keeps another (came_amd.state_layout), and the next step from the
converted state matches the CPU oracle stepped from the same converted state.

Tolerances: those of the parity tests (tests/parity.py for full8bit, tests/test_gpu_8bit2d.py for
8bit2d); the conversion itself is checked to within half a quantisation step of the target blocks.
"""
import math

import pytest
import torch

import came_amd
from came_amd import state_layout as SL
from oracle import came8_oracle as orc
from tests import parity as P
from tests import test_gpu_8bit2d as T2

pytestmark = pytest.mark.gpu

HP = dict(lr=1e-3, weight_decay=1e-2)
Q8_KEYS = ("exp_avg_q", "exp_avg_absmax", "factored_row_q", "factored_row_absmax", "factored_col_q",
           "factored_col_absmax")


def _params(shapes, dt, seed):
    return [torch.nn.Parameter(t.cuda()) for t in P.make_params(shapes, dt, seed)]


def _grads(shapes, dt, seed):
    gen = torch.Generator().manual_seed(seed)
    return [P.heavy_grad(gen, s, dt) for s in shapes]


def _run(opt, ps, grads):
    for p, g in zip(ps, grads):
        p.grad = g.cuda()
    opt.step()
    torch.cuda.synchronize()


def _cpu_state(st: dict) -> dict:
    return {k: (v.detach().cpu().clone() if isinstance(v, torch.Tensor) else v) for k, v in st.items()}


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_8bit2d_checkpoint_loads_into_came8bit(dtype):
    dt = getattr(torch, dtype)
    shapes = [(40, 300), (64, 128), (17, 33)]
    src = _params(shapes, dt, seed=1)
    opt = came_amd.CAME8bit2D(src, **HP)
    for s in range(3):
        _run(opt, src, _grads(shapes, dt, 10 + s))
    sd = opt.state_dict()
    ps = [torch.nn.Parameter(p.detach().clone()) for p in src]
    opt2 = came_amd.CAME8bit(ps, **HP)
    opt2.load_state_dict(sd)
    for i, (p, q) in enumerate(zip(src, ps)):
        st2d, st = opt.state[p], opt2.state[q]
        assert st["_mode"] == "full8bit" and st["factored"] and st["step"] == 0
        for k in Q8_KEYS:
            assert st[k].is_cuda and st[k].dtype in (torch.int8, torch.uint8, torch.float32), k
        # row/column states carried code for code; the momentum within half a step of its new blocks
        assert torch.equal(st["factored_row_q"][1], st2d["exp_avg_res_row_q"])
        assert torch.equal(st["factored_col_q"][0], st2d["exp_avg_sq_col_q"])
        m2d = SL.state_values(_cpu_state(st2d), shapes[i])["exp_avg"]
        mf = orc.dequantize_blockwise(st["exp_avg_q"].cpu(), st["exp_avg_absmax"].cpu(), signed=True, block_size=256)
        half = st["exp_avg_absmax"].cpu().repeat_interleave(256)[: m2d.numel()].reshape(m2d.shape) / 127 / 2
        assert ((mf - m2d).abs() <= half * 1.0001).all()
    # the next step from the converted state, against the oracle stepped from the same state
    refs = [_cpu_state({"p": q.data})["p"] for q in ps]
    sts = [_cpu_state(opt2.state[q]) for q in ps]
    grads = _grads(shapes, dt, 20)
    _run(opt2, ps, grads)
    for i, (q, r, g, st) in enumerate(zip(ps, refs, grads, sts)):
        st["step"] = 0
        cap = {}
        before = r.double()
        orc.full8bit_step(r, g, st, capture=cap, **P.oracle_hp(HP))
        where = f"8bit2d->full8bit {dtype} tensor {i} {shapes[i]}"
        P.compare_states(opt2.state[q], st, code_frac=1.5e-2, abs_rel=1e-6, where=where, ref_fp32=cap, tie_tol=2e-4)
        tainted = opt2.state[q]["exp_avg_q"].cpu() != st["exp_avg_q"]
        P.check_untainted_params(q.data, r, tainted, where, (r.double() - before).abs())


def test_came8bit_checkpoint_loads_into_came8bit2d():
    dt = torch.float32
    shapes = [(40, 300), (33, 64)]
    src = _params(shapes, dt, seed=2)
    opt = came_amd.CAME8bit(src, **HP)
    for s in range(3):
        _run(opt, src, _grads(shapes, dt, 30 + s))
    sd = opt.state_dict()
    ps = [torch.nn.Parameter(p.detach().clone()) for p in src]
    opt2 = came_amd.CAME8bit2D(ps, **HP)
    opt2.load_state_dict(sd)
    for p, q, s in zip(src, ps, shapes):
        st = opt2.state[q]
        assert st["_mode"] == "8bit2d" and "step" not in st and st["rows"] == s[0]
        assert torch.equal(st["exp_avg_sq_row_q"], opt.state[p]["factored_row_q"][0])
        assert st["res_col_partial"].numel() == math.ceil(s[0] / 16) * s[1]
    refs = [q.data.detach().cpu().clone() for q in ps]
    sts = []
    for q, s in zip(ps, shapes):
        st = orc.init_8bit2d_state(s)
        for k in T2.PERSIST:
            st[k] = opt2.state[q][k].detach().cpu().clone()
        sts.append(st)
    grads = _grads(shapes, dt, 40)
    _run(opt2, ps, grads)
    for i, (q, r, g, st) in enumerate(zip(ps, refs, grads, sts)):
        cap = {}
        before = r.double()
        orc.came8bit2d_step(r, g, st, capture=cap, **P.oracle_hp(HP))
        where = f"full8bit->8bit2d tensor {i} {shapes[i]}"
        T2._compare(opt2.state[q], st, cap, where)
        tainted = opt2.state[q]["exp_avg_q"].cpu() != st["exp_avg_q"]
        P.check_untainted_params(q.data, r, tainted, where, (r.double() - before).abs())


def test_without_conversion_a_foreign_state_resets_as_in_the_reference():
    """CAME8bit.py:757-759: a state of another _mode is cleared and initialised again by the next step."""
    dt = torch.float32
    shapes = [(40, 300)]
    src = _params(shapes, dt, seed=3)
    opt = came_amd.CAME8bit2D(src, **HP)
    _run(opt, src, _grads(shapes, dt, 50))
    sd = opt.state_dict()
    a = [torch.nn.Parameter(p.detach().clone()) for p in src]
    b = [torch.nn.Parameter(p.detach().clone()) for p in src]
    oa = came_amd.CAME8bit(a, **HP)
    oa.load_state_dict(sd, convert_layouts=False)
    assert oa.state[a[0]]["_mode"] == "8bit2d"
    ob = came_amd.CAME8bit(b, **HP)
    g = _grads(shapes, dt, 51)
    _run(oa, a, g)
    _run(ob, b, g)
    assert torch.equal(a[0].data, b[0].data)
    for k in Q8_KEYS:
        assert torch.equal(oa.state[a[0]][k], ob.state[b[0]][k]), k
    assert oa.state[a[0]]["step"] == 1


def _nd_checkpoint(shape, B, seed):
    """A state dict as the reference's CUDA N-D path leaves it (CAME8bitFull.py:790-829): per-matrix
    blocks, (2*prefix, n) row/column batches, its flags and shape keys."""
    P_, R, C = math.prod(shape[:-2]), shape[-2], shape[-1]
    gen = torch.Generator().manual_seed(seed)
    m = torch.randn(shape, generator=gen) * 1e-3
    rows = torch.rand((2 * P_, R), generator=gen) + 0.5
    cols = torch.rand((2 * P_, C), generator=gen) + 0.5
    qs, am = zip(*(orc.quantize_blockwise(m.reshape(P_, R * C)[i], signed=True, block_size=B) for i in range(P_)))
    rq, ra = zip(*(orc.quantize_blockwise(rows[i], signed=False, block_size=B) for i in range(2 * P_)))
    cq, ca = zip(*(orc.quantize_blockwise(cols[i], signed=False, block_size=B) for i in range(2 * P_)))
    st = {"step": 5, "_mode": "full8bit", "RMS": 0, "factored": True, "_cuda_factored_nd_ext_path": True,
          "_cuda_factored_nd_chunked_ext_path": False, "prefix_batch": P_, "matrix_rows": R, "matrix_cols": C,
          "exp_avg_q": torch.stack(qs).reshape(shape), "exp_avg_absmax": torch.stack(am),
          "factored_row_q": torch.stack(rq), "factored_row_absmax": torch.stack(ra),
          "factored_col_q": torch.stack(cq), "factored_col_absmax": torch.stack(ca)}
    group = {"lr": 1e-3, "eps": (1e-30, 1e-16), "clip_threshold": 1.0, "betas": (0.9, 0.999, 0.9999),
             "weight_decay": 1e-2, "block_size": B, "params": [0]}
    return {"state": {0: st}, "param_groups": [group]}


# Shapes over every route the per-matrix blocks take: rows and columns in partial blocks per matrix (the
# factor kernel's per-matrix block ranges), rows that straddle blocks (pass 2's unaligned variant), momentum
# blocks ending inside a matrix (the per-block parameter pass), tiny matrices (one thread per matrix),
# blocks that coincide with flat ones (the band passes, where the layouts agree), a block size that is not
# a power of two (every tensor on the per-block pass), fp32 and bf16.
ND_CASES = [((3, 40, 24), 64, "float32"), ((2, 5, 33, 7), 16, "float32"), ((4, 100, 100), 256, "bfloat16"),
            ((3, 64, 4096), 256, "bfloat16"), ((2, 3, 5), 4, "float32"), ((3, 40, 24), 100, "float32"),
            ((5, 300, 520), 256, "float32"), ((3, 129, 1001), 256, "bfloat16")]


@pytest.mark.parametrize("convert", [True, False])
@pytest.mark.parametrize("shape,B,dtype", ND_CASES)
def test_nd_per_matrix_checkpoint_steps_in_place(shape, B, dtype, convert):
    """A state dict of the reference's CUDA N-D path (per-matrix blocks, CAME8bitFull.py:790-842) loads into
    CAME8bitFull and is stepped in place (CAME8_STATE_Q8_MATRIX), whether or not layouts are converted: three
    steps, each teacher-forced against the oracle's per-matrix step, under the parity tolerances; the state
    keeps the reference's shapes, keys and views."""
    dt = getattr(torch, dtype)
    P_, R, C = math.prod(shape[:-2]), shape[-2], shape[-1]
    sd = _nd_checkpoint(shape, B, seed=4)
    p = torch.nn.Parameter(P.make_params([shape], dt, seed=5)[0].cuda())
    opt = came_amd.CAME8bitFull([p], lr=1e-3, weight_decay=1e-2, block_size=B)
    opt.load_state_dict(sd, convert_layouts=convert)
    ref_state = _cpu_state(opt.state[p])
    r = p.data.detach().cpu().clone()
    ohp = P.oracle_hp(dict(lr=1e-3, weight_decay=1e-2, block_size=B))
    check = T2_tight(f"nd per-matrix {shape} B={B} {dtype} convert={convert}", B)
    for step in range(3):
        with torch.no_grad():  # teacher forcing
            p.data.copy_(r.to(dt).cuda() if r.dtype != dt else r.cuda())
            for k in Q8_KEYS:
                opt.state[p][k].copy_(ref_state[k].cuda())
        g = _grads([shape], dt, 60 + step)
        _run(opt, [p], g)
        cap = {}
        before = r.double()
        orc.full8bit_step(r, g[0], ref_state, capture=cap, **ohp)
        check(step + 1, 0, p.data, r, opt.state[p], ref_state, (r.double() - before).abs(), cap)
    st = opt.state[p]
    assert SL.layout_of(st) == "full8bit-nd" and st["step"] == 8
    assert st["exp_avg_absmax"].shape == (P_, math.ceil(R * C / B))
    assert st["factored_row_absmax"].shape == (2 * P_, math.ceil(R / B))
    assert st["factored_col_absmax"].shape == (2 * P_, math.ceil(C / B))
    assert st["exp_avg_res_row_q"].shape == (P_, R)
    assert st["exp_avg_res_row_q"].data_ptr() == st["factored_row_q"].data_ptr() + P_ * R


def T2_tight(tag, B):
    from tests.test_gpu_parity import _tight_step_check
    return _tight_step_check(tag, block=B)


def test_nd_per_matrix_checkpoint_converts_for_camecuda():
    """CAMECUDA keeps fp32 states: a per-matrix checkpoint converts to them, each value the per-matrix
    dequantisation of its code (done by torch on the GPU here, on the CPU in the expectation: within
    1e-6 relative; the conversion's formula is pinned on the CPU in tests/test_state_layout.py)."""
    shape, B = (3, 40, 24), 64
    sd = _nd_checkpoint(shape, B, seed=8)
    ex = SL.state_values(sd["state"][0], shape, B)
    p = torch.nn.Parameter(P.make_params([shape], torch.float32, seed=9)[0].cuda())
    opt = came_amd.CAMECUDA([p], lr=1e-3, weight_decay=1e-2)
    opt.load_state_dict(sd)
    st = opt.state[p]
    assert st["_mode"] == "cudafp"
    torch.testing.assert_close(st["exp_avg"].cpu(), ex["exp_avg"], rtol=1e-6, atol=0)
    for k in ("sq_row", "res_row", "sq_col", "res_col"):
        torch.testing.assert_close(st[f"exp_avg_{k}"].cpu(), ex[k], rtol=1e-6, atol=0, msg=k)
