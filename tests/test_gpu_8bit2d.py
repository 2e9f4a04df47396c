"""GPU parity of the 8bit2d step (came_amd.CAME8bit2D) against the CPU restatement of the reference's
CUDA 8bit2d step (oracle.came8bit2d_step; reference came_cuda/csrc/came_kernels.cu:2584-2780,
3333-3367, launch order :3599-4040).

Tolerances (written here):
  * int8 momentum and uint8 row/column codes: never more than 1 apart; every differing code sits
    within TIE_TOL of a rounding tie of the oracle's scaled value (x * (1/absmax)) * Q; of those not
    at a tie to within EXACT_TIE, at most max(2, CODE_FRAC * n) differ.  The GPU sums rows and
    columns in another order than the oracle, so the values it quantises differ from the oracle's
    by a few ulps.  Structured gradients put many values exactly at a tie (one +-1e3 outlier per row
    makes the row's residual state half the block's absmax, code 127.5): those may all flip.
  * tile and block scales (absmax): within 1e-6 relative.
  * parameters: fp32 within 1e-5 relative to |p| plus the step's movement, bf16/fp16 within 1 ulp,
    on every element whose momentum code came out equal (the 8bit2d parameter write reads the
    requantised momentum, so an element whose code is one apart moves by absmax/127 * rr * cr * lr
    more or less; those are counted, not bounded).
Every step is teacher-forced: the GPU starts it from the oracle's parameters and state.
"""
import pytest
import torch

import came_amd
from oracle import came8_oracle as orc
from tests import parity as P

pytestmark = pytest.mark.gpu

PERSIST = ("exp_avg_q", "exp_avg_absmax") + tuple(
    f"exp_avg_{k}_{s}" for k in ("sq_row", "sq_col", "res_row", "res_col") for s in ("q", "absmax"))
CAPTURED = {"exp_avg_q": "exp_avg", "exp_avg_sq_row_q": "sq_row", "exp_avg_sq_col_q": "sq_col",
            "exp_avg_res_row_q": "res_row", "exp_avg_res_col_q": "res_col"}
# A differing code must sit within TIE_TOL code units of a rounding tie of the oracle's value: the
# reference's float sums (atomics of unfixed order on the GPU) and the oracle's differ by a few ulps,
# which moves a scaled value by ~1e-4 at most (the most seen here: 1.07e-4); codes off an exact tie
# (EXACT_TIE) may be at most CODE_FRAC of a state (the most seen: 1.0%).
TIE_TOL = 2e-4
EXACT_TIE = 1e-4
CODE_FRAC = 1.5e-2
SHAPES = [(64, 2048), (1000, 3), (3, 5000), (33, 5461), (130, 1024), (17, 17), (1, 1), (16, 16), (257, 129),
          (4097, 129), (48, 4100), (37, 400), (5, 48), (40, 3072)]


def _ohp(hp):
    h = P.oracle_hp(hp)
    return h


def _scaled(k: str, st: dict, cap: dict) -> torch.Tensor:
    """The oracle's pre-rounding code value (x * (1/absmax)) * Q for every code of `k`."""
    x = cap[CAPTURED[k]].float()
    if k == "exp_avg_q":
        rows, cols = x.shape
        tile = (torch.arange(rows)[:, None] // 16) * st["tile_cols"] + (torch.arange(cols)[None, :] // 16)
        a = st["exp_avg_absmax"][tile]
        q = 127.0
    else:
        a = st[k.replace("_q", "_absmax")].repeat_interleave(256)[: x.numel()]
        q = 255.0
    return (x * (torch.ones_like(a) / a)) * q


def _compare(gs: dict, st: dict, cap: dict, where: str) -> None:
    for k in PERSIST:
        g, r = gs[k].detach().cpu(), st[k]
        assert g.dtype == r.dtype and tuple(g.shape) == tuple(r.shape), f"{where}/{k}: {g.dtype}{tuple(g.shape)}"
        if k.endswith("_q"):
            _, mx = P.code_mismatch(g, r)
            assert mx <= 1, f"{where}/{k}: a code differs by {mx}"
            if mx:
                sc = _scaled(k, st, cap).reshape(r.shape)
                dist = (sc - sc.floor() - 0.5).abs()
                diff = g.to(torch.int32) != r.to(torch.int32)
                worst = dist[diff].max().item()
                print(f"[ties] {where}/{k}: {int(diff.sum())} of {g.numel()} codes differ, worst distance from a "
                      f"tie {worst:.2e}", flush=True)
                assert worst <= TIE_TOL, f"{where}/{k}: a differing code is {worst:.2e} from a rounding tie"
                off_tie = int((diff & (dist > EXACT_TIE)).sum())
                n = max(1, g.numel())
                assert off_tie <= max(2.0, CODE_FRAC * n), f"{where}/{k}: {off_tie} of {n} codes differ off a tie"
        else:
            m, _ = P.rel_err(g, r)
            assert m <= 1e-6, f"{where}/{k}: scale rel err {m:.3e}"


def _teacher_forced(shapes, dtype, steps, hp, seed, grad_fn=None):
    dt = getattr(torch, dtype)
    refs = P.make_params(shapes, dt, seed=seed)
    gen = torch.Generator().manual_seed(seed + 1)
    grad_fn = grad_fn or P.heavy_grad
    grads = [[grad_fn(gen, s, dt) for s in shapes] for _ in range(steps)]
    ps = [torch.nn.Parameter(r.clone().cuda()) for r in refs]
    opt = came_amd.CAME8bit2D(ps, **hp)
    ohp = _ohp(hp)
    sts = [orc.init_8bit2d_state(s) for s in shapes]
    flips = []
    for step in range(steps):
        with torch.no_grad():
            for p, r, st in zip(ps, refs, sts):
                p.data.copy_(r.cuda())
                gst = opt.state[p]
                if len(gst):
                    for k in PERSIST:
                        gst[k].copy_(st[k].cuda())
        for p, g in zip(ps, grads[step]):
            p.grad = g.cuda()
        opt.step()
        torch.cuda.synchronize()
        for i, (p, r, g, st) in enumerate(zip(ps, refs, grads[step], sts)):
            before = r.double()
            cap = {}
            orc.came8bit2d_step(r, g, st, capture=cap, **ohp)
            where = f"8bit2d {dtype} step {step + 1} tensor {i} {tuple(r.shape)}"
            gs = opt.state[p]
            assert gs["_mode"] == "8bit2d" and "step" not in gs
            _compare(gs, st, cap, where)
            flipped = gs["exp_avg_q"].cpu() != st["exp_avg_q"]
            flips.append(float(flipped.float().mean()))
            # the parameter write uses the requantised momentum: a code one apart (at a tie) moves the
            # element by exactly one code step, lr * rr_i * cr_j * absmax / 127, no more
            rows, cols = r.shape
            tile = (torch.arange(rows)[:, None] // 16) * st["tile_cols"] + (torch.arange(cols)[None, :] // 16)
            step_q = hp["lr"] * cap["res_factor"].double().abs() * st["exp_avg_absmax"][tile].double() / 127.0
            P.check_params_bound(p.data, r, step_q * flipped, where, (r.double() - before).abs(), tol=1e-5,
                                 scale=1.01)
    return flips


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_8bit2d_teacher_forced_vs_oracle(dtype):
    flips = _teacher_forced(SHAPES, dtype, 4, dict(lr=1e-3, weight_decay=1e-2), seed=51)
    assert max(flips) <= CODE_FRAC


def test_8bit2d_betas_no_weight_decay_gaussian_grads():
    def gauss(gen, s, dt):
        return (torch.randn(s, generator=gen) * 2e-4).to(dt)
    _teacher_forced([(256, 1024), (40, 72), (11008 // 8, 512)], "float32", 3,
                    dict(lr=2e-4, betas=(0.9, 0.95, 0.995), weight_decay=0.0), seed=53, grad_fn=gauss)


def test_8bit2d_zero_and_constant_gradients():
    """All-zero gradient matrices (row means 0: the mean-of-rows rule r = 1) and constant ones."""
    def special(gen, s, dt):
        k = int(torch.randint(0, 2, (1,), generator=gen))
        return (torch.zeros(s) if k == 0 else torch.full(s, 3e-3)).to(dt)
    _teacher_forced([(32, 48), (5, 300)], "float32", 3, dict(lr=1e-3, weight_decay=1e-2), seed=57, grad_fn=special)


def test_8bit2d_free_running_ten_steps():
    """Ten steps from a fresh state without teacher forcing stay close to the oracle."""
    shapes = [(256, 1024), (100, 37)]
    hp = dict(lr=2e-4, weight_decay=1e-2)
    refs = P.make_params(shapes, torch.float32, seed=61)
    gen = torch.Generator().manual_seed(62)
    ps = [torch.nn.Parameter(r.clone().cuda()) for r in refs]
    opt = came_amd.CAME8bit2D(ps, **hp)
    sts = [orc.init_8bit2d_state(s) for s in shapes]
    for _ in range(10):
        gs = [torch.randn(s, generator=gen) * 1e-3 for s in shapes]
        for p, g in zip(ps, gs):
            p.grad = g.cuda()
        opt.step()
        for r, g, st in zip(refs, gs, sts):
            orc.came8bit2d_step(r, g, st, **_ohp(hp))
    torch.cuda.synchronize()
    for p, r, st in zip(ps, refs, sts):
        _, nr = P.rel_err(p.data, r)
        assert nr <= 1e-4, nr
        frac, _ = P.code_mismatch(opt.state[p]["exp_avg_q"], st["exp_avg_q"])
        assert frac <= 1e-3, frac


def test_8bit2d_state_layout_and_state_dict_round_trip():
    """State keys, dtypes and shapes are the reference's (came8bit2d_state.py:33-75); a state dict saved
    after two steps loads into a fresh optimizer (bf16 parameters: the fp32 scratch tensors keep
    their dtype) and the next step matches the original optimizer's bit for bit."""
    shapes = [(40, 72), (33, 130)]
    refs = P.make_params(shapes, torch.bfloat16, seed=71)
    gen = torch.Generator().manual_seed(72)
    grads = [[(torch.randn(s, generator=gen) * 1e-3).to(torch.bfloat16) for s in shapes] for _ in range(3)]
    a = [torch.nn.Parameter(r.clone().cuda()) for r in refs]
    oa = came_amd.CAME8bit2D(a, lr=1e-3, weight_decay=1e-2)
    for s in range(2):
        for p, g in zip(a, grads[s]):
            p.grad = g.cuda()
        oa.step()
    st = oa.state[a[0]]
    ref_keys = {"_mode", "exp_avg_q", "exp_avg_absmax", "r_factor", "c_factor", "r_res_factor", "c_res_factor",
                "res_row_sum", "res_col_sum", "res_row_partial", "res_col_partial", "sum_sq_row", "sum_update",
                "sum_update_partial", "sum_res_row", "rows", "cols", "tile_rows", "tile_cols", "num_tiles"}
    ref_keys |= {f"exp_avg_{k}_{s}" for k in ("sq_row", "sq_col", "res_row", "res_col") for s in ("q", "absmax")}
    assert set(st.keys()) == ref_keys
    assert st["res_row_partial"].numel() == 5 * 40 and st["res_col_partial"].numel() == 3 * 72
    sd = oa.state_dict()
    b = [torch.nn.Parameter(p.detach().clone()) for p in a]
    ob = came_amd.CAME8bit2D(b, lr=1e-3, weight_decay=1e-2)
    ob.load_state_dict(sd)
    for k, v in oa.state[a[0]].items():
        w = ob.state[b[0]][k]
        if isinstance(v, torch.Tensor):
            assert w.dtype == v.dtype and w.shape == v.shape, k
        else:
            assert w == v, k
    for p, q, g in zip(a, b, grads[2]):
        p.grad, q.grad = g.cuda(), g.cuda()
    oa.step()
    ob.step()
    torch.cuda.synchronize()
    for p, q in zip(a, b):
        assert torch.equal(p.data, q.data)
        for k in PERSIST:
            assert torch.equal(oa.state[p][k], ob.state[q][k]), k


def test_8bit2d_errors_match_reference():
    p1 = torch.nn.Parameter(torch.zeros(8, device="cuda"))
    p1.grad = torch.zeros(8, device="cuda")
    with pytest.raises(NotImplementedError, match="supports 2D parameters only"):
        came_amd.CAME8bit2D([p1], lr=1e-3).step()
    p2 = torch.nn.Parameter(torch.zeros(8, 8, device="cuda"))
    p2.grad_dtype = None  # torch otherwise refuses a gradient of another dtype
    p2.grad = torch.zeros(8, 8, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="Expected g.dtype == p.dtype"):
        came_amd.CAME8bit2D([p2], lr=1e-3).step()
    p3 = torch.nn.Parameter(torch.zeros(8, 8, device="cuda"))
    p3.grad = torch.zeros(8, 8, device="cuda")
    opt = came_amd.CAME8bit2D([p3], lr=1e-3)
    opt.step()
    opt.state[p3]["res_row_partial"] = torch.zeros(3, device="cuda")  # too small for 8 rows x 1 tile column
    with pytest.raises(RuntimeError, match="res_row_partial is too small"):
        opt.step()


def _misaligned(t: torch.Tensor) -> torch.Tensor:
    """A contiguous copy of `t` that starts one element past a 16-byte boundary."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = buf[1:].view(t.shape)
    v.copy_(t)
    return v


def _bits(t: torch.Tensor) -> torch.Tensor:
    """The raw bits of a tensor (NaN compares equal to a NaN of the same bits)."""
    if t.dtype in (torch.float32,):
        return t.view(torch.int32)
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16)
    return t


def _forms_bitwise(shapes, dtype, grads, wd=1e-2):
    """Runs the steps of `grads` three ways (aligned: vector momentum pass and parameter write;
    parameter one element off a 16-byte boundary: scalar parameter write; momentum codes 8 bytes off
    one: scalar momentum pass too) and checks that parameters and states agree bit for bit."""
    dt = getattr(torch, dtype)
    refs = P.make_params(shapes, dt, seed=81)
    runs = {}
    for mode in ("aligned", "param_off", "codes_off"):
        ps = []
        for r in refs:
            d = r.clone().cuda()
            ps.append(torch.nn.Parameter(_misaligned(d) if mode == "param_off" else d))
        opt = came_amd.CAME8bit2D(ps, lr=1e-3, weight_decay=wd)
        for p, g in zip(ps, grads[0]):
            p.grad = g.cuda()
        opt.prime_for_cuda_graph()  # creates the states
        if mode == "codes_off":
            for p in ps:
                q = opt.state[p]["exp_avg_q"]
                buf = torch.zeros(q.numel() + 8, dtype=torch.int8, device="cuda")
                opt.state[p]["exp_avg_q"] = buf[8:].view(q.shape)
                assert opt.state[p]["exp_avg_q"].data_ptr() % 16 == 8
        for step in range(len(grads)):
            for p, g in zip(ps, grads[step]):
                p.grad = g.cuda()
            opt.step()
        torch.cuda.synchronize()
        runs[mode] = [(p.data.cpu(), {k: opt.state[p][k].cpu() for k in PERSIST}) for p in ps]
    for mode in ("param_off", "codes_off"):
        for i, ((pa, sa), (pb, sb)) in enumerate(zip(runs["aligned"], runs[mode])):
            assert torch.equal(_bits(pa), _bits(pb)), f"{mode} tensor {i}: parameters differ"
            for k in PERSIST:
                assert torch.equal(_bits(sa[k]), _bits(sb[k])), f"{mode} tensor {i}: {k} differs"
    return runs


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_8bit2d_vector_and_scalar_forms_agree_bitwise(dtype):
    """Rows that are a whole number of tiles (C % 16 == 0) with 16-byte aligned buffers take the vector
    momentum pass and parameter write; a parameter one element off a 16-byte boundary takes the scalar
    parameter write, and momentum codes 8 bytes off one take the scalar momentum pass too (pass 1,
    which needs only 8-byte aligned codes, stays the same).  Both forms run the same arithmetic in
    the same order, so three steps must agree bit for bit."""
    dt = getattr(torch, dtype)
    shapes = [(64, 2048), (37, 400), (5, 48), (130, 1024), (40, 3072)]
    gen = torch.Generator().manual_seed(82)
    grads = [[P.heavy_grad(gen, s, dt) for s in shapes] for _ in range(3)]
    _forms_bitwise(shapes, dtype, grads)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_8bit2d_forms_agree_on_special_tiles(dtype):
    """The vector momentum pass quantises a tile through a rounding constant when the tile holds no
    infinity or NaN and 1/absmax is finite, and through rint and the clamp otherwise; the scalar pass
    always takes the second way.  Tiles of zeros, of subnormal gradients (absmax subnormal, so
    1/absmax overflows, and numerators below the reciprocal division's range), a tensor with a NaN
    and one with an infinity must give the same bits both ways."""
    dt = getattr(torch, dtype)
    shapes = [(64, 2048), (48, 256), (32, 512), (32, 512)]
    gen = torch.Generator().manual_seed(83)
    grads = []
    for _ in range(2):
        gs = [P.heavy_grad(gen, s, dt) for s in shapes]
        gs[0][0:16, 0:16] = 0
        gs[0][16:32, 32:48] = 1e-39
        gs[0][33, 100] = 1e-39
        gs[1][16:32, 16:32] = 1e-38
        gs[2][5, 7] = float("nan")
        gs[3][9, 300] = float("inf")
        grads.append(gs)
    runs = _forms_bitwise(shapes, dtype, grads)
    p0, s0 = runs["aligned"][0]
    assert torch.isfinite(p0.float()).all() and (s0["exp_avg_q"][0:16, 0:16] == 0).all()
    assert (s0["exp_avg_q"][16:32, 32:48] != 0).any()
