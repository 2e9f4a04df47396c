"""GPU parity of CAMECUDA (fp32 optimizer states) against the CPU oracle's restatement of the
reference's generic fp32-state step (came_pytorch/CAMECUDA.py:275-326; oracle.fp32_state_step).

Tolerances (written here):
  * fp32 row / column states: |d| <= 1e-5 * (|x_ref| + 1e-2 * rms(x_ref)).  The GPU sums rows and
    columns in another order than torch's CPU kernels, so means and everything downstream of them
    can differ by a few ulps.
  * momentum m = b1*m_old + (1-b1)*u: the same bound with |x_ref| replaced by the size of the two
    terms, |b1*m_old| + |m - b1*m_old| (where they nearly cancel, an ulp of u is large next to m).
  * parameters: as for the 8-bit step (parity.check_untainted_params): fp32 within 1e-5 relative to
    |p| plus the step's movement, bf16 within 1 ulp.
Every step is teacher-forced (both sides start from the oracle's state) in parity mode
(``reference_norm``, the reference's float32 summation order of the update-RMS norm).
"""
import pytest
import torch

import came_amd
from oracle import came8_oracle as orc
from tests import parity as P

pytestmark = pytest.mark.gpu

STATE_KEYS = ("exp_avg", "exp_avg_sq_row", "exp_avg_sq_col", "exp_avg_res_row", "exp_avg_res_col", "exp_avg_sq")
# (2, 3, 5, 7), (16, 3, 3, 3) and (20, 8, 1, 1) are tensors of tiny matrices (one thread per matrix);
# (5, 11008) and (2, 20000) have rows wider than one sweep of the residual pass (column segments)
SHAPES = [(1,), (255,), (4097,), (1000, 3), (3, 5000), (64, 2048), (2, 3, 5, 7), (33, 5461), (130, 1024), (4, 4096),
          (16, 3, 3, 3), (20, 8, 1, 1), (5, 11008), (2, 20000)]


def _close(g: torch.Tensor, r: torch.Tensor, where: str, tol: float = 1e-5, scale: torch.Tensor | None = None):
    g, r = g.detach().cpu().double(), r.detach().double()
    assert g.shape == r.shape, where
    if r.numel() == 0:
        return
    rms = r.pow(2).mean().sqrt().item()
    size = r.abs() if scale is None else scale
    err = ((g - r).abs() / (size + 1e-2 * rms + 1e-38)).max().item()
    assert err <= tol, f"{where}: rel err {err:.3e} > {tol}"


def _run(shapes, dtype, steps, hp, seed):
    dt = getattr(torch, dtype)
    ref_p = P.make_params(shapes, dt, seed=seed)
    gen = torch.Generator().manual_seed(seed + 1)
    grads = [[P.heavy_grad(gen, s, dt) for s in shapes] for _ in range(steps)]
    gpu_p = [torch.nn.Parameter(p.clone().to("cuda")) for p in ref_p]
    opt = came_amd.CAMECUDA(gpu_p, **hp)
    ohp = {k: v for k, v in P.oracle_hp(hp).items() if k != "block_size"}
    ref_st = [orc.init_fp32_state(s) for s in shapes]
    for step in range(steps):
        # teacher forcing: the GPU starts the step from the oracle's parameters and states
        for p, rp, st in zip(gpu_p, ref_p, ref_st):
            p.data.copy_(rp.to("cuda"))
            p.grad = None
        for p, g in zip(gpu_p, grads[step]):
            p.grad = g.to("cuda")
        if step > 0:
            for p, st in zip(gpu_p, ref_st):
                for k in STATE_KEYS:
                    if k in st:
                        opt.state[p][k].copy_(st[k].to("cuda"))
        opt.step()
        torch.cuda.synchronize()
        for i, (p, rp, g, st) in enumerate(zip(gpu_p, ref_p, grads[step], ref_st)):
            before = rp.double()
            m_old = st["exp_avg"].double() * ohp["beta1"]
            orc.fp32_state_step(rp, g, st, **ohp)
            m_new = st["exp_avg"].double()
            m_size = m_old.abs() + (m_new - m_old).abs()
            where = f"CAMECUDA {dtype} step {step + 1} tensor {i} {tuple(rp.shape)}"
            gs = opt.state[p]
            assert gs["_mode"] == "cudafp" and gs["step"] == st["step"] and gs["factored"] == st["factored"]
            for k in STATE_KEYS:
                if k in st:
                    assert gs[k].dtype == torch.float32, f"{where}/{k}"
                    _close(gs[k], st[k], f"{where}/{k}", scale=m_size if k == "exp_avg" else None)
            P.check_untainted_params(p.data, rp, torch.zeros(rp.shape, dtype=torch.bool), where,
                                     (rp.double() - before).abs(), tol=1e-5)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16", "float16"])
def test_camecuda_teacher_forced_vs_oracle(dtype):
    _run(SHAPES, dtype, 4, dict(lr=1e-3, weight_decay=1e-2), seed=31)


def test_camecuda_betas_and_no_weight_decay():
    _run([(96, 1024), (40, 72), (300,)], "float32", 3,
         dict(lr=2e-4, betas=(0.9, 0.95, 0.995), weight_decay=0.0), seed=37)


def test_camecuda_default_norm_free_running_close():
    """Default mode (fp64 clip norm) over 5 free-running steps stays close to the oracle."""
    shapes = [(256, 1024), (1024,)]
    ref_p = P.make_params(shapes, torch.float32, seed=41)
    gen = torch.Generator().manual_seed(43)
    gpu_p = [torch.nn.Parameter(p.clone().cuda()) for p in ref_p]
    opt = came_amd.CAMECUDA(gpu_p, lr=2e-4, weight_decay=1e-2)
    ohp = {k: v for k, v in P.oracle_hp(dict(lr=2e-4, weight_decay=1e-2)).items() if k != "block_size"}
    sts = [orc.init_fp32_state(s) for s in shapes]
    for _ in range(5):
        gs = [torch.randn(s, generator=gen) * 1e-3 for s in shapes]
        for p, g in zip(gpu_p, gs):
            p.grad = g.cuda()
        opt.step()
        for rp, g, st in zip(ref_p, gs, sts):
            orc.fp32_state_step(rp, g, st, **ohp)
    torch.cuda.synchronize()
    for p, rp in zip(gpu_p, ref_p):
        _, nr = P.rel_err(p.data, rp)
        assert nr <= 1e-5, nr
