"""Shared helpers for the parity tests: run the GPU optimizer and the CPU oracle on the same inputs
and compare state and parameters under the tolerances the tests state."""
from __future__ import annotations

import math

import numpy as np
import torch

from collections import namedtuple

from oracle import came8_oracle as orc

Lockstep = namedtuple("Lockstep", "gpu_param ref_param gpu_state ref_state tainted flips movement bound")

HP_DEFAULTS = dict(lr=None, eps=(1e-30, 1e-16), clip_threshold=1.0, betas=(0.9, 0.999, 0.9999),
                   weight_decay=0.0, block_size=256)


def oracle_hp(hp: dict) -> dict:
    h = dict(HP_DEFAULTS)
    h.update(hp)
    b1, b2, b3 = h["betas"]
    return dict(beta1=b1, beta2=b2, beta3=b3, eps0=h["eps"][0], eps1=h["eps"][1], lr=h["lr"],
                clip_threshold=h["clip_threshold"], weight_decay=h["weight_decay"], block_size=h["block_size"])


STATE_KEYS = ("exp_avg_q", "exp_avg_absmax", "factored_row_q", "factored_row_absmax", "factored_col_q",
              "factored_col_absmax", "exp_avg_sq_q", "exp_avg_sq_absmax")


def code_mismatch(a: torch.Tensor, b: torch.Tensor):
    """(fraction of codes that differ, max |difference|)."""
    a = a.detach().cpu().to(torch.int32).reshape(-1)
    b = b.detach().cpu().to(torch.int32).reshape(-1)
    if a.numel() == 0:
        return 0.0, 0
    d = (a - b).abs()
    return float((d != 0).float().mean()), int(d.max())


def rel_err(a: torch.Tensor, b: torch.Tensor):
    """(max elementwise |a-b|/|b| over |b| > tiny, ||a-b|| / ||b||)."""
    a = a.detach().cpu().double().reshape(-1)
    b = b.detach().cpu().double().reshape(-1)
    if a.numel() == 0:
        return 0.0, 0.0
    nb = b.norm().item()
    normrel = (a - b).norm().item() / nb if nb > 0 else (a - b).norm().item()
    mask = b.abs() > 1e-30
    if mask.any():
        m = ((a - b).abs()[mask] / b.abs()[mask]).max().item()
    else:
        m = 0.0
    m = max(m, (a - b).abs()[~mask].max().item() if (~mask).any() else 0.0)
    return m, normrel


def param_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max_i |a_i - b_i| / (|b_i| + 1e-2 * rms(b)) for fp32 parameters.

    A bound of 1e-5 on this reads "within 1e-5 relative, or within ~1e-7 of the tensor's RMS"
    (about one fp32 ulp at the parameter scale).  The floor matters where p - lr*step cancels to
    a value near zero: there a one-ulp difference in the step direction is a large relative
    difference of the (tiny) result while being an ulp-level difference of the update.
    """
    a = a.detach().cpu().double().reshape(-1)
    b = b.detach().cpu().double().reshape(-1)
    if a.numel() == 0:
        return 0.0
    rms = b.pow(2).mean().sqrt().item()
    return ((a - b).abs() / (b.abs() + 1e-2 * rms + 1e-38)).max().item()


def lowp_close(a: torch.Tensor, b: torch.Tensor) -> bool:
    """bf16/fp16 parameters: every element within 1 ulp, or (cancellation to near zero) within 1e-7 of the RMS."""
    ai = a.detach().cpu().contiguous().view(torch.int16).to(torch.int32).reshape(-1)
    bi = b.detach().cpu().contiguous().view(torch.int16).to(torch.int32).reshape(-1)
    if ai.numel() == 0:
        return True

    def ordered(x):
        return torch.where(x < 0, -(x & 0x7FFF), x)

    ulps = (ordered(ai) - ordered(bi)).abs()
    af, bf = a.detach().cpu().double().reshape(-1), b.detach().cpu().double().reshape(-1)
    rms = bf.pow(2).mean().sqrt().item()
    ok = (ulps <= 1) | ((af - bf).abs() <= 1e-7 * rms)
    return bool(ok.all())


def ulp_diff_lowp(a: torch.Tensor, b: torch.Tensor) -> int:
    """Max distance in units in the last place between two bf16/fp16 tensors of the same dtype."""
    ai = a.detach().cpu().contiguous().view(torch.int16).to(torch.int32).reshape(-1)
    bi = b.detach().cpu().contiguous().view(torch.int16).to(torch.int32).reshape(-1)

    def ordered(x):  # sign-magnitude -> two's complement ordering
        return torch.where(x < 0, -(x & 0x7FFF), x)

    if ai.numel() == 0:
        return 0
    return int((ordered(ai) - ordered(bi)).abs().max())


def _ref_values(k: str, ref_fp32: dict):
    """fp32 values the reference quantised into code array `k` (stacked like the codes)."""
    if k == "exp_avg_q":
        return ref_fp32["exp_avg"], True
    if k == "exp_avg_sq_q":
        return ref_fp32["sq"], False
    if k == "factored_row_q":
        return torch.stack([ref_fp32["sq_row"], ref_fp32["res_row"]]), False
    if k == "factored_col_q":
        return torch.stack([ref_fp32["sq_col"], ref_fp32["res_col"]]), False
    raise KeyError(k)


def tie_distance(k: str, ref_state: dict, ref_fp32: dict, block: int) -> torch.Tensor:
    """|frac(scaled) - 0.5| of the reference's scaled value (x / absmax) * Q for every code of `k`."""
    vals, signed = _ref_values(k, ref_fp32)
    ak = k.replace("_q", "_absmax")
    absmax = ref_state[ak]
    rows = vals.reshape(absmax.shape[0], -1) if absmax.dim() == 2 else vals.reshape(1, -1)
    am = absmax.reshape(rows.shape[0], -1)
    out = []
    for rv, a in zip(rows, am):
        scale = a.repeat_interleave(block)[: rv.numel()]
        scaled = (rv.float() / scale) * (127.0 if signed else 255.0)
        out.append((scaled - scaled.floor() - 0.5).abs())
    return torch.stack(out).reshape(ref_state[k].shape)


def compare_states(gpu_state: dict, ref_state: dict, *, code_frac: float, abs_rel: float, where: str,
                   ref_fp32: dict | None = None, tie_tol: float | None = None, block: int = 256,
                   max_code_diff: int = 1):
    """Codes: never more than 1 apart, at most max(8, code_frac * n) differ, and (given the oracle's
    pre-quantisation values) every differing code sits within `tie_tol` of a rounding tie of the
    reference's scaled value; block scales within `abs_rel` relative."""
    report = {}
    for k in STATE_KEYS:
        if k not in ref_state:
            continue
        g, r = gpu_state[k].detach().cpu(), ref_state[k]
        assert g.dtype == r.dtype and tuple(g.shape) == tuple(r.shape), f"{where}/{k}: {g.dtype}{tuple(g.shape)} vs {r.dtype}{tuple(r.shape)}"
        if k.endswith("_q"):
            frac, mx = code_mismatch(g, r)
            report[k] = (frac, mx)
            assert mx <= max_code_diff, f"{where}/{k}: a code differs by {mx}"
            if ref_fp32 is not None and tie_tol is not None and mx > 0:
                dist = tie_distance(k, ref_state, ref_fp32, block)
                diff = g.to(torch.int32) != r.to(torch.int32)
                worst = dist[diff].max().item()
                report[k] = (frac, mx, worst)
                print(f"[ties] {where}/{k}: {int(diff.sum())} of {g.numel()} codes differ, worst distance from a "
                      f"tie {worst:.2e}", flush=True)
                assert worst <= tie_tol, f"{where}/{k}: a differing code is {worst:.2e} from a rounding tie (> {tie_tol})"
            n = max(1, g.numel())  # small state arrays: a handful of exact ties is not a fraction
            assert frac * n <= max(8.0, code_frac * n), f"{where}/{k}: {frac:.3e} of codes differ (bound {code_frac})"
        else:
            m, _ = rel_err(g, r)
            report[k] = m
            assert m <= abs_rel, f"{where}/{k}: block scale rel err {m:.3e} > {abs_rel}"
    return report


def make_params(shapes, dtype, seed, device="cpu"):
    gen = torch.Generator().manual_seed(seed)
    return [(torch.randn(s, generator=gen) * 0.02).to(dtype) for s in shapes]


# Tie-dense clip-norm chains: bf16 gradients m * 2^(k - 20), m an integer in [64, 127] (7 significant bits),
# k uniform in [-8, 0], random signs.  Under a power-of-two factor the update u keeps those bits, so each
# u^2 has at most 14 significant bits and its lowest set bit lies at one of nine exponents: wherever the
# running sum's unit is twice that bit, the fused multiply-add lands exactly half-way (a rounding tie).
# TIE_DENSE_STATE makes the factors powers of two in the first step with betas[1] = 0.5: row states 255
# (every row alike: r_i = 1) and column states 128 (c_j = rsqrt(0.5 * 128) = 1/8), which g^2 <= 2^-26
# does not move.
TIE_DENSE_BETAS = (0.9, 0.5, 0.9999)


def tie_dense_grad(gen, shape):
    n = math.prod(shape)
    m = torch.randint(64, 128, (n,), generator=gen).double()
    k = torch.randint(-8, 1, (n,), generator=gen).double()
    sign = torch.where(torch.rand(n, generator=gen) < 0.5, -1.0, 1.0).double()
    return (sign * m * torch.exp2(k - 20)).reshape(shape).to(torch.bfloat16)


# The tie-dense case of the GPU walk test and its counts under the replay rules (the C model of
# tests/native/norm_replay_model.c with exact estimates, pinned by tests/test_norm_replay_model.py): the
# most segments one of the eight chains replays (of 2048) and the most wavefront rounds those replays take.
TIE_SHAPE, TIE_SEED = (2048, 4096), 11
TIE_REPLAYS_MAX, TIE_ROUNDS_MAX = 1058, 14886


def tie_dense_state(state: dict) -> None:
    """Second-moment codes of a factored full8bit state (flat or GPU tensors) set to the power-of-two
    factor state described at TIE_DENSE_BETAS: rows 255, columns 128, absmax 255."""
    for key, code in (("factored_row", 255), ("factored_col", 128)):
        state[key + "_q"].view(2, -1)[0].fill_(code)
        state[key + "_absmax"].view(2, -1)[0].fill_(255.0)


def heavy_grad(gen, shape, dtype):
    """Student-t(2) * 1e-3 with 10% exact zeros and ~1 outlier of +-1e3 per 256 elements."""
    z = torch.randn(shape, generator=gen)
    chi = torch.randn((2,) + tuple(shape), generator=gen)
    g = z / torch.sqrt((chi ** 2).mean(dim=0)) * 1e-3
    g = torch.where(torch.rand(shape, generator=gen) < 0.1, torch.zeros_like(g), g)
    flat = g.reshape(-1)
    n = flat.numel()
    if n >= 16:
        pick = torch.randint(0, n, (max(1, n // 256),), generator=gen)
        flat[pick] = torch.where(torch.rand(pick.shape, generator=gen) < 0.5, -1e3, 1e3)
    return g.to(dtype)


class DriftBound:
    """Per-element allowance for a free-running GPU trajectory that parts from the reference only
    through 8-bit codes that came out one apart at rounding ties (each such code is checked to sit
    at a tie by the teacher-forced tests).

    After step t both sides' states are dequantised: the momentum difference |dm| (exact, from both
    sides' codes and scales) enters step t + 1 as beta1 * |dm|; a second-moment state that differs
    by a relative d perturbs the next update u by beta2 * d / 2 (through the rsqrt), and a residual
    state by beta3 * d / 2 the residual factor rf.  Step t + 1 then moves the parameter by lr * rf * m,
    so its difference grows by at most lr * (|rf| * E + |rf * m| * rho_res) with
    E = beta1 * |dm| + (1 - beta1) * |u| * rho_u, and weight decay scales what is carried.  First
    order: the caller allows twice the accumulated bound."""

    def __init__(self, shape, factored, hp):
        self.factored = factored
        self.b1, self.b2 = hp["beta1"], hp["beta2"]
        self.b3, self.lr, self.wd = hp["beta3"], hp["lr"], hp["weight_decay"]
        self.bs = hp["block_size"]
        z = lambda: torch.zeros(shape, dtype=torch.float64)  # noqa: E731
        self.D, self.Em, self.rho_u, self.rho_res = z(), z(), z(), z()

    def _deq(self, q, a, signed):
        return orc.dequantize_blockwise(q.detach().cpu(), a.detach().cpu(), signed=signed, block_size=self.bs).double()

    def _rel(self, gq, ga, rq, ra):
        r = self._deq(rq, ra, False)
        return (self._deq(gq, ga, False) - r).abs() / r.abs().clamp_min(1e-30)

    def update(self, gpu_state, ref_state, cap):
        """After both sides took step t (cap: the oracle's capture of step t)."""
        u = cap["update"].double().abs()
        em = self.Em + (1.0 - self.b1) * u * self.rho_u
        if self.factored:
            rf = cap["res_factor"].double().abs()
            dstep = rf * em + rf * cap["exp_avg"].double().abs() * self.rho_res
        else:
            dstep = em
        self.D = self.D * abs(1.0 - self.lr * self.wd) + self.lr * dstep
        g, r = gpu_state, ref_state
        self.Em = self.b1 * (self._deq(g["exp_avg_q"], g["exp_avg_absmax"], True)
                             - self._deq(r["exp_avg_q"], r["exp_avg_absmax"], True)).abs()
        if self.factored:
            d = [self._rel(g[f"factored_{k}_q"][j], g[f"factored_{k}_absmax"][j], r[f"factored_{k}_q"][j],
                           r[f"factored_{k}_absmax"][j]) for j in (0, 1) for k in ("row", "col")]
            self.rho_u = 0.5 * self.b2 * (d[0].unsqueeze(-1) + d[1].unsqueeze(-2))
            self.rho_res = 0.5 * self.b3 * (d[2].unsqueeze(-1) + d[3].unsqueeze(-2))
        else:
            self.rho_u = 0.5 * self.b2 * self._rel(g["exp_avg_sq_q"], g["exp_avg_sq_absmax"], r["exp_avg_sq_q"],
                                                   r["exp_avg_sq_absmax"])


def check_params_bound(gp: torch.Tensor, rp: torch.Tensor, bound: torch.Tensor, where: str,
                       movement: torch.Tensor, tol: float = 1e-5, scale: float = 2.0) -> float:
    """Every element: |dp| <= tol * (|p_ref| + movement + 1e-2 * rms(p_ref)) + scale * bound (DriftBound:
    first order, hence twice); bf16/fp16: or within 1 ulp, and an element with an allowance also gets
    the ulp its final rounding may add.  Returns the fraction of elements with a nonzero allowance."""
    g = gp.detach().cpu().reshape(-1)
    r = rp.detach().cpu().reshape(-1)
    rd, gd = r.double(), g.double()
    rms = rd.pow(2).mean().sqrt().item()
    allow = tol * (rd.abs() + movement.reshape(-1) + 1e-2 * rms) + scale * bound.reshape(-1)
    if r.dtype != torch.float32:
        ulp = (torch.nextafter(r.abs(), torch.full_like(r, float("inf"))) - r.abs()).double()
        allow = allow + torch.where(bound.reshape(-1) > 0, ulp, torch.zeros_like(ulp))
    dp = (gd - rd).abs()
    ok = dp <= allow
    if r.dtype != torch.float32:
        ai = g.contiguous().view(torch.int16).to(torch.int32)
        bi = r.contiguous().view(torch.int16).to(torch.int32)
        ordered = lambda x: torch.where(x < 0, -(x & 0x7FFF), x)  # noqa: E731
        ok |= (ordered(ai) - ordered(bi)).abs() <= 1
    if not bool(ok.all()):
        k = int((~ok).nonzero()[0])
        raise AssertionError(f"{where}: element {k}: |dp| {dp[k].item():.3e} > allowed {allow[k].item():.3e} "
                             f"(drift allowance {bound.reshape(-1)[k].item():.3e}); {int((~ok).sum())} elements")
    return float((bound > 0).double().mean())


def run_oracle(params, grads_per_step, hp: dict, steps: int):
    """CPU oracle over `steps` steps; returns (params, states)."""
    ohp = oracle_hp(hp)
    ps = [p.clone() for p in params]
    sts = [orc.init_full8bit_state(p.shape, ohp["block_size"]) for p in ps]
    for s in range(steps):
        for p, g, st in zip(ps, grads_per_step[s], sts):
            orc.full8bit_step(p, g, st, **ohp)
    return ps, sts


def run_gpu(cls, params, grads_per_step, hp: dict, steps: int, exact_norm=False, device="cuda"):
    ps = [torch.nn.Parameter(p.clone().to(device)) for p in params]
    kw = {k: v for k, v in hp.items()}
    opt = cls(ps, **kw)
    opt.exact_norm = exact_norm
    for s in range(steps):
        for p, g in zip(ps, grads_per_step[s]):
            p.grad = g.to(device)
        opt.step()
    torch.cuda.synchronize()
    return ps, opt


def run_lockstep(cls, params, grads_per_step, hp: dict, steps: int, exact_norm=False, device="cuda"):
    """GPU optimizer and CPU oracle side by side on the same inputs.

    Returns, per tensor: (gpu_param, ref_param, gpu_state, ref_state, tainted, flips) where
    `tainted` marks elements whose inputs to a later step differed because an 8-bit code of
    theirs (momentum, or the row/column second-moment or residual state of their row/column)
    came out one apart at an earlier step, `flips` is the per-step fraction of differing
    momentum codes, and `bound` the per-element drift allowance those differences add (DriftBound).
    """
    ohp = oracle_hp(hp)
    ps = [torch.nn.Parameter(p.clone().to(device)) for p in params]
    opt = cls(ps, **hp)
    opt.exact_norm = exact_norm
    refs = [p.clone() for p in params]
    sts = [orc.init_full8bit_state(p.shape, ohp["block_size"]) for p in refs]
    tainted = [torch.zeros(p.shape, dtype=torch.bool) for p in params]
    movement = [torch.zeros(p.shape, dtype=torch.float64) for p in params]
    bounds = [DriftBound(p.shape, st["factored"], ohp) for p, st in zip(params, sts)]
    flips = [[] for _ in params]
    for s in range(steps):
        for p, g in zip(ps, grads_per_step[s]):
            p.grad = g.to(device)
        opt.step()
        torch.cuda.synchronize()
        for i, (r, g, st) in enumerate(zip(refs, grads_per_step[s], sts)):
            before = r.double()
            cap = {}
            orc.full8bit_step(r, g, st, capture=cap, exact_norm=exact_norm, **ohp)
            movement[i] += (r.double() - before).abs()
            gs = opt.state[ps[i]]
            bounds[i].update(gs, st, cap)
            dq = gs["exp_avg_q"].cpu() != st["exp_avg_q"]
            flips[i].append(float(dq.float().mean()))
            t = dq.clone()
            if st["factored"]:
                shape = tuple(r.shape)
                rowd = (gs["factored_row_q"].cpu() != st["factored_row_q"]).any(dim=0)  # shape[:-1]
                cold = (gs["factored_col_q"].cpu() != st["factored_col_q"]).any(dim=0)  # shape[:-2]+(C,)
                t |= rowd.unsqueeze(-1).expand(shape)
                t |= cold.unsqueeze(-2).expand(shape)
            else:
                t |= gs["exp_avg_sq_q"].cpu() != st["exp_avg_sq_q"]
            tainted[i] |= t
    return [Lockstep(ps[i].data, refs[i], opt.state[ps[i]], sts[i], tainted[i], flips[i], movement[i], bounds[i].D)
            for i in range(len(ps))]


def check_untainted_params(gp: torch.Tensor, rp: torch.Tensor, tainted: torch.Tensor, where: str,
                           movement: torch.Tensor | None = None, tol: float = 1e-5) -> float:
    """Untainted elements, fp32: |dp| <= 1e-5 * (|p_ref| + sum_steps |p_ref step change|) + 1e-7 * rms(p_ref);
    bf16/fp16: within 1 ulp, or within that bound.  Returns the tainted fraction.

    Relative to the movement as well as to the value: where lr*|step| is comparable to or larger
    than |p| (small matrices, whose residual factors are large), an ulp-level relative difference
    of the update is that large relative to the parameter scale."""
    keep = ~tainted.reshape(-1)
    g = gp.detach().cpu().reshape(-1)
    r = rp.detach().cpu().reshape(-1)
    mv = torch.zeros(r.shape, dtype=torch.float64) if movement is None else movement.reshape(-1)
    if keep.any():
        rd, gd = r.double(), g.double()
        rms = rd.pow(2).mean().sqrt().item()
        err = ((gd - rd).abs() / (rd.abs() + mv + 1e-2 * rms + 1e-38))
        if r.dtype == torch.float32:
            worst = err[keep].max().item()
            assert worst <= tol, f"{where}: untainted param err {worst:.3e} > {tol}"
        else:
            ai = g.contiguous().view(torch.int16).to(torch.int32)
            bi = r.contiguous().view(torch.int16).to(torch.int32)
            ordered = lambda x: torch.where(x < 0, -(x & 0x7FFF), x)  # noqa: E731
            ulps = (ordered(ai) - ordered(bi)).abs()
            ok = (ulps <= 1) | (err <= tol)
            assert bool(ok[keep].all()), f"{where}: untainted low-precision params beyond 1 ulp (max {int(ulps[keep].max())})"
    return float(tainted.float().mean())


def run_teacher_forced(cls, params, grads_per_step, hp: dict, steps: int, exact_norm=False, device="cuda",
                       check=None):
    """Every step starts the GPU from the oracle's state and parameters of the previous step, so each
    step's arithmetic is compared on identical inputs (no divergence carried from earlier code flips).
    Both sides take the reference's float32 norm by default, and the exactly rounded norm with
    exact_norm=True (the library's opt-in mode and the oracle's matching variant).
    `check(step, i, gpu_param, ref_param, gpu_state, ref_state, movement)` is called per tensor."""
    ohp = oracle_hp(hp)
    ps = [torch.nn.Parameter(p.clone().to(device)) for p in params]
    opt = cls(ps, **hp)
    opt.exact_norm = exact_norm
    refs = [p.clone() for p in params]
    sts = [orc.init_full8bit_state(p.shape, ohp["block_size"]) for p in refs]
    for s in range(steps):
        with torch.no_grad():
            for p, r, st in zip(ps, refs, sts):
                p.data.copy_(r.to(device))
                gst = opt.state[p]
                if len(gst):
                    for k in STATE_KEYS:
                        if k in st:
                            gst[k].copy_(st[k].to(device))
        for p, g in zip(ps, grads_per_step[s]):
            p.grad = g.to(device)
        opt.step()
        torch.cuda.synchronize()
        for i, (r, g, st) in enumerate(zip(refs, grads_per_step[s], sts)):
            before = r.double()
            cap = {}
            orc.full8bit_step(r, g, st, capture=cap, exact_norm=exact_norm, **ohp)
            mv = (r.double() - before).abs()
            if check is not None:
                check(s + 1, i, ps[i].data, r, opt.state[ps[i]], st, mv, cap)
    return ps, opt, refs, sts
