"""Write golden vectors for the CAME 8-bit CPU oracle from the reference's own CPU path.

Run in the build container only (the reference tree is not present on GPU boxes):

    PYTHONDONTWRITEBYTECODE=1 python tests/golden/make_golden.py

It imports the reference package read-only from ``/root/reference`` and drives
``CAME8bitFull`` / ``CAME8bit`` / ``CAME8bitMemory`` on CPU tensors, which
routes every parameter through ``CAME8bitFull._step_param``'s pure-torch branch
(reference ``came_pytorch/CAME8bitFull.py:1006-1075``; ``CAME8bit.py:749-861``
falls through to it for CPU tensors).  The multi-step composite with
quantisation feedback has no closed form, so these vectors are what pins the
oracle (``oracle/came8_oracle.py``) for it.

Outputs (numpy ``.npz``, no pickles):
  * ``golden_small.npz``  -- inputs and full outputs after step 1 and step 10
    for a set of small and ragged shapes;
  * ``golden_c1_digest.npz`` -- SHA-256 digests plus a strided sample of the
    config-1 run (2048x2048 fp32 weight + 2048 bias, 10 steps);
  * ``golden_camecuda.npz`` -- the same as ``golden_small.npz`` for the
    reference's ``CAMECUDA`` on CPU tensors, whose fp32-state step is its
    pure-torch ``_step_param_generic`` (``came_pytorch/CAMECUDA.py:275-326``).

``--camecuda`` writes only ``golden_camecuda.npz``.
All runs use ``torch.set_num_threads(4)`` so that torch's parallel reductions
split the same way when the oracle replays them.
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"
THREADS = 4

# (name, class, shapes, p dtype, grad kind, hyper-parameters)
SMALL_CASES = [
    ("full_ragged_fp32", "CAME8bitFull",
     [(1,), (3,), (255,), (257,), (1000, 3), (3, 517), (129, 257), (2, 3, 5, 7), (4, 1, 1), (64, 64)],
     "float32", "normal", dict(lr=2e-4, weight_decay=1e-2)),
    ("came8bit_heavy_fp32", "CAME8bit",
     [(5,), (300,), (17, 300), (260, 9), (3, 3, 4, 4), (1, 1)],
     "float32", "heavy", dict(lr=1e-3, weight_decay=0.0)),
    ("memory_bf16", "CAME8bitMemory",
     [(64, 96), (96,), (33, 65)],
     "bfloat16", "normal", dict(lr=2e-4, weight_decay=1e-2, betas=(0.9, 0.95, 0.995))),
    ("full_zero_grads", "CAME8bitFull",
     [(40,), (31, 45)],
     "float32", "zero", dict(lr=1e-3, weight_decay=1e-1)),
    ("came8bit_bs64_clip", "CAME8bit",
     [(100,), (70, 130)],
     "float32", "normal", dict(lr=5e-4, weight_decay=1e-2, block_size=64, clip_threshold=0.5)),
]
NSTEPS = 10

# CAMECUDA (fp32 states) on CPU tensors: (name, shapes, p dtype, grad kind, hyper-parameters)
CAMECUDA_CASES = [
    ("cudafp_ragged_fp32", [(1,), (3,), (255,), (257,), (1000, 3), (3, 517), (129, 257), (2, 3, 5, 7), (4, 1, 1)],
     "float32", "normal", dict(lr=2e-4, weight_decay=1e-2)),
    ("cudafp_heavy_bf16", [(5,), (300,), (17, 300), (260, 9), (3, 3, 4, 4), (1, 1)],
     "bfloat16", "heavy", dict(lr=1e-3, weight_decay=1e-2, betas=(0.9, 0.95, 0.995))),
    ("cudafp_clip_fp32", [(100,), (70, 130)],
     "float32", "normal", dict(lr=5e-4, weight_decay=0.0, clip_threshold=0.5)),
]


def make_grad(gen: torch.Generator, shape, kind: str, dtype: torch.dtype) -> torch.Tensor:
    if kind == "normal":
        g = torch.randn(shape, generator=gen) * 1e-3
    elif kind == "heavy":
        # Student-t(2) scaled by 1e-3, 10% exact zeros, occasional 1e3 outliers
        z = torch.randn(shape, generator=gen)
        chi = torch.randn((2,) + tuple(shape), generator=gen)
        t = z / torch.sqrt((chi ** 2).mean(dim=0))
        g = t * 1e-3
        mask = torch.rand(shape, generator=gen) < 0.1
        g = torch.where(mask, torch.zeros_like(g), g)
        flat = g.reshape(-1)
        if flat.numel() >= 16:
            pick = torch.randint(0, flat.numel(), (max(1, flat.numel() // 256),), generator=gen)
            sign = torch.where(torch.rand(pick.shape, generator=gen) < 0.5, -1.0, 1.0)
            flat[pick] = 1e3 * sign
    elif kind == "zero":
        g = torch.zeros(shape)
    else:
        raise ValueError(kind)
    return g.to(dtype)


def state_arrays(prefix: str, state: dict, out: dict) -> None:
    for k, v in state.items():
        if isinstance(v, torch.Tensor):
            if k in ("exp_avg_sq_row_q", "exp_avg_res_row_q", "exp_avg_sq_col_q", "exp_avg_res_col_q",
                     "exp_avg_sq_row_absmax", "exp_avg_res_row_absmax", "exp_avg_sq_col_absmax",
                     "exp_avg_res_col_absmax"):
                continue  # views of factored_* tensors
            arr = v.detach().cpu()
            if arr.dtype == torch.bfloat16:
                arr = arr.view(torch.int16)
            out[f"{prefix}/{k}"] = arr.numpy().copy()
        elif isinstance(v, (bool, int, float)):
            out[f"{prefix}/{k}"] = np.array(v)


def p_array(p: torch.Tensor) -> np.ndarray:
    t = p.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)
    return t.numpy().copy()


def run_small(mod, out: dict, meta: dict) -> None:
    for ci, (name, cls_name, shapes, pdt, kind, hp) in enumerate(SMALL_CASES):
        dtype = getattr(torch, pdt)
        gen = torch.Generator().manual_seed(1000 + ci)
        params = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(dtype)) for s in shapes]
        for i, p in enumerate(params):
            out[f"{name}/p0/{i}"] = p_array(p)
        opt = getattr(mod, cls_name)(params, **hp)
        for step in range(1, NSTEPS + 1):
            for i, (p, s) in enumerate(zip(params, shapes)):
                g = make_grad(gen, s, kind, dtype)
                out[f"{name}/g{step}/{i}"] = p_array(g)
                p.grad = g
            opt.step()
            if step in (1, NSTEPS):
                for i, p in enumerate(params):
                    out[f"{name}/p{step}/{i}"] = p_array(p)
                    state_arrays(f"{name}/s{step}/{i}", opt.state[p], out)
        meta[name] = dict(cls=cls_name, shapes=[list(s) for s in shapes], dtype=pdt, grad=kind, hp=hp,
                          steps=NSTEPS)


def run_camecuda(mod, out: dict, meta: dict) -> None:
    for ci, (name, shapes, pdt, kind, hp) in enumerate(CAMECUDA_CASES):
        dtype = getattr(torch, pdt)
        gen = torch.Generator().manual_seed(2000 + ci)
        params = [torch.nn.Parameter((torch.randn(s, generator=gen) * 0.02).to(dtype)) for s in shapes]
        for i, p in enumerate(params):
            out[f"{name}/p0/{i}"] = p_array(p)
        opt = mod.CAMECUDA(params, **hp)
        for step in range(1, NSTEPS + 1):
            for i, (p, s) in enumerate(zip(params, shapes)):
                g = make_grad(gen, s, kind, dtype)
                out[f"{name}/g{step}/{i}"] = p_array(g)
                p.grad = g
            opt.step()
            if step in (1, NSTEPS):
                for i, p in enumerate(params):
                    out[f"{name}/p{step}/{i}"] = p_array(p)
                    state_arrays(f"{name}/s{step}/{i}", opt.state[p], out)
        meta[name] = dict(cls="CAMECUDA", shapes=[list(s) for s in shapes], dtype=pdt, grad=kind, hp=hp,
                          steps=NSTEPS)


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def c1_inputs():
    """Config 1: fp32 2048x2048 weight + 2048 bias, params N(0, 0.02^2) seed 0, grads N(0, 1e-3^2) seed 1+step."""
    gen = torch.Generator().manual_seed(0)
    w = torch.randn(2048, 2048, generator=gen) * 0.02
    b = torch.randn(2048, generator=gen) * 0.02
    return w, b


def c1_grads(step: int):
    gen = torch.Generator().manual_seed(1 + step)
    return torch.randn(2048, 2048, generator=gen) * 1e-3, torch.randn(2048, generator=gen) * 1e-3


def run_c1(mod, out: dict, meta: dict) -> None:
    w, b = c1_inputs()
    params = [torch.nn.Parameter(w.clone()), torch.nn.Parameter(b.clone())]
    opt = mod.CAME8bit(params, lr=2e-4, weight_decay=1e-2, betas=(0.9, 0.999, 0.9999), eps=(1e-30, 1e-16))
    digests = {}
    for step in range(1, NSTEPS + 1):
        gw, gb = c1_grads(step)
        params[0].grad, params[1].grad = gw, gb
        opt.step()
        if step in (1, NSTEPS):
            for i, p in enumerate(params):
                digests[f"s{step}/p{i}"] = digest(p.data)
                for k, v in opt.state[p].items():
                    if isinstance(v, torch.Tensor) and v.dim() > 0 and not k.startswith("exp_avg_sq_row") \
                            and not k.startswith("exp_avg_res_") and not k.startswith("exp_avg_sq_col"):
                        digests[f"s{step}/p{i}/{k}"] = digest(v)
                out[f"c1/s{step}/p{i}/sample"] = p.data.reshape(-1)[::997].numpy().copy()
                st = opt.state[p]
                out[f"c1/s{step}/p{i}/exp_avg_q_sample"] = st["exp_avg_q"].reshape(-1)[::997].numpy().copy()
                out[f"c1/s{step}/p{i}/exp_avg_absmax"] = st["exp_avg_absmax"].numpy().copy()
                if st["factored"]:
                    for k in ("factored_row_q", "factored_row_absmax", "factored_col_q", "factored_col_absmax"):
                        out[f"c1/s{step}/p{i}/{k}"] = st[k].numpy().copy()
                else:
                    for k in ("exp_avg_sq_q", "exp_avg_sq_absmax"):
                        out[f"c1/s{step}/p{i}/{k}"] = st[k].numpy().copy()
    out["c1/digests_json"] = np.array(json.dumps(digests, sort_keys=True))
    meta["c1"] = dict(cls="CAME8bit", steps=NSTEPS, lr=2e-4, weight_decay=1e-2)


def main() -> None:
    torch.set_num_threads(THREADS)
    sys.path.insert(0, REF)
    import came_pytorch as mod  # noqa: E402  (reference, read-only, CPU path only)

    meta = {"torch": torch.__version__, "threads": THREADS, "reference": REF}
    out: dict = {}
    if "--camecuda" in sys.argv[1:]:
        run_camecuda(mod, out, meta)
        out["meta_json"] = np.array(json.dumps(meta, sort_keys=True))
        np.savez_compressed(os.path.join(HERE, "golden_camecuda.npz"), **out)
        print("wrote", os.path.join(HERE, "golden_camecuda.npz"))
        return
    run_small(mod, out, meta)
    out["meta_json"] = np.array(json.dumps(meta, sort_keys=True))
    np.savez_compressed(os.path.join(HERE, "golden_small.npz"), **out)

    out = {}
    run_c1(mod, out, meta)
    np.savez_compressed(os.path.join(HERE, "golden_c1_digest.npz"), **out)
    print("wrote golden fixtures:", sorted(os.listdir(HERE)))


if __name__ == "__main__":
    main()
