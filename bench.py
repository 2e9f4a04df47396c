#!/usr/bin/env python3
"""Benchmark of the CAME 8-bit optimizer step on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c4] [--no-cpu-baseline]

Workload (default, the headline config c4): a Llama-7B-shape parameter set -- 32 layers, d=4096,
SwiGLU FFN 11008, vocab 32000 embedding and lm_head, RMSNorm weights; 291 tensors, 6,738,415,616
bf16 parameters with bf16 gradients ~ N(0, 2e-4^2) -- stepped by ``came_amd.CAME8bit``
(lr 2e-4, weight decay 1e-2, betas (0.9, 0.999, 0.9999), int8 blockwise momentum, block 256).
Parameters ~ N(0, 0.02^2); inputs are generated on the GPU before timing and stay resident.

A "step" is one full optimizer step over every tensor.  The timed region is exactly K steps,
bracketed by torch.cuda.synchronize().  Printed as one JSON line:
  value      algorithmic HBM GB/s of the whole step = compulsory bytes per step / step time,
             compulsory bytes (per factored R x C tensor of N elements):
               N*(s_g + 2*s_p + 2) + 8*ceil(N/256) + 4*(R+C) + 16*(ceil(R/256)+ceil(C/256))
             per 1-D tensor of n elements: n*(s_g + 2*s_p + 4) + 16*ceil(n/256)
  roofline   the dominant kernel (most device time): its algorithmic bytes per launch over its
             average launch time, both measured live with HIP events on the launch stream
             (came8_profile_*) over up to 5 further steps after the timed ones, against MI355X's
             8 TB/s HBM peak
  cpu_baseline  the CPU oracle (oracle/came8_oracle.py, op-for-op restatement of the reference's
             pure-PyTorch path) timed on this host on a bounded sample of the same workload
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

METRIC = "CAME8bit step time (ms) + achieved HBM GB/s, Llama-7B param set, 1 MI355X"
HBM_PEAK_GBS = 8000.0

# HBM-side bytes per launch of the dominant kernel, from rocprofv3 FETCH_SIZE / WRITE_SIZE runs of this
# bench (calibrated against a copy of known size: fetch x2, write x1); the summary, with its commands,
# is the file named in "source".  Re-measured whenever that kernel changes.
PROFILED_TRAFFIC = {
    ("c4", "pass3"): {"read": 34.107e9, "write": 20.342e9, "source": "profiles/c4_step_hbm_traffic.md"},
}


# ------------------------------------------------------------------------------------ workloads
def llama_shapes(layers, d, ffn, vocab):
    shapes = [(vocab, d)]
    for _ in range(layers):
        shapes += [(d, d), (d, d), (d, d), (d, d), (ffn, d), (ffn, d), (d, ffn), (d,), (d,)]
    shapes += [(d,), (vocab, d)]
    return shapes


def gpt2_medium_shapes():
    d, L, V, P = 1024, 24, 50257, 1024
    shapes = [(V, d), (P, d)]
    for _ in range(L):
        shapes += [(d,), (d,), (3 * d, d), (3 * d,), (d, d), (d,), (d,), (d,), (4 * d, d), (4 * d,), (d, 4 * d), (d,)]
    shapes += [(d,), (d,)]
    return shapes


def ragged_shapes(seed=0):
    """The ragged stress set (config c5): 500 tensors -- 250 1-D lengths U{1..4097}; the 2-D shapes 1000x3, 3x50257 and
    4097x129; conv weights 320x320x3x3 and 1280x640x1x1; 245 2-D shapes with rows and columns drawn from
    [1, 5000] outside multiples of 64."""
    gen = torch.Generator().manual_seed(seed)
    shapes = [(int(n),) for n in torch.randint(1, 4098, (250,), generator=gen)]
    shapes += [(1000, 3), (3, 50257), (4097, 129), (320, 320, 3, 3), (1280, 640, 1, 1)]
    while len(shapes) < 500:
        r, c = (int(x) for x in torch.randint(1, 5001, (2,), generator=gen))
        if r % 64 and c % 64:
            shapes.append((r, c))
    return shapes


def heavy_grad(shape, gen, dtype, device="cuda"):
    """1e-3 * Student-t(nu=2) (a normal over sqrt(Exp(1)), i.e. over sqrt(chi2_2 / 2)), 10% exact zeros,
    and in each flat block of 256 elements, with probability 1/2, one element set to +-1e3."""
    n = math.prod(shape)
    z = torch.randn(n, device=device, generator=gen)
    e = torch.rand(n, device=device, generator=gen).clamp_min_(1e-30).log_().neg_()
    g = z.div_(e.sqrt_()).mul_(1e-3)
    g.masked_fill_(torch.rand(n, device=device, generator=gen) < 0.1, 0.0)
    nb = (n + 255) // 256
    pos = torch.arange(nb, device=device) * 256 + torch.randint(0, 256, (nb,), device=device, generator=gen)
    pick = (torch.rand(nb, device=device, generator=gen) < 0.5) & (pos < n)
    sign = torch.where(torch.rand(nb, device=device, generator=gen) < 0.5, -1e3, 1e3)
    g[pos[pick]] = sign[pick]
    return g.reshape(shape).to(dtype)


def grad_stds(gspec, n, seed=1):
    """Per-tensor gradient standard deviations for a config's gradient spec: a float (the same for every
    tensor), None (heavy_grad, no std), or ("loguniform", base, lo, hi): base * 10^U(lo, hi) per tensor,
    drawn from a CPU generator of its own (N(0, 1e-3^2) times a per-tensor scale
    log-uniform in [1e-5, 1e-2])."""
    if gspec is None or isinstance(gspec, float):
        return [gspec] * n
    kind, base, lo, hi = gspec
    assert kind == "loguniform", gspec
    gen = torch.Generator().manual_seed(seed)
    u = torch.rand(n, generator=gen, dtype=torch.float64)
    return [base * 10.0 ** (lo + (hi - lo) * float(x)) for x in u]


CONFIGS = {
    # name: (workload label, shapes, param dtype, grad dtype, grad spec (grad_stds), optimizer, hparams)
    "c4": ("llama7b-shape/CAME8bit/bf16", lambda: llama_shapes(32, 4096, 11008, 32000), torch.bfloat16,
           torch.bfloat16, 2e-4, "CAME8bit", dict(lr=2e-4, weight_decay=1e-2, betas=(0.9, 0.999, 0.9999))),
    "c3": ("llama1b-style/CAME8bitMemory/bf16", lambda: llama_shapes(24, 2048, 5461, 32000), torch.bfloat16,
           torch.bfloat16, 5e-4, "CAME8bitMemory", dict(lr=2e-4, weight_decay=1e-2, betas=(0.9, 0.95, 0.995))),
    "c2": ("gpt2-medium/CAME8bit/fp32", gpt2_medium_shapes, torch.float32, torch.float32, ("loguniform", 1e-3, -5, -2),
           "CAME8bit", dict(lr=2e-4, weight_decay=1e-2)),
    "c1": ("2048x2048+2048/CAME8bit/fp32", lambda: [(2048, 2048), (2048,)], torch.float32, torch.float32, 1e-3,
           "CAME8bit", dict(lr=2e-4, weight_decay=1e-2)),
    # the Llama-7B matrices stepped by CAME8bit2D (8bit2d layout: momentum in 16x16 tiles; 2-D only)
    "c4_2d": ("llama7b-shape matrices/CAME8bit2D/bf16",
              lambda: [s for s in llama_shapes(32, 4096, 11008, 32000) if len(s) == 2], torch.bfloat16,
              torch.bfloat16, 2e-4, "CAME8bit2D", dict(lr=2e-4, weight_decay=1e-2, betas=(0.9, 0.999, 0.9999))),
    # the same Llama-7B set stepped by CAMECUDA (fp32 optimizer states)
    "c4fp": ("llama7b-shape/CAMECUDA/bf16", lambda: llama_shapes(32, 4096, 11008, 32000), torch.bfloat16,
             torch.bfloat16, 2e-4, "CAMECUDA", dict(lr=2e-4, weight_decay=1e-2, betas=(0.9, 0.999, 0.9999))),
    # the ragged stress set, heavy-tailed gradients, CAME8bitFull
    "c5": ("ragged-500/CAME8bitFull/fp32", ragged_shapes, torch.float32, torch.float32, None, "CAME8bitFull",
           dict(lr=2e-4, weight_decay=1e-2)),
}


def esize(dt):
    return torch.tensor([], dtype=dt).element_size()


def compulsory_bytes(shapes, pdt, gdt, block=256, fp32_state=False, tiles=False):
    """Bytes every step must move: gradient read, parameter and momentum codes read and written, momentum
    scales (one per block of 256, or per 16x16 tile with `tiles`) read and written, row/column states."""
    sg, sp = esize(gdt), esize(pdt)
    tot = 0
    for s in shapes:
        n = math.prod(s)
        if tiles:
            r, c = s
            tot += n * (sg + 2 * sp + 2) + 8 * math.ceil(r / 16) * math.ceil(c / 16) + 4 * (r + c) \
                + 16 * (math.ceil(r / block) + math.ceil(c / block))
            continue
        if fp32_state:  # fp32 momentum (and 1-D second moment) read and written; fp32 row/col states
            if len(s) >= 2:
                pr, pc = math.prod(s[:-1]), math.prod(s[:-2]) * s[-1]
                tot += n * (sg + 2 * sp + 8) + 16 * (pr + pc)
            else:
                tot += n * (sg + 2 * sp + 16)
            continue
        if len(s) >= 2:
            pr, pc = math.prod(s[:-1]), math.prod(s[:-2]) * s[-1]
            tot += n * (sg + 2 * sp + 2) + 8 * math.ceil(n / block) + 4 * (pr + pc) \
                + 16 * (math.ceil(pr / block) + math.ceil(pc / block))
        else:
            tot += n * (sg + 2 * sp + 4) + 16 * math.ceil(n / block)
    return tot


# --------------------------------------------------------------------------------- CPU baseline
CPU_SAMPLE_MAX = 400_000_000  # elements the CPU baseline steps (about 10-20 s of CPU work in all)


def sample_index(cfg_name, shapes):
    """Indices of the tensors the CPU baseline steps (cpu_sample)."""
    idx = list(range(len(shapes)))
    if sum(math.prod(s) for s in shapes) <= CPU_SAMPLE_MAX:
        return idx
    if cfg_name in ("c3", "c4", "c4fp"):
        return idx[:10] + idx[-2:]
    k = 1
    while sum(math.prod(shapes[i]) for i in idx[::k]) > CPU_SAMPLE_MAX:
        k += 1
    return idx[::k]


def cpu_sample(cfg_name, shapes):
    """The tensors the CPU baseline steps: the whole workload when it is small enough; for the
    Llama-shaped sets the embedding, the first decoder layer, the final norm and the lm_head (the
    other layers repeat the first); otherwise every k-th tensor."""
    idx = sample_index(cfg_name, shapes)
    sample = [shapes[i] for i in idx]
    if len(idx) == len(shapes):
        return sample, "the whole workload"
    if cfg_name in ("c3", "c4", "c4fp"):
        return sample, "embedding + decoder layer 0 + final norm + lm_head"
    return sample, f"every {idx[1] - idx[0]}-th tensor"


def cpu_model_name() -> str:
    """lscpu's model name (the host CPU), else /proc/cpuinfo's."""
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            return next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "unknown")
    except OSError:
        return "unknown"


def cpu_baseline(cfg_name, shapes, pdt, gdt, gstd, hp, fp32_state=False, tiles=False):
    """Time the CPU oracle on a bounded sample of the workload (cpu_sample): one warm-up step, then
    the median of three; returns the cpu_baseline object."""
    from oracle import came8_oracle as orc

    sample, how = cpu_sample(cfg_name, shapes)
    gen = torch.Generator().manual_seed(123)
    params = [(torch.randn(s, generator=gen) * 0.02).to(pdt) for s in sample]
    stds = dict(zip(range(len(shapes)), grad_stds(gstd, len(shapes))))
    pick = sample_index(cfg_name, shapes)
    grads = [(torch.randn(s, generator=gen) * (stds[i] or 1e-3)).to(gdt) for s, i in zip(sample, pick)]
    b1, b2, b3 = hp.get("betas", (0.9, 0.999, 0.9999))
    ohp = dict(beta1=b1, beta2=b2, beta3=b3, eps0=1e-30, eps1=1e-16, lr=hp["lr"], clip_threshold=1.0,
               weight_decay=hp.get("weight_decay", 0.0), block_size=256)
    if fp32_state:
        states = [orc.init_fp32_state(s) for s in sample]
        ohp.pop("block_size")
        step_fn = orc.fp32_state_step
    elif tiles:
        states = [orc.init_8bit2d_state(s) for s in sample]
        step_fn = orc.came8bit2d_step
    else:
        states = [orc.init_full8bit_state(s) for s in sample]
        step_fn = orc.full8bit_step
    # every core this process may run on: os.cpu_count(), within the affinity mask and the host's
    # OMP_NUM_THREADS (the box's share of a shared host)
    host = os.cpu_count() or 1
    cores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else host
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        cores = min(cores, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(max(1, min(host, cores)))
    times = []
    for it in range(4):
        t0 = time.perf_counter()
        for p, g, st in zip(params, grads, states):
            step_fn(p, g, st, **ohp)
        times.append(time.perf_counter() - t0)
        print(f"[bench] cpu baseline step {it}: {times[-1] * 1e3:.0f} ms", file=sys.stderr, flush=True)
    t = sorted(times[1:])[1]  # the first step allocates; the median of the next three
    nbytes = compulsory_bytes(sample, pdt, gdt, fp32_state=fp32_state, tiles=tiles)
    n_sample = sum(math.prod(s) for s in sample)
    n_total = sum(math.prod(s) for s in shapes)
    return {
        "value": round(nbytes / t / 1e9, 4),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "cpu_model": cpu_model_name(),
        "kind": "port",
        "sample": f"{how}: {len(sample)} tensors, {n_sample} elements of {cfg_name}; the oracle's step, one warm-up "
                  f"then the median of 3: {t * 1e3:.1f} ms; the whole workload extrapolated by element count: "
                  f"{t * n_total / n_sample * 1e3:.0f} ms/step",
        "ms_per_step_extrapolated": round(t * n_total / n_sample * 1e3, 1),
        "os_cpu_count": host,
        "torch_threads": torch.get_num_threads(),
    }


# ------------------------------------------------------------------------------------------ main
def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="c4", choices=sorted(CONFIGS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--exact-norm", action="store_true",
                    help="the opt-in clip norm (exactly rounded fp64 sum) instead of the reference's fp32 order")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="instead of the step, copy a MIB-sized device buffer --steps times (a plain copy "
                         "kernel of known bytes, to scale the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (--gpus {args.gpus} requested); across GPUs the "
              "optimizer step shards by tensor (each GPU steps its own tensors, no exchange during the step)",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").random_()
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        dt = (time.perf_counter() - t0) / args.steps
        print(json.dumps({"copy_calibration_bytes_read": n, "copy_calibration_bytes_written": n,
                          "ms_per_copy": round(dt * 1e3, 4), "GBps_read_plus_write": round(2 * n / dt / 1e9, 1)}))
        return

    import came_amd
    from came_amd import _lib

    label, shapes_fn, pdt, gdt, gstd, cls_name, hp = CONFIGS[args.config]
    shapes = shapes_fn()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    gen = torch.Generator(device=dev).manual_seed(0)
    params, grads = [], []
    for s, std in zip(shapes, grad_stds(gstd, len(shapes))):
        p = torch.randn(s, device=dev, dtype=torch.float32, generator=gen).mul_(0.02).to(pdt)
        if std is None:
            g = heavy_grad(s, gen, gdt, device=dev)
        else:
            g = torch.randn(s, device=dev, dtype=torch.float32, generator=gen).mul_(std).to(gdt)
        params.append(torch.nn.Parameter(p))
        params[-1].grad = g
        grads.append(g)
    opt = getattr(came_amd, cls_name)(params, **hp)
    opt.exact_norm = bool(args.exact_norm)
    print(f"[bench] {label}: {len(shapes)} tensors, {sum(math.prod(s) for s in shapes)} params; warmup {args.warmup}",
          file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        opt.step()
    torch.cuda.synchronize()

    # the timed steps run exactly as a user's would (no per-kernel events)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        opt.step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    # then a few more steps with every launch bracketed by HIP events on its stream, for the
    # per-kernel times and the roofline of the dominant kernel
    prof_steps = max(1, min(args.steps, 5))
    _lib.profile_enable(True)
    _lib.profile_read(reset=True)
    for _ in range(prof_steps):
        opt.step()
    torch.cuda.synchronize()
    phases = _lib.profile_read(reset=True)
    _lib.profile_enable(False)
    # the other clip-norm mode on the same optimizer, for comparison (not the reported value)
    other_ms = None
    if cls_name != "CAME8bit2D":
        opt.exact_norm = not bool(args.exact_norm)
        for _ in range(2):
            opt.step()
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        for _ in range(args.steps):
            opt.step()
        torch.cuda.synchronize()
        other_ms = (time.perf_counter() - t2) * 1e3 / args.steps
        opt.exact_norm = bool(args.exact_norm)

    ms = (t1 - t0) * 1e3 / args.steps
    fp32_state = cls_name == "CAMECUDA"
    tiles = cls_name == "CAME8bit2D"
    nbytes = compulsory_bytes(shapes, pdt, gdt, fp32_state=fp32_state, tiles=tiles)
    value = nbytes / (ms / 1e3) / 1e9
    dom = max(phases.items(), key=lambda kv: kv[1][1])
    dname, (dl, dms, dbytes) = dom
    achieved = (dbytes / dl) / (dms / dl / 1e3) / 1e9
    phase_rep = {k: {"launches_per_step": v[0] / prof_steps, "ms_per_step": round(v[1] / prof_steps, 4),
                     "alg_GBps": round(v[2] / (v[1] / 1e3) / 1e9, 1) if v[2] > 0 and v[1] > 0 else None}
                 for k, v in sorted(phases.items(), key=lambda kv: -kv[1][1])}
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02^2) params, "
                + ("heavy-tailed Student-t(2)" if gstd is None else f"N(0,{gstd:g}^2)" if isinstance(gstd, float)
                   else f"N(0,{gstd[1]:g}^2) x per-tensor 10^U({gstd[2]},{gstd[3]})")
                + " grads, resident in HBM)",
        "config": {
            "workload": label,
            "tensors": len(shapes),
            "params": sum(math.prod(s) for s in shapes),
            "param_dtype": str(pdt).replace("torch.", ""),
            "grad_dtype": str(gdt).replace("torch.", ""),
            "state": "fp32 momentum + fp32 row/col factors" if fp32_state
            else "int8 momentum in 16x16 tiles + uint8 row/col factors, block 256" if tiles
            else "int8 momentum + uint8 row/col factors, block 256",
            "clip_norm": "exact fp64 (opt-in)" if args.exact_norm else "reference fp32 order (default)",
            "compulsory_bytes_per_step": nbytes,
            "step_roofline_frac": round(value / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dname,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (PROFILED_TRAFFIC[(args.config, dname)]["read"] + PROFILED_TRAFFIC[(args.config, dname)]["write"])
            if (args.config, dname) in PROFILED_TRAFFIC else None,
            "traffic_source": PROFILED_TRAFFIC.get((args.config, dname), {}).get("source"),
            "alg_bytes_per_launch": dbytes / dl,
            "avg_launch_ms": round(dms / dl, 4),
        },
        "phases": phase_rep,
    }
    if other_ms is not None:
        out["other_clip_mode"] = {
            "clip_norm": "reference fp32 order (default)" if args.exact_norm else "exact fp64 (opt-in)",
            "ms_per_step": round(other_ms, 4)}
    if not args.no_cpu_baseline:
        print("[bench] timing the CPU oracle on a sample", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline(args.config, shapes, pdt, gdt, gstd, hp, fp32_state=fp32_state,
                                           tiles=tiles)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
