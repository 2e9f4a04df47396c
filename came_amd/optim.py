"""CAME 8-bit optimizers whose step runs in libcame8 (hand-written HIP kernels for MI355X).

Drop-in replacements for the reference classes of the same names:

  * ``CAME8bitFull``   -- came_pytorch/CAME8bitFull.py:39-120 (constructor), :748-937 (state),
                          :939-1118 (step)
  * ``CAME8bit``       -- came_pytorch/CAME8bit.py:24-206 (constructor and kwarg validation),
                          :672-693 (prime_for_cuda_graph), :712-912 (step)
  * ``CAME8bitMemory`` -- came_pytorch/CAME8bitMemory.py:17-52 (constructor), :390-447 (state),
                          :559-635 (step)

Same constructor arguments, defaults and ``ValueError`` texts, same param-group
keys, same per-parameter state keys, dtypes and shapes as the reference's
full8bit layout (flat row-major 256-element blocks, ``CAME8bitFull.py:748-788``).
Each ``step()`` hands every parameter of a param group to ONE ``came8_step``
call (include/came8.h), which runs the whole update as a few multi-tensor
launches on the current stream: no per-parameter launches, no host sync.

Parameters must live on the GPU; there is no CPU path (the reference's CPU
arithmetic is the test oracle, not part of this package).
"""
from __future__ import annotations

import ctypes
import math
import time
import warnings
import weakref
from collections import Counter, defaultdict
from itertools import chain

import torch
import torch.optim

from . import _lib
from . import state_layout
from .blockwise_quantization import init_batched_qstate, init_qstate, num_blocks

_DTYPE_CODE = {torch.float32: _lib.CAME8_F32, torch.bfloat16: _lib.CAME8_BF16, torch.float16: _lib.CAME8_F16}

_VIEW_KEYS = (
    "exp_avg_sq_row_q", "exp_avg_res_row_q", "exp_avg_sq_col_q", "exp_avg_res_col_q",
    "exp_avg_sq_row_absmax", "exp_avg_res_row_absmax", "exp_avg_sq_col_absmax", "exp_avg_res_col_absmax",
)


# The reference's per-parameter routing flags.  Its CPU path writes every one as False
# (CAME8bitFull.py:783-787, 921; CAME8bitMemory.py:431-447; CAMECUDA.py:117-118); so does this build,
# whose kernels read none of the per-tensor scratch buffers a True flag promises the reference.
_FACTORED_FLAGS = ("_cuda_factored_fastpath", "_cuda_factored_nd_ext_path", "_cuda_factored_nd_chunked_ext_path",
                   "_cuda_factored_ext_path")
_NONFACTORED_FLAGS = ("_cuda_nonfactored_fastpath",)
_FP32_FLAGS = ("_cuda_fp_factored_fastpath", "_cuda_fp_nonfactored_fastpath")
# Per-tensor scratch the reference's CUDA paths keep in the state (CAME8bitFull.py:790-937,
# CAMECUDA.py:120-140; 12-16 bytes per element).  A state loaded from such a run drops them (the
# library's workspace replaces them) and its flags are set False, so the state saved back loads in the
# reference, which then takes its generic path.
_REFERENCE_SCRATCH_KEYS = (
    "exp_avg_fp32", "scratch_fp32", "grad_fp32", "update_fp32", "_cuda_nonfactored_update_fp16",
    "row_factor_fp32", "col_factor_fp32", "row_mean_fp32", "factored_row_fp32", "factored_col_fp32",
    "row_absmax_scratch", "reduce_partial", "sum_row_state", "sum_update", "sum_update_partial",
    "sum_update_slice", "sum_update_chunk", "sum_update_equiv", "row_workspace", "col_workspace",
    "param_workspace", "matrix_rows", "matrix_cols", "prefix_batch", "nd_chunk_size",
    "_cuda_factored_nd_chunked_direct_row_sum",
)


def _release_workspace(ptr: int) -> None:
    try:
        _lib.load().came8_release_workspace(ptr)
    except Exception:  # interpreter shutdown
        pass


class _Came8Base(torch.optim.Optimizer):
    """Shared step machinery: state layout, descriptor table, workspace, one library call per group."""

    _MODE = "full8bit"                 # state["_mode"] of this optimizer's layout
    # layouts the library steps in place (state_layout.layout_of): this optimizer's own, and for full8bit
    # the reference CUDA N-D path's per-matrix blocks (CAME8_STATE_Q8_MATRIX)
    _IN_PLACE = ("full8bit", "full8bit-nd")
    _STATE_KIND = _lib.CAME8_STATE_Q8  # how the library reads the state pointers
    _VIEWS_BEFORE_FLAGS = False        # the reference's key order (CAME8bitMemory: views first)

    def _validate_and_defaults(self, lr, eps, clip_threshold, betas, weight_decay, block_size):
        # came_pytorch/CAME8bitFull.py:73-91
        if lr is None or lr <= 0.0:
            raise ValueError(f"lr must be > 0, got {lr}")
        if clip_threshold <= 0.0:
            raise ValueError(f"clip_threshold must be > 0, got {clip_threshold}")
        if len(eps) != 2:
            raise ValueError(f"eps must be a tuple of length 2, got eps={eps}")
        if len(betas) != 3:
            raise ValueError(f"betas must be a tuple of length 3, got betas={betas}")
        if block_size <= 0:
            raise ValueError(f"block_size must be > 0, got {block_size}")
        return dict(
            lr=float(lr),
            eps=(float(eps[0]), float(eps[1])),
            clip_threshold=float(clip_threshold),
            betas=(float(betas[0]), float(betas[1]), float(betas[2])),
            weight_decay=float(weight_decay),
            block_size=int(block_size),
        )

    # ------------------------------------------------------------------ state
    @staticmethod
    def _bind_factored_views(state: dict) -> None:
        """Views of the stacked row/col states (CAME8bitFull.py:214-223; per-matrix layout :188-210)."""
        if state_layout.layout_of(state) == "full8bit-nd":
            P, R, C = state["prefix_batch"], state["matrix_rows"], state["matrix_cols"]
            rq = state["factored_row_q"].view(2, P, R)
            cq = state["factored_col_q"].view(2, P, C)
            ra = state["factored_row_absmax"].view(2, P, -1)
            ca = state["factored_col_absmax"].view(2, P, -1)
            state["exp_avg_sq_row_q"], state["exp_avg_res_row_q"] = rq[0], rq[1]
            state["exp_avg_sq_col_q"], state["exp_avg_res_col_q"] = cq[0], cq[1]
            state["exp_avg_sq_row_absmax"], state["exp_avg_res_row_absmax"] = ra[0], ra[1]
            state["exp_avg_sq_col_absmax"], state["exp_avg_res_col_absmax"] = ca[0], ca[1]
            state["exp_avg_q_batched"] = state["exp_avg_q"].view(P, R, C)
            for k, n in (("row", R), ("col", C)):
                if f"{k}_factor_fp32" in state:  # the reference's scratch, kept for its round trip
                    state[f"{k}_factor_batched"] = state[f"{k}_factor_fp32"].view(P, n)
            return
        state["exp_avg_sq_row_q"] = state["factored_row_q"][0]
        state["exp_avg_res_row_q"] = state["factored_row_q"][1]
        state["exp_avg_sq_col_q"] = state["factored_col_q"][0]
        state["exp_avg_res_col_q"] = state["factored_col_q"][1]
        state["exp_avg_sq_row_absmax"] = state["factored_row_absmax"][0]
        state["exp_avg_res_row_absmax"] = state["factored_row_absmax"][1]
        state["exp_avg_sq_col_absmax"] = state["factored_col_absmax"][0]
        state["exp_avg_res_col_absmax"] = state["factored_col_absmax"][1]

    def _init_state(self, state: dict, grad: torch.Tensor, block_size: int) -> None:
        """The reference's full8bit layout (CAME8bitFull.py:748-788, 919-923)."""
        state["step"] = 0
        state["_mode"] = "full8bit"
        state["RMS"] = 0
        state["exp_avg_q"], state["exp_avg_absmax"] = init_qstate(
            grad.shape, device=grad.device, signed=True, block_size=block_size)
        factored = len(grad.shape) >= 2
        state["factored"] = factored
        if factored:
            row_shape = grad.shape[:-1]
            col_shape = grad.shape[:-2] + grad.shape[-1:]
            state["factored_row_q"], state["factored_row_absmax"] = init_batched_qstate(
                row_shape, batch_size=2, device=grad.device, signed=False, block_size=block_size)
            state["factored_col_q"], state["factored_col_absmax"] = init_batched_qstate(
                col_shape, batch_size=2, device=grad.device, signed=False, block_size=block_size)
            if self._VIEWS_BEFORE_FLAGS:
                self._bind_factored_views(state)
            for k in _FACTORED_FLAGS:
                state[k] = False
            self._bind_factored_views(state)
        else:
            state["exp_avg_sq_q"], state["exp_avg_sq_absmax"] = init_qstate(
                grad.shape, device=grad.device, signed=False, block_size=block_size)
            for k in _NONFACTORED_FLAGS:
                state[k] = False

    def _check_state(self, p: torch.Tensor, state: dict, block_size: int) -> None:
        if tuple(state["exp_avg_q"].shape) != tuple(p.shape):
            raise RuntimeError("Parameter shape changed; this optimizer does not support resizing 8-bit state.")
        if (state["exp_avg_absmax"].numel() != num_blocks(p.numel(), block_size)
                and state_layout.layout_of(state) != "full8bit-nd"):
            raise RuntimeError("block_size changed after the 8-bit state was created; the state layout is fixed.")
        if state["exp_avg_q"].device != p.device:
            raise RuntimeError("optimizer state lives on a different device than its parameter")
        if state.get("factored") and "factored_row_absmax" in state:
            rows = math.prod(p.shape[:-1])
            cols = math.prod(p.shape[:-2]) * p.shape[-1]
            if state_layout.layout_of(state) == "full8bit-nd":
                # per-matrix blocks: [2*P][blocks of R] and [2*P][blocks of C] scales, [P][blocks of R*C]
                P, R, C = math.prod(p.shape[:-2]), p.shape[-2], p.shape[-1]
                if (p.dim() < 3 or (state.get("prefix_batch"), state.get("matrix_rows"), state.get("matrix_cols"))
                        != (P, R, C)):
                    raise RuntimeError("per-matrix state does not match this parameter's matrices")
                want = {"exp_avg_absmax": P * num_blocks(R * C, block_size),
                        "factored_row_absmax": 2 * P * num_blocks(R, block_size),
                        "factored_col_absmax": 2 * P * num_blocks(C, block_size),
                        "factored_row_q": 2 * rows, "factored_col_q": 2 * cols}
                for key, n in want.items():
                    if state[key].numel() != n:
                        raise RuntimeError(f"{key} does not have the per-matrix layout of this parameter "
                                           f"(block size {block_size})")
                return
            # the flat layout: [2][blocks of the P*R row states] and [2][blocks of the P*C column states]
            for key, n in (("factored_row", rows), ("factored_col", cols)):
                if (state[f"{key}_q"].numel() != 2 * n
                        or state[f"{key}_absmax"].numel() != 2 * num_blocks(n, block_size)):
                    raise RuntimeError(f"{key} state does not have the flat full8bit layout of this parameter")

    # -------------------------------------------------------------- checkpoint
    def load_state_dict(self, state_dict: dict, convert_layouts: bool = True) -> None:
        """torch's loader casts every floating state tensor to the parameter dtype.  Every state tensor of
        these optimizers has a dtype of its own (int8/uint8 codes, fp32 scales and fp32 states, whatever
        the parameter dtype), so each is put back as saved, on the parameter's device.

        A state saved in another of the reference's layouts (the 8bit2d tiles its CUDA path keeps for
        2-D parameters, the per-matrix blocks of its CUDA N-D path, fp32 CAMECUDA states, or full8bit
        states under CAME8bit2D / CAMECUDA) is converted into this optimizer's layout
        (``state_layout.convert_state``), so the momentum and second moments carry over.  With
        ``convert_layouts=False`` such a state is left as loaded, and, as in the reference
        (CAME8bit.py:757-759), re-initialised by the next step; that includes the reference CUDA N-D
        path's per-matrix blocks (``_mode`` "full8bit" with ``_cuda_factored_nd_ext_path``), which no
        kernel here steps in place."""
        saved_groups = state_dict["param_groups"]
        saved_state = state_dict["state"]
        super().load_state_dict(state_dict)
        id_map = dict(zip(chain.from_iterable(g["params"] for g in saved_groups),
                          chain.from_iterable(g["params"] for g in self.param_groups)))
        for k, st in saved_state.items():
            p = id_map.get(k)
            if p is None or p not in self.state:
                continue
            live = self.state[p]
            for key, v in st.items():
                if isinstance(v, torch.Tensor):
                    live[key] = v.detach().to(device=p.device).clone()
                # torch's loader rebuilds iterables element-wise, which turns the string "_mode" into a
                # generator (and a mode mismatch would reset the state on the next step): plain values
                # are restored as saved
                elif isinstance(v, (str, bool, int, float)):
                    live[key] = v
            self._after_load(live)
            if convert_layouts:
                self._adopt_layout(p, live)

    def _group_of(self, p: torch.Tensor) -> dict:
        for g in self.param_groups:
            if any(q is p for q in g["params"]):
                return g
        raise KeyError("parameter is in no param group")

    def _adopt_layout(self, p: torch.Tensor, state: dict) -> None:
        """Convert a loaded state of another layout into this optimizer's (see load_state_dict)."""
        src = state_layout.layout_of(state)
        if not src or src in self._IN_PLACE or (self._MODE == "8bit2d" and p.dim() != 2):
            return
        if src == "8bit1d" and self._MODE == "full8bit" and p.dim() == 1:
            # the reference CAME8bit's 1-D batched-path states (CAME8bit.py:252-262) keep full8bit's
            # 1-D tensors under another _mode: relabelled, codes untouched
            state["_mode"] = "full8bit"
            for k in ("_cuda_nonfactored_batched_fastpath", "_cuda_nonfactored_multitensor_fastpath",
                      "_cuda_batched_update_fp16"):
                state.pop(k, None)
            self._after_load(state)
            return
        block_size = int(self._group_of(p).get("block_size", 256))
        new = state_layout.convert_state(state, tuple(p.shape), self._MODE, block_size)
        state.clear()
        if self._MODE == "8bit2d":
            init_8bit2d_state(state, p.data, block_size=256)
            for key, v in new.items():
                if isinstance(v, torch.Tensor):
                    state[key].copy_(v.reshape(state[key].shape))
        else:
            state.update(new)
        self._after_load(state)

    def _after_load(self, state: dict) -> None:
        self._drop_reference_scratch(state)
        if state.get("factored") and "factored_row_q" in state:
            self._bind_factored_views(state)

    def _drop_reference_scratch(self, state: dict) -> None:
        # a state already in this optimizer's own layout (not the reference's per-matrix N-D blocks,
        # which load_state_dict converts next, and not 8bit2d, whose state keeps its partial buffers)
        if self._MODE != "8bit2d" and state_layout.layout_of(state) == self._MODE:
            for k in _REFERENCE_SCRATCH_KEYS:
                state.pop(k, None)
            flags = _FP32_FLAGS if self._MODE == "cudafp" else (
                _FACTORED_FLAGS if state.get("factored") else _NONFACTORED_FLAGS)
            for k in flags:
                state[k] = False

    # ------------------------------------------------------------------- step
    def _group_hparams(self, group: dict) -> _lib.Came8HParams:
        b1, b2, b3 = group["betas"]
        e0, e1 = group["eps"]
        flags = _lib.CAME8_FLAG_EXACT_NORM if getattr(self, "exact_norm", False) else 0
        return _lib.Came8HParams(float(group["lr"]), float(b1), float(b2), float(b3), float(e0), float(e1),
                                 float(group["clip_threshold"]), float(group["weight_decay"]),
                                 int(group["block_size"]), flags)

    def _workspace(self, group: dict, device: torch.device, descs, n: int, block_size: int):
        """(workspace tensor, tag) for one param group on `device`, grown when its tensor list needs
        more.

        The workspace holds the group's launch plan between steps and nothing else writes to it; each
        allocation gets a fresh tag, so the library never trusts a plan left in reused memory.  Each
        param group has a workspace of its own: groups that shared one would replace each other's
        plan on every step (an upload, and a wait for the previous one, per group and step).
        """
        lib = _lib.load()
        need = ctypes.c_size_t(0)
        _lib.check(lib.came8_workspace_size(descs, n, block_size, ctypes.byref(need)), "came8_workspace_size")
        cache = self.__dict__.setdefault("_came8_workspaces", {})
        key = (device, id(group))
        ent = cache.get(key)
        if ent is None:  # a new group (or groups replaced by load_state_dict): drop workspaces of gone groups
            live = {id(g) for g in self.param_groups}
            for k in [k for k in cache if k[1] not in live]:
                lib.came8_release_workspace(cache.pop(k)[0].data_ptr())
        if ent is None or ent[0].numel() < need.value:
            if ent is not None:
                lib.came8_release_workspace(ent[0].data_ptr())
            ws = torch.empty(max(int(need.value), 256), dtype=torch.uint8, device=device)
            weakref.finalize(ws, _release_workspace, ws.data_ptr())
            ent = (ws, _lib.new_workspace_tag())
            cache[key] = ent
        return ent

    def _prepare_param(self, p: torch.Tensor, block_size: int):
        grad = p.grad
        if grad.is_sparse:
            raise RuntimeError("CAME does not support sparse gradients.")
        if not p.is_cuda:
            raise RuntimeError(
                f"{type(self).__name__} (came_amd) runs the step on the GPU; got a parameter on {p.device}")
        if p.dtype not in _DTYPE_CODE or grad.dtype not in _DTYPE_CODE:
            raise RuntimeError(f"unsupported dtype: param {p.dtype}, grad {grad.dtype} "
                               "(float32, bfloat16 and float16 are supported)")
        if grad.shape != p.shape:
            raise RuntimeError(f"grad shape {tuple(grad.shape)} does not match param shape {tuple(p.shape)}")
        state = self.state[p]
        # another layout (a different _mode, or the reference CUDA N-D path's per-matrix blocks under
        # _mode "full8bit") starts over, as the reference does (CAME8bit.py:757-759)
        if len(state) == 0 or state_layout.layout_of(state) not in self._IN_PLACE:
            state.clear()
            self._init_state(state, grad, block_size)
        self._check_state(p, state, block_size)
        return state, grad

    def _group_block_size(self, group: dict) -> int:
        return int(group["block_size"])

    @staticmethod
    def _is_factored(state: dict) -> bool:
        return bool(state["factored"])

    @staticmethod
    def _count_step(state: dict) -> None:
        state["step"] += 1

    def _fill_desc(self, d, p: torch.Tensor, state: dict) -> None:
        """State pointers of one tensor in the full8bit layout (include/came8.h: came8_tensor)."""
        d.exp_avg_q = state["exp_avg_q"].data_ptr()
        d.exp_avg_absmax = state["exp_avg_absmax"].data_ptr()
        if state["factored"]:
            d.row_q = state["factored_row_q"].data_ptr()
            d.row_absmax = state["factored_row_absmax"].data_ptr()
            d.col_q = state["factored_col_q"].data_ptr()
            d.col_absmax = state["factored_col_absmax"].data_ptr()
        else:
            d.row_q = state["exp_avg_sq_q"].data_ptr()
            d.row_absmax = state["exp_avg_sq_absmax"].data_ptr()

    @torch.no_grad()
    def _step_group(self, group: dict, params: list, plan_only: bool = False) -> None:
        """One came8_step per device over the group's params; with plan_only the library builds and
        uploads the launch plan and launches nothing (states are created, step counts not advanced)."""
        block_size = self._group_block_size(group)
        hp = self._group_hparams(group)
        if plan_only:
            hp.flags |= _lib.CAME8_FLAG_PLAN_ONLY
        by_device: dict = defaultdict(list)
        for p in params:
            by_device[p.device].append(p)
        lib = _lib.load()
        for device, plist in by_device.items():
            items = []
            for p in plist:
                state, grad = self._prepare_param(p, block_size)
                if not plan_only:
                    self._count_step(state)
                if p.numel() == 0:
                    continue
                items.append((p, state, grad))
            if not items:
                continue
            n = len(items)
            descs, keep, copyback = self._descriptors(items, block_size)
            ws, tag = self._workspace(group, device, descs, n, block_size)
            with torch.cuda.device(device):
                stream = torch.cuda.current_stream(device).cuda_stream
                _lib.check(lib.came8_step(descs, n, ctypes.byref(hp), ws.data_ptr(), ws.numel(), tag, stream),
                           "came8_step")
            if plan_only:
                continue
            self.__dict__.setdefault("_came8_last_step", {})[(device, id(group))] = [p for p, _, _ in items]
            for p, pd in copyback:
                p.data.copy_(pd)

    def _fp16_update_tensors(self, items: list, block_size: int) -> list:
        """Which of the (param, state, grad) items take the reference's fp16-update rounding of the 1-D update
        (CAME8_TENSOR_FP16_UPDATE): with cuda_nonfactored_use_fp16_update every unfactored tensor, as the
        reference's CAME8bitFull nonfactored CUDA step selects its fp16-update kernel for all of them
        (CAME8bitFull.py:485-490)."""
        on = bool(getattr(self, "cuda_nonfactored_use_fp16_update", False)) and self._STATE_KIND == _lib.CAME8_STATE_Q8
        return [on and not self._is_factored(st) for _, st, _ in items]

    def _descriptors(self, items: list, block_size: int = 256):
        """came8_tensor descriptors of (param, state, grad) triples (include/came8.h), the contiguous
        gradient copies they point to, and (param, contiguous copy) pairs to write back after the step."""
        descs = (_lib.Came8Tensor * len(items))()
        keep, copyback = [], []
        fp16u = self._fp16_update_tensors(items, block_size)
        for i, (p, state, grad) in enumerate(items):
            pd = p.data
            if not pd.is_contiguous():
                pd = pd.contiguous()
                copyback.append((p, pd))
            g = grad if grad.is_contiguous() else grad.contiguous()
            keep.append(g)
            d = descs[i]
            d.param = pd.data_ptr()
            d.grad = g.data_ptr()
            d.param_dtype = _DTYPE_CODE[p.dtype]
            d.grad_dtype = _DTYPE_CODE[g.dtype]
            d.state_kind = (_lib.CAME8_STATE_Q8_MATRIX if self._STATE_KIND == _lib.CAME8_STATE_Q8
                            and state_layout.layout_of(state) == "full8bit-nd" else self._STATE_KIND)
            if self._is_factored(state):
                shape = tuple(p.shape)
                d.prefix = math.prod(shape[:-2])
                d.rows, d.cols = shape[-2], shape[-1]
                d.factored = 1
            else:
                d.prefix, d.rows, d.cols = 1, 1, p.numel()
                d.factored = 0
            d.tensor_flags = _lib.CAME8_TENSOR_FP16_UPDATE if fp16u[i] else 0
            self._fill_desc(d, p, state)
        return descs, keep, copyback

    def last_clip_divisors(self, group_index: int = 0) -> dict:
        """{param: clip divisor max(rms(u) / clip_threshold, 1)} of the param group's last step, read
        back from the device (came8_read_clip; synchronises with the current stream)."""
        group = self.param_groups[group_index]
        lib = _lib.load()
        out = {}
        for (device, gid), plist in self.__dict__.get("_came8_last_step", {}).items():
            if gid != id(group):
                continue
            ws, tag = self.__dict__["_came8_workspaces"][(device, gid)]
            vals = (ctypes.c_float * len(plist))()
            with torch.cuda.device(device):
                stream = torch.cuda.current_stream(device).cuda_stream
                _lib.check(lib.came8_read_clip(ws.data_ptr(), tag, len(plist), vals, stream), "came8_read_clip")
            out.update({p: float(v) for p, v in zip(plist, vals)})
        return out

    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        timing = self._dispatch_timing_is_enabled()
        t0 = time.perf_counter()
        count = 0
        for group in self.param_groups:
            params = []
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("CAME does not support sparse gradients.")
                params.append(p)
            if params:
                self._step_group(group, params)
                count += len(params)
        if timing:
            self._benchmark_dispatch_timing_last = {
                "came8_step_host_time_ms": (time.perf_counter() - t0) * 1000.0,
                "came8_step_param_count": count,
            }
        return loss

    def _dispatch_timing_is_enabled(self) -> bool:
        return bool(getattr(self, "_benchmark_dispatch_timing", False))


class CAME8bitFull(_Came8Base):
    """All-state blockwise 8-bit CAME (reference came_pytorch/CAME8bitFull.py:39)."""

    def __init__(
        self,
        params,
        lr: float,
        eps: tuple[float, float] = (1e-30, 1e-16),
        clip_threshold: float = 1.0,
        betas: tuple[float, float, float] = (0.9, 0.999, 0.9999),
        weight_decay: float = 0.0,
        block_size: int = 256,
        prefer_factored_cuda_ext_path: bool = True,
        cuda_factored_nd_chunk_size_override: int | None = None,
        cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel: int | None = None,
        cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel: int | None = None,
        cuda_nonfactored_use_fp16_update: bool = False,
    ):
        defaults = self._validate_and_defaults(lr, eps, clip_threshold, betas, weight_decay, block_size)
        super().__init__(params, defaults)
        # Accepted for signature compatibility (CAME8bitFull.py:92-120); apart from
        # cuda_nonfactored_use_fp16_update they tuned the reference's per-parameter CUDA chains and
        # select nothing here, but their validation is kept.
        self.prefer_factored_cuda_ext_path = bool(prefer_factored_cuda_ext_path)
        self.cuda_factored_nd_chunk_size_override = (
            None if cuda_factored_nd_chunk_size_override is None else int(cuda_factored_nd_chunk_size_override))
        self.cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel = (
            None if cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel is None
            else int(cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel))
        self.cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel = (
            None if cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel is None
            else int(cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel))
        # the one that changes numerics: 1-D tensors take the reference's fp16-update variant
        # (CAME8_FLAG_FP16_UPDATE); settable after construction as well
        self.cuda_nonfactored_use_fp16_update = bool(cuda_nonfactored_use_fp16_update)
        if self.cuda_factored_nd_chunk_size_override is not None and self.cuda_factored_nd_chunk_size_override <= 0:
            raise ValueError("cuda_factored_nd_chunk_size_override must be positive when set")
        self.cuda_factored_nd_chunked_direct_row_sum = not (
            self.cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel is None
            and self.cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel is None)
        self.track_cuda_rms_state = False
        # the clip's update norm: the reference's own fp32 order (default), or with exact_norm = True
        # the exactly rounded fp64 sum (one pass over the gradients less; not the reference's value)
        self.exact_norm = False


class CAME8bitMemory(CAME8bitFull):
    """8-bit CAME with compact state (reference came_pytorch/CAME8bitMemory.py:17).

    The reference shares scratch buffers per device between parameters; here every param group's
    step uses one workspace per optimizer and device, so the same holds by construction.

    The reference's CUDA path steps 1-D tensors with its fp16-update kernels whatever the arguments
    (CAME8bitMemory.py:524-557); its CPU path, which this class follows by default, does not.  Set
    ``opt.cuda_nonfactored_use_fp16_update = True`` for the CUDA path's rounding.
    """

    def __init__(
        self,
        params,
        lr: float,
        eps: tuple[float, float] = (1e-30, 1e-16),
        clip_threshold: float = 1.0,
        betas: tuple[float, float, float] = (0.9, 0.999, 0.9999),
        weight_decay: float = 0.0,
        block_size: int = 256,
    ):
        super().__init__(params, lr=lr, eps=eps, clip_threshold=clip_threshold, betas=betas,
                         weight_decay=weight_decay, block_size=block_size,
                         prefer_factored_cuda_ext_path=False, cuda_nonfactored_use_fp16_update=False)

    _VIEWS_BEFORE_FLAGS = True  # CAME8bitMemory.py:423-436


class CAME8bit(CAME8bitFull):
    """Single-entry 8-bit CAME (reference came_pytorch/CAME8bit.py:24).

    Every parameter, whatever its rank, takes the full8bit state layout and the one multi-tensor
    step; the reference's per-rank dispatch knobs are validated and recorded but select nothing.
    """

    CUDA_1D_RUNTIME_MODE_DEFAULT = "default"
    CUDA_1D_RUNTIME_MODE_REPEATED_FP16_PAIRMIN = "repeated_fp16_pairmin"
    CUDA_ND_RUNTIME_MODE_DEFAULT = "default"
    CUDA_ND_RUNTIME_MODE_CHUNK32_LARGE_DIRECT_ROW_SUM = "chunk32_large_direct_row_sum"
    EXPLICIT_USER_FACING_KWARGS = frozenset({
        "prefer_cuda_fast_path", "prefer_cuda_2d_fast_path", "prefer_factored_cuda_ext_path",
        "cuda_1d_runtime_mode", "cuda_nd_runtime_mode", "cuda_graph_compatible",
    })
    EXPERIMENTAL_CUDA_TUNING_DEFAULTS = {
        "prefer_cuda_1d_batched_fast_path": False,
        "prefer_cuda_1d_multitensor_fast_path": False,
        "cuda_1d_batched_use_fp16_update": False,
        "cuda_1d_batched_chunk_size": 8,
        "cuda_1d_batched_min_bucket_size": 4,
        "cuda_1d_batched_min_numel": 1024,
        "cuda_1d_batched_max_numel": 65536,
        "cuda_factored_nd_chunk_size_override": None,
        "cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel": None,
        "cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel": None,
        "cuda_nonfactored_use_fp16_update": False,
    }

    def __init__(
        self,
        params,
        lr: float,
        eps: tuple[float, float] = (1e-30, 1e-16),
        clip_threshold: float = 1.0,
        betas: tuple[float, float, float] = (0.9, 0.999, 0.9999),
        weight_decay: float = 0.0,
        block_size: int = 256,
        prefer_cuda_fast_path: bool = True,
        prefer_cuda_2d_fast_path: bool | None = None,
        prefer_cuda_1d_fast_path: bool | None = None,
        prefer_cuda_1d_batched_fast_path: bool = False,
        prefer_cuda_1d_multitensor_fast_path: bool = False,
        cuda_1d_batched_use_fp16_update: bool = False,
        cuda_1d_batched_chunk_size: int = 8,
        cuda_1d_batched_min_bucket_size: int = 4,
        cuda_1d_batched_min_numel: int = 1024,
        cuda_1d_batched_max_numel: int = 65536,
        cuda_1d_runtime_mode: str = CUDA_1D_RUNTIME_MODE_DEFAULT,
        prefer_factored_cuda_ext_path: bool = True,
        cuda_factored_nd_chunk_size_override: int | None = None,
        cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel: int | None = None,
        cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel: int | None = None,
        cuda_nd_runtime_mode: str = CUDA_ND_RUNTIME_MODE_DEFAULT,
        cuda_nonfactored_use_fp16_update: bool = False,
        cuda_graph_compatible: bool = False,
    ):
        # validation order and messages follow CAME8bit.py:94-206
        if cuda_1d_runtime_mode not in {self.CUDA_1D_RUNTIME_MODE_DEFAULT,
                                        self.CUDA_1D_RUNTIME_MODE_REPEATED_FP16_PAIRMIN}:
            raise ValueError(
                "cuda_1d_runtime_mode must be one of "
                f"{self.CUDA_1D_RUNTIME_MODE_DEFAULT!r}, {self.CUDA_1D_RUNTIME_MODE_REPEATED_FP16_PAIRMIN!r}; "
                f"got {cuda_1d_runtime_mode!r}")
        if cuda_nd_runtime_mode not in {self.CUDA_ND_RUNTIME_MODE_DEFAULT,
                                        self.CUDA_ND_RUNTIME_MODE_CHUNK32_LARGE_DIRECT_ROW_SUM}:
            raise ValueError(
                "cuda_nd_runtime_mode must be one of "
                f"{self.CUDA_ND_RUNTIME_MODE_DEFAULT!r}, {self.CUDA_ND_RUNTIME_MODE_CHUNK32_LARGE_DIRECT_ROW_SUM!r}; "
                f"got {cuda_nd_runtime_mode!r}")
        overrides = self._experimental_cuda_tuning_overrides(
            prefer_cuda_1d_batched_fast_path=prefer_cuda_1d_batched_fast_path,
            prefer_cuda_1d_multitensor_fast_path=prefer_cuda_1d_multitensor_fast_path,
            cuda_1d_batched_use_fp16_update=cuda_1d_batched_use_fp16_update,
            cuda_1d_batched_chunk_size=cuda_1d_batched_chunk_size,
            cuda_1d_batched_min_bucket_size=cuda_1d_batched_min_bucket_size,
            cuda_1d_batched_min_numel=cuda_1d_batched_min_numel,
            cuda_1d_batched_max_numel=cuda_1d_batched_max_numel,
            cuda_factored_nd_chunk_size_override=cuda_factored_nd_chunk_size_override,
            cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel=(
                cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel),
            cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel=(
                cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel),
            cuda_nonfactored_use_fp16_update=cuda_nonfactored_use_fp16_update,
        )
        if overrides:
            warnings.warn(
                "CAME8bit low-level CUDA tuning kwargs are experimental and intended for "
                "benchmark/diagnostic use: " + ", ".join(overrides)
                + ". Prefer cuda_1d_runtime_mode/cuda_nd_runtime_mode for tracked user-facing opt-ins.",
                RuntimeWarning, stacklevel=2)
        eff_1d_fast = prefer_cuda_1d_fast_path
        eff_1d_batched = prefer_cuda_1d_batched_fast_path
        eff_1d_mt = prefer_cuda_1d_multitensor_fast_path
        eff_1d_fp16 = cuda_1d_batched_use_fp16_update
        eff_min_bucket = cuda_1d_batched_min_bucket_size
        eff_nd_chunk = cuda_factored_nd_chunk_size_override
        eff_nd_min = cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel
        eff_nf_fp16 = cuda_nonfactored_use_fp16_update
        if cuda_1d_runtime_mode == self.CUDA_1D_RUNTIME_MODE_REPEATED_FP16_PAIRMIN:
            eff_1d_fast = eff_1d_batched = eff_1d_mt = eff_1d_fp16 = True
            eff_min_bucket = 2
            eff_nf_fp16 = True
        if cuda_nd_runtime_mode == self.CUDA_ND_RUNTIME_MODE_CHUNK32_LARGE_DIRECT_ROW_SUM:
            eff_nd_chunk = 32
            eff_nd_min = 256 * 256
        super().__init__(
            params, lr=lr, eps=eps, clip_threshold=clip_threshold, betas=betas, weight_decay=weight_decay,
            block_size=block_size, prefer_factored_cuda_ext_path=prefer_factored_cuda_ext_path,
            cuda_factored_nd_chunk_size_override=eff_nd_chunk,
            cuda_factored_nd_chunked_direct_row_sum_min_matrix_numel=eff_nd_min,
            cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel=cuda_factored_nd_chunked_direct_row_sum_max_matrix_numel,
            cuda_nonfactored_use_fp16_update=eff_nf_fp16,
        )
        self.cuda_1d_runtime_mode = cuda_1d_runtime_mode
        self.cuda_nd_runtime_mode = cuda_nd_runtime_mode
        self.prefer_cuda_fast_path = bool(prefer_cuda_fast_path)
        self.prefer_cuda_2d_fast_path = (
            self.prefer_cuda_fast_path if prefer_cuda_2d_fast_path is None else bool(prefer_cuda_2d_fast_path))
        self.prefer_cuda_1d_batched_fast_path = bool(eff_1d_batched)
        self.prefer_cuda_1d_multitensor_fast_path = bool(eff_1d_mt)
        self.cuda_1d_batched_use_fp16_update = bool(eff_1d_fp16)
        self.prefer_cuda_1d_fast_path = (
            self.prefer_cuda_1d_batched_fast_path if eff_1d_fast is None else bool(eff_1d_fast))
        self.cuda_1d_batched_chunk_size = int(cuda_1d_batched_chunk_size)
        self.cuda_1d_batched_min_bucket_size = int(eff_min_bucket)
        self.cuda_1d_batched_min_numel = int(cuda_1d_batched_min_numel)
        self.cuda_1d_batched_max_numel = int(cuda_1d_batched_max_numel)
        if self.cuda_1d_batched_chunk_size <= 0:
            raise ValueError("cuda_1d_batched_chunk_size must be positive")
        if self.cuda_1d_batched_min_bucket_size <= 0:
            raise ValueError("cuda_1d_batched_min_bucket_size must be positive")
        if self.cuda_1d_batched_min_numel <= 0 or self.cuda_1d_batched_max_numel < self.cuda_1d_batched_min_numel:
            raise ValueError("cuda_1d_batched_min_numel/max_numel must define a positive range")
        self.cuda_graph_compatible = bool(cuda_graph_compatible)
        self.experimental_cuda_tuning_overrides = overrides

    @classmethod
    def _experimental_cuda_tuning_overrides(cls, **kwargs) -> tuple[str, ...]:
        return tuple(k for k, default in cls.EXPERIMENTAL_CUDA_TUNING_DEFAULTS.items() if kwargs[k] != default)

    @torch.no_grad()
    def _fp16_update_tensors(self, items: list, block_size: int) -> list:
        """The reference's per-tensor choice of the fp16-update kernels (CAME8bit.py:224-245 predicates,
        :712-861 per-parameter routing, :862-891 bucket flush, :441-529 multi-tensor step).  A contiguous
        1-D CUDA tensor:

        - with prefer_cuda_1d_fast_path, in the batched size range [cuda_1d_batched_min_numel,
          cuda_1d_batched_max_numel] under prefer_cuda_1d_batched_fast_path, and in a bucket of at least
          cuda_1d_batched_min_bucket_size tensors of its device, dtype and length: the multi-tensor kernels
          when prefer_cuda_1d_multitensor_fast_path is set, fp16 update iff cuda_1d_batched_use_fp16_update;
          else the batched kernel, whose update is always fp32;
        - otherwise (the single-tensor 1-D path or the full8bit direct path): fp16 update iff
          cuda_nonfactored_use_fp16_update.

        Other tensors (factored, or not contiguous: the reference's generic path) keep the fp32 update."""
        def fast_1d(p, g):
            return p.is_cuda and p.dim() == 1 and p.is_contiguous() and g.is_contiguous()

        def batched(p, g):
            return (self.prefer_cuda_1d_fast_path and self.prefer_cuda_1d_batched_fast_path and fast_1d(p, g)
                    and self.cuda_1d_batched_min_numel <= p.numel() <= self.cuda_1d_batched_max_numel
                    and block_size > 0)

        buckets = Counter((p.device, p.dtype, p.numel()) for p, st, g in items
                          if not self._is_factored(st) and batched(p, g))
        out = []
        for p, st, g in items:
            if self._is_factored(st) or not fast_1d(p, g):
                out.append(False)
            elif batched(p, g) and buckets[(p.device, p.dtype, p.numel())] >= self.cuda_1d_batched_min_bucket_size:
                out.append(self.prefer_cuda_1d_multitensor_fast_path and self.cuda_1d_batched_use_fp16_update)
            else:
                out.append(bool(self.cuda_nonfactored_use_fp16_update))
        return out

    def prime_for_cuda_graph(self) -> None:
        """Create every state, the workspace and its uploaded launch plan before capture
        (CAME8bit.py:672-693), so that a captured step only enqueues kernel launches."""
        for group in self.param_groups:
            params = []
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.grad.is_sparse:
                    raise RuntimeError("CAME does not support sparse gradients.")
                if not (p.data.is_contiguous() and p.grad.is_contiguous()):
                    raise RuntimeError("CUDA graph capture requires contiguous parameter and gradient tensors.")
                params.append(p)
            if params:
                self._step_group(group, params, plan_only=True)


# state tensors of the fp32-state layout (all fp32, whatever the parameter dtype)
_FP32_STATE_KEYS = ("exp_avg", "exp_avg_sq_row", "exp_avg_sq_col", "exp_avg_res_row", "exp_avg_res_col", "exp_avg_sq")


class CAMECUDA(_Came8Base):
    """CAME with fp32 optimizer state (reference came_pytorch/CAMECUDA.py:16).

    Same constructor arguments, ``ValueError`` texts, param-group keys and per-parameter state as
    the reference (CAMECUDA.py:27-56, 83-104: ``step``, ``_mode`` = "cudafp", ``factored``,
    ``exp_avg`` and ``exp_avg_sq_row/col`` + ``exp_avg_res_row/col`` for ndim >= 2 or ``exp_avg_sq``
    for 1-D, all fp32).  The arithmetic is the reference's ``_step_param_generic``
    (CAMECUDA.py:275-326) -- the 8-bit step's with the states kept in fp32 -- run for every
    parameter of a group by one ``came8_step`` call with fp32 states.  The reference's per-tensor
    CUDA scratch buffers (``scratch_fp32`` and the like) are not kept: the library's workspace
    replaces them, and a state dict without them loads in the reference (it then takes its
    generic path).
    """

    _MODE = "cudafp"
    _IN_PLACE = ("cudafp",)
    _STATE_KIND = _lib.CAME8_STATE_FP32
    _WORK_BLOCK = 256  # shapes the library's work decomposition only; fp32 states have no blocks

    def __init__(
        self,
        params,
        lr: float,
        eps: tuple[float, float] = (1e-30, 1e-16),
        clip_threshold: float = 1.0,
        betas: tuple[float, float, float] = (0.9, 0.999, 0.9999),
        weight_decay: float = 0.0,
    ):
        # came_pytorch/CAMECUDA.py:37-56
        if lr is None or lr <= 0.0:
            raise ValueError(f"lr must be > 0, got {lr}")
        if clip_threshold <= 0.0:
            raise ValueError(f"clip_threshold must be > 0, got {clip_threshold}")
        if len(eps) != 2:
            raise ValueError(f"eps must be a tuple of length 2, got eps={eps}")
        if len(betas) != 3:
            raise ValueError(f"betas must be a tuple of length 3, got betas={betas}")
        if not all(0.0 <= beta <= 1.0 for beta in betas):
            raise ValueError(f"betas must be in [0, 1], got betas={betas}")
        defaults = dict(
            lr=float(lr),
            eps=(float(eps[0]), float(eps[1])),
            clip_threshold=float(clip_threshold),
            betas=(float(betas[0]), float(betas[1]), float(betas[2])),
            weight_decay=float(weight_decay),
        )
        super().__init__(params, defaults)
        # the clip's update norm: the reference's own fp32 order (default), or with exact_norm = True
        # the exactly rounded fp64 sum (one pass over the gradients less; not the reference's value)
        self.exact_norm = False

    @property
    def supports_memory_efficient_fp16(self):
        return True

    @property
    def supports_flat_params(self):
        return False

    def _group_block_size(self, group: dict) -> int:
        return self._WORK_BLOCK

    def _group_hparams(self, group: dict) -> _lib.Came8HParams:
        b1, b2, b3 = group["betas"]
        e0, e1 = group["eps"]
        flags = _lib.CAME8_FLAG_EXACT_NORM if getattr(self, "exact_norm", False) else 0
        return _lib.Came8HParams(float(group["lr"]), float(b1), float(b2), float(b3), float(e0), float(e1),
                                 float(group["clip_threshold"]), float(group["weight_decay"]),
                                 self._WORK_BLOCK, flags)

    def _init_state(self, state: dict, grad: torch.Tensor, block_size: int) -> None:
        """The reference's fp32 layout (CAMECUDA.py:83-104)."""
        state["step"] = 0
        state["_mode"] = "cudafp"
        state["factored"] = grad.dim() >= 2
        shape = tuple(grad.shape)
        state["exp_avg"] = torch.zeros(shape, device=grad.device, dtype=torch.float32)
        if state["factored"]:
            row_shape, col_shape = shape[:-1], shape[:-2] + shape[-1:]
            for k, sh in (("exp_avg_sq_row", row_shape), ("exp_avg_sq_col", col_shape),
                          ("exp_avg_res_row", row_shape), ("exp_avg_res_col", col_shape)):
                state[k] = torch.zeros(sh, device=grad.device, dtype=torch.float32)
        else:
            state["exp_avg_sq"] = torch.zeros(shape, device=grad.device, dtype=torch.float32)
        for k in _FP32_FLAGS:
            state[k] = False

    def _check_state(self, p: torch.Tensor, state: dict, block_size: int) -> None:
        if tuple(state["exp_avg"].shape) != tuple(p.shape):
            raise RuntimeError("Parameter shape changed; the optimizer state no longer matches it.")
        for k in _FP32_STATE_KEYS:
            v = state.get(k)
            if v is None:
                continue
            if v.device != p.device:
                raise RuntimeError("optimizer state lives on a different device than its parameter")
            if v.dtype != torch.float32 or not v.is_contiguous():
                state[k] = v.to(dtype=torch.float32).contiguous()

    def _fill_desc(self, d, p: torch.Tensor, state: dict) -> None:
        """fp32 state pointers (include/came8.h: came8_tensor with CAME8_STATE_FP32)."""
        d.exp_avg_q = state["exp_avg"].data_ptr()
        d.exp_avg_absmax = None
        if state["factored"]:
            d.row_q = state["exp_avg_sq_row"].data_ptr()
            d.row_absmax = state["exp_avg_res_row"].data_ptr()
            d.col_q = state["exp_avg_sq_col"].data_ptr()
            d.col_absmax = state["exp_avg_res_col"].data_ptr()
        else:
            d.row_q = state["exp_avg_sq"].data_ptr()
            d.row_absmax = None

    def _after_load(self, state: dict) -> None:
        self._drop_reference_scratch(state)


_TILE_2D = 16


def init_8bit2d_state(state: dict, p_data: torch.Tensor, *, block_size: int = 256) -> None:
    """The reference's 8bit2d state of a 2-D parameter (came_pytorch/came8bit2d_state.py:33-75): the
    persistent tensors, the per-parameter scratch tensors the reference keeps in the state (the
    library uses ``res_row_partial`` / ``res_col_partial`` as its tile sums; the others stay
    unwritten, so a state dict saved here steps unchanged in the reference) and the shape keys.
    There is no ``step`` key."""
    rows, cols = p_data.shape
    dev = p_data.device
    tr, tc = math.ceil(rows / _TILE_2D), math.ceil(cols / _TILE_2D)
    state["_mode"] = "8bit2d"
    state["exp_avg_q"] = torch.zeros_like(p_data, dtype=torch.int8)
    state["exp_avg_absmax"] = torch.zeros((tr * tc,), device=dev, dtype=torch.float32)  # 0: no momentum yet
    for k, n in (("sq_row", rows), ("sq_col", cols), ("res_row", rows), ("res_col", cols)):
        state[f"exp_avg_{k}_q"], state[f"exp_avg_{k}_absmax"] = init_qstate(
            (n,), device=dev, signed=False, block_size=block_size)
    f32 = dict(device=dev, dtype=torch.float32)
    for k, n in (("r_factor", rows), ("c_factor", cols), ("r_res_factor", rows), ("c_res_factor", cols),
                 ("res_row_sum", rows), ("res_col_sum", cols), ("res_row_partial", tc * rows),
                 ("res_col_partial", tr * cols), ("sum_sq_row", 1), ("sum_update", 1),
                 ("sum_update_partial", (rows * cols + 255) // 256), ("sum_res_row", 1)):
        state[k] = torch.empty((n,), **f32)
    state.update(rows=rows, cols=cols, tile_rows=tr, tile_cols=tc, num_tiles=tr * tc)


def validate_8bit2d_state(state: dict, p_data: torch.Tensor) -> None:
    """came_pytorch/came8bit2d_state.py:78-87 (same messages)."""
    rows, cols = p_data.shape
    tr, tc = math.ceil(rows / _TILE_2D), math.ceil(cols / _TILE_2D)
    if state["rows"] != rows or state["cols"] != cols:
        raise RuntimeError("Parameter shape changed; this optimizer does not support resizing 8-bit state.")
    if state["tile_rows"] != tr or state["tile_cols"] != tc or state["num_tiles"] != tr * tc:
        raise RuntimeError("Tile layout changed; this optimizer does not support resizing 8-bit state.")


class CAME8bit2D(_Came8Base):
    """CAME with int8 momentum in 16x16 tiles, 2-D CUDA parameters only (reference
    came_pytorch/CAME8bit2D.py:9).

    Same constructor arguments, defaults and errors (CAME8bit2D.py:19-50, 52-72, 74-131), same
    state keys (came8bit2d_state.py:33-75; no ``step``).  The arithmetic is the reference's CUDA
    8bit2d step (``came2d_step``, came_cuda/csrc/came_bindings.cpp:617-759): float32 EMAs of the row
    and column states, momentum quantised per 16x16 tile with a tile absmax that starts at 0,
    multiplicative weight decay and the parameter written from the requantised momentum.  Every
    parameter of a param group is stepped by one ``came8_step`` call.
    """

    _MODE = "8bit2d"
    _IN_PLACE = ("8bit2d",)
    _STATE_KIND = _lib.CAME8_STATE_8BIT2D

    def __init__(
        self,
        params,
        lr: float,
        eps: tuple[float, float] = (1e-30, 1e-16),
        clip_threshold: float = 1.0,
        betas: tuple[float, float, float] = (0.9, 0.999, 0.9999),
        weight_decay: float = 0.0,
        block_size: int = 256,
        cuda_graph_compatible: bool = False,
    ):
        # came_pytorch/CAME8bit2D.py:30-50
        if lr is None or lr <= 0.0:
            raise ValueError(f"lr must be > 0, got {lr}")
        if clip_threshold <= 0.0:
            raise ValueError(f"clip_threshold must be > 0, got {clip_threshold}")
        if len(eps) != 2:
            raise ValueError(f"eps must be a tuple of length 2, got eps={eps}")
        if len(betas) != 3:
            raise ValueError(f"betas must be a tuple of length 3, got betas={betas}")
        if block_size != 256:
            raise ValueError("Only block_size=256 is supported in this minimal implementation.")
        defaults = dict(
            lr=float(lr),
            eps=(float(eps[0]), float(eps[1])),
            clip_threshold=float(clip_threshold),
            betas=(float(betas[0]), float(betas[1]), float(betas[2])),
            weight_decay=float(weight_decay),
            block_size=int(block_size),
        )
        super().__init__(params, defaults)
        self.cuda_graph_compatible = bool(cuda_graph_compatible)

    @staticmethod
    def _is_factored(state: dict) -> bool:
        return True

    @staticmethod
    def _count_step(state: dict) -> None:
        pass  # the 8bit2d state keeps no step count

    def _check_grad(self, p: torch.Tensor) -> None:
        # came_pytorch/CAME8bit2D.py:89-101
        if p.dim() != 2:
            raise NotImplementedError("CAME8bit2D currently supports 2D parameters only.")
        if not p.is_cuda:
            raise NotImplementedError("CAME8bit2D requires CUDA parameters.")
        if p.grad.is_sparse:
            raise RuntimeError("CAME does not support sparse gradients.")
        if p.grad.dtype != p.dtype:
            raise RuntimeError(f"Expected g.dtype == p.dtype, got {p.grad.dtype} vs {p.dtype}")
        if self.cuda_graph_compatible and not (p.data.is_contiguous() and p.grad.is_contiguous()):
            raise RuntimeError("CUDA graph capture requires contiguous parameter and gradient tensors.")

    def _init_state(self, state: dict, grad: torch.Tensor, block_size: int) -> None:
        init_8bit2d_state(state, grad, block_size=block_size)

    def _check_state(self, p: torch.Tensor, state: dict, block_size: int) -> None:
        """Shape keys as the reference checks them, then every buffer the library will write: dtype,
        device, contiguity and size (the reference's own checks, came_bindings.cpp:657-714)."""
        validate_8bit2d_state(state, p.data)
        rows, cols = p.shape
        tr, tc = state["tile_rows"], state["tile_cols"]
        nbr, nbc = num_blocks(rows, block_size), num_blocks(cols, block_size)
        need = {"exp_avg_q": (torch.int8, rows * cols), "exp_avg_absmax": (torch.float32, tr * tc),
                "exp_avg_sq_row_q": (torch.uint8, rows), "exp_avg_res_row_q": (torch.uint8, rows),
                "exp_avg_sq_col_q": (torch.uint8, cols), "exp_avg_res_col_q": (torch.uint8, cols),
                "exp_avg_sq_row_absmax": (torch.float32, nbr), "exp_avg_res_row_absmax": (torch.float32, nbr),
                "exp_avg_sq_col_absmax": (torch.float32, nbc), "exp_avg_res_col_absmax": (torch.float32, nbc),
                "res_row_partial": (torch.float32, tc * rows), "res_col_partial": (torch.float32, tr * cols)}
        for k, (dt, n) in need.items():
            v = state.get(k)
            if not isinstance(v, torch.Tensor):
                raise RuntimeError(f"8bit2d state is missing {k}")
            if v.device != p.device:
                raise RuntimeError("optimizer state lives on a different device than its parameter")
            if v.dtype != dt:
                raise RuntimeError(f"{k} must be {str(dt).replace('torch.', '')}, got {v.dtype}")
            if not v.is_contiguous():
                raise RuntimeError(f"{k} must be contiguous")
            if v.numel() < n:
                raise RuntimeError(f"{k} is too small: {v.numel()} < {n}")
        if tuple(state["exp_avg_q"].shape) != tuple(p.shape):
            raise RuntimeError("exp_avg_q.shape must match p.shape")

    def _fill_desc(self, d, p: torch.Tensor, state: dict) -> None:
        """8bit2d state pointers (include/came8.h: came8_tensor with CAME8_STATE_8BIT2D)."""
        d.exp_avg_q = state["exp_avg_q"].data_ptr()
        d.exp_avg_absmax = state["exp_avg_absmax"].data_ptr()
        d.row_q = state["exp_avg_sq_row_q"].data_ptr()
        d.row_absmax = state["exp_avg_sq_row_absmax"].data_ptr()
        d.col_q = state["exp_avg_sq_col_q"].data_ptr()
        d.col_absmax = state["exp_avg_sq_col_absmax"].data_ptr()
        d.res_row_q = state["exp_avg_res_row_q"].data_ptr()
        d.res_row_absmax = state["exp_avg_res_row_absmax"].data_ptr()
        d.res_col_q = state["exp_avg_res_col_q"].data_ptr()
        d.res_col_absmax = state["exp_avg_res_col_absmax"].data_ptr()
        d.res_row_partial = state["res_row_partial"].data_ptr()
        d.res_col_partial = state["res_col_partial"].data_ptr()

    def _after_load(self, state: dict) -> None:
        pass

    @torch.no_grad()
    def step(self, closure=None):
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is not None:
                    self._check_grad(p)
        return super().step(closure)

    @torch.no_grad()
    def prime_for_cuda_graph(self) -> None:
        """Create every state, the workspace and its uploaded launch plan before capture
        (came_pytorch/CAME8bit2D.py:52-72, same messages)."""
        for group in self.param_groups:
            params = []
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.dim() != 2:
                    raise RuntimeError("CUDA graph capture for CAME8bit2D requires 2D parameters.")
                if not p.is_cuda:
                    raise RuntimeError("CUDA graph capture for CAME8bit2D requires CUDA parameters.")
                if p.grad.is_sparse:
                    raise RuntimeError("CAME does not support sparse gradients.")
                if p.grad.dtype != p.dtype:
                    raise RuntimeError(f"Expected g.dtype == p.dtype, got {p.grad.dtype} vs {p.dtype}")
                if not (p.data.is_contiguous() and p.grad.is_contiguous()):
                    raise RuntimeError("CUDA graph capture requires contiguous parameter and gradient tensors.")
                params.append(p)
            if params:
                self._step_group(group, params, plan_only=True)
