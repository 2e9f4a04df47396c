"""CPU-side checks of the product package: the C-ABI library loads and exports every symbol
include/came8.h declares, argument validation returns the documented error codes before any device
work, and the optimizer classes keep the reference's constructor validation and state layout."""
import ctypes
import json
import os
import re
import warnings

import numpy as np
import pytest
import torch

import came_amd
from came_amd import _lib as L
from oracle import came8_oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _header_functions():
    src = open(os.path.join(ROOT, "include", "came8.h")).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(came8_\w+)\s*\(", src, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = L.load()
    declared = _header_functions()
    assert set(declared) == set(L.EXPORTED_SYMBOLS), declared
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.came8_abi_version() == L.ABI_VERSION == 5
    assert b"gfx950" in lib.came8_version()


def _desc(shape, dtype=L.CAME8_F32, fake=0x100000):
    d = L.Came8Tensor()
    d.param, d.grad = fake, fake + 0x10000000
    d.exp_avg_q, d.exp_avg_absmax = fake + 0x20000000, fake + 0x30000000
    d.row_q, d.row_absmax = fake + 0x40000000, fake + 0x50000000
    if len(shape) >= 2:
        d.col_q, d.col_absmax = fake + 0x60000000, fake + 0x70000000
        d.prefix = int(torch.tensor(shape[:-2]).prod().item()) if len(shape) > 2 else 1
        d.rows, d.cols, d.factored = shape[-2], shape[-1], 1
    else:
        d.prefix, d.rows, d.cols, d.factored = 1, 1, shape[0], 0
    d.param_dtype = d.grad_dtype = dtype
    return d


def test_workspace_size_host_only():
    lib = L.load()
    arr = (L.Came8Tensor * 3)(_desc((4096, 4096), L.CAME8_BF16), _desc((4096,)), _desc((2, 3, 5, 7)))
    out = ctypes.c_size_t(0)
    assert lib.came8_workspace_size(arr, 3, 256, ctypes.byref(out)) == L.CAME8_OK
    # column partials dominate: 3 arrays of (4096/256 bands of 2^20/4096 rows) x 4096 fp32 for the matrix
    assert 3 * 16 * 4096 * 4 < out.value < 64 << 20
    assert lib.came8_workspace_size(arr, 0, 256, ctypes.byref(out)) == L.CAME8_OK


@pytest.mark.parametrize("bad", ["block", "shape", "dtype", "null"])
def test_invalid_arguments_are_rejected(bad):
    lib = L.load()
    d = _desc((8, 8))
    block = 256
    if bad == "block":
        block = 0
    elif bad == "shape":
        d.rows = 0
    elif bad == "dtype":
        d.grad_dtype = 7
    else:
        d.exp_avg_q = 0
    arr = (L.Came8Tensor * 1)(d)
    out = ctypes.c_size_t(0)
    assert lib.came8_workspace_size(arr, 1, block, ctypes.byref(out)) == L.CAME8_EINVAL
    assert lib.came8_last_error()
    hp = L.Came8HParams(1e-3, 0.9, 0.999, 0.9999, 1e-30, 1e-16, 1.0, 0.0, block, 0)
    assert lib.came8_step(arr, 1, ctypes.byref(hp), 0x1000, 1 << 30, 0, None) == L.CAME8_EINVAL


def test_step_rejects_small_workspace_and_bad_hparams():
    lib = L.load()
    arr = (L.Came8Tensor * 1)(_desc((64, 64)))
    hp = L.Came8HParams(1e-3, 0.9, 0.999, 0.9999, 1e-30, 1e-16, 1.0, 0.0, 256, 0)
    assert lib.came8_step(arr, 1, ctypes.byref(hp), 0x1000, 16, 0, None) == L.CAME8_ESPACE
    hp.lr = 0.0
    assert lib.came8_step(arr, 1, ctypes.byref(hp), 0x1000, 1 << 30, 0, None) == L.CAME8_EINVAL
    hp.lr, hp.clip_threshold = 1e-3, -1.0
    assert lib.came8_step(arr, 1, ctypes.byref(hp), 0x1000, 1 << 30, 0, None) == L.CAME8_EINVAL


# --- constructor validation: messages of came_pytorch/CAME8bitFull.py:73-82, CAME8bit.py:94-206 ---
P0 = [torch.nn.Parameter(torch.zeros(2, 2))]


@pytest.mark.parametrize("cls", ["CAME8bit", "CAME8bitFull", "CAME8bitMemory"])
@pytest.mark.parametrize("kw,msg", [
    (dict(lr=0.0), "lr must be > 0"),
    (dict(lr=1e-3, clip_threshold=0.0), "clip_threshold must be > 0"),
    (dict(lr=1e-3, eps=(1e-30,)), "eps must be a tuple of length 2"),
    (dict(lr=1e-3, betas=(0.9, 0.99)), "betas must be a tuple of length 3"),
    (dict(lr=1e-3, block_size=0), "block_size must be > 0"),
])
def test_constructor_validation(cls, kw, msg):
    with pytest.raises(ValueError, match=msg):
        getattr(came_amd, cls)(P0, **kw)


def test_came8bit_mode_validation_and_warning():
    with pytest.raises(ValueError, match="cuda_1d_runtime_mode must be one of"):
        came_amd.CAME8bit(P0, lr=1e-3, cuda_1d_runtime_mode="nope")
    with pytest.raises(ValueError, match="cuda_nd_runtime_mode must be one of"):
        came_amd.CAME8bit(P0, lr=1e-3, cuda_nd_runtime_mode="nope")
    with pytest.raises(ValueError, match="cuda_1d_batched_chunk_size must be positive"):
        came_amd.CAME8bit(P0, lr=1e-3, cuda_1d_batched_chunk_size=0)
    with pytest.warns(RuntimeWarning, match="experimental"):
        opt = came_amd.CAME8bit(P0, lr=1e-3, cuda_1d_batched_chunk_size=4)
    assert opt.experimental_cuda_tuning_overrides == ("cuda_1d_batched_chunk_size",)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        opt = came_amd.CAME8bit(P0, lr=1e-3, cuda_1d_runtime_mode="repeated_fp16_pairmin")
    assert opt.cuda_1d_batched_min_bucket_size == 2 and opt.prefer_cuda_1d_fast_path
    opt = came_amd.CAME8bit(P0, lr=1e-3, cuda_nd_runtime_mode="chunk32_large_direct_row_sum")
    assert opt.cuda_factored_nd_chunk_size_override == 32
    assert opt.param_groups[0]["block_size"] == 256
    assert set(opt.param_groups[0]) >= {"lr", "eps", "clip_threshold", "betas", "weight_decay", "block_size"}


def test_cpu_parameters_are_refused():
    p = torch.nn.Parameter(torch.zeros(4, 4))
    opt = came_amd.CAME8bitFull([p], lr=1e-3)
    p.grad = torch.zeros(4, 4)
    with pytest.raises(RuntimeError, match="GPU"):
        opt.step()


@pytest.mark.parametrize("shape", [(7,), (5, 9), (2, 3, 5, 7), (300, 1000)])
@pytest.mark.parametrize("block", [256, 64])
def test_state_layout_matches_reference(shape, block):
    opt = came_amd.CAME8bitFull([torch.nn.Parameter(torch.zeros(shape))], lr=1e-3, block_size=block)
    st = {}
    opt._init_state(st, torch.zeros(shape), block)
    ref = orc.init_full8bit_state(shape, block)
    for k, v in ref.items():
        assert k in st, k
        if isinstance(v, torch.Tensor):
            assert st[k].dtype == v.dtype and tuple(st[k].shape) == tuple(v.shape), k
            assert torch.equal(st[k], v), k
        else:
            assert st[k] == v, k
    if len(shape) >= 2:
        assert st["exp_avg_res_col_q"].data_ptr() == st["factored_col_q"][1].data_ptr()


_VIEWS = {"exp_avg_sq_row_q", "exp_avg_res_row_q", "exp_avg_sq_col_q", "exp_avg_res_col_q",
          "exp_avg_sq_row_absmax", "exp_avg_res_row_absmax", "exp_avg_sq_col_absmax", "exp_avg_res_col_absmax"}


def _golden_key_sets(path, case):
    """{tensor index: {key: value or None}} of the reference's states after step 1, as the golden file
    recorded them: every key but the views of the stacked row/column states and the _mode string."""
    z = np.load(path)
    out = {}
    pre = f"{case}/s1/"
    for k in z.keys():
        if k.startswith(pre):
            i, key = k[len(pre):].split("/", 1)
            v = z[k]
            out.setdefault(int(i), {})[key] = v.item() if v.ndim == 0 and v.dtype == np.bool_ else None
    return out


@pytest.mark.parametrize("case", ["full_ragged_fp32", "came8bit_heavy_fp32", "memory_bf16", "came8bit_bs64_clip"])
def test_state_key_set_matches_reference(golden_dir, case):
    """Each state holds exactly the reference's keys (golden_small.npz, written by the reference's own CPU
    path), its CUDA routing flags included with the reference's CPU values (all False), plus _mode and,
    for factored tensors, the eight views."""
    meta = json.loads(str(np.load(os.path.join(golden_dir, "golden_small.npz"))["meta_json"]))[case]
    ref = _golden_key_sets(os.path.join(golden_dir, "golden_small.npz"), case)
    cls = getattr(came_amd, meta["cls"])
    block = meta["hp"].get("block_size", 256)
    for i, shape in enumerate(meta["shapes"]):
        p = torch.nn.Parameter(torch.zeros(shape))
        opt = cls([p], lr=1e-3, block_size=block) if meta["cls"] != "CAME8bitMemory" else cls([p], lr=1e-3)
        st = {}
        opt._init_state(st, torch.zeros(shape), block)
        want = set(ref[i]) | {"_mode"} | (_VIEWS if len(shape) >= 2 else set())
        assert set(st) == want, (case, shape, sorted(set(st) ^ want))
        for k, v in ref[i].items():
            if v is not None:  # the boolean flags
                assert st[k] is v, (case, shape, k, st[k], v)


def test_camecuda_state_key_set_matches_reference(golden_dir):
    path = os.path.join(golden_dir, "golden_camecuda.npz")
    meta = json.loads(str(np.load(path)["meta_json"]))
    for case, m in meta.items():
        if not isinstance(m, dict) or "shapes" not in m:
            continue
        ref = _golden_key_sets(path, case)
        for i, shape in enumerate(m["shapes"]):
            opt = came_amd.CAMECUDA([torch.nn.Parameter(torch.zeros(shape))], lr=1e-3)
            st = {}
            opt._init_state(st, torch.zeros(shape), 256)
            assert set(st) == set(ref[i]) | {"_mode"}, (case, shape, sorted(set(st) ^ (set(ref[i]) | {"_mode"})))
            for k, v in ref[i].items():
                if v is not None:
                    assert st[k] is v, (case, shape, k)


def test_loaded_reference_cuda_state_drops_its_scratch():
    """A state saved by the reference's CUDA path (flags True, per-tensor fp32 scratch) loads with the flags
    False and the scratch dropped (the library's workspace replaces it)."""
    p = torch.nn.Parameter(torch.zeros(40, 60))
    opt = came_amd.CAME8bitFull([p], lr=1e-3)
    st = {}
    opt._init_state(st, torch.zeros(40, 60), 256)
    saved = {k: v for k, v in st.items() if k not in _VIEWS}
    saved["_cuda_factored_fastpath"] = saved["_cuda_factored_ext_path"] = True
    saved["exp_avg_fp32"] = torch.zeros(40, 60)
    saved["scratch_fp32"] = torch.zeros(40, 60)
    saved["sum_update"] = torch.zeros(1)
    sd = {"state": {0: saved}, "param_groups": [dict(opt.state_dict()["param_groups"][0])]}
    opt2 = came_amd.CAME8bitFull([p], lr=1e-3)
    opt2.load_state_dict(sd)
    live = opt2.state[p]
    assert set(live) == set(st), sorted(set(live) ^ set(st))
    assert live["_cuda_factored_fastpath"] is False and live["_cuda_factored_ext_path"] is False


def test_load_state_dict_keeps_dtypes_mode_and_copies():
    """torch's loader would cast codes and fp32 block scales to the parameter dtype and turn the
    "_mode" string into a generator; the loaded state must equal the saved one, in its own memory."""
    ps = [torch.nn.Parameter(torch.randn(130, 260).bfloat16()), torch.nn.Parameter(torch.randn(260).bfloat16())]
    opt = came_amd.CAME8bitFull(ps, lr=2e-4)
    for p in ps:
        opt._init_state(opt.state[p], p, 256)
        opt.state[p]["exp_avg_absmax"].uniform_(0.1, 1.0)
        opt.state[p]["exp_avg_q"].random_(-127, 128)
        opt.state[p]["step"] = 7
    sd = opt.state_dict()
    ps2 = [torch.nn.Parameter(p.data.clone()) for p in ps]
    opt2 = came_amd.CAME8bitFull(ps2, lr=2e-4)
    opt2.load_state_dict(sd)
    for p, p2 in zip(ps, ps2):
        a, b = opt.state[p], opt2.state[p2]
        assert b["_mode"] == "full8bit" and b["step"] == 7 and b["factored"] == a["factored"]
        for k, v in a.items():
            if isinstance(v, torch.Tensor):
                assert b[k].dtype == v.dtype and torch.equal(b[k], v), k
                if k in ("exp_avg_q", "exp_avg_absmax"):
                    assert b[k].data_ptr() != v.data_ptr(), k
        if a["factored"]:
            assert b["exp_avg_res_row_q"].data_ptr() == b["factored_row_q"][1].data_ptr()


# ---------------------------------------------------------------------------------- CAMECUDA
@pytest.mark.parametrize("kw,msg", [
    (dict(lr=0.0), "lr must be > 0"),
    (dict(lr=1e-3, clip_threshold=0.0), "clip_threshold must be > 0"),
    (dict(lr=1e-3, eps=(1e-30,)), "eps must be a tuple of length 2"),
    (dict(lr=1e-3, betas=(0.9, 0.99)), "betas must be a tuple of length 3"),
    (dict(lr=1e-3, betas=(0.9, 1.5, 0.99)), r"betas must be in \[0, 1\]"),
])
def test_camecuda_constructor_validation(kw, msg):
    with pytest.raises(ValueError, match=msg):
        came_amd.CAMECUDA(P0, **kw)


def test_camecuda_group_keys_and_properties():
    opt = came_amd.CAMECUDA(P0, lr=1e-3, weight_decay=0.1)
    assert set(opt.param_groups[0]) == {"params", "lr", "eps", "clip_threshold", "betas", "weight_decay"}
    assert opt.supports_memory_efficient_fp16 and not opt.supports_flat_params


@pytest.mark.parametrize("shape", [(7,), (5, 9), (2, 3, 5, 7)])
def test_camecuda_state_layout_matches_reference(shape):
    opt = came_amd.CAMECUDA([torch.nn.Parameter(torch.zeros(shape))], lr=1e-3)
    st = {}
    opt._init_state(st, torch.zeros(shape), 256)
    ref = orc.init_fp32_state(shape)
    assert set(st) == set(ref)
    for k, v in ref.items():
        if isinstance(v, torch.Tensor):
            assert st[k].dtype == torch.float32 and tuple(st[k].shape) == tuple(v.shape), k
        else:
            assert st[k] == v, k


def test_camecuda_load_state_dict_keeps_fp32_states():
    ps = [torch.nn.Parameter(torch.randn(30, 20).bfloat16()), torch.nn.Parameter(torch.randn(20).bfloat16())]
    opt = came_amd.CAMECUDA(ps, lr=2e-4)
    for p in ps:
        opt._init_state(opt.state[p], p, 256)
        opt.state[p]["exp_avg"].normal_()
        opt.state[p]["step"] = 3
    ps2 = [torch.nn.Parameter(p.data.clone()) for p in ps]
    opt2 = came_amd.CAMECUDA(ps2, lr=2e-4)
    opt2.load_state_dict(opt.state_dict())
    for p, p2 in zip(ps, ps2):
        a, b = opt.state[p], opt2.state[p2]
        assert b["_mode"] == "cudafp" and b["step"] == 3
        for k, v in a.items():
            if isinstance(v, torch.Tensor):
                assert b[k].dtype == torch.float32 and torch.equal(b[k], v), k


def test_fp32_state_kind_checks():
    lib = L.load()
    size = ctypes.c_size_t(0)
    d = _desc((64, 64))
    d.state_kind = 7
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(d), 1, 256, ctypes.byref(size)) == L.CAME8_EINVAL
    assert b"state_kind" in lib.came8_last_error()
    d.state_kind = L.CAME8_STATE_FP32
    d.exp_avg_absmax = None  # not used by fp32 states
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(d), 1, 256, ctypes.byref(size)) == L.CAME8_OK
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(d), 1, 100, ctypes.byref(size)) == L.CAME8_EINVAL
    v = _desc((33,))
    v.state_kind = L.CAME8_STATE_FP32
    v.exp_avg_absmax = v.row_absmax = None
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(v), 1, 256, ctypes.byref(size)) == L.CAME8_OK


# ---------------------------------------------------------------------------------- CAME8bit2D
def _desc2d(shape, fake=0x100000):
    d = _desc(shape, fake=fake)
    d.state_kind = L.CAME8_STATE_8BIT2D
    d.res_row_q, d.res_row_absmax = fake + 0x80000000, fake + 0x90000000
    d.res_col_q, d.res_col_absmax = fake + 0xA0000000, fake + 0xB0000000
    return d


def test_8bit2d_state_kind_checks():
    """came2d_step's rules (came_bindings.cpp:617-714): 2-D only, block_size 256, every state given."""
    lib = L.load()
    size = ctypes.c_size_t(0)
    d = _desc2d((100, 300))
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(d), 1, 256, ctypes.byref(size)) == L.CAME8_OK
    ws_own = size.value
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(d), 1, 128, ctypes.byref(size)) == L.CAME8_EINVAL
    assert b"block_size=256" in lib.came8_last_error()
    d.res_col_absmax = None
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(d), 1, 256, ctypes.byref(size)) == L.CAME8_EINVAL
    assert b"residual" in lib.came8_last_error()
    n = _desc2d((2, 3, 5, 7))
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(n), 1, 256, ctypes.byref(size)) == L.CAME8_EINVAL
    v = _desc2d((33,))
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(v), 1, 256, ctypes.byref(size)) == L.CAME8_EINVAL
    # the caller's tile partial buffers replace the workspace's copy: R*ceil(C/16) + C*ceil(R/16) floats
    d = _desc2d((100, 300))
    d.res_row_partial = 0x7000000000
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(d), 1, 256, ctypes.byref(size)) == L.CAME8_EINVAL
    d.res_col_partial = 0x7100000000
    assert lib.came8_workspace_size((L.Came8Tensor * 1)(d), 1, 256, ctypes.byref(size)) == L.CAME8_OK
    assert ws_own - size.value >= 4 * (100 * 19 + 300 * 7)


@pytest.mark.parametrize("kw,msg", [
    (dict(lr=0.0), "lr must be > 0"),
    (dict(lr=1e-3, clip_threshold=0.0), "clip_threshold must be > 0"),
    (dict(lr=1e-3, eps=(1e-30,)), "eps must be a tuple of length 2"),
    (dict(lr=1e-3, betas=(0.9, 0.999)), "betas must be a tuple of length 3"),
    (dict(lr=1e-3, block_size=128), "Only block_size=256 is supported"),
])
def test_came8bit2d_constructor_validation(kw, msg):
    with pytest.raises(ValueError, match=msg):
        came_amd.CAME8bit2D([torch.nn.Parameter(torch.zeros(4, 4))], **kw)


def test_came8bit2d_group_keys_and_cpu_refusal():
    p = torch.nn.Parameter(torch.zeros(4, 4))
    opt = came_amd.CAME8bit2D([p], lr=1e-3, weight_decay=0.1, cuda_graph_compatible=True)
    g = opt.param_groups[0]
    assert {k: g[k] for k in ("lr", "eps", "clip_threshold", "betas", "weight_decay", "block_size")} == dict(
        lr=1e-3, eps=(1e-30, 1e-16), clip_threshold=1.0, betas=(0.9, 0.999, 0.9999), weight_decay=0.1,
        block_size=256)
    assert opt.cuda_graph_compatible is True
    p.grad = torch.zeros(4, 4)
    with pytest.raises(NotImplementedError, match="requires CUDA parameters"):
        opt.step()
    with pytest.raises(RuntimeError, match="requires CUDA parameters"):
        opt.prime_for_cuda_graph()


def test_came8bit2d_state_layout_matches_oracle_init():
    """init_8bit2d_state (the product) and the oracle's restatement of came8bit2d_state.py:33-75 agree on
    every persistent key, dtype, shape and initial value; the reference's scratch keys are present."""
    from came_amd.optim import init_8bit2d_state
    for shape in [(37, 50), (1, 1), (16, 33), (4097, 129)]:
        st = {}
        init_8bit2d_state(st, torch.zeros(shape))
        ref = orc.init_8bit2d_state(shape)
        for k, v in ref.items():
            if isinstance(v, torch.Tensor):
                assert st[k].dtype == v.dtype and st[k].shape == v.shape and torch.equal(st[k], v), k
            else:
                assert st[k] == v, k
        extra = set(st) - set(ref)
        assert extra == set(orc.SCRATCH_8BIT2D_KEYS)
        assert "step" not in st
