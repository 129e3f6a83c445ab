"""CPU tests of the drop-in boundary: constructor, param_groups, state_dict, C ABI exports.

No GPU work runs here.  The library is loaded (it links the HIP runtime but
touches no device) to check that every symbol include/mi_adamw.h declares is
exported and that the host-side chunk-table helper is right.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np
import pytest
import torch

import mi_adamw
from mi_adamw import _lib
from mi_adamw.optimizer import _hyper
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mi_adamw.h")


def _params():
    return [torch.nn.Parameter(torch.randn(10, 3)), torch.nn.Parameter(torch.randn(4))]


@pytest.mark.parametrize("fused", [False, True, None])
def test_defaults_and_param_groups_match_torch(fused):
    """main.py:177 passes fused=args.fused: either value builds the same defaults and
    param_groups as torch's AdamW (the step is fused either way)."""
    ours = mi_adamw.FusedAdamW(_params(), lr=6e-4, weight_decay=0.1, fused=fused)
    ref = torch.optim.AdamW(_params(), lr=6e-4, weight_decay=0.1, fused=fused)
    assert ours.defaults == ref.defaults
    assert ours.param_groups[0].keys() == ref.param_groups[0].keys()
    for k in ref.param_groups[0]:
        if k != "params":
            assert ours.param_groups[0][k] == ref.param_groups[0][k]
    assert ours.state_dict() == ref.state_dict()
    assert mi_adamw.AdamW is mi_adamw.FusedAdamW
    assert isinstance(ours, torch.optim.Optimizer)


@pytest.mark.parametrize("kwargs", [
    dict(lr=-1.0), dict(eps=-1e-8), dict(betas=(1.0, 0.999)), dict(betas=(0.9, -0.1)),
    dict(weight_decay=-0.1), dict(betas=(0.9, torch.tensor(0.99))),
    dict(lr=torch.tensor([1e-3, 2e-3])),
    dict(lr=torch.tensor(1e-3), foreach=True),
])
def test_invalid_arguments_raise_like_torch(kwargs):
    with pytest.raises((ValueError, RuntimeError)) as ref:
        torch.optim.AdamW(_params(), **kwargs)
    with pytest.raises(type(ref.value)) as ours:
        mi_adamw.FusedAdamW(_params(), **kwargs)
    assert str(ours.value) == str(ref.value)


@pytest.mark.parametrize("kwargs", [dict(differentiable=True),
                                    dict(betas=(torch.tensor(0.9), torch.tensor(0.999)))])
def test_unsupported_flags_fail_loudly(kwargs):
    with pytest.raises(NotImplementedError):
        mi_adamw.FusedAdamW(_params(), **kwargs)


def test_capturable_groups_must_agree():
    opt = mi_adamw.FusedAdamW(_params(), capturable=True)
    assert opt.capturable and opt.param_groups[0]["capturable"] is True
    with pytest.raises(NotImplementedError, match="capturable"):
        opt.add_param_group({"params": _params(), "capturable": False})
    with pytest.raises(NotImplementedError, match="capturable"):
        mi_adamw.FusedAdamW([{"params": _params()}, {"params": _params(), "capturable": True}])
    assert len(opt.param_groups) == 1


def test_capturable_group_constants():
    """The capturable chain's per-group constants: betas, 1-beta1, 1-beta2 and eps
    rounded to fp32; a float lr with its host weight-decay factor; a CPU tensor lr by
    value; a device lr by pointer (not built without a GPU)."""
    from mi_adamw.optimizer import _capt_hyper
    f32 = np.float32
    g = dict(lr=6e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, maximize=True)
    h = _capt_hyper(g, torch.device("cpu"))
    assert (h.beta1, h.beta2) == (float(f32(0.9)), float(f32(0.999)))
    assert h.lerp_w == float(f32(1 - 0.9)) and h.one_minus_beta2 == float(f32(1 - 0.999))
    assert h.eps == float(f32(1e-8)) and h.grad_sign == -1.0
    assert h.lr_mode == _lib.LR_FLOAT and h.lr == float(f32(6e-4))
    assert h.wd_factor == float(f32(1 - 6e-4 * 0.1))
    h = _capt_hyper(dict(g, lr=torch.tensor(6e-4), weight_decay=0.0), torch.device("cpu"))
    assert h.lr_mode == _lib.LR_VALUE and h.lr == float(f32(6e-4)) and h.wd_factor == 1.0
    h = _capt_hyper(dict(g, lr=torch.tensor(6e-4)), torch.device("cpu"))
    assert h.wd_factor == float((1 - torch.tensor(6e-4) * 0.1).item())
    with pytest.raises(NotImplementedError, match="float32"):
        _capt_hyper(dict(g, lr=torch.tensor(6e-4, dtype=torch.float64)), torch.device("cpu"))


def test_fused_chain_group_set():
    """fused=True's per-group set: lr, betas, weight decay and eps as the float64 values
    torch._fused_adamw_ receives, the step count as fp32, maximize as the sign; a CPU
    tensor lr by value (the op's tensor-lr overload takes lr.item()); on a CPU device a
    device lr is never formed."""
    from mi_adamw.optimizer import _fused_hyper
    g = dict(lr=6e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, maximize=True)
    h = _fused_hyper(g, 1001.0, torch.device("cpu"))
    assert (h.lr, h.beta1, h.beta2, h.weight_decay, h.eps) == (6e-4, 0.9, 0.999, 0.1, 1e-8)
    assert h.step == 1001.0 and h.grad_sign == -1.0 and not h.lr_ptr
    h = _fused_hyper(dict(g, lr=torch.tensor(6e-4), maximize=False), 3.0, torch.device("cpu"))
    assert h.lr == float(np.float32(6e-4)) and h.grad_sign == 1.0 and not h.lr_ptr
    h = _fused_hyper(dict(g, lr=torch.tensor(6e-4, dtype=torch.float64)), 3.0,
                     torch.device("cpu"))
    assert h.lr == 6e-4
    assert ctypes.sizeof(h) == 56


@pytest.mark.parametrize("view", ["strided", "transposed", "wrong_dtype"])
def test_state_entries_are_made_dense_for_the_kernel(view):
    """A state entry put into the dict as a strided view, a transposed view or another
    dtype is replaced by a dense copy of the state dtype with the same values before its
    pointer goes into a table (the kernel reads numel contiguous elements from it)."""
    p = torch.nn.Parameter(torch.randn(6, 5))
    opt = mi_adamw.FusedAdamW([p])
    vals = torch.randn(6, 5)
    if view == "strided":
        base = torch.full((60,), 7.0)
        t = base[::2]
        t.copy_(vals.reshape(-1))
    elif view == "transposed":
        t = vals.t().contiguous().t()
    else:
        t = vals.double()
    st = {"exp_avg": t}
    out = opt._state_tensor(p, st, "exp_avg")
    assert out.is_contiguous() and out.dtype == torch.float32 and st["exp_avg"] is out
    assert torch.equal(out.reshape(-1), vals.reshape(-1).float())
    if view == "strided":
        assert out.data_ptr() != base.data_ptr()


def test_extra_options_are_validated():
    with pytest.raises(ValueError):
        mi_adamw.FusedAdamW(_params(), max_grad_norm=0.0)
    with pytest.raises(ValueError):
        mi_adamw.FusedAdamW(_params(), state_dtype=torch.float16)
    with pytest.raises(ValueError):
        mi_adamw.FusedAdamW(_params(), chunk_elems=1000)
    for bad in (-1, 1.5, "4"):
        with pytest.raises(ValueError, match="place_trials"):
            mi_adamw.FusedAdamW(_params(), place_trials=bad)
    with pytest.raises(NotImplementedError, match="place_trials"):
        mi_adamw.FusedAdamW(_params(), place_trials=2, amsgrad=True)
    capt = mi_adamw.FusedAdamW(_params(), place_trials=2, capturable=True)
    assert capt.place_trials == 2 and capt.captured is False
    opt = mi_adamw.FusedAdamW(_params(), place_trials=4)
    assert opt.place_trials == 4 and opt.placement is None


def test_step_on_cpu_params_raises_before_touching_state():
    params = _params()
    opt = mi_adamw.FusedAdamW(params)
    for p in params:
        p.grad = torch.randn_like(p)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        opt.step()
    assert len(opt.state) == 0


def test_step_without_grads_is_a_noop():
    opt = mi_adamw.FusedAdamW(_params())
    assert opt.step() is None
    assert opt.step(lambda: 3.0) == 3.0
    assert len(opt.state) == 0


def test_sparse_grad_raises_like_torch():
    p = torch.nn.Parameter(torch.randn(4, 3))
    p.grad = torch.randn(4, 3).to_sparse()
    with pytest.raises(RuntimeError, match="sparse"):
        mi_adamw.FusedAdamW([p]).step()


def test_add_param_group_and_zero_grad():
    params = _params()
    opt = mi_adamw.FusedAdamW(params, lr=1e-3)
    opt.add_param_group({"params": [torch.nn.Parameter(torch.randn(5))], "lr": 2e-3})
    assert len(opt.param_groups) == 2
    assert opt.param_groups[1]["lr"] == 2e-3
    assert opt.param_groups[1]["betas"] == (0.9, 0.999)
    for g in opt.param_groups:
        for p in g["params"]:
            p.grad = torch.ones_like(p)
    opt.zero_grad()
    assert all(p.grad is None for g in opt.param_groups for p in g["params"])


def test_load_torch_state_dict_on_cpu_keeps_torch_layout():
    """A torch AdamW state dict (CPU) loads; steps live in the packed CPU buffer."""
    ref_params = _params()
    ref = torch.optim.AdamW(ref_params, lr=1e-3, fused=False)
    for p in ref_params:
        p.grad = torch.randn_like(p)
    ref.step()
    ref.step()
    ours = mi_adamw.FusedAdamW([torch.nn.Parameter(p.detach().clone()) for p in ref_params],
                               lr=1e-3, fused=False)
    ours.load_state_dict(ref.state_dict())
    sd = ours.state_dict()
    for i, st in sd["state"].items():
        assert float(st["step"]) == 2.0
        assert st["step"].dtype == torch.float32 and st["step"].device.type == "cpu"
        assert torch.equal(st["exp_avg"], ref.state[ref_params[i]]["exp_avg"])
    # Steps of different params are independent tensors in the saved dict.
    assert sd["state"][0]["step"] is not sd["state"][1]["step"]
    sd["state"][0]["step"] += 1
    assert float(sd["state"][1]["step"]) == 2.0


def test_bf16_state_dict_loads_as_bf16():
    ref_params = _params()
    ref = torch.optim.AdamW(ref_params, lr=1e-3)
    for p in ref_params:
        p.grad = torch.randn_like(p)
    ref.step()
    ours = mi_adamw.FusedAdamW([torch.nn.Parameter(p.detach().clone()) for p in ref_params],
                               lr=1e-3, state_dtype=torch.bfloat16)
    ours.load_state_dict(ref.state_dict())
    for p in ours.param_groups[0]["params"]:
        assert ours.state[p]["exp_avg"].dtype == torch.bfloat16
        assert ours.state[p]["exp_avg_sq"].dtype == torch.bfloat16


@pytest.mark.parametrize("lr,betas,eps,wd,step,maximize", [
    (3e-4, (0.9, 0.95), 1e-8, 0.1, 1.0, False),
    (6e-4, (0.9, 0.999), 1e-8, 0.1, 7.0, False),
    (1e-3, (0.3, 0.95), 1e-6, 0.0, 1000.0, True),
    (0.0, (0.9, 0.999), 1e-8, 0.1, 2.0, False),
    (3e-4, (0.9, 0.95), 1e-8, 0.1, 16777217.0, False),
])
def test_product_scalars_equal_oracle_scalars(lr, betas, eps, wd, step, maximize):
    """The product's per-step fp32 scalars equal the oracle's (pinned by the golden tests)."""
    group = dict(lr=lr, betas=betas, eps=eps, weight_decay=wd, maximize=maximize)
    step = float(np.float32(step))
    ours = _hyper(group, step)
    ref = O.hyper_from_group(lr, betas[0], betas[1], eps, wd, step, maximize)
    assert ours.wd_factor == ref.wd_factor
    assert ours.lerp_w == ref.lerp_w
    assert ours.beta2 == ref.beta2
    assert ours.one_minus_beta2 == ref.one_minus_beta2
    assert ours.inv_bc2_sqrt == float(np.float32(1.0 / ref.bc2_sqrt))
    assert ours.eps == ref.eps
    assert ours.neg_step_size == ref.neg_step_size
    assert ours.grad_sign == ref.grad_sign


def _header_functions():
    text = open(HEADER).read()
    return re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(mi_adamw_[a-z_0-9]+)\s*\(", text, re.M)


def test_library_exports_every_header_symbol():
    lib = _lib.load()
    names = _header_functions()
    assert set(names) == set(_lib.EXPORTS)
    for name in names:
        assert hasattr(lib, name), name
    assert _lib.version().startswith(f"mi_adamw {_lib.ABI_VERSION} gfx950")


def test_header_structs_match_bindings():
    text = open(HEADER).read()
    assert f"#define MI_ADAMW_ABI_VERSION {_lib.ABI_VERSION}" in text
    assert f"#define MI_ADAMW_MAX_HYPER {_lib.MAX_HYPER}" in text
    assert f"#define MI_ADAMW_MAX_NORM_BLOCKS {_lib.MAX_NORM_BLOCKS}" in text
    assert f"#define MI_ADAMW_CHUNK_QUANTUM {_lib.CHUNK_QUANTUM}" in text
    assert ctypes.sizeof(_lib.TensorRow) == 64
    assert ctypes.sizeof(_lib.Hyper) == 8 * 4
    # Field order of mi_adamw_tensor, as declared in the header.
    body = text[text.index("typedef struct mi_adamw_tensor {"):text.index("} mi_adamw_tensor;")]
    fields = re.findall(r"\*?\s*(\w+);", body)
    assert fields == [f for f, _ in _lib.TensorRow._fields_]
    assert f"#define MI_ADAMW_F_AMSGRAD (1 << 3)" in text and _lib.F_AMSGRAD == 1 << 3
    body = text[text.index("typedef struct mi_adamw_capt_hyper {"):
                text.index("} mi_adamw_capt_hyper;")]
    assert re.findall(r"\*?\s*(\w+);", body) == [f for f, _ in _lib.CaptHyper._fields_]
    for name in ("LR_FLOAT", "LR_VALUE", "LR_DEVICE"):
        assert f"#define MI_ADAMW_{name} {getattr(_lib, name)}" in text


def test_table_rows_are_built_field_by_field_on_cpu():
    """The tensor tables the optimizer and the clip hand the kernels, built on
    CPU tensors (no launch): every field lands where the row layout puts it."""
    from mi_adamw import clip as C
    from mi_adamw.optimizer import _ROW_DTYPE, _Rec
    assert _ROW_DTYPE.names == tuple(f for f, _ in _lib.TensorRow._fields_)
    assert _ROW_DTYPE.itemsize == ctypes.sizeof(_lib.TensorRow)
    grads = [torch.zeros(10), torch.zeros(4097), torch.zeros(0)]
    launch = C._tables(grads, torch.device("cpu"), 0)
    rows = launch.host_rows
    assert len(rows) == 2
    assert list(rows["grad"]) == [grads[0].data_ptr(), grads[1].data_ptr()]
    assert list(rows["numel"]) == [10, 4097]
    assert list(rows["max_exp_avg_sq"]) == [0, 0]
    assert launch.n_chunks == 1 + 2

    params = [torch.nn.Parameter(torch.zeros(6)), torch.nn.Parameter(torch.zeros(5))]
    opt = mi_adamw.FusedAdamW([dict(params=params[:1], amsgrad=True),
                               dict(params=params[1:])])
    entries = []
    for gi, p in enumerate(params):
        rec = _Rec(gi, p, opt._slots[id(p)])
        rec.st = opt.state[p]
        opt._init_state(p, rec.st, gi == 0)
        entries.append((rec, torch.zeros_like(p)))
    ams_rows = opt._tensor_rows(entries[:1], [0], True)[0]
    plain_rows = opt._tensor_rows(entries[1:], [0], False)[0]
    st0, st1 = opt.state[params[0]], opt.state[params[1]]
    assert ams_rows["max_exp_avg_sq"][0] == st0["max_exp_avg_sq"].data_ptr() != 0
    assert ams_rows["exp_avg_sq"][0] == st0["exp_avg_sq"].data_ptr()
    assert plain_rows["max_exp_avg_sq"][0] == 0 and "max_exp_avg_sq" not in st1
    assert list(plain_rows["numel"]) == [5] and list(ams_rows["numel"]) == [6]
    row = opt._row_struct(type("L", (), {"host_rows": ams_rows})())
    assert row.max_exp_avg_sq == st0["max_exp_avg_sq"].data_ptr() and row.numel == 6
    # A state tensor of the wrong size is refused before any pointer reaches a kernel;
    # one of the wrong dtype or layout is converted in place.
    st1["exp_avg"] = torch.zeros(4)
    with pytest.raises(RuntimeError, match="elements"):
        opt._tensor_rows(entries[1:], [0], False)
    st1["exp_avg"] = torch.zeros(10, dtype=torch.float64)[::2]
    rows = opt._tensor_rows(entries[1:], [0], False)[0]
    assert st1["exp_avg"].dtype == torch.float32 and st1["exp_avg"].is_contiguous()
    assert rows["exp_avg"][0] == st1["exp_avg"].data_ptr()


def test_launch_rows_refresh_keeps_the_chunk_table():
    """When only pointers move, a launch takes new rows and keeps its chunk table; a
    change of tensor sizes is refused, so the caller rebuilds."""
    from mi_adamw.optimizer import _ROW_DTYPE, _Launch
    rows = np.zeros(3, dtype=_ROW_DTYPE)
    rows["grad"] = [4096, 8192, 12288]
    rows["numel"] = [5, 4097, 9000]
    launch = _Launch(rows, 4096, torch.device("cpu"))
    chunks = launch.chunks
    assert launch.n_chunks == 1 + 2 + 3
    moved = rows.copy()
    moved["grad"] = [65536, 131072, 196608]
    assert launch.set_rows(moved, torch.device("cpu"))
    assert launch.chunks is chunks
    assert list(launch.host_rows["grad"]) == [65536, 131072, 196608]
    assert bytes(launch.rows.numpy()) == moved.tobytes()
    resized = moved.copy()
    resized["numel"][1] = 4096
    assert not launch.set_rows(resized, torch.device("cpu"))


def test_moved_gradients_are_patched_into_the_rows():
    """Only the gradient column (and its alignment flag) changes when gradients move;
    empty tensors have no row, so rows map back to their entries."""
    from mi_adamw.optimizer import _Rec
    params = [torch.nn.Parameter(torch.zeros(n)) for n in (6, 0, 4097)]
    opt = mi_adamw.FusedAdamW(params)
    entries = []
    for p in params:
        rec = _Rec(0, p, opt._slots[id(p)])
        rec.st = opt.state[p]
        opt._init_state(p, rec.st, False)
        entries.append((rec, torch.zeros_like(p)))
    launch = opt._new_launch(entries, [0, 0, 0], False, torch.device("cpu"))
    assert list(launch.src) == [0, 2] and launch.n_rows == 2
    before = launch.host_rows.copy()
    chunks = launch.chunks
    new = np.array([1 << 20, 2 << 20, (3 << 20) + 4], dtype=np.uint64)   # the last misaligned
    launch.patch_grads(new, torch.device("cpu"))
    rows = launch.host_rows
    assert list(rows["grad"]) == [1 << 20, (3 << 20) + 4]
    assert list(rows["flags"]) == [_lib.T_VEC, 0]
    for f in ("param", "exp_avg", "exp_avg_sq", "numel", "hyper"):
        assert np.array_equal(rows[f], before[f])
    assert launch.chunks is chunks and bytes(launch.rows.numpy()) == rows.tobytes()


def test_build_chunks_helper():
    lib = _lib.load()
    numels = np.array([0, 1, 65536, 65537, 3 * 65536 - 5], dtype=np.int64)
    n = lib.mi_adamw_build_chunks(numels.ctypes.data, len(numels), 65536, None, 0)
    assert n == 0 + 1 + 1 + 2 + 3
    out = np.zeros(2 * n, dtype=np.int32)
    assert lib.mi_adamw_build_chunks(numels.ctypes.data, len(numels), 65536, out.ctypes.data, n) == n
    rows = out.reshape(-1, 2).tolist()
    assert rows == [[1, 0], [2, 0], [3, 0], [3, 1], [4, 0], [4, 1], [4, 2]]
    # Rejected: chunk size not a multiple of the quantum, too small a buffer, negative sizes.
    assert lib.mi_adamw_build_chunks(numels.ctypes.data, len(numels), 1024, None, 0) == _lib.E_INVALID
    assert lib.mi_adamw_build_chunks(numels.ctypes.data, len(numels), 65536, out.ctypes.data,
                                     n - 1) == _lib.E_INVALID
    bad = np.array([-1], dtype=np.int64)
    assert lib.mi_adamw_build_chunks(bad.ctypes.data, 1, 65536, None, 0) == _lib.E_INVALID


def test_abi_rejects_bad_arguments_without_launching():
    lib = _lib.load()
    h = (_lib.Hyper * 1)()
    # NULL tables, zero chunks, too many hyper sets, bad chunk size: all rejected on the host.
    assert lib.mi_adamw_step(None, None, 1, 65536, h, 1, None, 0, 0, 0, None) == _lib.E_INVALID
    assert lib.mi_adamw_step(1, 1, 1, 65536, h, 17, None, 0, 0, 0, None) == _lib.E_INVALID
    assert lib.mi_adamw_step(1, 1, 1, 1000, h, 1, None, 0, 0, 0, None) == _lib.E_INVALID
    assert lib.mi_adamw_step(1, 1, 0, 65536, h, 1, None, 0, 0, 0, None) == _lib.E_INVALID
    assert lib.mi_adamw_step(1, 1, 1, 65536, h, 1, None, 7, 0, 0, None) == _lib.E_INVALID
    assert lib.mi_adamw_step(1, 1, 1, 65536, h, 1, None, 0, _lib.F_CLIP, 0, None) == _lib.E_INVALID
    assert lib.mi_adamw_step(1, 1, 1, 65536, h, 1, None, 0, 1 << 5, 0, None) == _lib.E_INVALID
    assert lib.mi_adamw_grad_norm(1, 1, 0, 65536, 1.0, 1, 1, 1, None) == _lib.E_INVALID
    assert lib.mi_adamw_grad_norm_flat(None, 10, 65536, 1.0, 1, 1, 1, None) == _lib.E_INVALID
    assert lib.mi_adamw_scale_grads(1, 1, 1, 65536, None, None) == _lib.E_INVALID
    row = _lib.TensorRow(param=16, grad=32, exp_avg=48, exp_avg_sq=64, param_copy=0, numel=10,
                         hyper=0, flags=_lib.T_VEC)
    # Flat entry: a bf16 copy requested without a copy pointer, and a misaligned pointer.
    assert lib.mi_adamw_step_flat(ctypes.byref(row), h, None, 65536, 0, _lib.F_BF16_COPY, 0,
                                  None) == _lib.E_INVALID
    # amsgrad without a max_exp_avg_sq pointer, then with a misaligned one.
    assert lib.mi_adamw_step_flat(ctypes.byref(row), h, None, 65536, 0, _lib.F_AMSGRAD, 0,
                                  None) == _lib.E_INVALID
    row.max_exp_avg_sq = 84
    assert lib.mi_adamw_step_flat(ctypes.byref(row), h, None, 65536, 0, _lib.F_AMSGRAD, 0,
                                  None) == _lib.E_ALIGN
    row.max_exp_avg_sq = 0
    row.grad = 36
    assert lib.mi_adamw_step_flat(ctypes.byref(row), h, None, 65536, 0, 0, 0, None) == _lib.E_ALIGN
    assert "invalid" in _lib.strerror(_lib.E_INVALID)


def test_deepcopy_and_pickle_give_a_working_optimizer():
    """torch optimizers survive copy.deepcopy and pickling (Optimizer.__getstate__);
    FusedAdamW's own options and bookkeeping come back with them."""
    import copy
    import pickle
    params = [torch.nn.Parameter(torch.randn(4, 3)), torch.nn.Parameter(torch.randn(5))]
    ref = torch.optim.AdamW(params, lr=1e-3, fused=False)
    for p in params:
        p.grad = torch.randn_like(p)
    ref.step()
    opt = mi_adamw.FusedAdamW(params, lr=1e-3, fused=False, max_grad_norm=0.5, bf16_copy=True,
                              state_dtype=torch.bfloat16, chunk_elems=8192)
    opt.load_state_dict(ref.state_dict())
    for clone in (copy.deepcopy(opt), pickle.loads(pickle.dumps(opt))):
        assert (clone.max_grad_norm, clone.bf16_copy, clone.state_dtype, clone.chunk_elems) == \
            (0.5, True, torch.bfloat16, 8192)
        cps = clone.param_groups[0]["params"]
        assert all(q is not p for q, p in zip(cps, params))
        for q, p in zip(cps, params):
            st = clone.state[q]
            assert float(st["step"]) == 1.0
            assert st["step"] is clone._step_views[clone._slots[id(q)]]   # re-homed
            assert st["exp_avg"].dtype == torch.bfloat16
            assert torch.equal(st["exp_avg"], opt.state[p]["exp_avg"])
            assert torch.equal(clone.bf16_param(q), q.detach().bfloat16())
        assert clone.state_dict()["param_groups"] == opt.state_dict()["param_groups"]


def test_flat_layout_makes_no_per_parameter_copies():
    """With flat_buffer=True the bf16 copies live in the flat copy buffer only."""
    if not torch.cuda.is_available():
        opt = mi_adamw.FusedAdamW([torch.nn.Parameter(torch.zeros(3))], bf16_copy=True)
        assert len(opt._copies) == 1
        with pytest.raises(RuntimeError, match="ROCm GPU"):
            mi_adamw.FusedAdamW([torch.nn.Parameter(torch.zeros(3))], bf16_copy=True,
                                flat_buffer=True)


def test_capturable_launch_maps_rows_to_step_slots_on_cpu():
    """A capturable launch (built on CPU tensors, no kernel): one row per non-empty
    tensor, always as tables (each tensor has its own device step count), and a
    step index giving each row its parameter's slot in the packed step buffer."""
    from mi_adamw.optimizer import _Rec
    params = [torch.nn.Parameter(torch.zeros(n)) for n in (6, 0, 4097, 3)]
    opt = mi_adamw.FusedAdamW(params, capturable=True)
    entries = []
    for p in params:
        rec = _Rec(0, p, opt._slots[id(p)])
        rec.st = opt.state[p]
        opt._init_state(p, rec.st, False)
        entries.append((rec, torch.zeros_like(p)))
    launch = opt._new_launch(entries, [0] * 4, False, torch.device("cpu"))
    assert launch.tables and launch.n_rows == 3
    assert list(launch.host_rows["numel"]) == [6, 4097, 3]
    # uploaded as raw bytes; the kernel reads them as int32
    assert launch.step_index.view(torch.int32).tolist() == [opt._slots[id(params[i])]
                                                            for i in (0, 2, 3)]
    one = opt._new_launch(entries[2:3], [0], False, torch.device("cpu"))
    assert one.tables and one.n_rows == 1
    assert one.step_index.view(torch.int32).tolist() == [opt._slots[id(params[2])]]
    # the state's step tensors are views of the packed buffer, as torch's capturable layout
    # has one 0-d fp32 step per parameter
    for p in params:
        st = opt.state[p]["step"]
        assert st.dim() == 0 and st.dtype == torch.float32
        assert st.data_ptr() == opt._steps[opt._slots[id(p)]].data_ptr()


def test_param_groups_from_generators_and_named_parameters():
    """A group dict holding a generator, and torch's (name, parameter) pairs, register
    every parameter, with and without bf16 copies (the copy check must not consume
    the generator)."""
    m = torch.nn.Linear(4, 3)
    for copy in (False, True):
        o = mi_adamw.FusedAdamW([{"params": m.parameters()}], bf16_copy=copy)
        assert len(o.param_groups[0]["params"]) == 2
        o.add_param_group({"params": (p for p in [torch.nn.Parameter(torch.zeros(5))])})
        assert len(o.param_groups[1]["params"]) == 1
        # named groups (torch refuses to mix them with unnamed ones, and so do we)
        o = mi_adamw.FusedAdamW(m.named_parameters(), bf16_copy=copy)
        assert o.param_groups[0]["param_names"] == ["weight", "bias"]
        assert [id(p) for p in o.param_groups[0]["params"]] == [id(m.weight), id(m.bias)]
        if copy:
            assert o.bf16_param(m.weight).dtype == torch.bfloat16


def test_bench_bytes_per_parameter():
    """bench.py's algorithmic bytes per parameter, per configuration: p, g, m, v read and
    p, m, v written once each (fp32 4 B, bf16 moments 2 B), +2 B for the bf16 copy,
    +4 B for the norm pass's read of g, +4 B when the clipped g is stored back."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    expected = {"125m-step1": 28, "125m-clip": 32, "350m-master-clip-copy": 34,
                "1.3b-bf16state-copy": 22, "1.3b-bf16state-copy-clip": 26,
                "1.3b-bf16state-copy-clip-flat": 26, "6.7b-flat-clip-copy": 34,
                "125m-clip-fused-chain": 32, "1.3b-bf16state-copy-clip-fused-chain": 26,
                "6.7b-flat-clip-copy-fused-chain": 34}
    assert set(expected) == set(bench.CONFIGS)
    # the headline is the largest configuration; every other one is in the default sweep
    # but the headline's set in the fused=True chain, which only --sweep asks for
    assert bench.DEFAULT_CONFIG == "6.7b-flat-clip-copy"
    assert (set(bench.CONFIGS) - set(bench.DEFAULT_SWEEP) - {bench.DEFAULT_CONFIG}
            == {"6.7b-flat-clip-copy-fused-chain"})
    assert set(bench.DEFAULT_CPU) <= set(bench.CONFIGS)
    # a fused-chain configuration is its base configuration in the other chain
    for name, cfg in bench.CONFIGS.items():
        assert cfg[-1] == name.endswith("-fused-chain")
        if cfg[-1]:
            assert bench.CONFIGS[name[:-len("-fused-chain")]][:-1] == cfg[:-1]
    for name, total in expected.items():
        _, clip, state, copy, *_ = bench.CONFIGS[name]
        step, update = bench.bytes_per_param(clip, state, copy)
        assert step == total and update == total - (4 if clip else 0), name
        step_w, update_w = bench.bytes_per_param(clip, state, copy, write_grads=True)
        assert (step_w, update_w) == (step + 4, update + 4), name


def test_bench_cpu_host_record_and_streamed_baseline():
    """The CPU baseline's host record (physical and logical cores from /proc/cpuinfo) and
    the streamed full-set timing on a small set, with a pool smaller than the set."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    info = bench.host_cpu()
    assert info["affinity_cpus"] >= 1 and info["logical_cpus"] >= info["physical_cores"] >= 1
    from mi_adamw.workloads import GPTShape, SHAPES
    threads = torch.get_num_threads()
    try:
        SHAPES["gpt-tiny"] = GPTShape("gpt-tiny", layers=2, hidden=64, heads=2, ffn=256,
                                      vocab=1000, positions=128)
        bench.CONFIGS["tiny-clip"] = ("gpt-tiny", True, "fp32", False, False, 1000, 1e-2,
                                      False)
        n = SHAPES["gpt-tiny"].numel()
        cb = bench.cpu_baseline("tiny-clip", batch_params=70_000, warmup=1, reps=2)
    finally:
        SHAPES.pop("gpt-tiny", None)
        bench.CONFIGS.pop("tiny-clip", None)
        torch.set_num_threads(threads)
    assert cb["kind"] == "reference" and cb["unit"] == "GB/s" and cb["value"] > 0
    assert cb["cores"] == (info["physical_cores"] or info["affinity_cpus"])
    assert f"{n} params" in cb["sample"] and "streamed in" in cb["sample"]
    assert abs(cb["params_per_s"] - n / cb["ms_per_step"] * 1e3) <= 1e-3 * cb["params_per_s"]


def test_step_hooks_and_scheduler_see_step():
    """step() is the Optimizer's hooked step: pre/post hooks run, and LambdaLR (main.py:178-180)
    sees it called, so it raises no order warning.  No gradients: nothing reaches the GPU."""
    import warnings
    p = torch.nn.Parameter(torch.randn(4))
    opt = mi_adamw.FusedAdamW([p], lr=6e-4, weight_decay=0.1, fused=False)
    calls = []
    opt.register_step_pre_hook(lambda o, a, k: calls.append("pre"))
    opt.register_step_post_hook(lambda o, a, k: calls.append("post"))
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda it: min(1.0, it / 10))
    assert opt.param_groups[0]["lr"] == 0.0
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        assert opt.step() is None
        sched.step()
    assert calls == ["pre", "post"]
    assert opt.param_groups[0]["lr"] == pytest.approx(6e-5)
