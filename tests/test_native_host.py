"""The native host path's checks on the CPU (mi_adamw._host, csrc/host.cpp).

A plan for one table-free launch (one row, which lives on the host) is built over CPU
tensors, so prepare() runs every check, the step counting and the row patching without
any GPU call.  It must report READY when nothing moved, READY_MOVED after a new gradient
tensor (and patch the host row), and FALLBACK, with nothing changed, for everything it
must leave to the general path.  A plan over device tables calls mi_adamw_set_grads for
moved gradients; bound to a stub that fails, prepare() must report ERROR with the
library's code and change nothing, and the optimizer must raise and drop its tables.
"""
from __future__ import annotations

import ctypes
import types

import numpy as np
import pytest
import torch

from mi_adamw import _lib
from mi_adamw.optimizer import _ROW_DTYPE, FusedAdamW


class _Setup:
    def __init__(self, n_params: int = 1, same_hyper: bool = True, n: int = 1000,
                 tables: bool = False):
        self.host = _lib.host()
        self.params = [torch.nn.Parameter(torch.randn(n)) for _ in range(n_params)]
        for p in self.params:
            p.grad = torch.randn(n)
        self.steps = torch.full((n_params,), 7.0)
        self.states = [{"step": self.steps[i], "exp_avg": torch.zeros(n), "exp_avg_sq": torch.zeros(n)}
                       for i in range(n_params)]
        n_rows = n_params if tables else 1
        self.rows = np.zeros(n_rows, dtype=_ROW_DTYPE)
        for i in range(n_rows):
            p, st = self.params[i], self.states[i]
            self.rows[i] = (p.data_ptr(), p.grad.data_ptr(), st["exp_avg"].data_ptr(),
                            st["exp_avg_sq"].data_ptr(), 0, 0, n, 0, _lib.T_VEC)
        r = self.rows[0]
        self.flat_row = _lib.TensorRow(param=int(r["param"]), grad=int(r["grad"]),
                                       exp_avg=int(r["exp_avg"]), exp_avg_sq=int(r["exp_avg_sq"]),
                                       param_copy=0, max_exp_avg_sq=0, numel=n, hyper=0,
                                       flags=_lib.T_VEC)
        n_hyper = 1 if same_hyper else n_params
        self.hyper_steps = np.zeros(n_hyper, dtype=np.float64)
        hypers = [0 if same_hyper else i for i in range(n_params)]
        if tables:
            # the device table's address is only handed to mi_adamw_set_grads, which the
            # tests below replace with a stub that never reads it
            row_of = list(range(n_params))
            launch = (True, 0x1000, 0x2000, 1, n_params, self.rows.ctypes.data, 0, 0)
        else:
            row_of = [0] + [-1] * (n_params - 1)
            launch = (False, 0, 0, 1, 1, self.rows.ctypes.data, ctypes.addressof(self.flat_row), 0)
        self.plan = self.host.plan(
            list(self.params), list(self.states), list(range(n_params)), hypers, row_of,
            [True] * n_params, [p.grad.data_ptr() for p in self.params], False,
            (self.steps.data_ptr(), self.steps.numel()),
            (self.hyper_steps.ctypes.data, n_hyper), launch,
            (4096, 0, 0, 0, True, 1.0, 1.0, 0, 0, 0, 123, False),
            (self.rows, self.steps, self.hyper_steps))

    def prepare(self, stream: int = 123) -> int:
        return self.host.prepare(self.plan, stream)


def test_ready_advances_the_step_counts():
    s = _Setup(n_params=3)
    assert s.prepare() == s.host.READY
    assert s.steps.tolist() == [8.0, 8.0, 8.0]
    assert s.hyper_steps.tolist() == [8.0]
    assert s.prepare() == s.host.READY
    assert s.steps.tolist() == [9.0, 9.0, 9.0]
    assert float(s.states[1]["step"]) == 9.0          # the state's step is a view of the buffer


def test_moved_gradient_patches_the_host_row():
    s = _Setup()
    p = s.params[0]
    p.grad = torch.randn(p.shape)                      # as backward allocates after zero_grad
    assert s.prepare() == s.host.READY_MOVED
    assert int(s.rows[0]["grad"]) == p.grad.data_ptr()
    assert int(s.rows[0]["flags"]) == (_lib.T_VEC if p.grad.data_ptr() % 16 == 0 else 0)
    assert s.prepare() == s.host.READY                 # the plan now holds the new address
    # a misaligned gradient view clears the vector flag
    base = torch.randn(p.numel() + 1)
    p.grad = base[1:]
    assert p.grad.data_ptr() % 16 != 0
    assert s.prepare() == s.host.READY_MOVED
    assert int(s.rows[0]["flags"]) == 0
    assert s.steps.tolist() == [10.0]


def _unchanged(s, before_steps):
    assert s.steps.tolist() == before_steps


@pytest.mark.parametrize("change", ["grad None", "grad non-contiguous", "grad dtype", "p.data",
                                    "p.data narrowed", "p.data re-strided", "grad narrowed",
                                    "state replaced", "state data", "state re-strided",
                                    "state narrowed", "step replaced", "other stream"])
def test_every_other_change_falls_back_untouched(change):
    s = _Setup(n_params=2)
    assert s.prepare() == s.host.READY
    before = s.steps.tolist()
    rows_before = s.rows.copy()
    p = s.params[1]
    stream = 123
    if change == "grad None":
        p.grad = None
    elif change == "grad non-contiguous":
        p.grad = torch.randn(2 * p.numel())[::2]
        assert not p.grad.is_contiguous()
    elif change == "grad dtype":
        # torch refuses a grad of another dtype on assignment; a complex parameter's
        # view does not arise here, so swap the parameter's storage dtype instead
        with torch.no_grad():
            p.data = p.data.double()
        p.grad = torch.randn(p.shape, dtype=torch.float64)
    elif change == "p.data":
        with torch.no_grad():
            p.data = p.data.clone()
    elif change == "p.data narrowed":
        # same address, fewer elements: the row (and the state) still cover the old size
        ptr = p.data_ptr()
        with torch.no_grad():
            p.data = p.data[:p.numel() // 2]
        assert p.data_ptr() == ptr
        p.grad = torch.randn(p.shape)
    elif change == "p.data re-strided":
        # same address and element count, elements in another order (a transposed view):
        # the row steps by memory position, so it no longer pairs p with a dense gradient
        ptr = p.data_ptr()
        with torch.no_grad():
            p.data = p.data.as_strided((p.numel() // 2, 2), (1, p.numel() // 2))
        assert p.data_ptr() == ptr and not p.is_contiguous()
        p.grad = torch.randn(p.shape)
    elif change == "grad narrowed":
        # a gradient whose storage is smaller than the row (torch checks shapes on
        # assignment, .data of the gradient is not checked)
        p.grad.data = torch.randn(p.numel() // 2)
    elif change == "state replaced":
        s.states[1]["exp_avg"] = s.states[1]["exp_avg"].clone()
    elif change == "state data":
        s.states[1]["exp_avg_sq"].data = torch.zeros(p.numel())
    elif change == "state re-strided":
        # same object, address and element count, elements in another order
        v = s.states[1]["exp_avg_sq"]
        ptr = v.data_ptr()
        v.data = v.data.as_strided((v.numel() // 2, 2), (1, v.numel() // 2))
        assert v.data_ptr() == ptr and not v.is_contiguous()
    elif change == "state narrowed":
        # same object and address, fewer elements than the row reads
        m = s.states[1]["exp_avg"]
        ptr = m.data_ptr()
        m.data = m.data[:m.numel() // 2]
        assert m.data_ptr() == ptr
    elif change == "step replaced":
        s.states[1]["step"] = torch.tensor(8.0)
    elif change == "other stream":
        stream = 456
    assert s.prepare(stream) == s.host.FALLBACK
    _unchanged(s, before)
    assert np.array_equal(s.rows, rows_before)


def test_a_group_with_two_step_counts_falls_back():
    s = _Setup(n_params=2)
    s.steps[1] = 3.0
    assert s.prepare() == s.host.FALLBACK
    assert s.steps.tolist() == [7.0, 3.0]
    # in separate hyperparameter sets the two counts are fine
    t = _Setup(n_params=2, same_hyper=False)
    t.steps[1] = 3.0
    assert t.prepare() == t.host.READY
    assert t.steps.tolist() == [8.0, 4.0] and t.hyper_steps.tolist() == [8.0, 4.0]


def test_plan_refuses_bad_entries():
    host = _lib.host()
    p = torch.nn.Parameter(torch.randn(4))
    steps = torch.zeros(1)
    hs = np.zeros(1)
    rows = np.zeros(1, dtype=_ROW_DTYPE)
    row = _lib.TensorRow()
    common = dict(steps=(steps.data_ptr(), 1), hs=(hs.ctypes.data, 1))
    bad_state = {"step": steps[0], "exp_avg": "not a tensor", "exp_avg_sq": torch.zeros(4)}
    with pytest.raises(ValueError):
        host.plan([p], [bad_state], [0], [0], [0], [True], [0], False, common["steps"],
                  common["hs"], (False, 0, 0, 1, 1, rows.ctypes.data, ctypes.addressof(row), 0),
                  (4096, 0, 0, 0, False, 0.0, 1.0, 0, 0, 0, 0, False), ())
    good_state = {"step": steps[0], "exp_avg": torch.zeros(4), "exp_avg_sq": torch.zeros(4)}
    with pytest.raises(ValueError):         # slot outside the step buffer
        host.plan([p], [good_state], [5], [0], [0], [True], [0], False, common["steps"],
                  common["hs"], (False, 0, 0, 1, 1, rows.ctypes.data, ctypes.addressof(row), 0),
                  (4096, 0, 0, 0, False, 0.0, 1.0, 0, 0, 0, 0, False), ())


_SET_GRADS = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32,
                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p)


@pytest.fixture
def failing_set_grads():
    """The host extension bound to a stub mi_adamw_set_grads that returns the codes in
    `codes` in turn (the library's other entry points stay bound); rebound to the
    library afterwards."""
    host = _lib.host()
    lib = _lib.load()
    real = [ctypes.cast(getattr(lib, name), ctypes.c_void_p).value for name in _lib.HOST_BINDINGS]
    codes, calls = [], []

    def stub(rows, n_rows, n, prow, pgrad, pvec, stream):
        calls.append(n)
        return codes.pop(0)

    fn = _SET_GRADS(stub)
    host.bind(ctypes.cast(fn, ctypes.c_void_p).value, *real[1:])
    try:
        yield codes, calls
    finally:
        host.bind(*real)


def test_a_failed_gradient_patch_is_an_error_and_changes_nothing(failing_set_grads):
    codes, calls = failing_set_grads
    s = _Setup(n_params=3, tables=True)
    assert s.prepare() == s.host.READY
    assert calls == []                                  # nothing moved, nothing patched
    steps, hsteps, rows = s.steps.tolist(), s.hyper_steps.tolist(), s.rows.copy()
    for p in s.params:
        p.grad = torch.randn(p.shape)
    # 1 is hipErrorInvalidValue and 2 hipErrorOutOfMemory: the same integers as FALLBACK
    # and READY_MOVED, which must not be how they read
    for code in (1, 2, _lib.E_INVALID):
        codes.append(code)
        assert s.prepare() == s.host.ERROR
        assert s.host.last_error(s.plan) == code
        assert s.steps.tolist() == steps and s.hyper_steps.tolist() == hsteps
        assert np.array_equal(s.rows, rows)
    assert calls == [3, 3, 3]
    codes.append(_lib.OK)
    assert s.prepare() == s.host.READY_MOVED        # the plan still knows the old addresses
    assert [int(r) for r in s.rows["grad"]] == [p.grad.data_ptr() for p in s.params]
    assert s.steps.tolist() == [x + 1 for x in steps]


def test_the_optimizer_raises_and_drops_its_tables_on_a_failed_patch(failing_set_grads):
    codes, _ = failing_set_grads
    s = _Setup(n_params=2, tables=True)
    cache = types.SimpleNamespace(grads=[p.grad.data_ptr() for p in s.params])
    fast = types.SimpleNamespace(plan=s.plan, cache=cache)
    opt = types.SimpleNamespace(_fast=fast, _launch_cache=cache, native_steps=0)
    assert FusedAdamW._fast_prepare(opt, fast, s.host, 123) is True
    assert opt.native_steps == 1
    steps = s.steps.tolist()
    s.params[1].grad = torch.randn(s.params[1].shape)
    codes.append(2)
    with pytest.raises(_lib.MiAdamwError, match=r"mi_adamw_set_grads failed: .*\(code 2\)"):
        FusedAdamW._fast_prepare(opt, fast, s.host, 123)
    assert opt._fast is None and opt._launch_cache is None and opt.native_steps == 1
    assert s.steps.tolist() == steps
    # another stream: the general path takes the step
    opt2 = types.SimpleNamespace(_fast=fast, _launch_cache=cache, native_steps=0)
    assert FusedAdamW._fast_prepare(opt2, fast, s.host, 456) is False
    assert opt2._fast is fast and opt2.native_steps == 0
