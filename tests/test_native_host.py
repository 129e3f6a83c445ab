"""The native host path's checks on the CPU (mi_adamw._host, csrc/host.cpp).

A plan for one table-free launch (one row, which lives on the host) is built over CPU
tensors, so prepare() runs every check, the step counting and the row patching without
any GPU call.  It must report READY when nothing moved, READY_MOVED after a new gradient
tensor (and patch the host row), and FALLBACK, with nothing changed, for everything it
must leave to the general path.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from mi_adamw import _lib
from mi_adamw.optimizer import _ROW_DTYPE


class _Setup:
    def __init__(self, n_params: int = 1, same_hyper: bool = True, n: int = 1000):
        self.host = _lib.host()
        self.params = [torch.nn.Parameter(torch.randn(n)) for _ in range(n_params)]
        for p in self.params:
            p.grad = torch.randn(n)
        self.steps = torch.full((n_params,), 7.0)
        self.states = [{"step": self.steps[i], "exp_avg": torch.zeros(n), "exp_avg_sq": torch.zeros(n)}
                       for i in range(n_params)]
        self.rows = np.zeros(1, dtype=_ROW_DTYPE)
        p0 = self.params[0]
        self.rows[0] = (p0.data_ptr(), p0.grad.data_ptr(), self.states[0]["exp_avg"].data_ptr(),
                        self.states[0]["exp_avg_sq"].data_ptr(), 0, 0, n, 0, _lib.T_VEC)
        r = self.rows[0]
        self.flat_row = _lib.TensorRow(param=int(r["param"]), grad=int(r["grad"]),
                                       exp_avg=int(r["exp_avg"]), exp_avg_sq=int(r["exp_avg_sq"]),
                                       param_copy=0, max_exp_avg_sq=0, numel=n, hyper=0,
                                       flags=_lib.T_VEC)
        n_hyper = 1 if same_hyper else n_params
        self.hyper_steps = np.zeros(n_hyper, dtype=np.float64)
        hypers = [0 if same_hyper else i for i in range(n_params)]
        row_of = [0] + [-1] * (n_params - 1)
        self.plan = self.host.plan(
            list(self.params), list(self.states), list(range(n_params)), hypers, row_of,
            [True] * n_params, [p.grad.data_ptr() for p in self.params], False,
            (self.steps.data_ptr(), self.steps.numel()),
            (self.hyper_steps.ctypes.data, n_hyper),
            (False, 0, 0, 1, 1, self.rows.ctypes.data, ctypes.addressof(self.flat_row), 0),
            (4096, 0, 0, 0, True, 1.0, 1.0, 0, 0, 0, 123),
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
                                    "p.data narrowed", "grad narrowed", "state replaced",
                                    "state data", "step replaced", "other stream"])
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
    elif change == "grad narrowed":
        # a gradient whose storage is smaller than the row (torch checks shapes on
        # assignment, .data of the gradient is not checked)
        p.grad.data = torch.randn(p.numel() // 2)
    elif change == "state replaced":
        s.states[1]["exp_avg"] = s.states[1]["exp_avg"].clone()
    elif change == "state data":
        s.states[1]["exp_avg_sq"].data = torch.zeros(p.numel())
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
                  (4096, 0, 0, 0, False, 0.0, 1.0, 0, 0, 0, 0), ())
    good_state = {"step": steps[0], "exp_avg": torch.zeros(4), "exp_avg_sq": torch.zeros(4)}
    with pytest.raises(ValueError):         # slot outside the step buffer
        host.plan([p], [good_state], [5], [0], [0], [True], [0], False, common["steps"],
                  common["hs"], (False, 0, 0, 1, 1, rows.ctypes.data, ctypes.addressof(row), 0),
                  (4096, 0, 0, 0, False, 0.0, 1.0, 0, 0, 0, 0), ())
