"""The allocation-free entry point mlg_logsoftmax_topk_noalloc (static device scratch)
against mlg_logsoftmax_topk with a caller workspace: identical values and indices, on two
calls in a row (the second smaller, so stale scratch from the first would show), and the
row limit refused before anything runs."""
import ctypes as C

import numpy as np
import pytest
import torch

import malaga_amd as M
from malaga_amd import _lib

pytestmark = pytest.mark.gpu


def ptr(t):
    return C.c_void_p(t.data_ptr())


def run_both(lib, x, k, mask):
    rows, V = x.shape
    xd = torch.from_numpy(x).cuda()
    work = torch.zeros(lib.mlg_logsoftmax_topk_scratch(rows, k) // 4 + 1, device="cuda")
    v_ref = torch.zeros((rows, k), device="cuda")
    i_ref = torch.zeros((rows, k), dtype=torch.int32, device="cuda")
    _lib.check(lib.mlg_logsoftmax_topk(ptr(xd), rows, V, k, mask, ptr(work), ptr(v_ref), ptr(i_ref), None))
    v = torch.full((rows, k), 7.0, device="cuda")
    i = torch.full((rows, k), 7, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    lib.mlg_debug_fail_alloc_after(0)  # any library allocation inside the call would now fail
    try:
        _lib.check(lib.mlg_logsoftmax_topk_noalloc(ptr(xd), rows, V, k, mask, ptr(v), ptr(i), None))
        torch.cuda.synchronize()
    finally:
        lib.mlg_debug_fail_alloc_after(-1)
    return v_ref.cpu().numpy(), i_ref.cpu().numpy(), v.cpu().numpy(), i.cpu().numpy()


def test_noalloc_topk_equals_workspace_entry():
    M._Ctx(0)  # a context makes device 0 current, as a model would
    lib = _lib.load()
    rng = np.random.default_rng(17)
    for rows, V, k, mask in ((256, 256206, 8, 2), (5, 3001, 4, -1)):  # the second call smaller
        x = rng.normal(0, 3, (rows, V)).astype(np.float32)
        x[0, 77] = x[0, 33] = 40.0  # a tie: the lower index first
        vr, ir, v, i = run_both(lib, x, k, mask)
        assert np.array_equal(ir, i)
        assert np.array_equal(vr.view(np.uint32), v.view(np.uint32))
        assert i[0, :2].tolist() == [33, 77]


def test_noalloc_topk_refuses_rows_beyond_the_scratch():
    lib = _lib.load()
    x = torch.zeros((257, 16), device="cuda")
    v = torch.zeros((257, 2), device="cuda")
    i = torch.zeros((257, 2), dtype=torch.int32, device="cuda")
    st = lib.mlg_logsoftmax_topk_noalloc(ptr(x), 257, 16, 2, -1, ptr(v), ptr(i), None)
    assert st == _lib.ERR_INVALID
    assert b"256-row static scratch" in lib.mlg_last_error()
