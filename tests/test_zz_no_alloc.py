"""Allocation-free TP backward (o2mi_tp_backward_noalloc_f32) against the
workspace entry point o2mi_tp_backward_f32, both called through the C ABI.

The scratch entry point shares one device array per GPU between calls, so
each case makes two calls in a row, the second with fewer rows: the second
must not see anything the first left behind.  dx and dy are per-row results
and must be bitwise equal; dw is bitwise equal when the workspace entry
point's partial rows fit in the scratch (then both use the same grid), else
within the parity gate (normalized max error <= 1e-5).
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import o2_oracle as O

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 64 << 20          # O2MI_TP_SCRATCH_BYTES of include/ictc_o2_hp_amd.h


def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _both(plan, x, y, w, g, needed):
    lib = plan._lib
    n = x.shape[0]
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ref = [torch.full_like(x, 7.0), torch.full_like(y, 7.0), torch.full_like(w, 7.0)]
    new = [torch.full_like(x, -3.0), torch.full_like(y, -3.0), torch.full_like(w, -3.0)]
    ws_bytes = plan.workspace_bytes(n)
    ws = torch.empty(max(1, ws_bytes // 4), dtype=torch.float32, device=x.device)
    rc = lib.o2mi_tp_backward_f32(plan.handle, _ptr(x), _ptr(y), _ptr(w), _ptr(g),
                                  *[_ptr(t) for t in ref], _ptr(ws), ws_bytes, n, needed, stream)
    assert rc == 0, lib.o2mi_last_error()
    rc = lib.o2mi_tp_backward_noalloc_f32(plan.handle, _ptr(x), _ptr(y), _ptr(w), _ptr(g),
                                          *[_ptr(t) for t in new], n, needed, stream)
    assert rc == 0, lib.o2mi_last_error()
    torch.cuda.synchronize()
    return ref, new, ws_bytes


@pytest.mark.parametrize("channels,m_max,parity,rows", [
    (128, 6, "full", (131072, 3001)),     # the headline plan at full size, then fewer rows
    (32, 2, "canonical", (40000, 77)),
    (17, 3, "full", (5000, 1)),
    (256, 4, "canonical", (9000, 640)),
    (128, 8, "full", (20000, 333)),       # 128-lane backward tiles; grid cut to the scratch
])
def test_noalloc_backward_matches_workspace_backward(channels, m_max, parity, rows):
    from ictc_o2_hp import _native
    print(f"noalloc case C{channels} m{m_max} {parity} rows {rows}", flush=True)
    plan = _native.TPNativePlan(channels, m_max, parity, "component", 0)
    gen = torch.Generator(device="cuda").manual_seed(channels * 100 + m_max)
    w = torch.randn(plan.weight_numel, device="cuda", generator=gen) * 0.05
    for n in rows:
        x, y, g = (torch.randn((n, plan.width), device="cuda", generator=gen) for _ in range(3))
        ref, new, ws_bytes = _both(plan, x, y, w, g, 7)
        assert torch.equal(ref[0], new[0]) and torch.equal(ref[1], new[1])
        if ws_bytes <= SCRATCH_BYTES:
            assert torch.equal(ref[2], new[2])
        else:
            err = O.normalized_error(ref[2].double().cpu().numpy(), new[2].double().cpu().numpy())
            assert err <= 1e-5, err


def test_noalloc_backward_roles_and_empty_input():
    """Role subsets leave unrequested outputs untouched; N = 0 writes dw = 0."""
    from ictc_o2_hp import _native
    plan = _native.TPNativePlan(24, 3, "full", "component", 0)
    gen = torch.Generator(device="cuda").manual_seed(5)
    w = torch.randn(plan.weight_numel, device="cuda", generator=gen)
    x, y, g = (torch.randn((700, plan.width), device="cuda", generator=gen) for _ in range(3))
    for needed in (4, 1, 6):
        ref, new, _ = _both(plan, x, y, w, g, needed)
        for role, (a, b) in enumerate(zip(ref, new)):
            if needed & (1 << role):
                assert torch.equal(a, b)
            else:
                assert bool((b == -3.0).all())
    dw = torch.full((plan.weight_numel,), 5.0, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = plan._lib.o2mi_tp_backward_noalloc_f32(plan.handle, None, None, _ptr(w), None, None,
                                                None, _ptr(dw), 0, 7, stream)
    assert rc == 0
    torch.cuda.synchronize()
    assert bool((dw == 0).all())


def test_noalloc_backward_matches_oracle():
    """Against the fp64 oracle, on rows the scratch also held a larger call's data."""
    from ictc_o2_hp import _native
    plan = _native.TPNativePlan(16, 4, "full", "component", 0)
    oplan = O.OraclePlan(16, 4, "full")
    rng = np.random.default_rng(11)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    w64 = rng.standard_normal(plan.weight_numel) * 0.1
    w = torch.from_numpy(w64).float().cuda()
    for n in (20000, 33):
        x64, y64, g64 = (rng.standard_normal((n, plan.width)) for _ in range(3))
        x, y, g = (torch.from_numpy(a).float().cuda() for a in (x64, y64, g64))
        outs = [torch.empty_like(x), torch.empty_like(y), torch.empty_like(w)]
        rc = plan._lib.o2mi_tp_backward_noalloc_f32(plan.handle, _ptr(x), _ptr(y), _ptr(w),
                                                    _ptr(g), *[_ptr(t) for t in outs], n, 7,
                                                    stream)
        assert rc == 0, plan._lib.o2mi_last_error()
        torch.cuda.synchronize()
        xf, yf, gf = (a.astype(np.float32).astype(np.float64) for a in (x64, y64, g64))
        wf = w64.astype(np.float32).astype(np.float64)
        ref = O.backward(oplan, xf, yf, wf, gf)
        for r, a in zip(ref, outs):
            assert O.normalized_error(r, a.double().cpu().numpy()) <= 1e-5
