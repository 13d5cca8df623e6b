"""torch.library ops of the radial affine map fused with a V=1 uvu product.

Schemas follow the reference (``radial_streamed.py:81-146``):

* ``radial_stream_forward(left, angular, radial, alpha, bias, info,
  coefficients, first_order, second_order, metadata_id, has_bias,
  save_first) -> (out, cached_weights)``
* ``radial_stream_backward(left, angular, radial, alpha, bias,
  cached_weights, grad_output, info, coefficients, first_order,
  second_order, metadata_id, has_bias, needed=31) -> (gx, gy, gr, ga, gb)``
  with ``needed`` bits x=1, angular=2, hidden=4, alpha=8, bias=16; roles not
  requested come back as size-0 tensors.

Structures with a fused gfx950 kernel (``o2mi_radial_*``: the weights are
generated on the matrix cores and consumed in registers) never materialise
weights, so ``cached_weights`` is always empty here.  Other structures run
the same contract on the GPU as bounded row blocks: an fp32 GEMM for the
block's weights, then the uvu kernels (``radial_streamed.py:37-57``).
"""
from __future__ import annotations

import ctypes
import threading

import torch
import torch.nn.functional as F

from . import _native, uvu_ops

NAMESPACE = uvu_ops.NAMESPACE
# Row blocks of the composed path: at most this many generated weight floats
# (2 GiB; the block's weight adjoint takes as much again) and rows.  Small
# blocks starve the GEMMs and multiply launches: at C = 256 with 254 paths a
# 64 MiB budget gave 258-row blocks and a 36% slower full VJP.
_BLOCK_WEIGHT_FLOATS = 1 << 29
_MAX_BLOCK_ROWS = 16384

_STRUCTURES: dict = {}
_PLANS: dict = {}
_LOCK = threading.Lock()


def register_structure(metadata_id: int, channels: int, m_max: int, parity: str,
                       m_max_in2: int, parity_in2: str) -> None:
    """Record the uvu structure behind ``metadata_id`` (set by the module)."""
    with _LOCK:
        _STRUCTURES[metadata_id] = (channels, m_max, _native.PARITY[parity], m_max_in2,
                                    _native.PARITY[parity_in2])


def fused_plan(metadata_id: int, hidden: int):
    """Plan handle of the fused kernels, or None when none is compiled."""
    key = (metadata_id, hidden)
    with _LOCK:
        if key in _PLANS:
            return _PLANS[key]
        structure = _STRUCTURES.get(metadata_id)
        plan = None
        if structure is not None:
            lib = _native.library()
            handle = ctypes.c_void_p()
            status = lib.o2mi_radial_plan_create(*structure, hidden, ctypes.byref(handle))
            if status == _native.O2MI_OK:
                plan = handle
            elif status != -2:  # O2MI_ERR_UNSUPPORTED: use the composed path
                _native.check(status, "o2mi_radial_plan_create")
        _PLANS[key] = plan
        return plan


def _block_rows(weight_numel: int) -> int:
    return max(1, min(_MAX_BLOCK_ROWS, _BLOCK_WEIGHT_FLOATS // max(1, weight_numel)))


def _aligned(t: torch.Tensor) -> torch.Tensor:
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _ptr(t):
    return t.data_ptr() if t is not None and t.numel() else None


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _check_operands(*tensors):
    device = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda" or t.device != device:
            raise ValueError("radial ops need CUDA(HIP) tensors on one device")
        if t.dtype != torch.float32 and t.dtype != torch.int32:
            raise ValueError("radial kernels compute in float32")


def _forward_impl(left, angular, radial, alpha, bias, info, coefficients, first_order,
                  second_order, metadata_id, has_bias):
    _check_operands(left, angular, radial, alpha, coefficients)
    result = torch.empty_like(left)
    rows = left.shape[0]
    if rows == 0:
        return result
    plan = fused_plan(metadata_id, radial.shape[1])
    if plan is not None:
        left, radial, alpha = _aligned(left), _aligned(radial), _aligned(alpha)
        angular = angular.contiguous()
        with torch.cuda.device(left.device):
            _native.check(_native.library().o2mi_radial_forward_f32(
                plan, left.data_ptr(), angular.data_ptr(), radial.data_ptr(), alpha.data_ptr(),
                _ptr(bias) if has_bias else None, coefficients.data_ptr(), result.data_ptr(),
                rows, _stream(left.device)), "o2mi_radial_forward_f32")
        return result
    step = _block_rows(alpha.shape[0])
    for start in range(0, rows, step):
        end = min(rows, start + step)
        weights = F.linear(radial[start:end], alpha, bias if has_bias else None)
        uvu_ops._forward_into(left[start:end].contiguous(), angular[start:end].contiguous(),
                              weights, info, coefficients, first_order, second_order,
                              metadata_id, False, result[start:end])
    return result


def _backward_impl(left, angular, radial, alpha, bias, grad_output, info, coefficients,
                   first_order, second_order, metadata_id, has_bias, needed):
    _check_operands(left, angular, radial, alpha, coefficients, grad_output)
    has_bias = has_bias and bias.numel() > 0
    if not has_bias:
        needed &= ~16
    gx = torch.empty_like(left) if needed & 1 else left.new_empty(0)
    gy = torch.empty_like(angular) if needed & 2 else angular.new_empty(0)
    gr = torch.empty_like(radial) if needed & 4 else radial.new_empty(0)
    ga = torch.empty_like(alpha) if needed & 8 else alpha.new_empty(0)
    gb = torch.empty_like(bias) if needed & 16 else bias.new_empty(0)
    rows = left.shape[0]
    if needed == 0:
        return gx, gy, gr, ga, gb
    plan = fused_plan(metadata_id, radial.shape[1])
    if plan is not None:
        lib = _native.library()
        left, radial, alpha = _aligned(left), _aligned(radial), _aligned(alpha)
        grad_output = _aligned(grad_output)
        angular = angular.contiguous()
        with torch.cuda.device(left.device):  # workspace size and launch on one device
            ws_bytes = int(lib.o2mi_radial_backward_workspace_bytes(plan, rows, needed))
            workspace = torch.empty(max(4, (ws_bytes + 3) // 4), dtype=torch.float32,
                                    device=left.device)
            _native.check(lib.o2mi_radial_backward_f32(
                plan, left.data_ptr(), angular.data_ptr(), radial.data_ptr(), alpha.data_ptr(),
                _ptr(bias) if has_bias else None, coefficients.data_ptr(),
                grad_output.data_ptr(), _ptr(gx), _ptr(gy), _ptr(gr), _ptr(ga), _ptr(gb),
                workspace.data_ptr(), ws_bytes, rows, needed, _stream(left.device)),
                "o2mi_radial_backward_f32")
        return gx, gy, gr, ga, gb
    if needed & 8:
        ga.zero_()
    if needed & 16:
        gb.zero_()
    tp_needed = (needed & 3) | (4 if needed & 28 else 0)
    step = _block_rows(alpha.shape[0])
    for start in range(0, rows, step):
        end = min(rows, start + step)
        hidden = radial[start:end]
        weights = (F.linear(hidden, alpha, bias if has_bias else None) if needed & 3
                   else alpha.new_empty((end - start, alpha.shape[0])))
        bx = gx[start:end] if needed & 1 else gx
        by = gy[start:end] if needed & 2 else gy
        bw = (left.new_empty((end - start, alpha.shape[0])) if tp_needed & 4
              else left.new_empty(0))
        uvu_ops._backward_into(left[start:end].contiguous(), angular[start:end].contiguous(),
                               weights, grad_output[start:end].contiguous(), info, coefficients,
                               first_order, second_order, metadata_id, False, tp_needed,
                               bx, by, bw)
        if needed & 4:
            torch.mm(bw, alpha, out=gr[start:end])
        if needed & 8:
            ga.addmm_(bw.t(), hidden)
        if needed & 16:
            gb.add_(bw.sum(0))
    return gx, gy, gr, ga, gb


@torch.library.custom_op(NAMESPACE + "::radial_stream_forward", mutates_args=())
def radial_forward(left: torch.Tensor, angular: torch.Tensor, radial: torch.Tensor,
                   alpha: torch.Tensor, bias: torch.Tensor, info: torch.Tensor,
                   coefficients: torch.Tensor, first_order: torch.Tensor,
                   second_order: torch.Tensor, metadata_id: int, has_bias: bool,
                   save_first: bool) -> tuple[torch.Tensor, torch.Tensor]:
    result = _forward_impl(left, angular, radial, alpha, bias, info, coefficients, first_order,
                           second_order, metadata_id, has_bias)
    return result, alpha.new_empty(0)


@radial_forward.register_fake
def _radial_forward_fake(left, angular, radial, alpha, bias, info, coefficients, first_order,
                         second_order, metadata_id, has_bias, save_first):
    return torch.empty_like(left), alpha.new_empty(0)


@torch.library.custom_op(NAMESPACE + "::radial_stream_backward", mutates_args=())
def radial_backward(left: torch.Tensor, angular: torch.Tensor, radial: torch.Tensor,
                    alpha: torch.Tensor, bias: torch.Tensor, cached_weights: torch.Tensor,
                    grad_output: torch.Tensor, info: torch.Tensor, coefficients: torch.Tensor,
                    first_order: torch.Tensor, second_order: torch.Tensor, metadata_id: int,
                    has_bias: bool, needed: int = 31
                    ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                               torch.Tensor]:
    return _backward_impl(left, angular, radial, alpha, bias, grad_output.contiguous(), info,
                          coefficients, first_order, second_order, metadata_id, has_bias,
                          needed)


@radial_backward.register_fake
def _radial_backward_fake(left, angular, radial, alpha, bias, cached_weights, grad_output, info,
                          coefficients, first_order, second_order, metadata_id, has_bias,
                          needed=31):
    if not (has_bias and bias.numel() > 0):
        needed &= ~16
    return tuple(torch.empty_like(v) if needed & (1 << i) else v.new_empty(0)
                 for i, v in enumerate((left, angular, radial, alpha, bias)))


def _mask(flags) -> int:
    return sum(int(bool(f)) << i for i, f in enumerate(flags))


def _forward_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs[:9])
    ctx.metadata_id, ctx.has_bias = inputs[9], inputs[10]


def _forward_backward(ctx, grad_output, _cache_grad):
    left, angular, radial, alpha, bias, info, coefficients, first_order, second_order = \
        ctx.saved_tensors
    roles = uvu_ops.required_gradients((left, angular, radial, alpha, bias),
                                       ctx.needs_input_grad[:5])
    grads = radial_backward(left, angular, radial, alpha, bias, alpha.new_empty(0),
                            grad_output.contiguous(), info, coefficients, first_order,
                            second_order, ctx.metadata_id, ctx.has_bias, _mask(roles))
    return (*(g if r else None for g, r in zip(grads, roles)),
            None, None, None, None, None, None, None)


radial_forward.register_autograd(_forward_backward, setup_context=_forward_setup)


def _backward_setup(ctx, inputs, output):
    (left, angular, radial, alpha, bias, _cached, grad_output, info, coefficients, first_order,
     second_order, metadata_id, has_bias, needed) = inputs
    ctx.save_for_backward(left, angular, radial, alpha, bias, grad_output, info, coefficients,
                          first_order, second_order)
    ctx.metadata_id, ctx.has_bias = metadata_id, has_bias
    ctx.set_materialize_grads(False)


def _backward_backward(ctx, d_left, d_angular, d_radial, d_alpha, d_bias):
    """Second order by multilinearity: out = f(x, y, r a^T + b) is linear in x,
    in y and in the generated weights, so each incoming cotangent turns into
    one first-order call with that operand replaced (``radial_streamed.py:167-207``)."""
    (left, angular, radial, alpha, bias, grad_output, info, coefficients, first_order,
     second_order) = ctx.saved_tensors
    wanted = uvu_ops.required_gradients(
        (left, angular, radial, alpha, bias, grad_output),
        (*ctx.needs_input_grad[:5], ctx.needs_input_grad[6]))
    total = [None] * 6
    tables = (info, coefficients, first_order, second_order)

    def add(operands, roles, has_bias):
        x, y, r, a, b = operands
        roles = [i for i in roles if wanted[i]]
        if roles:
            grads = radial_backward(x, y, r, a, b, a.new_empty(0), grad_output, *tables,
                                    ctx.metadata_id, has_bias, _mask(i in roles for i in range(5)))
            for i in roles:
                total[i] = grads[i] if total[i] is None else total[i] + grads[i]
        if wanted[5]:
            value, _ = radial_forward(x, y, r, a, b, *tables, ctx.metadata_id, has_bias, False)
            total[5] = value if total[5] is None else total[5] + value

    empty_bias = bias.new_empty(0)
    if d_left is not None:
        add((d_left.contiguous(), angular, radial, alpha, bias), (1, 2, 3, 4), ctx.has_bias)
    if d_angular is not None:
        add((left, d_angular.contiguous(), radial, alpha, bias), (0, 2, 3, 4), ctx.has_bias)
    if d_radial is not None:
        add((left, angular, d_radial.contiguous(), alpha, empty_bias), (0, 1, 3), False)
    if d_alpha is not None or d_bias is not None:
        probe_alpha = d_alpha.contiguous() if d_alpha is not None else torch.zeros_like(alpha)
        with_bias = d_bias is not None and ctx.has_bias
        probe_bias = d_bias.contiguous() if with_bias else empty_bias
        add((left, angular, radial, probe_alpha, probe_bias), (0, 1, 2), with_bias)
    return (*total[:5], None, total[5], None, None, None, None, None, None, None)


radial_backward.register_autograd(_backward_backward, setup_context=_backward_setup)


# ---------------------------------------------------------------------------
# Gathered first input: edge e reads row index[e] of a node table.  The fused
# kernels address the table directly (the gathered rows are never
# materialised); the table's adjoint is the per-edge adjoint summed onto table
# rows in a fixed order (graph_ops).  Not in the reference, which gathers with
# torch indexing outside its radial chain (docs/RADIAL.md:97-99).

_TABLE_BYTES_LIMIT = 1 << 31


def _gather_fused(table, metadata_id, hidden):
    plan = fused_plan(metadata_id, hidden)
    if plan is None or table.numel() * 4 >= _TABLE_BYTES_LIMIT or table.shape[0] == 0:
        return None
    return plan


def _gather_forward_impl(table, index, angular, radial, alpha, bias, info, coefficients,
                         first_order, second_order, metadata_id, has_bias):
    from . import graph_ops
    _check_operands(table, angular, radial, alpha, coefficients)
    rows = index.shape[0]
    result = table.new_empty((rows, table.shape[1]))
    if rows == 0:
        return result
    plan = _gather_fused(table, metadata_id, radial.shape[1])
    if plan is None:
        left = graph_ops._gather_rows(table, index)
        return _forward_impl(left, angular, radial, alpha, bias, info, coefficients, first_order,
                             second_order, metadata_id, has_bias)
    table, radial, alpha = _aligned(table), _aligned(radial), _aligned(alpha)
    angular = angular.contiguous()
    with torch.cuda.device(table.device):
        _native.check(_native.library().o2mi_radial_forward_gather_f32(
            plan, table.data_ptr(), table.shape[0], index.data_ptr(), angular.data_ptr(),
            radial.data_ptr(), alpha.data_ptr(), _ptr(bias) if has_bias else None,
            coefficients.data_ptr(), result.data_ptr(), rows, _stream(table.device)),
            "o2mi_radial_forward_gather_f32")
    return result


def _gather_backward_impl(table, index, angular, radial, alpha, bias, grad_output, info,
                          coefficients, first_order, second_order, metadata_id, has_bias, needed):
    from . import graph_ops
    _check_operands(table, angular, radial, alpha, coefficients, grad_output)
    rows = index.shape[0]
    plan = _gather_fused(table, metadata_id, radial.shape[1])
    if plan is None or rows == 0:
        left = graph_ops._gather_rows(table, index)
        gx, gy, gr, ga, gb = _backward_impl(left, angular, radial, alpha, bias, grad_output,
                                            info, coefficients, first_order, second_order,
                                            metadata_id, has_bias, needed)
    else:
        has_bias = has_bias and bias.numel() > 0
        if not has_bias:
            needed &= ~16
        width = table.shape[1]
        gx = table.new_empty((rows, width)) if needed & 1 else table.new_empty(0)
        gy = torch.empty_like(angular) if needed & 2 else angular.new_empty(0)
        gr = torch.empty_like(radial) if needed & 4 else radial.new_empty(0)
        ga = torch.empty_like(alpha) if needed & 8 else alpha.new_empty(0)
        gb = torch.empty_like(bias) if needed & 16 else bias.new_empty(0)
        if needed:
            lib = _native.library()
            table, radial, alpha = _aligned(table), _aligned(radial), _aligned(alpha)
            grad_output = _aligned(grad_output)
            angular = angular.contiguous()
            with torch.cuda.device(table.device):  # workspace size and launch on one device
                ws_bytes = int(lib.o2mi_radial_backward_workspace_bytes(plan, rows, needed))
                workspace = torch.empty(max(4, (ws_bytes + 3) // 4), dtype=torch.float32,
                                        device=table.device)
                _native.check(lib.o2mi_radial_backward_gather_f32(
                    plan, table.data_ptr(), table.shape[0], index.data_ptr(), angular.data_ptr(),
                    radial.data_ptr(), alpha.data_ptr(), _ptr(bias) if has_bias else None,
                    coefficients.data_ptr(), grad_output.data_ptr(), _ptr(gx), _ptr(gy),
                    _ptr(gr), _ptr(ga), _ptr(gb), workspace.data_ptr(), ws_bytes, rows, needed,
                    _stream(table.device)), "o2mi_radial_backward_gather_f32")
    if needed & 1:
        order, offsets = graph_ops.csr_runs(index, table.shape[0])
        g_table = graph_ops.segment_sum_native(gx, order, offsets, table.shape[0])
    else:
        g_table = table.new_empty(0)
    return g_table, gy, gr, ga, gb


@torch.library.custom_op(NAMESPACE + "::radial_gather_forward", mutates_args=())
def radial_gather_forward(table: torch.Tensor, index: torch.Tensor, angular: torch.Tensor,
                          radial: torch.Tensor, alpha: torch.Tensor, bias: torch.Tensor,
                          info: torch.Tensor, coefficients: torch.Tensor,
                          first_order: torch.Tensor, second_order: torch.Tensor,
                          metadata_id: int, has_bias: bool) -> torch.Tensor:
    return _gather_forward_impl(table, index, angular, radial, alpha, bias, info, coefficients,
                                first_order, second_order, metadata_id, has_bias)


@radial_gather_forward.register_fake
def _radial_gather_forward_fake(table, index, angular, radial, alpha, bias, info, coefficients,
                                first_order, second_order, metadata_id, has_bias):
    return table.new_empty((index.shape[0], table.shape[1]))


@torch.library.custom_op(NAMESPACE + "::radial_gather_backward", mutates_args=())
def radial_gather_backward(table: torch.Tensor, index: torch.Tensor, angular: torch.Tensor,
                           radial: torch.Tensor, alpha: torch.Tensor, bias: torch.Tensor,
                           grad_output: torch.Tensor, info: torch.Tensor,
                           coefficients: torch.Tensor, first_order: torch.Tensor,
                           second_order: torch.Tensor, metadata_id: int, has_bias: bool,
                           needed: int = 31
                           ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor,
                                      torch.Tensor]:
    return _gather_backward_impl(table, index, angular, radial, alpha, bias,
                                 grad_output.contiguous(), info, coefficients, first_order,
                                 second_order, metadata_id, has_bias, needed)


@radial_gather_backward.register_fake
def _radial_gather_backward_fake(table, index, angular, radial, alpha, bias, grad_output, info,
                                 coefficients, first_order, second_order, metadata_id, has_bias,
                                 needed=31):
    if not (has_bias and bias.numel() > 0):
        needed &= ~16
    return tuple(torch.empty_like(v) if needed & (1 << i) else v.new_empty(0)
                 for i, v in enumerate((table, angular, radial, alpha, bias)))


def _gather_forward_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs[:10])
    ctx.metadata_id, ctx.has_bias = inputs[10], inputs[11]


def _gather_forward_backward(ctx, grad_output):
    (table, index, angular, radial, alpha, bias, info, coefficients, first_order,
     second_order) = ctx.saved_tensors
    needs = ctx.needs_input_grad
    roles = uvu_ops.required_gradients((table, angular, radial, alpha, bias),
                                       (needs[0], needs[2], needs[3], needs[4], needs[5]))
    grads = radial_gather_backward(table, index, angular, radial, alpha, bias,
                                   grad_output.contiguous(), info, coefficients, first_order,
                                   second_order, ctx.metadata_id, ctx.has_bias, _mask(roles))
    g = [gr if r else None for gr, r in zip(grads, roles)]
    return (g[0], None, g[1], g[2], g[3], g[4], None, None, None, None, None, None)


radial_gather_forward.register_autograd(_gather_forward_backward,
                                        setup_context=_gather_forward_setup)


def _gather_backward_setup(ctx, inputs, output):
    (table, index, angular, radial, alpha, bias, grad_output, info, coefficients, first_order,
     second_order, metadata_id, has_bias, needed) = inputs
    ctx.save_for_backward(table, index, angular, radial, alpha, bias, grad_output, info,
                          coefficients, first_order, second_order)
    ctx.metadata_id, ctx.has_bias, ctx.needed = metadata_id, has_bias, needed
    ctx.set_materialize_grads(False)


def _gather_backward_backward(ctx, d_table, d_angular, d_radial, d_alpha, d_bias):
    """Second order through the differentiable composition: the table adjoint
    is scatter_add(first-order input adjoint of gather(table)), and gather and
    scatter_add are each other's adjoints, so the radial op's own second order
    (``_backward_backward``) supplies every term."""
    from . import graph_ops
    (table, index, angular, radial, alpha, bias, grad_output, info, coefficients, first_order,
     second_order) = ctx.saved_tensors
    cot = (d_table, d_angular, d_radial, d_alpha, d_bias)
    selected = [i for i, c in enumerate(cot) if c is not None and c.numel()]
    needs = ctx.needs_input_grad
    positions = (0, 2, 3, 4, 5, 6)          # table, angular, radial, alpha, bias, grad_output
    if not selected or not any(needs[p] for p in positions):
        return (None,) * 14
    with torch.enable_grad():
        leaves = [v.detach().requires_grad_(bool(needs[p]))
                  for v, p in zip((table, angular, radial, alpha, bias, grad_output), positions)]
        t, y, r, a, b, go = leaves
        left = graph_ops._gather_rows(t, index)
        mask = sum(1 << i for i in selected)
        grads = radial_backward(left, y, r, a, b, a.new_empty(0), go, info, coefficients,
                                first_order, second_order, ctx.metadata_id, ctx.has_bias, mask)
        outs = list(grads)
        if mask & 1:
            outs[0] = graph_ops._scatter_add_rows(grads[0], index, table.shape[0])
        wrt = [v for v in leaves if v.requires_grad]
        got = torch.autograd.grad([outs[i] for i in selected], wrt,
                                  [cot[i].contiguous() for i in selected], allow_unused=True)
    it = iter(got)
    mapped = [next(it) if v.requires_grad else None for v in leaves]
    result = [None] * 14
    for value, p in zip(mapped, positions):
        result[p] = value
    return tuple(result)


radial_gather_backward.register_autograd(_gather_backward_backward,
                                         setup_context=_gather_backward_setup)
