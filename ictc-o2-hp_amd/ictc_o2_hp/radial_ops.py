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
# Row blocks of the composed path: at most this many generated weight floats.
_BLOCK_WEIGHT_FLOATS = 1 << 24
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
        ws_bytes = int(lib.o2mi_radial_backward_workspace_bytes(plan, rows, needed))
        workspace = torch.empty(max(4, (ws_bytes + 3) // 4), dtype=torch.float32,
                                device=left.device)
        with torch.cuda.device(left.device):
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
