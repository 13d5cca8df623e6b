"""torch.library ops over the C ABI: ``o2_forward`` and ``o2_backward``.

Schemas follow the reference's ops (``triton_o2.py:786-794``, ``:878-887``):
``o2_forward(left, right, weight, path_info, path_coefficients, metadata_id)``
and ``o2_backward(left, right, weight, grad_output, path_info,
path_coefficients, metadata_id) -> (grad_left, grad_right, grad_weight)``.
``metadata_id`` indexes this process's plan registry; ``path_info`` and
``path_coefficients`` are the reference's int32 [P, 25] / f32 [P, 4] path
metadata, carried for schema compatibility (the compiled kernels embed the
same table).  Each op has a fake implementation and autograd, so
``torch.compile(fullgraph=True)`` traces through it; the backward's own
derivative (second order) is built from the same two ops by multilinearity
(the reference differentiates its PyTorch algebra, ``triton_o2.py:1035-1069``).

Outputs and workspaces come from torch's caching allocator; kernels run on
the current stream.  A CUDA tensor without the built library raises.
"""
from __future__ import annotations

import threading
from dataclasses import dataclass, field
from typing import Dict

import torch

from . import __version__
from . import _native
from .plan import TPPlan

NAMESPACE = "ictc_o2_hp_v" + __version__.replace(".", "_")


@dataclass
class _Registered:
    plan: TPPlan
    layout: int
    native: Dict[int, _native.TPNativePlan] = field(default_factory=dict)


_REGISTRY: Dict[int, _Registered] = {}
_REGISTRY_LOCK = threading.Lock()


def register(plan: TPPlan, layout: int) -> int:
    """Register a module's plan; returns its ``metadata_id``."""
    with _REGISTRY_LOCK:
        metadata_id = len(_REGISTRY)
        _REGISTRY[metadata_id] = _Registered(plan, layout)
    return metadata_id


def registered(metadata_id: int) -> _Registered:
    return _REGISTRY[metadata_id]


def _native_plan(metadata_id: int) -> _native.TPNativePlan:
    entry = _REGISTRY[metadata_id]
    native = entry.native.get(0)
    if native is None:
        with _REGISTRY_LOCK:
            native = entry.native.get(0)
            if native is None:
                plan = entry.plan
                native = _native.TPNativePlan(plan.channels, plan.m_max, plan.parity,
                                              plan.normalization, entry.layout)
                if native.width != plan.width or native.weight_numel != plan.weight_numel:
                    raise _native.NativeLibraryError("compiled plan disagrees with the host plan")
                entry.native[0] = native
    return native


def _check_inputs(*tensors: torch.Tensor) -> None:
    device = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda" or t.device != device:
            raise ValueError("o2 ops need CUDA(HIP) tensors on one device")
        if t.dtype != torch.float32:
            raise ValueError("o2 ops compute in float32")
        if not t.is_contiguous():
            raise ValueError("o2 ops need contiguous tensors")


def _launcher(native: _native.TPNativePlan, path_info: torch.Tensor,
              path_coefficients: torch.Tensor, device: torch.device):
    """The compiled kernels of the plan, or (m_max beyond the compiled plans)
    the table-driven kernels reading the op's own path tables on ``device``."""
    if native.compiled:
        return native
    n_paths = path_info.shape[0] if path_info.dim() == 2 else -1
    if (path_info.dtype != torch.int32 or path_info.dim() != 2 or path_info.shape[1] != 25
            or path_coefficients.dtype != torch.float32
            or tuple(path_coefficients.shape) != (n_paths, 4)):
        raise ValueError("path_info / path_coefficients must be int32 [P, 25] / float32 [P, 4]")
    if path_info.device != device or path_coefficients.device != device:
        raise ValueError("the path tables must be on the operands' device")
    info, coef = path_info.contiguous(), path_coefficients.contiguous()
    call = _native.TablesCall(native, info.data_ptr(), coef.data_ptr(), n_paths)
    call.keep = (info, coef)
    return call


def _check_shapes(op: str, native, left, right, weight, grad_output=None) -> None:
    """The kernels read x, y (and the cotangent) as [N, W] rows and w as P_w
    floats: anything else is refused before a launch."""
    ok = (left.dim() == 2 and left.shape[1] == native.width and right.shape == left.shape
          and weight.numel() == native.weight_numel
          and (grad_output is None or grad_output.shape == left.shape))
    if not ok:
        raise ValueError(f"{op}: shapes do not match the plan")


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


@torch.library.custom_op(NAMESPACE + "::o2_forward", mutates_args=())
def o2_forward(left: torch.Tensor, right: torch.Tensor, weight: torch.Tensor,
               path_info: torch.Tensor, path_coefficients: torch.Tensor,
               metadata_id: int) -> torch.Tensor:
    native = _native_plan(metadata_id)
    _check_shapes("o2_forward", native, left, right, weight)
    _check_inputs(left, right, weight)
    n_rows = left.shape[0]
    out = torch.empty_like(left)
    kernels = _launcher(native, path_info, path_coefficients, left.device)
    with torch.cuda.device(left.device):
        kernels.forward(left.data_ptr(), right.data_ptr(), weight.data_ptr(), out.data_ptr(),
                        n_rows, _stream(left.device))
    return out


@o2_forward.register_fake
def _o2_forward_fake(left, right, weight, path_info, path_coefficients, metadata_id):
    return torch.empty_like(left)


@torch.library.custom_op(NAMESPACE + "::o2_backward", mutates_args=())
def o2_backward(left: torch.Tensor, right: torch.Tensor, weight: torch.Tensor,
                grad_output: torch.Tensor, path_info: torch.Tensor,
                path_coefficients: torch.Tensor,
                metadata_id: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    grad_output = grad_output.contiguous()
    native = _native_plan(metadata_id)
    _check_shapes("o2_backward", native, left, right, weight, grad_output)
    _check_inputs(left, right, weight, grad_output)
    n_rows = left.shape[0]
    grad_left = torch.empty_like(left)
    grad_right = torch.empty_like(right)
    grad_weight = torch.empty_like(weight)
    kernels = _launcher(native, path_info, path_coefficients, left.device)
    # The workspace size depends on the device's CU count: query it on the
    # tensors' device, like the launch.
    with torch.cuda.device(left.device):
        ws_bytes = kernels.workspace_bytes(n_rows)
        workspace = torch.empty(max(1, (ws_bytes + 3) // 4), dtype=torch.float32,
                                device=left.device)
        kernels.backward(left.data_ptr(), right.data_ptr(), weight.data_ptr(),
                        grad_output.data_ptr(), grad_left.data_ptr(), grad_right.data_ptr(),
                        grad_weight.data_ptr(), workspace.data_ptr(), ws_bytes, n_rows, 7,
                        _stream(left.device))
    return grad_left, grad_right, grad_weight


@o2_backward.register_fake
def _o2_backward_fake(left, right, weight, grad_output, path_info, path_coefficients,
                      metadata_id):
    return torch.empty_like(left), torch.empty_like(right), torch.empty_like(weight)


def _forward_setup(ctx, inputs, output):
    left, right, weight, path_info, path_coefficients, metadata_id = inputs
    ctx.save_for_backward(left, right, weight, path_info, path_coefficients)
    ctx.metadata_id = metadata_id


def _forward_backward(ctx, grad_output):
    left, right, weight, path_info, path_coefficients = ctx.saved_tensors
    grads = o2_backward(left, right, weight, grad_output, path_info, path_coefficients,
                        ctx.metadata_id)
    return (*grads, None, None, None)


o2_forward.register_autograd(_forward_backward, setup_context=_forward_setup)


def _backward_setup(ctx, inputs, output):
    left, right, weight, grad_output, path_info, path_coefficients, metadata_id = inputs
    ctx.save_for_backward(left, right, weight, grad_output, path_info, path_coefficients)
    ctx.metadata_id = metadata_id
    ctx.set_materialize_grads(False)


def _backward_backward(ctx, dd_left, dd_right, dd_weight):
    """Second order by multilinearity.  out = F(x, y, w) is linear in each of
    x, y and w, and the first VJP is (F_x^T g, F_y^T g, F_w^T g), so

        <dd_x, dx> + <dd_y, dy> + <dd_w, dw>
            = <g, F(dd_x, y, w) + F(x, dd_y, w) + F(x, y, dd_w)>.

    Each incoming cotangent is one first-order call with that operand
    replaced: its VJP gives the gradients of the two other operands and its
    value the gradient of g.  The calls are the kernel ops themselves, so
    higher orders compose.  (The reference differentiates its PyTorch algebra
    here, ``triton_o2.py:1041-1064``; the results agree to fp32 rounding.)"""
    left, right, weight, grad_output, path_info, path_coefficients = ctx.saved_tensors
    wanted = ctx.needs_input_grad[:4]
    total = [None] * 4

    def add(x, y, w, roles):
        roles = [i for i in roles if wanted[i]]
        if roles:
            grads = o2_backward(x, y, w, grad_output, path_info, path_coefficients,
                                ctx.metadata_id)
            for i in roles:
                total[i] = grads[i] if total[i] is None else total[i] + grads[i]
        if wanted[3]:
            value = o2_forward(x, y, w, path_info, path_coefficients, ctx.metadata_id)
            total[3] = value if total[3] is None else total[3] + value

    if dd_left is not None:
        add(dd_left.contiguous(), right, weight, (1, 2))
    if dd_right is not None:
        add(left, dd_right.contiguous(), weight, (0, 2))
    if dd_weight is not None:
        add(left, right, dd_weight.contiguous(), (0, 1))
    return (*total, None, None, None)


o2_backward.register_autograd(_backward_backward, setup_context=_backward_setup)
