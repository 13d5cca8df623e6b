"""Deterministic node <-> edge row movement for message passing.

``gather_rows(table, index)`` is ``table[index]`` for a 2-D table and 1-D
int64 index; ``scatter_add_rows(rows, index, n)`` sums ``rows[e]`` into row
``index[e]`` of an ``[n, width]`` result.  Each is the other's adjoint, so
both are differentiable to any order.  The reference leaves this data movement
outside its radial chain (docs/RADIAL.md:97-99) and a PyTorch model does it
with indexing, whose backward is an atomic ``index_put``/``index_add``
(summation order not fixed).  Here, on CUDA(HIP) float32 tensors:

* the gather is one HIP kernel (``o2mi_rows_gather_f32``);
* the scatter-add sorts the index once (stable ``argsort``), finds each
  table row's run with ``searchsorted`` and sums every run in increasing edge
  order (``o2mi_rows_segment_sum_f32``): bitwise reproducible, no atomics.

An index outside ``[0, n)`` gathers a zero row and is dropped by the
scatter-add (torch indexing would raise instead).  Other devices and dtypes
use ``index_select`` / ``index_add``.
"""
from __future__ import annotations

import torch

from . import _native
from .ops import NAMESPACE


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _native_ok(*tensors) -> bool:
    return all(t.device.type == "cuda" for t in tensors) and tensors[0].dtype == torch.float32


def _check(table_or_rows: torch.Tensor, index: torch.Tensor) -> None:
    if table_or_rows.ndim != 2:
        raise ValueError("rows must be a 2-D [rows, width] tensor")
    if index.ndim != 1 or index.dtype not in (torch.int64, torch.int32):
        raise ValueError("index must be a 1-D int64 or int32 tensor")
    if index.device != table_or_rows.device:
        raise ValueError("index and rows must be on the same device")


def csr_runs(index: torch.Tensor, n: int):
    """(order, offsets): a stable sort of the edges by index and, for each of
    the ``n`` table rows, the run ``order[offsets[r]:offsets[r+1]]`` of its
    edges (indices outside ``[0, n)`` fall outside every run)."""
    index = index.to(torch.int64)
    order = torch.argsort(index, stable=True)
    bounds = torch.arange(n + 1, device=index.device, dtype=torch.int64)
    offsets = torch.searchsorted(index[order], bounds)
    return order, offsets


def segment_sum_native(rows: torch.Tensor, order: torch.Tensor, offsets: torch.Tensor,
                       n: int) -> torch.Tensor:
    """HIP segment sum of ``rows`` over the runs of ``csr_runs`` (float32)."""
    rows = rows.contiguous()
    out = rows.new_empty((n, rows.shape[1]))
    if n == 0:
        return out
    with torch.cuda.device(rows.device):
        _native.check(_native.library().o2mi_rows_segment_sum_f32(
            rows.data_ptr() if rows.numel() else None, rows.shape[0], rows.shape[1],
            order.data_ptr() if order.numel() else None, offsets.data_ptr(), n,
            out.data_ptr(), _stream(rows.device)), "o2mi_rows_segment_sum_f32")
    return out


@torch.library.custom_op(NAMESPACE + "::gather_rows", mutates_args=())
def _gather_rows(table: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    out = table.new_empty((index.shape[0], table.shape[1]))
    if table.shape[0] == 0:
        return table.new_zeros((index.shape[0], table.shape[1]))
    if not _native_ok(table):
        valid = (index >= 0) & (index < table.shape[0])
        picked = table.index_select(0, torch.where(valid, index, torch.zeros_like(index)))
        return picked * valid.unsqueeze(1).to(table.dtype)
    if out.numel() == 0:
        return out
    table = table.contiguous()
    with torch.cuda.device(table.device):
        _native.check(_native.library().o2mi_rows_gather_f32(
            table.data_ptr() if table.numel() else None, table.shape[0],
            index.data_ptr(), index.shape[0], table.shape[1], out.data_ptr(),
            _stream(table.device)), "o2mi_rows_gather_f32")
    return out


@_gather_rows.register_fake
def _gather_rows_fake(table, index):
    return table.new_empty((index.shape[0], table.shape[1]))


@torch.library.custom_op(NAMESPACE + "::scatter_add_rows", mutates_args=())
def _scatter_add_rows(rows: torch.Tensor, index: torch.Tensor, n: int) -> torch.Tensor:
    if not _native_ok(rows):
        valid = (index >= 0) & (index < n)
        out = rows.new_zeros((n, rows.shape[1]))
        return out.index_add(0, index[valid], rows[valid])
    order, offsets = csr_runs(index, n)
    return segment_sum_native(rows, order, offsets, n)


@_scatter_add_rows.register_fake
def _scatter_add_rows_fake(rows, index, n):
    return rows.new_empty((n, rows.shape[1]))


def _gather_setup(ctx, inputs, output):
    table, index = inputs
    ctx.save_for_backward(index)
    ctx.rows = table.shape[0]


def _gather_backward(ctx, grad):
    (index,) = ctx.saved_tensors
    return _scatter_add_rows(grad.contiguous(), index, ctx.rows), None


def _scatter_setup(ctx, inputs, output):
    _rows, index, _n = inputs
    ctx.save_for_backward(index)


def _scatter_backward(ctx, grad):
    (index,) = ctx.saved_tensors
    return _gather_rows(grad.contiguous(), index), None, None


_gather_rows.register_autograd(_gather_backward, setup_context=_gather_setup)
_scatter_add_rows.register_autograd(_scatter_backward, setup_context=_scatter_setup)


def gather_rows(table: torch.Tensor, index: torch.Tensor) -> torch.Tensor:
    """``table[index]`` ([len(index), width]) with a deterministic backward."""
    _check(table, index)
    return _gather_rows(table, index.to(torch.int64).contiguous())


def scatter_add_rows(rows: torch.Tensor, index: torch.Tensor, n: int) -> torch.Tensor:
    """``zeros(n, width).index_add(0, index, rows)`` summed in a fixed order."""
    _check(rows, index)
    if index.shape[0] != rows.shape[0]:
        raise ValueError("index must have one entry per row")
    if n < 0:
        raise ValueError("n must be non-negative")
    return _scatter_add_rows(rows, index.to(torch.int64).contiguous(), int(n))
