"""RadialUvuTensorProduct: a radial network's final affine layer fused with a
V=1 O(2) uvu product (Parity-LRX/ICTC-O2-HP ``radial_uvu.py:10-66``).

``forward(left, angular, radial_hidden)`` equals
``tp(left, angular, radial_out(radial_hidden))``.  CUDA(HIP) float32 with a
``UvuTensorProduct`` runs the ``radial_stream_forward`` op, whose gfx950
kernels generate each edge's weights on the matrix cores and consume them in
registers; other dtypes, devices and a ``ReferenceUvuTensorProduct`` use the
original differentiable composition.

``forward(table, angular, radial_hidden, left_index=index)`` (an extension:
the reference gathers outside its chain, docs/RADIAL.md:97-99) equals
``tp(table[index], angular, radial_out(radial_hidden))`` for a node table
``[nodes, input1_dimension]`` and int64/int32 edge index ``[edges]``: the
fused kernels read the table rows directly, and the table's gradient sums the
edge adjoints onto table rows in a fixed order (``graph_ops``), so it is
bitwise reproducible.  An index outside ``[0, nodes)`` reads a zero row.

``out_index=dst, out_rows=n`` (with or without ``left_index``) returns the
edge -> node aggregation ``[n, input1_dimension]``: each edge's output summed
onto row ``dst[e]`` in increasing edge order (``graph_ops.scatter_add_rows``,
deterministic; its backward gathers the node cotangent).  An index outside
``[0, n)`` is dropped.
"""
from __future__ import annotations

import torch

from .uvu_o2 import ReferenceUvuTensorProduct, UvuTensorProduct


class RadialUvuTensorProduct(torch.nn.Module):
    """Equivalent to ``tp(left, angular, radial_out(radial_hidden))``.

    ``tp`` must use one second-input channel and external per-edge weights;
    ``radial_out`` is reused as is (``radial_uvu.py:21-34``).
    """

    def __init__(self, tp: ReferenceUvuTensorProduct, radial_out: torch.nn.Linear):
        super().__init__()
        if not isinstance(tp, ReferenceUvuTensorProduct):
            raise TypeError("tp must be an O(2) uvu tensor product")
        if tp.channels_in2 != 1 or tp.shared_weights or tp.internal_weights:
            raise ValueError("radial fusion requires V=1 and external per-edge TP weights")
        if not isinstance(radial_out, torch.nn.Linear):
            raise TypeError("radial_out must be the final torch.nn.Linear of the radial network")
        if radial_out.out_features != tp.weight_numel:
            raise ValueError("radial_out.out_features must equal tp.weight_numel")
        if radial_out.in_features < 1:
            raise ValueError("radial_out must have at least one input feature")
        self.tp = tp
        self.radial_out = radial_out
        if isinstance(tp, UvuTensorProduct):
            from . import radial_ops
            radial_ops.register_structure(tp._kernel_metadata_id, tp.channels, tp.m_max,
                                          tp.parity, tp.m_max_in2, tp.parity_in2)

    def forward(self, left, angular, radial_hidden, *, left_index=None, out_index=None,
                out_rows=None):
        if (out_index is None) != (out_rows is None):
            raise ValueError("out_index and out_rows must be given together")
        if out_index is not None:
            if out_index.ndim != 1 or out_index.dtype not in (torch.int64, torch.int32):
                raise ValueError("out_index must be a 1-D int64 or int32 tensor")
            if int(out_rows) < 0:
                raise ValueError("out_rows must be non-negative")
            edges = self.forward(left, angular, radial_hidden, left_index=left_index)
            if edges.ndim != 2 or out_index.shape[0] != edges.shape[0]:
                raise ValueError("out_index must have one entry per edge of [edges, dim] inputs")
            if out_index.device != edges.device:
                raise ValueError("out_index must be on the inputs' device")
            from . import graph_ops
            return graph_ops.scatter_add_rows(edges, out_index, int(out_rows))
        if left_index is not None:
            return self._forward_gathered(left, left_index, angular, radial_hidden)
        tp = self.tp
        if left.ndim < 1 or left.shape[-1] != tp.input1_dimension:
            raise ValueError("left has the wrong final dimension")
        if angular.shape != (*left.shape[:-1], tp.input2_dimension):
            raise ValueError("angular must have the same batch shape and configured dimension")
        if radial_hidden.shape != (*left.shape[:-1], self.radial_out.in_features):
            raise ValueError(
                "radial_hidden must have the same batch shape and affine input dimension")
        if not left.is_floating_point():
            raise TypeError("radial uvu operands must be real floating-point tensors")
        operands = [angular, radial_hidden, self.radial_out.weight, tp._coefficients]
        if self.radial_out.bias is not None:
            operands.append(self.radial_out.bias)
        if any(v.device != left.device or v.dtype != left.dtype for v in operands):
            raise ValueError("all operands and modules must have the same device and dtype")
        if (left.device.type != "cuda" or left.dtype != torch.float32
                or not isinstance(tp, UvuTensorProduct)):
            return tp(left, angular, self.radial_out(radial_hidden))
        from .radial_ops import radial_forward
        bias = self.radial_out.bias
        result, _ = radial_forward(
            left.reshape(-1, tp.input1_dimension).contiguous(),
            angular.reshape(-1, tp.input2_dimension).contiguous(),
            radial_hidden.reshape(-1, self.radial_out.in_features).contiguous(),
            self.radial_out.weight.contiguous(),
            bias.contiguous() if bias is not None else self.radial_out.weight.new_empty(0),
            tp._path_info, tp._coefficients, tp._first_order, tp._second_order,
            tp._kernel_metadata_id, bias is not None,
            torch.is_grad_enabled() and (left.requires_grad or angular.requires_grad))
        return result.reshape(*left.shape[:-1], tp.representation_dimension)

    def _forward_gathered(self, table, index, angular, radial_hidden):
        tp = self.tp
        if table.ndim != 2 or table.shape[-1] != tp.input1_dimension:
            raise ValueError("with left_index, left must be a [rows, input1_dimension] table")
        if index.ndim != 1 or index.dtype not in (torch.int64, torch.int32):
            raise ValueError("left_index must be a 1-D int64 or int32 tensor")
        if index.device != table.device:
            raise ValueError("left_index must be on the table's device")
        edges = index.shape[0]
        if angular.shape != (edges, tp.input2_dimension):
            raise ValueError("angular must be [len(left_index), input2_dimension]")
        if radial_hidden.shape != (edges, self.radial_out.in_features):
            raise ValueError("radial_hidden must be [len(left_index), radial_out.in_features]")
        if not table.is_floating_point():
            raise TypeError("radial uvu operands must be real floating-point tensors")
        operands = [angular, radial_hidden, self.radial_out.weight, tp._coefficients]
        if self.radial_out.bias is not None:
            operands.append(self.radial_out.bias)
        if any(v.device != table.device or v.dtype != table.dtype for v in operands):
            raise ValueError("all operands and modules must have the same device and dtype")
        from . import graph_ops
        if (table.device.type != "cuda" or table.dtype != torch.float32
                or not isinstance(tp, UvuTensorProduct)):
            left = graph_ops.gather_rows(table, index)
            return tp(left, angular, self.radial_out(radial_hidden))
        from .radial_ops import radial_gather_forward
        bias = self.radial_out.bias
        return radial_gather_forward(
            table.contiguous(), index.to(torch.int64).contiguous(), angular.contiguous(),
            radial_hidden.contiguous(), self.radial_out.weight.contiguous(),
            bias.contiguous() if bias is not None else self.radial_out.weight.new_empty(0),
            tp._path_info, tp._coefficients, tp._first_order, tp._second_order,
            tp._kernel_metadata_id, bias is not None)
