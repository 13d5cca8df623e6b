"""ICTC-O2 HP on AMD Instinct MI355X: Cartesian O(2) tensor products.

Drop-in for Parity-LRX/ICTC-O2-HP's public operators.  CUDA(HIP) float32
inputs run hand-written gfx950 kernels through the C ABI in
``libictc_o2_hp_amd.so``; other devices and dtypes use the differentiable
PyTorch algebra, as the reference does.
"""

__version__ = "0.1.6.dev0"
__all__ = [
    "TensorProduct", "TupleTensorProduct", "ComponentMajorTensorProduct",
    "ReferenceTensorProduct", "UvuTensorProduct", "ReferenceUvuTensorProduct", "__version__",
    "RadialUvuTensorProduct", "gather_rows", "scatter_add_rows",
]


def __getattr__(name):
    # Lazy exports: importing the package needs neither the GPU nor the library.
    if name == "ReferenceTensorProduct":
        from .reference import ReferenceTensorProduct
        return ReferenceTensorProduct
    if name == "RadialUvuTensorProduct":
        from .radial_uvu import RadialUvuTensorProduct
        return RadialUvuTensorProduct
    if name in {"gather_rows", "scatter_add_rows"}:
        from . import graph_ops
        return getattr(graph_ops, name)
    if name in {"UvuTensorProduct", "ReferenceUvuTensorProduct"}:
        from . import uvu_o2
        return getattr(uvu_o2, name)
    if name in {"TensorProduct", "TupleTensorProduct", "ComponentMajorTensorProduct"}:
        from . import api
        return getattr(api, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
