"""MI355X-native diffusion-LLM attention path (drop-in for the attention layer
of dLLM-Serve): ``Attention`` / ``Context`` / ``SparseConfig`` backed by
hand-written gfx950 HIP kernels behind a C ABI."""

from .utils.context import Context, get_context, set_context, reset_context  # noqa: F401
from .sparse.state import SparseConfig, PerRequestSparseState  # noqa: F401

__all__ = ["Context", "get_context", "set_context", "reset_context", "SparseConfig", "PerRequestSparseState"]
