"""MI355X (gfx950) fp32 GRU training path: hand-written HIP kernels behind a
C ABI (librnn_kernel_amd.so), with an nn.GRU-compatible PyTorch front end."""
from .gru import (
    GRU,
    GRUFunction,
    MAX_HIDDEN_SIZE,
    from_torch_gru,
    gru_forward_inference,
    is_available,
    is_supported_gru,
)

__all__ = [
    "GRU",
    "GRUFunction",
    "MAX_HIDDEN_SIZE",
    "from_torch_gru",
    "gru_forward_inference",
    "is_available",
    "is_supported_gru",
]
