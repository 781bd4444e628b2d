"""MI355X (gfx950) fp32 GRU training path: hand-written HIP kernels behind a
C ABI (librnn_kernel_amd.so), with an nn.GRU-compatible PyTorch front end."""
from .gru import (
    GRU,
    GRUFunction,
    MAX_HIDDEN_SIZE,
    RecurrenceAbortedError,
    check_recurrences,
    from_torch_gru,
    gru_forward_inference,
    is_available,
    is_supported_gru,
    set_strict,
)
from .train import AdamW, HeadFunction, LinearHead, MSELossFunction, mse_loss

__all__ = [
    "AdamW",
    "HeadFunction",
    "LinearHead",
    "MSELossFunction",
    "mse_loss",
    "GRU",
    "GRUFunction",
    "MAX_HIDDEN_SIZE",
    "RecurrenceAbortedError",
    "check_recurrences",
    "from_torch_gru",
    "gru_forward_inference",
    "is_available",
    "is_supported_gru",
    "set_strict",
]
