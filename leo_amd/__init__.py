"""leo_amd: an MI355X (gfx950) execution backend for Leo's per-byte training step.

The hot path -- delayed sparse recurrent delivery, eligibility traces, the
257-way readout/softmax/surprise and the batch-end lane-ordered delta mean -- runs
as hand-written HIP kernels in libleo_hip.so behind the C-ABI of
include/leo_hip.h. This package is the Python face of that boundary:

    Config        crates/leo-core/src/config.rs
    Model         crates/leo-core/src/model.rs (host layouts, seeded init)
    HipRuntime    crates/leo-core/src/backend.rs RuntimeBackend on the GPU
"""
from .config import Config, ConfigError
from .model import BEGIN_DOCUMENT, END_DOCUMENT, Model
from .native import FROZEN, PROVISIONAL, TRAINING, VERIFIED, LeoError
from .runtime import BatchReport, HipRuntime, StepMetrics

__all__ = [
    "BEGIN_DOCUMENT", "END_DOCUMENT", "FROZEN", "PROVISIONAL", "TRAINING", "VERIFIED",
    "BatchReport", "Config", "ConfigError", "HipRuntime", "LeoError", "Model", "StepMetrics",
]
