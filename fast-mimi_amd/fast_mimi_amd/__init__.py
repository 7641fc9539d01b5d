"""fast_mimi_amd — the Mimi codec encode/decode hot path on AMD MI355X (gfx950).

Same public surface as kadirnar/fast-mimi (``src/fast_mimi/__init__.py``):
configuration, model, output and streaming-cache types.  Compute runs in the hand-written HIP
library ``libfast_mimi_amd.so`` (C ABI: ``include/fast_mimi_amd.h``).
"""

from .config import (
    KYUTAI_MIMI_MODEL_ID,
    KYUTAI_MIMI_PARAMETER_COUNT,
    KYUTAI_MIMI_PARAMETER_FINGERPRINT,
    KYUTAI_MIMI_REVISION,
    KYUTAI_MIMI_WEIGHTS_SHA256,
    MimiConfig,
)
from .model import MimiDecoderOutput, MimiEncoderOutput, MimiModel, MimiOutput
from .streaming import MimiConv1dPaddingCache, MimiKVCache

__all__ = [
    "KYUTAI_MIMI_MODEL_ID",
    "KYUTAI_MIMI_PARAMETER_COUNT",
    "KYUTAI_MIMI_PARAMETER_FINGERPRINT",
    "KYUTAI_MIMI_REVISION",
    "KYUTAI_MIMI_WEIGHTS_SHA256",
    "MimiConfig",
    "MimiConv1dPaddingCache",
    "MimiDecoderOutput",
    "MimiEncoderOutput",
    "MimiKVCache",
    "MimiModel",
    "MimiOutput",
]
