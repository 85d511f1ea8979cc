"""Python host API over libgsample (the C ABI in include/gsample.h).

Mirrors the reference's decoding-policy surface (src/runtime/sampling.ts,
src/runtime/decoding.ts, src/runtime/generation-config.ts,
src/runtime/constraints.ts) with the same names, argument meaning and error
messages, and runs every sampling decision on the GPU through the C ABI.
torch is used only to own device memory; nothing here computes a sample on
the CPU. If the shared library is missing, importing the runtime raises.
"""
from __future__ import annotations

from .config import (  # noqa: F401
    DEFAULT_DECODING_CONFIG,
    DEFAULT_GENERATION_CONFIG,
    DecodingConfig,
    resolve_gemma_generation_config,
    uses_gemma_gpu_greedy,
    validate_decoding_config,
)
from . import vocab  # noqa: F401
from .runtime import (  # noqa: F401
    GS_F32,
    GS_BF16,
    GS_FLAG_DEAD_END,
    GS_FLAG_EMPTY_CANDIDATES,
    GS_FLAG_EXACT_PATH,
    GS_FLAG_GREEDY,
    GS_FLAG_NEAR_TIE,
    GS_FLAG_NONFINITE,
    GS_FLAG_TOPP_TIE,
    GS_FLAG_UNSUPPORTED,
    GS_FLAG_INVALID_SLOT,
    GS_FLAG_INDEX_CHECK,
    GSampleError,
    LIB_PATH,
    RowConfig,
    Sampler,
    SeededRandom,
    js_exp,
    js_log,
    library,
    sample_token,
    softcap,
    token_log_probability,
)
from .constraint import ByteDfa, CompiledByteConstraint, VocabBytes, mask_constraint_logits  # noqa: F401
from . import config, constraint, runtime, workloads  # noqa: F401,E402
