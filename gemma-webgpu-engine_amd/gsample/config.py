"""DecodingConfig and its validation, as in src/runtime/decoding.ts:1-59 and
src/runtime/generation-config.ts:47-77 (same field names, defaults, checks,
check order and messages)."""
from __future__ import annotations

import math
from dataclasses import dataclass, field, fields, replace
from typing import List

VOCAB_SIZE = 262144


@dataclass
class DecodingConfig:
    temperature: float = 0.8
    topK: int = 40
    topP: float = 0.95
    minP: float = 0.0
    typicalP: float = 1.0
    repetitionPenalty: float = 1.05
    repetitionWindow: int = 64
    frequencyPenalty: float = 0.0
    presencePenalty: float = 0.0
    maxNewTokens: int = 256
    seed: int = 42
    stopTokenIds: List[int] = field(default_factory=list)

    def merged(self, **overrides) -> "DecodingConfig":
        return replace(self, **overrides)


DEFAULT_DECODING_CONFIG = DecodingConfig()

DEFAULT_GENERATION_CONFIG = DecodingConfig(
    temperature=0.0,
    topK=0,
    topP=1.0,
    minP=0.0,
    typicalP=1.0,
    repetitionPenalty=1.0,
    repetitionWindow=0,
    frequencyPenalty=0.0,
    presencePenalty=0.0,
    maxNewTokens=256,
    stopTokenIds=[],
)


def _is_finite_number(x) -> bool:
    return isinstance(x, (int, float)) and not isinstance(x, bool) and math.isfinite(x)


def _is_integer(x) -> bool:
    if isinstance(x, bool):
        return False
    if isinstance(x, int):
        return True
    return isinstance(x, float) and math.isfinite(x) and float(x).is_integer()


def validate_decoding_config(partial: dict) -> dict:
    """validateDecodingConfig: {"ok": bool, "errors": [...]} in the reference's order."""
    names = {f.name for f in fields(DecodingConfig)}
    value = {f.name: getattr(DEFAULT_DECODING_CONFIG, f.name) for f in fields(DecodingConfig)}
    value.update({k: v for k, v in partial.items() if k in names})
    errors = []
    t = value["temperature"]
    if not _is_finite_number(t) or t < 0:
        errors.append("temperature must be >= 0")
    if not _is_integer(value["topK"]) or value["topK"] < 0:
        errors.append("topK must be a non-negative integer")
    for key in ("topP", "minP", "typicalP"):
        x = value[key]
        if not _is_finite_number(x) or x < 0 or x > 1:
            errors.append(f"{key} must be between 0 and 1")
    rp = value["repetitionPenalty"]
    if not _is_finite_number(rp) or rp <= 0:
        errors.append("repetitionPenalty must be > 0")
    if not _is_integer(value["repetitionWindow"]) or value["repetitionWindow"] < 0:
        errors.append("repetitionWindow must be a non-negative integer")
    fp = value["frequencyPenalty"]
    if not _is_finite_number(fp) or fp < 0:
        errors.append("frequencyPenalty must be finite and non-negative")
    pp = value["presencePenalty"]
    if not _is_finite_number(pp) or pp < 0:
        errors.append("presencePenalty must be finite and non-negative")
    if not _is_integer(value["maxNewTokens"]) or value["maxNewTokens"] < 1:
        errors.append("maxNewTokens must be a positive integer")
    if not _is_integer(value["seed"]):
        errors.append("seed must be an integer")
    stops = value["stopTokenIds"]
    if not isinstance(stops, (list, tuple)) or any(not _is_integer(t) or t < 0 for t in stops):
        errors.append("stopTokenIds must contain non-negative integers")
    return {"ok": len(errors) == 0, "errors": errors}


def resolve_gemma_generation_config(options: dict) -> DecodingConfig:
    """resolveGemmaGenerationConfig: generate() defaults, validation, stop-id bound."""
    names = {f.name for f in fields(DecodingConfig)}
    merged = {f.name: getattr(DEFAULT_GENERATION_CONFIG, f.name) for f in fields(DecodingConfig)}
    merged.update({k: v for k, v in options.items() if k in names})
    result = validate_decoding_config(merged)
    if not result["ok"]:
        raise ValueError(f"Invalid Gemma decoding config: {'; '.join(result['errors'])}")
    if any(t >= VOCAB_SIZE for t in merged["stopTokenIds"]):
        raise ValueError(f"Gemma stop token IDs must be below {VOCAB_SIZE}")
    merged["stopTokenIds"] = list(merged["stopTokenIds"])
    return DecodingConfig(**merged)


def uses_gemma_gpu_greedy(config: DecodingConfig) -> bool:
    """usesGemmaGpuGreedy (src/runtime/generation-config.ts:72-77)."""
    return (config.temperature == 0 and config.repetitionPenalty == 1 and config.frequencyPenalty == 0
            and config.presencePenalty == 0)
