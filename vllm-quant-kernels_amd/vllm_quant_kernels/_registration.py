"""Env-var driven registration of the OOT LogitsProcessor and the fused sampler.

Same names, truthy set and priority as the reference
(src/vllm_quant_kernels/_registration.py:7-81):
  lm_head: VLLM_USE_MXFP4_LMHEAD > VLLM_USE_MXFP8_LMHEAD > VLLM_USE_FP8_LMHEAD >
           VLLM_USE_W8A8_LMHEAD > VLLM_USE_INT8_LMHEAD
  sampler: VLLM_USE_FUSED_SAMPLER (independent, combinable)
Truthy values are 1/true/yes/on, case-insensitive; unset or empty is false.
"""
import os
import sys

_ENV_INT8 = "VLLM_USE_INT8_LMHEAD"
_ENV_W8A8 = "VLLM_USE_W8A8_LMHEAD"
_ENV_FP8 = "VLLM_USE_FP8_LMHEAD"
_ENV_MXFP8 = "VLLM_USE_MXFP8_LMHEAD"
_ENV_MXFP4 = "VLLM_USE_MXFP4_LMHEAD"
_ENV_SAMPLER = "VLLM_USE_FUSED_SAMPLER"

# lm_head env vars in priority order, with the mode name each selects
LMHEAD_PRIORITY = (
    (_ENV_MXFP4, "mxfp4"),
    (_ENV_MXFP8, "mxfp8"),
    (_ENV_FP8, "fp8"),
    (_ENV_W8A8, "w8a8"),
    (_ENV_INT8, "int8"),
)
ALL_ENV_VARS = tuple(v for v, _ in LMHEAD_PRIORITY) + (_ENV_SAMPLER,)


def _env_bool(name: str, default: bool = False) -> bool:
    val = os.environ.get(name, "")
    if val == "":
        return default
    return val.lower() in ("1", "true", "yes", "on")


def selected_lmhead_mode():
    """The lm_head mode the env vars select, or None when none is set."""
    for var, mode in LMHEAD_PRIORITY:
        if _env_bool(var):
            return mode
    return None


def _silence_unknown_env_warning() -> None:
    """Whitelist our env vars in vllm.envs so vLLM does not warn about them."""
    try:
        import vllm.envs as vllm_envs
        table = vllm_envs.environment_variables
        for var in ALL_ENV_VARS:
            if var not in table:
                table[var] = (lambda v=var: os.environ.get(v, ""))
    except Exception:
        pass  # vLLM without that table: only a cosmetic warning is lost


def register_all() -> None:
    """Register the replacements selected by the env vars (idempotent)."""
    _silence_unknown_env_warning()
    mode = selected_lmhead_mode()
    use_sampler = _env_bool(_ENV_SAMPLER)
    if mode is None and not use_sampler:
        print(
            f"[vllm-quant-kernels] Plugin loaded but disabled "
            f"(set {_ENV_MXFP4}=1 | {_ENV_MXFP8}=1 | {_ENV_FP8}=1 | {_ENV_W8A8}=1 | "
            f"{_ENV_INT8}=1 to enable quantized LM head, or {_ENV_SAMPLER}=1 to "
            f"enable the fused sampler).",
            file=sys.stderr, flush=True,
        )
        return
    if mode is not None:
        from ._quant import QuantizedLogitsProcessor  # noqa: F401  (registers the OOT class)
        print(
            f"[vllm-quant-kernels] Registered QuantizedLogitsProcessor as OOT "
            f"replacement for LogitsProcessor (dtype={mode}).",
            file=sys.stderr, flush=True,
        )
    if use_sampler:
        from ._sampler import install_fused_sampler
        install_fused_sampler()
