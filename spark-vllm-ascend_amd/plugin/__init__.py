"""vLLM general-plugin entry point of the MI355X Q4_0 decode path.

Mirrors the reference's entry point (src/spark_vllm_ascend/plugin/
__init__.py:1-7,60-87, declared at pyproject.toml:13-14 as
``vllm.general_plugins: spark2_5 = spark_vllm_ascend.plugin:register``):
importing this module touches the standard library only, and register() is
cheap, idempotent and safe to call in every vLLM process.

register() installs the decode path's operator surface:
  * the graph-safe torch custom ops ``torch.ops.smx.*`` (HIP kernels);
  * when vLLM is importable, the ``q4_0`` quantization config (Q4_0 linear
    method) in vLLM's quantization registry, unless vLLM already has one of
    that name and SMX_PLUGIN_OVERRIDE is not set.
It returns a dict naming what was registered.  The model class itself
(the reference registers ``Spark2_5ForCausalLM``) is outside the decode path
and is not registered here.
"""
from __future__ import annotations

import importlib
import importlib.util
import logging
import os

__all__ = ["OVERRIDE_ENV", "QUANT_NAME", "register"]

logger = logging.getLogger(__name__)

QUANT_NAME = "q4_0"
OVERRIDE_ENV = "SMX_PLUGIN_OVERRIDE"
_TRUE = frozenset({"1", "true", "yes", "on"})
_state: dict | None = None


def _override_requested() -> bool:
    return os.environ.get(OVERRIDE_ENV, "").strip().lower() in _TRUE


def _package() -> str:
    return __name__.rsplit(".", 1)[0]


def _register_vllm_quant(state: dict) -> None:
    if importlib.util.find_spec("vllm") is None:
        state["vllm"] = None
        return
    import vllm  # noqa: F401
    from vllm.model_executor.layers import quantization as q  # type: ignore

    linear = importlib.import_module(_package() + ".integration.linear")
    state["vllm"] = getattr(vllm, "__version__", "unknown")
    existing = getattr(q, "QUANTIZATION_METHODS", [])
    if QUANT_NAME in existing and not _override_requested():
        logger.info("smx plugin: quantization %r already known to vLLM; standing down "
                    "(set %s=1 to override)", QUANT_NAME, OVERRIDE_ENV)
        state["quant"] = None
        return
    q.register_quantization_config(QUANT_NAME)(linear.Q4_0Config)
    state["quant"] = QUANT_NAME


def register() -> dict:
    """Register the decode path's ops (and its vLLM hooks when vLLM is
    present).  Idempotent: later calls return the first call's result."""
    global _state
    if _state is not None:
        return _state
    state: dict = {"ops": None, "quant": None, "vllm": None}
    custom_ops = importlib.import_module(_package() + ".integration.custom_ops")
    custom_ops.register()
    state["ops"] = "smx"
    _register_vllm_quant(state)
    logger.info("smx plugin: registered %s", state)
    _state = state
    return state
