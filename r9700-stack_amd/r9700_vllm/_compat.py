"""vLLM is an optional dependency: the kernel layer, the experts' apply() and the tests run without it.

Everything vLLM-specific (quantization-config registration, the modular-kernel base class, the logger) is looked
up here lazily, so importing r9700_vllm never requires vLLM and never hides a missing kernel library.
"""
from __future__ import annotations

import logging

import torch


def vllm_available() -> bool:
    try:
        import vllm  # noqa: F401
        return True
    except Exception:
        return False


def get_logger(name: str):
    try:
        from vllm.logger import init_logger
        return init_logger("vllm." + name)
    except Exception:
        return logging.getLogger(name)


def register_custom_op(lib: torch.library.Library, name: str, fn, mutates_args: list[str], fake_impl) -> None:
    """torch.ops.<lib>.<name>: vLLM's direct_register_custom_op when vLLM is installed, else torch.library."""
    try:
        from vllm.utils.torch_utils import direct_register_custom_op
        direct_register_custom_op(name, fn, mutates_args=mutates_args, fake_impl=fake_impl, target_lib=lib)
        return
    except ImportError:
        pass
    schema = torch.library.infer_schema(fn, mutates_args=mutates_args)
    lib.define(name + schema)
    lib.impl(name, fn, "CUDA")
    lib._register_fake(name, fake_impl)
