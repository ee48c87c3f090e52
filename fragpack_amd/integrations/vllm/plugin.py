"""The ``vllm.general_plugins`` entry point.

Reference: fragpack/integrations/vllm/plugin.py.  Registration records the
backend's import path only: no kernels are loaded, no tracker is made and the
GPU is not touched until vLLM instantiates the backend.
"""

from __future__ import annotations

from fragpack_amd.integrations.vllm.compat import require_supported_vllm

BACKEND_PATH = "fragpack_amd.integrations.vllm.backend.FragPackAttentionBackend"


def register() -> None:
    """Check the installed vLLM release, then register the backend in the
    CUSTOM attention slot.

    Raises:
        RuntimeError: The installed vLLM is not the supported release (nothing
            is registered then).
    """
    require_supported_vllm()
    from vllm.v1.attention.backends.registry import AttentionBackendEnum, register_backend

    register_backend(AttentionBackendEnum.CUSTOM, BACKEND_PATH)


__all__ = ["BACKEND_PATH", "register"]
