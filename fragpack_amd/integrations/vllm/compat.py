"""Version-pinned adaptation of vLLM's V2 model runner.

Reference: fragpack/integrations/vllm/compat.py.  Attention backends never see
the scheduler output, but the store needs each step's open blocks; the
wrapper installed here feeds :class:`OpenBlocks` before every real model step.
That is a runtime patch of one vLLM release, so the release is checked first.

The reference pins the CUDA wheel "0.30.0+cu129".  This build runs on ROCm, so
it pins the same release built for ROCm: public version "0.30.0" with a local
label that starts with "rocm" (e.g. "0.30.0+rocm700").  CUDA wheels, other
releases and unlabelled source builds are rejected.  Checking the version
imports neither torch nor vLLM.
"""

from __future__ import annotations

import functools
from importlib import metadata
from typing import TYPE_CHECKING, Any

if TYPE_CHECKING:
    from fragpack_amd.integrations.vllm.lifecycle import OpenBlocks

SUPPORTED_VLLM_RELEASE = "0.30.0"
SUPPORTED_LOCAL_PREFIX = "rocm"
SUPPORTED_VLLM_VERSION = f"{SUPPORTED_VLLM_RELEASE}+{SUPPORTED_LOCAL_PREFIX}*"
_installed_tracker: OpenBlocks | None = None


def _supported(version: str) -> bool:
    release, _, local = version.partition("+")
    return release == SUPPORTED_VLLM_RELEASE and local.startswith(SUPPORTED_LOCAL_PREFIX)


def require_supported_vllm(*, use_v2_model_runner: bool | None = None) -> str:
    """Reject an absent or unsupported vLLM distribution, or a non-V2 runner.

    Args:
        use_v2_model_runner: The resolved runner choice; None (plugin
            discovery) checks the distribution only.

    Returns:
        The installed distribution version.

    Raises:
        RuntimeError: vLLM is not installed, or its version is not the pinned
            release for ROCm.
        ValueError: ``use_v2_model_runner`` is False.
    """
    try:
        installed = metadata.version("vllm")
    except metadata.PackageNotFoundError as exc:
        raise RuntimeError(f"FragPack requires vllm=={SUPPORTED_VLLM_VERSION}; vLLM is not installed") from exc
    if not _supported(installed):
        raise RuntimeError(
            f"FragPack requires vllm=={SUPPORTED_VLLM_VERSION}; found {installed}. "
            "Its V2 lifecycle adapter is release-specific."
        )
    if use_v2_model_runner is not None and not use_v2_model_runner:
        raise ValueError("FragPack attention needs the V2 model runner")
    return installed


def install_tracker(tracker: OpenBlocks, *, use_v2_model_runner: bool) -> None:
    """Wrap ``GPUModelRunner.execute_model`` once so that every real step
    updates ``tracker`` before the model runs (dummy runs pass straight
    through).

    Args:
        tracker: The worker's block tracker, shared with the backend.
        use_v2_model_runner: Must be True.

    Raises:
        RuntimeError: Unsupported distribution, or a different tracker is
            already installed (the backend would otherwise read a stale one).
        ValueError: The runner is not V2.

    Repeating the call with the installed tracker does nothing.  Call during
    worker initialisation, before model execution starts.
    """
    global _installed_tracker
    require_supported_vllm(use_v2_model_runner=use_v2_model_runner)
    if _installed_tracker is tracker:
        return
    if _installed_tracker is not None:
        raise RuntimeError("FragPack V2 lifecycle adapter already has a tracker")

    from vllm.v1.worker.gpu.model_runner import GPUModelRunner

    wrapped = GPUModelRunner.execute_model

    @functools.wraps(wrapped)
    def execute_model(self: Any, scheduler_output: Any, *args: Any, **kwargs: Any) -> Any:
        if not kwargs.get("dummy_run", False):
            tracker.update(scheduler_output)
        return wrapped(self, scheduler_output, *args, **kwargs)

    GPUModelRunner.execute_model = execute_model
    _installed_tracker = tracker


def installed_tracker() -> OpenBlocks | None:
    """The tracker the runner wrapper feeds, or None before installation."""
    return _installed_tracker


__all__ = ["SUPPORTED_VLLM_VERSION", "install_tracker", "installed_tracker", "require_supported_vllm"]
