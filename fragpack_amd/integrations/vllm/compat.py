"""The one vLLM release this integration patches, and the patch itself.

Reference interface: fragpack/integrations/vllm/compat.py
(``SUPPORTED_VLLM_VERSION``, ``require_supported_vllm``, ``install_tracker``,
``installed_tracker``).  Attention backends never see the scheduler output,
but the store needs each step's open blocks (:class:`OpenBlocks`), so the V2
model runner's ``execute_model`` is wrapped to feed the tracker before every
real step.  Wrapping a method of one release is version-specific: the release
is checked before anything is touched.

The reference pins the CUDA wheel "0.30.0+cu129"; this build runs on ROCm and
pins the same release's ROCm builds: public version "0.30.0" with a local
label starting "rocm" (e.g. "0.30.0+rocm700").  Checking the version imports
neither torch nor vLLM.
"""

from __future__ import annotations

from dataclasses import dataclass
import functools
from importlib import metadata
from typing import TYPE_CHECKING, Any, Callable

if TYPE_CHECKING:
    from fragpack_amd.integrations.vllm.lifecycle import OpenBlocks


@dataclass(frozen=True)
class _Pin:
    release: str
    local_prefix: str

    def __str__(self) -> str:
        return f"{self.release}+{self.local_prefix}*"

    def admits(self, version: str) -> bool:
        public, plus, local = version.partition("+")
        return public == self.release and bool(plus) and local.startswith(self.local_prefix)


_PIN = _Pin("0.30.0", "rocm")
SUPPORTED_VLLM_VERSION = str(_PIN)


class _RunnerPatch:
    """The installed wrapper: which tracker it feeds."""

    tracker: OpenBlocks | None = None

    @staticmethod
    def wrap(step: Callable[..., Any], tracker: OpenBlocks) -> Callable[..., Any]:
        @functools.wraps(step)
        def execute_model(runner: Any, scheduler_output: Any, *args: Any, **kwargs: Any) -> Any:
            if not kwargs.get("dummy_run", False):  # profiling / warm-up runs carry no real requests
                tracker.update(scheduler_output)
            return step(runner, scheduler_output, *args, **kwargs)

        return execute_model


def require_supported_vllm(*, use_v2_model_runner: bool | None = None) -> str:
    """The installed vLLM version, if it is the pinned release's ROCm build.

    Args:
        use_v2_model_runner: The resolved runner choice; None (plugin
            discovery) checks the distribution only.

    Raises:
        RuntimeError: vLLM is absent or is another build or release.
        ValueError: ``use_v2_model_runner`` is False.
    """
    try:
        found = metadata.version("vllm")
    except metadata.PackageNotFoundError as exc:
        raise RuntimeError(f"FragPack requires vllm=={SUPPORTED_VLLM_VERSION}; vLLM is not installed") from exc
    if not _PIN.admits(found):
        raise RuntimeError(f"FragPack requires vllm=={SUPPORTED_VLLM_VERSION}, found {found}: the runner patch "
                           "is release-specific")
    if use_v2_model_runner is False:
        raise ValueError("FragPack attention needs the V2 model runner")
    return found


def install_tracker(tracker: OpenBlocks, *, use_v2_model_runner: bool) -> None:
    """Feed ``tracker`` from every real model step (idempotent per tracker).

    Call during worker initialisation, before the model runs.

    Raises:
        RuntimeError: Unsupported vLLM, or another tracker is already installed
            (the backend would read a stale mirror).
        ValueError: The runner is not V2.
    """
    require_supported_vllm(use_v2_model_runner=use_v2_model_runner)
    if _RunnerPatch.tracker is tracker:
        return
    if _RunnerPatch.tracker is not None:
        raise RuntimeError("FragPack's V2 runner patch already has a tracker")
    from vllm.v1.worker.gpu.model_runner import GPUModelRunner

    GPUModelRunner.execute_model = _RunnerPatch.wrap(GPUModelRunner.execute_model, tracker)
    _RunnerPatch.tracker = tracker


def installed_tracker() -> OpenBlocks | None:
    """The tracker the runner patch feeds, or None before installation."""
    return _RunnerPatch.tracker


__all__ = ["SUPPORTED_VLLM_VERSION", "install_tracker", "installed_tracker", "require_supported_vllm"]
