"""Stand-in ``vllm`` modules for testing the integration without vLLM.

vLLM is not installed in this image.  The integration imports a handful of its
names (config helpers, the attention-backend base classes, the KV spec, the
V2 model runner, the backend registry); :func:`install` puts minimal modules
with those names into ``sys.modules`` through a pytest ``monkeypatch`` so
they disappear after the test.  The stand-ins carry only what the
integration reads: they are fixtures, not a vLLM model of behaviour.
"""

from __future__ import annotations

import enum
import re
import sys
from dataclasses import dataclass, field
from types import ModuleType, SimpleNamespace
from typing import Any, Generic, TypeVar

INTEGRATION_MODULES = (
    "fragpack_amd.integrations.vllm.backend",
    "fragpack_amd.integrations.vllm.compat",
    "fragpack_amd.integrations.vllm.plugin",
)

M = TypeVar("M")


class AttentionCGSupport(enum.Enum):
    NEVER = 0
    UNIFORM_SINGLE_TOKEN_DECODE = 1
    ALWAYS = 2


class AttentionType:
    DECODER = "decoder"
    ENCODER = "encoder"


class AttentionBackend:
    pass


class AttentionLayer:
    pass


class AttentionImpl(Generic[M]):
    pass


class AttentionMetadataBuilder(Generic[M]):
    def __init__(self, kv_cache_spec, layer_names, vllm_config, device) -> None:
        self.kv_cache_spec = kv_cache_spec
        self.layer_names = layer_names
        self.vllm_config = vllm_config
        self.device = device
        self.reorder_batch_threshold = None

    def _init_reorder_batch_threshold(self, threshold: int, supports_spec_as_decode: bool = False) -> None:
        self.reorder_batch_threshold = threshold


@dataclass
class CommonAttentionMetadata:
    query_start_loc: Any
    query_start_loc_cpu: Any
    seq_lens: Any
    seq_lens_cpu_upper_bound: Any
    num_reqs: int
    num_actual_tokens: int
    block_table_tensor: Any
    slot_mapping: Any


@dataclass(frozen=True)
class AttentionSpec:
    block_size: int
    num_kv_heads: int
    head_size: int
    dtype: Any = None
    num_head_slots: int | None = None
    state_content_bytes: int | None = None


class KVCacheLayout(enum.Enum):
    NHD = 0
    LBNHC = 1


class Attention:
    """A model's attention layer: its name and bound KV cache."""

    def __init__(self, layer_name: str, kv_cache: Any) -> None:
        self.layer_name = layer_name
        self.kv_cache = kv_cache


@dataclass
class VllmConfig:
    use_v2_model_runner: bool = True
    speculative_config: Any = None
    cache_config: Any = field(default_factory=lambda: SimpleNamespace(block_size=128))
    scheduler_config: Any = field(default_factory=lambda: SimpleNamespace(max_num_batched_tokens=2048,
                                                                          max_num_seqs=16))
    compilation_config: Any = field(default_factory=lambda: SimpleNamespace(max_cudagraph_capture_size=0))
    model_config: Any = field(default_factory=lambda: SimpleNamespace(max_model_len=4096))
    layers: dict = field(default_factory=dict)


def get_layers_from_vllm_config(config: VllmConfig, layer_type: type, layer_names: list[str]) -> dict:
    return {name: config.layers[name] for name in layer_names if isinstance(config.layers[name], layer_type)}


def extract_layer_index(name: str) -> int:
    found = re.findall(r"\.(\d+)\.", name)
    if len(found) != 1:
        raise ValueError(f"no single layer index in {name}")
    return int(found[0])


class GPUModelRunner:
    """Records the arguments of every model step."""

    def execute_model(self, scheduler_output: Any, *args: Any, **kwargs: Any) -> Any:
        return scheduler_output, args, kwargs


def _module(monkeypatch, name: str, **attrs: Any) -> ModuleType:
    mod = ModuleType(name)
    mod.__path__ = []  # a package, so submodules import
    for k, v in attrs.items():
        setattr(mod, k, v)
    monkeypatch.setitem(sys.modules, name, mod)
    return mod


def install(monkeypatch, version: str = "0.30.0+rocm700") -> SimpleNamespace:
    """Install the stand-ins and the distribution version; drop cached
    integration modules so that they import against the stand-ins.

    Returns:
        Handles of the stand-ins a test inspects (``registrations`` of the
        backend registry, the ``GPUModelRunner`` class).
    """
    from importlib import metadata

    real_version = metadata.version

    def version_of(name: str) -> str:
        return version if name == "vllm" else real_version(name)

    monkeypatch.setattr(metadata, "version", version_of)
    for name in INTEGRATION_MODULES:
        monkeypatch.delitem(sys.modules, name, raising=False)
    registrations: list[tuple[Any, str]] = []
    runner_cls = type("GPUModelRunner", (GPUModelRunner,), {})
    for pkg in ("vllm", "vllm.model_executor", "vllm.model_executor.layers", "vllm.model_executor.models",
                "vllm.v1", "vllm.v1.attention", "vllm.v1.attention.backends", "vllm.v1.worker",
                "vllm.v1.worker.gpu"):
        _module(monkeypatch, pkg)
    _module(monkeypatch, "vllm.config", VllmConfig=VllmConfig, get_layers_from_vllm_config=get_layers_from_vllm_config)
    _module(monkeypatch, "vllm.distributed", get_tensor_model_parallel_rank=lambda: 0)
    _module(monkeypatch, "vllm.model_executor.layers.attention", Attention=Attention)
    _module(monkeypatch, "vllm.model_executor.models.utils", extract_layer_index=extract_layer_index)
    _module(monkeypatch, "vllm.v1.attention.backend", AttentionBackend=AttentionBackend,
            AttentionCGSupport=AttentionCGSupport, AttentionImpl=AttentionImpl, AttentionLayer=AttentionLayer,
            AttentionMetadataBuilder=AttentionMetadataBuilder, AttentionType=AttentionType,
            CommonAttentionMetadata=CommonAttentionMetadata)
    _module(monkeypatch, "vllm.v1.kv_cache_interface", AttentionSpec=AttentionSpec, KVCacheLayout=KVCacheLayout)
    _module(monkeypatch, "vllm.v1.worker.gpu.model_runner", GPUModelRunner=runner_cls)
    _module(monkeypatch, "vllm.v1.attention.backends.registry",
            AttentionBackendEnum=SimpleNamespace(CUSTOM="custom-slot"),
            register_backend=lambda slot, path: registrations.append((slot, path)))
    return SimpleNamespace(registrations=registrations, GPUModelRunner=runner_cls)
