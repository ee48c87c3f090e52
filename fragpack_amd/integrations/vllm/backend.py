"""vLLM attention backend that keeps the KV cache FragPack-compressed in HBM.

Reference: fragpack/integrations/vllm/backend.py.  Same classes and the same
``--attention-backend CUSTOM`` contract; the step protocol itself lives in
:mod:`fragpack_amd.integrations.vllm.step` (vLLM-free), this module only
adapts vLLM's builder / impl / backend classes to it.

Each paged KV block holds, per layer, one page of
:func:`~fragpack_amd.ops.hbm_kv.page_bytes` shared by its ``2 H`` records, so
the same HBM holds more blocks than a BF16 cache.  Decode attention decodes
the records inside the attention kernel; prefill decodes context pages into a
BF16 workspace and runs the MFMA prefill kernel over it.  vLLM does not pass
the scheduler's open blocks to attention backends, so the model runner is
wrapped by the version-pinned adapter in ``compat``.

Requirements: V2 model runner, BF16 KV, head size 128, ``H * G`` query heads
with ``G`` dividing 8, block size 128, gfx950 (MI355X: vLLM reports
capability 9.5), no speculative decoding, a TP size that divides the KV
heads.  Calibrated tables come from ``FRAGPACK_TABLES``; each TP rank loads
its own heads' tables.
"""

from __future__ import annotations

import os
from dataclasses import replace
from typing import ClassVar

import torch
from vllm.config import VllmConfig, get_layers_from_vllm_config
from vllm.distributed import get_tensor_model_parallel_rank
from vllm.model_executor.layers.attention import Attention
from vllm.model_executor.models.utils import extract_layer_index
from vllm.v1.attention.backend import (
    AttentionBackend,
    AttentionCGSupport,
    AttentionImpl,
    AttentionLayer,
    AttentionMetadataBuilder,
    AttentionType,
    CommonAttentionMetadata,
)
from vllm.v1.kv_cache_interface import AttentionSpec, KVCacheLayout

from fragpack_amd.compression.attn_tables import load_tables
from fragpack_amd.integrations.vllm.compat import install_tracker, require_supported_vllm
from fragpack_amd.integrations.vllm.lifecycle import OpenBlocks
from fragpack_amd.integrations.vllm.step import (
    OVERFLOW_RECORDS,
    FragPackMetadata,
    FragPackRunner,
    PrefillGroup,
    layer_forward,
)
from fragpack_amd.ops.fused_attn_decode import GQA
from fragpack_amd.ops.hbm_kv import BLOCK_TOKENS, HEAD_DIM, page_bytes

_TRACKER = OpenBlocks(BLOCK_TOKENS)


class FragPackMetadataBuilder(AttentionMetadataBuilder[FragPackMetadata]):
    """Builds :class:`FragPackMetadata`; owns the store and the workspaces
    through a :class:`FragPackRunner`.  Model-runner thread only."""

    _cudagraph_support: ClassVar[AttentionCGSupport] = AttentionCGSupport.UNIFORM_SINGLE_TOKEN_DECODE

    def __init__(
        self,
        kv_cache_spec: AttentionSpec,
        layer_names: list[str],
        vllm_config: VllmConfig,
        device: torch.device,
    ) -> None:
        super().__init__(kv_cache_spec, layer_names, vllm_config, device)
        require_supported_vllm(use_v2_model_runner=vllm_config.use_v2_model_runner)
        if vllm_config.speculative_config is not None:
            raise ValueError("FragPack attention does not support speculative decoding")
        if vllm_config.cache_config.block_size != BLOCK_TOKENS:
            raise ValueError(f"FragPack attention needs --block-size {BLOCK_TOKENS}")
        self._init_reorder_batch_threshold(1, supports_spec_as_decode=False)
        install_tracker(_TRACKER, use_v2_model_runner=vllm_config.use_v2_model_runner)

        sched = vllm_config.scheduler_config
        capture = vllm_config.compilation_config.max_cudagraph_capture_size or 0
        kv_heads = kv_cache_spec.num_kv_heads
        self.layer_names = sorted(layer_names, key=extract_layer_index)
        path = os.environ.get("FRAGPACK_TABLES")
        if not path:
            raise ValueError("FRAGPACK_TABLES must point at calibrated FragPack tables (.npz)")
        # vLLM gives TP rank r the KV heads [r * H, (r + 1) * H)
        rank = get_tensor_model_parallel_rank()
        heads = slice(rank * kv_heads, (rank + 1) * kv_heads)
        tables = load_tables(path, device, heads)
        if tables.plut.shape[2] != kv_heads:
            raise ValueError(f"FragPack tables {path} do not cover KV heads {heads.start}..{heads.stop}")
        self.runner = FragPackRunner(
            kv_heads,
            tables,
            device,
            max_tokens=max(sched.max_num_batched_tokens, capture),
            max_reqs=max(sched.max_num_seqs, capture),
            max_model_len=vllm_config.model_config.max_model_len,
            overflow_records=int(os.environ.get("FRAGPACK_OVERFLOW", OVERFLOW_RECORDS)),
            layer_names=self.layer_names,
        )

    def build(
        self, common_prefix_len: int, common_attn_metadata: CommonAttentionMetadata, fast_build: bool = False
    ) -> FragPackMetadata:
        """Prepare the store for this step (also before a graph replay) and
        return every layer's metadata.  Raises ``StoreError`` on data loss."""
        return self._build(common_attn_metadata, capture=False)

    def build_for_cudagraph_capture(self, common_attn_metadata: CommonAttentionMetadata) -> FragPackMetadata:
        """Capture metadata: launch shapes only, store state untouched."""
        return self._build(common_attn_metadata, capture=True)

    def _build(self, cam: CommonAttentionMetadata, capture: bool) -> FragPackMetadata:
        layers = get_layers_from_vllm_config(self.vllm_config, Attention, self.layer_names)
        caches = [layers[name].kv_cache for name in self.layer_names]
        n = cam.num_reqs
        return self.runner.build(
            caches,
            cam.query_start_loc_cpu.numpy()[: n + 1],
            cam.seq_lens_cpu_upper_bound.numpy()[:n],
            cam.seq_lens,
            cam.block_table_tensor,
            cam.slot_mapping,
            _TRACKER.live_blocks(),
            capture=capture,
        )


class FragPackAttentionImpl(AttentionImpl[FragPackMetadata]):
    """Decoder self-attention over the FragPack HBM store.

    Args:
        num_heads: Query heads.
        head_size: 128.
        scale: Softmax scale.
        num_kv_heads: KV heads; ``num_heads / num_kv_heads`` must divide 8.
        alibi_slopes, sliding_window: Must be None.
        kv_cache_dtype: ``auto`` or ``bfloat16``.
        logits_soft_cap: None or 0.
        attn_type: Decoder.
        kv_sharing_target_layer_name: None.
    """

    def __init__(
        self,
        num_heads: int,
        head_size: int,
        scale: float,
        num_kv_heads: int | None = None,
        alibi_slopes: list[float] | None = None,
        sliding_window: int | None = None,
        kv_cache_dtype: str = "auto",
        logits_soft_cap: float | None = None,
        attn_type: str = AttentionType.DECODER,
        kv_sharing_target_layer_name: str | None = None,
        **kwargs: object,
    ) -> None:
        num_kv_heads = num_kv_heads or num_heads
        if num_heads % num_kv_heads or GQA % (num_heads // num_kv_heads) or head_size != HEAD_DIM:
            raise ValueError(f"FragPack attention needs a GQA group dividing {GQA} and head size {HEAD_DIM}")
        if alibi_slopes is not None or sliding_window is not None or logits_soft_cap:
            raise ValueError("FragPack attention supports plain causal attention only")
        if attn_type != AttentionType.DECODER or kv_sharing_target_layer_name is not None:
            raise ValueError("FragPack attention supports unshared decoder self-attention only")
        if kv_cache_dtype not in FragPackAttentionBackend.supported_kv_cache_dtypes:
            raise ValueError(f"FragPack attention stores BF16 KV, not {kv_cache_dtype}")
        self.num_heads = num_heads
        self.head_size = head_size
        self.scale = float(scale)
        self.num_kv_heads = num_kv_heads
        self.kv_cache_dtype = kv_cache_dtype

    def forward(
        self,
        layer: AttentionLayer,
        query: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        kv_cache: torch.Tensor,
        attn_metadata: FragPackMetadata,
        output: torch.Tensor,
        output_scale: torch.Tensor | None = None,
        output_block_scale: torch.Tensor | None = None,
    ) -> torch.Tensor:
        """Write this layer's new KV, attend, encode closed blocks; the last
        layer commits.  Graph-safe for decode-only batches."""
        if output_scale is not None or output_block_scale is not None:
            raise NotImplementedError("FragPack attention does not fuse output quantization")
        if attn_metadata is None:
            return output.zero_()
        li = attn_metadata.layer_index[layer.layer_name]
        return layer_forward(attn_metadata, li, query, key, value, output, self.scale)


class FragPackAttentionBackend(AttentionBackend):
    """FragPack-compressed HBM KV cache backend (``--attention-backend CUSTOM``)."""

    accept_output_buffer: bool = True
    forward_includes_kv_cache_update: bool = True
    supported_dtypes: ClassVar[list[torch.dtype]] = [torch.bfloat16]
    supported_kv_cache_dtypes: ClassVar[list[str]] = ["auto", "bfloat16"]

    @staticmethod
    def get_supported_kernel_block_sizes() -> list[int]:
        return [BLOCK_TOKENS]

    @staticmethod
    def get_name() -> str:
        return "CUSTOM"

    @staticmethod
    def get_impl_cls() -> type[FragPackAttentionImpl]:
        return FragPackAttentionImpl

    @staticmethod
    def get_builder_cls() -> type[FragPackMetadataBuilder]:
        return FragPackMetadataBuilder

    @classmethod
    def get_supported_head_sizes(cls) -> list[int]:
        return [HEAD_DIM]

    @classmethod
    def customize_spec(cls, spec: AttentionSpec) -> AttentionSpec:
        """One record page per block and layer: a single head slot of
        ``page_bytes(H) / 128`` bytes per token."""
        if spec.state_content_bytes is not None:
            return spec
        return replace(spec, num_head_slots=1, state_content_bytes=page_bytes(spec.num_kv_heads) // BLOCK_TOKENS)

    @classmethod
    def supported_kv_cache_layouts(cls) -> tuple[KVCacheLayout, ...]:
        """Layer-major: each layer's blocks are contiguous rows."""
        return (KVCacheLayout.LBNHC,)

    @classmethod
    def supports_compute_capability(cls, capability: object) -> bool:
        """gfx950 only (the kernels are built for it); vLLM on ROCm reports
        it as 9.5."""
        return (capability.major, capability.minor) == (9, 5)


__all__ = [
    "FragPackAttentionBackend",
    "FragPackAttentionImpl",
    "FragPackMetadata",
    "FragPackMetadataBuilder",
    "PrefillGroup",
]
