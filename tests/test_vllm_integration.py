"""Host-side contracts of the vLLM integration (no GPU, no vLLM).

Mirrors the reference's tests/unit/test_open_blocks.py and
tests/unit/test_vllm_compat.py: the open-block tracker, the version gate and
runner wrapper, lazy plugin registration.  Adds the capacity snapshot, the
step planner (decode split, closed-block count, prefill workspace groups,
checked against brute force) and the backend classes' validation, imported
against the stand-in vLLM modules of ``tests/fake_vllm.py``.
"""

from __future__ import annotations

import importlib
import sys
from types import SimpleNamespace

import numpy as np
import pytest

from fragpack_amd.integrations.vllm.lifecycle import OpenBlocks
from tests import fake_vllm


def _output(new=(), cached=(), finished=(), resumed=(), preempted=(), updates=None):
    """A scheduler output with the fields OpenBlocks reads.

    new: (req_id, block_ids, num_computed_tokens); cached: (req_id,
    num_computed_tokens, new_block_ids or None).
    """
    return SimpleNamespace(
        finished_req_ids=set(finished),
        preempted_req_ids=set(preempted),
        scheduled_new_reqs=[SimpleNamespace(req_id=r, block_ids=(list(b),), num_computed_tokens=c)
                            for r, b, c in new],
        block_table_updates={r: (ids,) for r, ids in updates.items()} if updates else None,
        scheduled_cached_reqs=SimpleNamespace(
            req_ids=[r for r, _, _ in cached],
            num_computed_tokens=[c for _, c, _ in cached],
            new_block_ids=[None if b is None else (list(b),) for _, _, b in cached],
            resumed_req_ids=set(resumed),
        ),
    )


# --- OpenBlocks (reference lifecycle.py) ---------------------------------------


def test_open_blocks_tracks_partial_block_of_each_writer():
    ob = OpenBlocks(128)
    ob.update(_output(new=(("a", [10, 11, 12], 0), ("b", [20], 0))))
    assert ob.live_blocks().tolist() == []
    ob.update(_output(cached=(("a", 200, None), ("b", 128, None))))
    assert ob.live_blocks().tolist() == [11]
    ob.update(_output(cached=(("a", 300, None), ("b", 129, [21]))))
    assert sorted(ob.live_blocks().tolist()) == [12, 21]


def test_open_blocks_reallocated_block_is_not_live_ahead_of_its_writer():
    ob = OpenBlocks(128)
    ob.update(_output(new=(("a", [10, 11], 0),)))
    ob.update(_output(cached=(("a", 200, None),)))
    assert ob.live_blocks().tolist() == [11]
    ob.update(_output(new=(("b", [30, 11], 0),), finished={"a"}))
    ob.update(_output(cached=(("b", 50, None),)))
    assert ob.live_blocks().tolist() == [30]


def test_open_blocks_resume_replaces_and_preemption_discards():
    ob = OpenBlocks(128)
    ob.update(_output(new=(("a", [10, 11], 0),)))
    ob.update(_output(cached=(("a", 150, None),)))
    ob.update(_output(cached=(("a", 130, [40, 41]),), resumed={"a"}))
    assert ob.live_blocks().tolist() == [41]
    ob.update(_output(preempted={"a"}, cached=(("a", 160, None),)))
    assert ob.live_blocks().tolist() == []
    ob.update(_output(preempted={"a"}, new=(("a", [50, 51], 140),)))
    assert ob.live_blocks().tolist() == [51]


def test_open_blocks_table_update_is_authoritative():
    ob = OpenBlocks(128)
    ob.update(_output(new=(("a", [10, 11], 150),)))
    ob.update(_output(cached=(("a", 150, [90]),), updates={"a": [40, 41]}))
    assert ob.live_blocks().tolist() == [41]
    ob.update(_output(cached=(("a", 260, None),)))
    assert ob.live_blocks().tolist() == []


def test_open_blocks_unallocated_next_block_and_bad_input():
    ob = OpenBlocks(128)
    ob.update(_output(new=(("a", [10], 130),)))  # next token's block not allocated yet
    assert ob.live_blocks().tolist() == []
    assert ob.live_blocks().dtype == np.int32
    bad = _output(cached=(("a", 131, None),))
    bad.scheduled_cached_reqs.new_block_ids.append(None)
    with pytest.raises(ValueError):
        ob.update(bad)
    with pytest.raises(ValueError):
        OpenBlocks(0)


# --- compat / plugin (reference compat.py, plugin.py) -----------------------------


def _step_output():
    return _output(new=(("a", [10, 11], 150),))


@pytest.mark.parametrize("version", ["0.29.0+rocm700", "0.30.0", "0.30.0+cu129", "0.31.0+rocm700"])
def test_other_distributions_are_rejected_before_runner_mutation(monkeypatch, version):
    fakes = fake_vllm.install(monkeypatch, version)
    compat = importlib.import_module("fragpack_amd.integrations.vllm.compat")
    original = fakes.GPUModelRunner.execute_model
    with pytest.raises(RuntimeError, match="release-specific"):
        compat.install_tracker(OpenBlocks(128), use_v2_model_runner=True)
    assert fakes.GPUModelRunner.execute_model is original


def test_rocm_build_of_pinned_release_is_accepted(monkeypatch):
    fake_vllm.install(monkeypatch, "0.30.0+rocm710")
    compat = importlib.import_module("fragpack_amd.integrations.vllm.compat")
    assert compat.require_supported_vllm() == "0.30.0+rocm710"
    with pytest.raises(ValueError, match="V2 model runner"):
        compat.require_supported_vllm(use_v2_model_runner=False)


def test_missing_distribution_has_actionable_error(monkeypatch):
    from importlib import metadata

    fake_vllm.install(monkeypatch)
    compat = importlib.import_module("fragpack_amd.integrations.vllm.compat")

    def missing(name):
        raise metadata.PackageNotFoundError(name)

    monkeypatch.setattr(metadata, "version", missing)
    with pytest.raises(RuntimeError, match="vLLM is not installed"):
        compat.require_supported_vllm()


def test_real_step_updates_tracker_before_the_model_and_forwards_arguments(monkeypatch):
    fakes = fake_vllm.install(monkeypatch)
    compat = importlib.import_module("fragpack_amd.integrations.vllm.compat")
    tracker = OpenBlocks(128)
    inner = fakes.GPUModelRunner.execute_model

    def observe(self, so, *args, **kwargs):
        assert tracker.live_blocks().tolist() == [11]
        return inner(self, so, *args, **kwargs)

    fakes.GPUModelRunner.execute_model = observe
    compat.install_tracker(tracker, use_v2_model_runner=True)
    step = _step_output()
    assert fakes.GPUModelRunner().execute_model(step, "x", flag=7) == (step, ("x",), {"flag": 7})
    assert compat.installed_tracker() is tracker


def test_dummy_step_bypasses_tracker(monkeypatch):
    fakes = fake_vllm.install(monkeypatch)
    compat = importlib.import_module("fragpack_amd.integrations.vllm.compat")
    tracker = OpenBlocks(128)
    tracker.update(_step_output())
    compat.install_tracker(tracker, use_v2_model_runner=True)
    assert fakes.GPUModelRunner().execute_model(None, dummy_run=True) == (None, (), {"dummy_run": True})
    assert tracker.live_blocks().tolist() == [11]


def test_installation_is_idempotent_and_rejects_a_second_tracker(monkeypatch):
    fakes = fake_vllm.install(monkeypatch)
    compat = importlib.import_module("fragpack_amd.integrations.vllm.compat")
    tracker = OpenBlocks(128)
    compat.install_tracker(tracker, use_v2_model_runner=True)
    wrapped = fakes.GPUModelRunner.execute_model
    compat.install_tracker(tracker, use_v2_model_runner=True)
    assert fakes.GPUModelRunner.execute_model is wrapped
    with pytest.raises(RuntimeError, match="already has a tracker"):
        compat.install_tracker(OpenBlocks(128), use_v2_model_runner=True)
    fakes.GPUModelRunner().execute_model(_step_output())
    assert tracker.live_blocks().tolist() == [11]


def test_plugin_registers_the_class_path_without_importing_the_backend(monkeypatch):
    fakes = fake_vllm.install(monkeypatch)
    plugin = importlib.import_module("fragpack_amd.integrations.vllm.plugin")
    backend_path = "fragpack_amd.integrations.vllm.backend"
    monkeypatch.setitem(sys.modules, backend_path, None)  # an import attempt would fail
    plugin.register()
    assert fakes.registrations == [("custom-slot", backend_path + ".FragPackAttentionBackend")]
    assert sys.modules[backend_path] is None


def test_plugin_rejects_an_unsupported_release_before_registration(monkeypatch):
    fakes = fake_vllm.install(monkeypatch, "0.31.0+rocm700")
    plugin = importlib.import_module("fragpack_amd.integrations.vllm.plugin")
    with pytest.raises(RuntimeError, match="release-specific"):
        plugin.register()
    assert fakes.registrations == []


# --- capacity (reference capacity.py) ---------------------------------------------


def test_capacity_snapshot_is_host_only_and_copied():
    from fragpack_amd.integrations.vllm import capacity

    cap = capacity.FragPackCapacity(blocks=10, block_tokens=128, layers=2, kv_heads=8, page_bytes=380928,
                                    raw_page_bytes=524288, memory={"arena": 1})
    capacity.publish_capacity(cap)
    assert capacity.get_capacity() is cap
    d = cap.to_dict()
    d["memory"]["arena"] = 2
    assert cap.memory["arena"] == 1
    with pytest.raises(Exception):
        cap.blocks = 3  # frozen


# --- step planner (reference backend.py:269-290, 398-446) -------------------------


def test_step_constants_match_the_store():
    from fragpack_amd.integrations.vllm import step
    from fragpack_amd.ops import hbm_kv

    assert (step.BLOCK_TOKENS, step.HEAD_DIM) == (hbm_kv.BLOCK_TOKENS, hbm_kv.HEAD_DIM)


def test_split_decodes():
    from fragpack_amd.integrations.vllm.step import split_decodes

    assert split_decodes(np.array([1, 1, 1])) == 3
    assert split_decodes(np.array([1, 1, 5, 1])) == 2
    assert split_decodes(np.array([7])) == 0
    assert split_decodes(np.array([], np.int64)) == 0


def test_closes_count_blocks_filled_this_step_brute_force():
    from fragpack_amd.integrations.vllm.step import plan_step

    rng = np.random.default_rng(7)
    for _ in range(200):
        R = int(rng.integers(1, 9))
        qlen = rng.integers(1, 400, R)
        qlen[: int(rng.integers(0, R + 1))] = 1
        prior = rng.integers(0, 2000, R)
        seq = prior + qlen
        qsl = np.concatenate(([0], np.cumsum(qlen)))
        hs = plan_step(qsl, seq, slot_rows=int(qsl[-1]) + 3, workspace_pages=64, max_tokens=4096)
        # a block closes when its 128th token (position 128k-1) is among the new ones
        brute = sum(1 for r in range(R) for pos in range(prior[r], seq[r]) if pos % 128 == 127)
        assert hs.closes == brute
        assert hs.max_close == min(brute, 4096)  # launched as planned: the exact count
        assert hs.num_tokens == qsl[-1]
        cap = plan_step(qsl, seq, slot_rows=int(qsl[-1]) + 3, workspace_pages=64, max_tokens=4096, capture=True)
        assert cap.max_close == min(max(brute, cap.num_decodes), 4096)  # covers every replay
        assert cap.prefills == []


def test_prefill_groups_pack_rows_in_order_within_the_workspace():
    from fragpack_amd.integrations.vllm.step import plan_step

    rng = np.random.default_rng(8)
    for _ in range(100):
        R = int(rng.integers(1, 12))
        nd = int(rng.integers(0, R))
        qlen = np.concatenate((np.ones(nd, np.int64), rng.integers(2, 700, R - nd)))
        seq = qlen + rng.integers(0, 900, R)
        qsl = np.concatenate(([0], np.cumsum(qlen)))
        ws = 16
        hs = plan_step(qsl, seq, int(qsl[-1]), ws, 8192)
        assert hs.num_decodes == nd
        rows = [r for g in hs.prefills for r in range(g.r0, g.r1)]
        assert rows == list(range(nd, R))
        for g in hs.prefills:
            pages = -(-seq[g.r0 : g.r1] // 128)
            assert pages.sum() <= ws or g.r1 - g.r0 == 1
            assert (g.tok0, g.tok1) == (qsl[g.r0], qsl[g.r1])
            assert g.cu_seqlens_q.tolist() == (qsl[g.r0 : g.r1 + 1] - qsl[g.r0]).tolist()
            assert g.seqused_k.tolist() == seq[g.r0 : g.r1].tolist()
            assert g.max_seqlen_q == int(qlen[g.r0 : g.r1].max())
            # workspace page j of row i holds the row's j-th block, pages used once
            used = []
            for i, r in enumerate(range(g.r0, g.r1)):
                for j in range(int(pages[i])):
                    wp = int(g.block_table[i, j])
                    assert (g.src_rows[wp], g.src_cols[wp]) == (r, j)
                    used.append(wp)
            assert sorted(used) == list(range(len(g.src_rows)))


def test_default_workspace_holds_a_step_of_fresh_prompts_in_one_group():
    from fragpack_amd.integrations.vllm.step import default_workspace_pages, plan_step

    rng = np.random.default_rng(9)
    for _ in range(200):
        max_len = int(rng.integers(1, 40)) * 100
        max_tokens, max_reqs = int(rng.integers(1, 9000)), int(rng.integers(1, 40))
        ws = default_workspace_pages(max_len, max_tokens, max_reqs)
        assert ws >= -(-max_len // 128)
        # fresh prompts (context = query, at least 2 tokens: 1 is a decode) within the
        # step budget, request count and model length
        R = int(rng.integers(1, max_reqs + 1))
        qlen = rng.integers(2, min(max_len, max(max_tokens // R, 2)) + 1, R)
        qlen = qlen[np.cumsum(qlen) <= max_tokens]
        if qlen.size == 0:
            continue
        qsl = np.concatenate(([0], np.cumsum(qlen)))
        hs = plan_step(qsl, qlen, int(qsl[-1]), ws, max_tokens)
        assert len(hs.prefills) == 1 and (hs.prefills[0].r0, hs.prefills[0].r1) == (0, qlen.size)
    # one max-length context always fits
    assert default_workspace_pages(8192, 512, 4) == 64
    assert default_workspace_pages(8320, 32768, 4) == 256 + 4


def test_prefill_longer_than_the_workspace_is_rejected():
    from fragpack_amd.integrations.vllm.step import plan_step

    with pytest.raises(ValueError, match="workspace"):
        plan_step(np.array([0, 600]), np.array([3000]), 600, workspace_pages=8, max_tokens=4096)
    hs = plan_step(np.array([0, 600]), np.array([3000]), 600, workspace_pages=8, max_tokens=4096, capture=True)
    assert hs.prefills == [] and hs.num_decodes == 0


# --- backend classes against the stand-in vLLM -----------------------------------


def test_backend_classes_and_impl_validation(monkeypatch):
    fake_vllm.install(monkeypatch)
    backend = importlib.import_module("fragpack_amd.integrations.vllm.backend")
    from fragpack_amd.ops.hbm_kv import page_bytes

    B = backend.FragPackAttentionBackend
    assert B.get_name() == "CUSTOM"
    assert B.get_supported_kernel_block_sizes() == [128] and B.get_supported_head_sizes() == [128]
    assert B.get_impl_cls() is backend.FragPackAttentionImpl
    assert B.get_builder_cls() is backend.FragPackMetadataBuilder
    spec = fake_vllm.AttentionSpec(block_size=128, num_kv_heads=8, head_size=128)
    custom = B.customize_spec(spec)
    assert custom.num_head_slots == 1 and custom.state_content_bytes * 128 == page_bytes(8)
    assert B.customize_spec(custom) is custom
    assert B.supports_compute_capability(SimpleNamespace(major=9, minor=5))
    assert not B.supports_compute_capability(SimpleNamespace(major=9, minor=4))
    impl = backend.FragPackAttentionImpl(32, 128, 0.1, 8)
    assert impl.num_kv_heads == 8
    for kwargs in ({"num_heads": 32, "head_size": 64, "num_kv_heads": 8},
                   {"num_heads": 48, "head_size": 128, "num_kv_heads": 3},  # G = 16
                   {"num_heads": 12, "head_size": 128, "num_kv_heads": 4},  # G = 3
                   {"num_heads": 8, "head_size": 128, "sliding_window": 64},
                   {"num_heads": 8, "head_size": 128, "logits_soft_cap": 30.0},
                   {"num_heads": 8, "head_size": 128, "kv_cache_dtype": "fp8"},
                   {"num_heads": 8, "head_size": 128, "attn_type": "encoder"}):
        with pytest.raises(ValueError):
            backend.FragPackAttentionImpl(scale=0.1, **kwargs)


def test_builder_rejects_unsupported_engine_settings(monkeypatch):
    fake_vllm.install(monkeypatch)
    backend = importlib.import_module("fragpack_amd.integrations.vllm.backend")
    spec = fake_vllm.AttentionSpec(block_size=128, num_kv_heads=2, head_size=128)
    names = ["model.layers.0.attn"]
    cases = [
        (fake_vllm.VllmConfig(use_v2_model_runner=False), ValueError, "V2"),
        (fake_vllm.VllmConfig(speculative_config=object()), ValueError, "speculative"),
        (fake_vllm.VllmConfig(cache_config=SimpleNamespace(block_size=16)), ValueError, "block-size"),
    ]
    for cfg, exc, match in cases:
        with pytest.raises(exc, match=match):
            backend.FragPackMetadataBuilder(spec, names, cfg, "cpu")
    monkeypatch.delenv("FRAGPACK_TABLES", raising=False)
    with pytest.raises(ValueError, match="FRAGPACK_TABLES"):
        backend.FragPackMetadataBuilder(spec, names, fake_vllm.VllmConfig(), "cpu")
