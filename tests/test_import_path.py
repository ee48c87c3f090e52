"""The reference's import path: ``fragpack.<module>`` resolves to this build.

A caller written against the reference imports ``fragpack.compression.*``,
``fragpack.ops.*`` and ``fragpack.integrations.vllm.*`` unchanged (reference:
fragpack/integrations/vllm/backend.py:37-60, plugin entry point
pyproject.toml ``fragpack.integrations.vllm.plugin:register``).  Each test
imports a reference module path, checks it is this build's module object,
and calls one of its functions.  No GPU.
"""

from __future__ import annotations

import importlib
import sys

import numpy as np
import pytest

from tests import fake_vllm

MODULES = [
    "fragpack.logging",
    "fragpack.compression",
    "fragpack.compression.attn_page",
    "fragpack.compression.attn_tables",
    "fragpack.ops",
    "fragpack.ops.fragpack_ext",
    "fragpack.ops.fused_attn_decode",
    "fragpack.ops.hbm_kv",
    "fragpack.integrations",
    "fragpack.integrations.vllm",
    "fragpack.integrations.vllm.capacity",
    "fragpack.integrations.vllm.compat",
    "fragpack.integrations.vllm.lifecycle",
]


@pytest.mark.parametrize("name", MODULES)
def test_reference_module_path_is_this_build(name):
    mod = importlib.import_module(name)
    assert mod is importlib.import_module("fragpack_amd" + name[len("fragpack"):])


def test_from_imports_and_calls():
    from fragpack.compression.attn_page import calibrate_table, decode_record, encode_record
    from fragpack.compression.attn_tables import calibrate, device_tables
    from fragpack.ops.fused_attn_decode import RecordTables, decode_units, workspace_elems
    from fragpack.ops.hbm_kv import HbmKvStore, page_bytes
    from fragpack_amd.ops.hbm_kv import HbmKvStore as Native

    assert HbmKvStore is Native and callable(device_tables) and RecordTables.__module__.startswith("fragpack_amd")
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((128, 128)) * 0.5).astype(np.float32).view(np.uint32)
    rec = (x >> 16).astype(np.uint16)
    table = calibrate_table((rec >> 8).astype(np.uint8))
    for kv in (0, 1):
        assert np.array_equal(decode_record(encode_record(rec, table, kv), table, kv), rec)
    dump = rec.reshape(1, 1, 1, 128, 1, 128).repeat(2, axis=2)
    assert calibrate(dump).shape == (1, 2, 1, 22)
    assert page_bytes(4) == 190464 and page_bytes(8) == 380928  # the reference page sizes, hbm_kv.py:87-99
    assert decode_units(4, 4, 256) >= 4
    o, m, p = workspace_elems(4, 16)
    assert o == 4 * 16 * 8 * 128 and m == 4 * 16 * 8 * 2 and p > 0


def test_logger_is_shared():
    from fragpack.logging import init_logger
    from fragpack_amd.logging import init_logger as native

    assert init_logger is native
    assert init_logger("fragpack.test").name == "fragpack_amd.fragpack.test"  # under the package handler


def test_reference_plugin_entry_point(monkeypatch):
    fakes = fake_vllm.install(monkeypatch)
    for name in list(sys.modules):
        if name.startswith("fragpack.integrations.vllm."):
            monkeypatch.delitem(sys.modules, name)
    plugin = importlib.import_module("fragpack.integrations.vllm.plugin")  # the reference's entry point
    plugin.register()
    assert [p for _, p in fakes.registrations] == [plugin.BACKEND_PATH]
    backend = importlib.import_module("fragpack.integrations.vllm.backend")
    assert backend.FragPackAttentionBackend.get_name() == "CUSTOM"


def test_unknown_module_still_fails():
    with pytest.raises(ModuleNotFoundError):
        importlib.import_module("fragpack.no_such_module")
