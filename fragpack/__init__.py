"""The reference's import path, ``fragpack.*``, served by this build.

Callers written against the reference import ``fragpack.compression.attn_tables``,
``fragpack.ops.hbm_kv``, ``fragpack.ops.fused_attn_decode``,
``fragpack.integrations.vllm.backend`` and so on (reference:
fragpack/integrations/vllm/backend.py:37-60, fragpack/ops/hbm_kv.py:177,
fragpack/ops/fused_attn_decode.py:105).  Every ``fragpack.<name>`` module is
the ``fragpack_amd.<name>`` module itself (the same object, registered under
both names), so state such as the loaded library, the logger registry and
class identity is shared whichever name a caller uses.  The vLLM plugin entry
point of the reference, ``fragpack.integrations.vllm.plugin:register``,
resolves the same way.
"""

from __future__ import annotations

import importlib
import importlib.abc
import importlib.machinery
import sys

_PREFIX = __name__ + "."
_TARGET = "fragpack_amd."

__version__ = "0.1.0"


class _Alias(importlib.abc.MetaPathFinder, importlib.abc.Loader):
    """Finds ``fragpack.X`` as ``fragpack_amd.X``: the loader returns the
    already imported target module, so nothing is executed twice."""

    def find_spec(self, fullname, path=None, target=None):
        if not fullname.startswith(_PREFIX):
            return None
        real = _TARGET + fullname[len(_PREFIX):]
        try:
            mod = importlib.import_module(real)
        except ModuleNotFoundError as e:
            if e.name == real:  # no such module here: let the import fail as usual
                return None
            raise
        return importlib.machinery.ModuleSpec(fullname, self, is_package=hasattr(mod, "__path__"))

    def create_module(self, spec):
        return importlib.import_module(_TARGET + spec.name[len(_PREFIX):])

    def exec_module(self, module):
        pass


if not any(isinstance(f, _Alias) for f in sys.meta_path):
    sys.meta_path.insert(0, _Alias())
