"""vLLM CUSTOM attention backend over the FragPack HBM store.

Mirrors fragpack/integrations/vllm (backend.py, compat.py, lifecycle.py,
capacity.py, plugin.py).  ``lifecycle``, ``capacity``, ``compat`` and
``plugin`` import neither torch nor vLLM at module level; ``step`` holds the
engine-independent per-step / per-layer logic; ``backend`` adapts it to vLLM's
attention-backend classes and needs vLLM installed.
"""
