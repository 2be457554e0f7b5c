"""MI355X-native paged-KV attention for LLMario's engine.

The product is the C-ABI library ``libllmario_hip.so`` (``include/llmario_hip.h``), built from
``csrc/`` with hipcc for gfx950. This package holds its sources, the build step, a ctypes
binding and a thin Python mirror of the engine's KV-cache/attention interface.
"""

from .kv import HipKvCache, KvFull, Layer, LmhError  # noqa: F401

__all__ = ["HipKvCache", "KvFull", "Layer", "LmhError"]
