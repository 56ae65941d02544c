"""MI355X (gfx950) implementation of router-ia's stateful hybrid-attention path.

Module names mirror the reference package (v2/src/router_ia) so callers of
``router_ia.qwen36_attention_cache`` switch by putting this directory's parent
(``router-ia_amd/``) first on ``sys.path``.  The arithmetic runs in the HIP
library built from ``router-ia_amd/csrc`` and bound in ``_native``.
"""

__all__ = ["qwen36_attention_cache", "batched_state", "kernels"]
