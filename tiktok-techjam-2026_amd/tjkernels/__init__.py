"""tjkernels -- MI355X-native (gfx950) fused Transformer forward.

Drop-in for the TechJam 2026 ``UserOptimizedTransformer`` hook
(torch_transformer_benchmark.py:182-204)::

    import tjkernels
    class UserOptimizedTransformer(BaselineTransformer):
        def forward(self, x, valid_token_mask=None):
            return tjkernels.forward(self, x, valid_token_mask)

Same public names as the reference package (tjkernels/__init__.py:16-19).
The engine reads the module's own parameters, so the harness's strict
``load_state_dict`` weight copy keeps working.  All compute runs in
hand-written HIP kernels from ``libtjk.so``; there is no CPU or torch
fallback.
"""

from .engine import forward, get_engine, reset_engines
from .modules import TransformerConfig, UserOptimizedTransformer
from .plans import Plan, select_plan

__all__ = ["forward", "get_engine", "reset_engines", "Plan", "select_plan",
           "TransformerConfig", "UserOptimizedTransformer"]
