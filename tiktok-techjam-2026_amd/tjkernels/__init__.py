"""MI355X (gfx950) implementation of the TechJam 2026 Transformer forward.

The harness swaps its baseline module for ``UserOptimizedTransformer``
(torch_transformer_benchmark.py:182-204); that hook only has to hand its
input to :func:`forward`, which looks up (or builds) the engine for the
module and runs it on the caller's stream.  The engine takes the weights
from the module's parameters at build time, so a module filled by the
harness's strict ``load_state_dict`` needs no extra step.

Every operation of the forward -- LayerNorm, the four projections, the
feed-forward block and attention -- is a HIP kernel of ``libtjk.so``
reached through the C-ABI in ``include/tjk.h``.  Shapes or tensors the
kernels do not take raise an error; nothing falls back to torch or to the
CPU.

Exported names follow the reference package (tjkernels/__init__.py:16-19):
``forward``, ``get_engine``, ``reset_engines``, ``Plan`` and
``select_plan``, plus the module and config classes the hook is built from.
"""

from .engine import forward, get_engine, reset_engines
from .modules import TransformerConfig, UserOptimizedTransformer
from .plans import Plan, select_plan

__all__ = ["forward", "get_engine", "reset_engines", "Plan", "select_plan",
           "TransformerConfig", "UserOptimizedTransformer"]
