"""MI355X-native deterministic fixed-point reductions for vLLM.

Importing the package registers the torch.ops.fxpr.* operators (HIP kernels
behind a C ABI, libfxpr_hip.so) and their fake impls, as importing the
reference package does (fxpr_vllm/__init__.py:1-2).
"""

from . import _lib  # noqa: F401
from . import library_ops  # noqa: F401
